"""Checkpoint linears on the GPU: every eligible linear of the committed fixture
(tests/golden/checkpoint_small.safetensors: GPTQ and comfy-kitchen W4A8 forms), packed tile-major by
mdx/checkpoint.py, through the W4A8 GEMV against the oracle on the row-major contract tensors, bit for
bit; and a full-width two-layer GPTQ checkpoint (GDN + attention, hidden 4096) loaded into the hybrid
decoder, whose decode equals that of the same weights packed directly."""
import os
import sys

import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits
from oracle import ref

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
FIX = os.path.join(HERE, "golden", "checkpoint_small.safetensors")


def test_fixture_linears_through_the_gemv(C, dev):
    from mdx import checkpoint, layout
    ck = checkpoint.Checkpoint(FIX)
    tiled, rep = ck.load(device=dev)
    g = torch.Generator().manual_seed(3)
    for p in rep.packed:
        w = tiled[p]
        row = ck.w4(p, tiled=False)
        for rows in (1, 8):
            print(f"case checkpoint linear {p} rows={rows}", flush=True)
            x = torch.randint(-128, 128, (rows, w.k), generator=g, dtype=torch.int8)
            xs = torch.rand(rows, generator=g) * 0.05 + 0.01
            out = torch.empty(rows, w.n, dtype=torch.bfloat16, device=dev)
            C.stream_gemv(x.to(dev), xs.to(dev), [w], [out])
            s = row.s.view(torch.uint8).numpy() if row.s.dtype == torch.float8_e4m3fn else row.s.float().numpy()
            s_f32 = ref.fp8e4m3_to_f32(s) if row.s.dtype == torch.float8_e4m3fn else s
            want = ref.w4a8_linear(x.numpy(), xs.numpy(), row.q.numpy(), s_f32, row.sc.numpy(),
                                   None if row.cb is None else row.cb.numpy(), row.group_size)
            assert_bits_equal(bits(out), want, f"{p} rows={rows}")


def test_full_width_gptq_checkpoint_in_the_decoder(C, dev, tmp_path):
    sys.path.insert(0, os.path.join(HERE, "golden"))
    from make_checkpoint_fixture import pack_int32
    from safetensors.torch import save_file
    from mdx import _lib, checkpoint, hybrid, layout
    cfg = hybrid.HybridConfig(layers=2, attn_every=2, cap=128, greedy=True)
    H, I, qd, kd = cfg.hidden, cfg.inter, cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    ch, hv = 2 * cfg.gdn_key_heads * 128 + cfg.gdn_value_heads * 128, cfg.gdn_value_heads * 128
    shapes = {"model.layers.0.linear_attn.in_proj_qkv": (ch, H), "model.layers.0.linear_attn.in_proj_z": (hv, H),
              "model.layers.0.linear_attn.out_proj": (H, hv), "model.layers.1.self_attn.q_proj": (qd, H),
              "model.layers.1.self_attn.k_proj": (kd, H), "model.layers.1.self_attn.v_proj": (kd, H),
              "model.layers.1.self_attn.o_proj": (H, qd)}
    for i in (0, 1):
        shapes.update({f"model.layers.{i}.mlp.gate_proj": (I, H), f"model.layers.{i}.mlp.up_proj": (I, H),
                       f"model.layers.{i}.mlp.down_proj": (H, I)})
    g = torch.Generator().manual_seed(8)
    t, direct = {}, {}
    for p, (N, K) in shapes.items():
        codes = torch.randint(0, 16, (K, N), generator=g)
        scales = (torch.rand(K // 128, N, generator=g) * 0.015 + 0.005).half()
        t[p + ".qweight"] = pack_int32(codes, 0)
        t[p + ".qzeros"] = pack_int32(torch.full((K // 128, N), 7), 1)
        t[p + ".scales"] = scales
        t[p + ".g_idx"] = torch.arange(K, dtype=torch.int32) // 128
        packed, s_rel, sch, _ = layout.gptq_pack((codes.t() - 8).to(torch.int8), scales.t().contiguous(), 128,
                                                 integral=False)
        direct[p] = layout.W4(layout.tile_major_codes(packed).to(dev), s_rel.to(dev), sch.to(dev), None,
                              _lib.LAYOUT_TILE, _lib.DECODE_AUTO)
    path = str(tmp_path / "w4_gptq_2layer.safetensors")
    save_file(t, path, metadata={"bits": "4", "group_size": "128", "sym": "true", "checkpoint_format": "gptq"})
    del t
    print("case full-width checkpoint load", flush=True)
    ck = checkpoint.Checkpoint(path)
    weights, rep = ck.load(device=dev)
    assert rep.fallback == {} and len(rep.packed) == len(shapes)
    plan, bad = checkpoint.plan_hybrid(rep, cfg)
    assert bad == {} and sorted(plan) == [0, 1]
    for p, w in weights.items():
        d = direct[p]
        assert torch.equal(w.q, d.q) and torch.equal(w.s, d.s) and torch.equal(w.sc, d.sc), p
    ms = []
    for src in ("checkpoint", "direct"):
        m = hybrid.HybridModel(cfg, dev, seed=12)
        if src == "checkpoint":
            m.load_w4(weights, plan)
        else:
            m.load_w4(direct, plan)
        m.prefill(torch.randint(0, cfg.vocab, (20,), generator=torch.Generator().manual_seed(6)))
        ms.append(m)
    for step in range(2):
        print(f"case full-width checkpoint step {step}", flush=True)
        for m in ms:
            m.step(m.parity)
            m.parity ^= 1
        torch.cuda.synchronize()
        a, b = ms
        assert torch.isfinite(a.logits.float()).all()
        assert torch.equal(a.result, b.result) and torch.equal(a.hbuf, b.hbuf) and torch.equal(a.logits, b.logits)
