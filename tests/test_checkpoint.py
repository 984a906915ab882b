"""On-disk W4A8 checkpoints (mdx/checkpoint.py) on the CPU, against the committed fixture
tests/golden/checkpoint_small.safetensors (written by tests/golden/make_checkpoint_fixture.py):

- the GPTQ word unpacking against a brute-force bit loop;
- every GPTQ linear packed into the contract keeps its codes exactly (code - 8 = the signed weight
  code) and its dequantised weights within the contract's rounding (the reference's A1 map: w8 =
  rint(q * s_rel), s_rel an fp16 ratio: |w8 * s_channel - q * s_g| <= (1/2 + 127 / 2048) s_channel);
- comfy-kitchen W4A8 tensors pass through bit for bit (only the codes are permuted tile-major);
- each ineligible linear is reported with the reason of the check it fails (act-order groups,
  asymmetric zeros, a bias, a negative fp8 scale), the dense tensor is not packed;
- the per-model plan: the fixture's two layers route whole under a matching shape config; a wrong
  intermediate size or a layer past the depth is reported."""
import os

import numpy as np
import pytest
import torch

from oracle import ref

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "checkpoint_small.safetensors")


def _ckpt():
    from mdx import checkpoint
    return checkpoint.Checkpoint(FIX)


def test_unpack_int32_nibbles_brute_force():
    from mdx import checkpoint
    g = torch.Generator().manual_seed(1)
    w = torch.randint(-2 ** 31, 2 ** 31 - 1, (3, 5), generator=g, dtype=torch.int64).to(torch.int32)
    rows = checkpoint.unpack_int32_nibbles(w, 0)
    cols = checkpoint.unpack_int32_nibbles(w, 1)
    for i in range(3):
        for n in range(5):
            u = int(w[i, n]) & 0xFFFFFFFF
            for j in range(8):
                nib = (u >> (4 * j)) & 15
                assert rows[8 * i + j, n] == nib and cols[i, 8 * n + j] == nib


def test_scan_and_fallback_reasons():
    ck = _ckpt()
    weights, rep = ck.load(tiled=False)
    f = rep.formats
    assert f["lm_head"] == "dense" and f["w4a8.a"] == "w4a8" and f["model.layers.0.mlp.down_proj"] == "gptq"
    assert rep.fallback == {"extra.act_order": "g_idx", "extra.asym": "zeros", "w4a8.bias": "bias",
                            "w4a8.bad_scale": "scale"}
    assert "lm_head" not in weights and set(weights) == set(rep.packed)
    assert len(rep.packed) == 13 + 1 + 2  # two layers, the extra layer 5 linear, two W4A8 linears


def _gptq_dense(ck, p):
    """Codes [N, K] (0..15) and the GPTQ dequantised weights (float64) of a fixture linear, by loops over
    the stored words (independent of the reader)."""
    qw = ck.tensor(p + ".qweight").to(torch.int64) & 0xFFFFFFFF
    K8, N = qw.shape
    codes = torch.empty(K8 * 8, N, dtype=torch.int64)
    for j in range(8):
        codes[j::8] = (qw >> (4 * j)) & 15
    s = ck.tensor(p + ".scales").double()
    G = K8 * 8 // s.shape[0]
    w = (codes - 8).double() * s.repeat_interleave(G, 0)
    return codes.t(), w.t(), G


@pytest.mark.parametrize("integral", [False, True])
def test_gptq_linears_keep_codes_and_scales(integral):
    from mdx import layout
    ck = _ckpt()
    for p, fmt in ck.linears().items():
        if fmt != "gptq" or p.startswith("extra"):
            continue
        w = ck.w4(p, tiled=False, integral=integral)
        codes, dense, G = _gptq_dense(ck, p)
        assert torch.equal(layout.unpack_codes(w.q).to(torch.int64), codes), p
        assert w.group_size == G
        w8 = ref.decode_w8(w.q.numpy(), w.s.float().numpy(), None, G).astype(np.float64)
        sch = w.sc.double().numpy()[:, None]
        err = np.abs(w8 * sch - dense.numpy())
        if integral:
            # s_rel = round(s_g / (smax / 15)): the group scale moves by at most smax / 30 per unit code
            smax = ck.tensor(p + ".scales").double().amax(0).numpy()[:, None]
            assert (err <= 8 * smax / 30 + 1e-12).all(), p
        else:
            # rint of q * s_rel (half a unit) plus s_rel's fp16 rounding (2^-11 relative, |q| s_rel <= 127)
            assert (err <= sch * (0.5 + 127 / 2048) * (1 + 1e-6)).all(), p


def test_w4a8_linears_pass_through_bit_for_bit():
    from mdx import layout
    ck = _ckpt()
    for p in ("w4a8.a", "w4a8.b"):
        w = ck.w4(p)  # tile-major
        assert torch.equal(layout.row_major_codes(w.q), ck.tensor(p + ".weight"))
        assert torch.equal(w.s.view(torch.uint8), ck.tensor(p + ".weight_scale").view(torch.uint8))
        assert torch.equal(w.sc, ck.tensor(p + ".s_channel")) and torch.equal(w.cb, ck.tensor(p + ".codebook"))
        assert w.group_size == 16


def test_live_quantized_tensor_and_int8_head_checks():
    from mdx import checkpoint
    ck = _ckpt()

    class P:
        scale = ck.tensor("w4a8.a.weight_scale")
        s_channel = ck.tensor("w4a8.a.s_channel")
        codebook = ck.tensor("w4a8.a.codebook")
        group_size, convrot_groupsize, mma_packed, transposed, correction = 16, 256, False, False, None

    class QT:
        _qdata = ck.tensor("w4a8.a.weight")
        _params = P()

    w = checkpoint.w4_from_quantized(QT(), tiled=False)
    assert torch.equal(w.q, QT._qdata)
    P.mma_packed = True
    with pytest.raises(checkpoint.Ineligible) as e:
        checkpoint.w4_from_quantized(QT())
    assert e.value.reason == "layout"
    q = torch.randint(-127, 128, (32, 512), dtype=torch.int8)
    s = torch.rand(32)
    w8, s8 = checkpoint.int8_head_from_tensorwise(q, s)
    assert torch.equal(s8, s) and w8.shape == q.shape
    with pytest.raises(checkpoint.Ineligible):
        checkpoint.int8_head_from_tensorwise(q, s, convrot=False)


def test_plan_hybrid_routes_whole_layers():
    from mdx import checkpoint, hybrid
    ck = _ckpt()
    _, rep = ck.load(tiled=False)
    cfg = hybrid.HybridConfig(layers=2, hidden=256, inter=256, heads=2, kv_heads=1, head_dim=128, gdn_key_heads=1,
                              gdn_value_heads=2, attn_every=2)
    plan, bad = checkpoint.plan_hybrid(rep, cfg)
    assert sorted(plan) == [0, 1]
    assert plan[0] == {"g": "model.layers.0.mlp.gate_proj", "u": "model.layers.0.mlp.up_proj",
                       "d": "model.layers.0.mlp.down_proj", "qkv": "model.layers.0.linear_attn.in_proj_qkv",
                       "z": "model.layers.0.linear_attn.in_proj_z", "o": "model.layers.0.linear_attn.out_proj"}
    assert set(plan[1]) == {"g", "u", "d", "q", "k", "v", "o"}
    assert bad == {"model.layers.5.mlp.gate_proj": "layer"}
    cfg.inter = 512
    plan, bad = checkpoint.plan_hybrid(rep, cfg)
    assert plan == {} and bad["model.layers.0.mlp.down_proj"] == "shape" and bad["model.layers.1.mlp.up_proj"] == "shape"
