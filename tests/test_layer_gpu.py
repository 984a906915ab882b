"""Decoder-layer segments on the GPU against the oracle's composition: layer_pre and layer_post bit for
bit (gated and ungated, full and compact H256), layer_gdn's pre part and post part bit for bit and its
GDN core within the float64 bound. Reference tests mirrored: tests/test_layer_post.py."""
import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits
from oracle import ref
from test_w4a8_gpu import random_w4, s_f32

pytestmark = pytest.mark.gpu


def _mats(g, shapes, fmt, dev, tiled):
    from mdx import layout
    ws = [random_w4(N, K, g, fmt) for N, K in shapes]
    cb = ws[0][3]
    args, dicts = [], []
    for q, s, c, _, G in ws:
        dicts.append(dict(packed=q.numpy(), s=s_f32(s), sch=c.numpy(), cb=None if cb is None else cb.numpy(), G=G))
        qq = layout.tile_major_codes(q) if tiled else q
        cbt = cb if cb is not None else torch.arange(-8, 8, dtype=torch.float32)
        args += [qq.to(dev), s.to(dev), c.to(dev), cbt.to(dev)]
    return args, dicts


@pytest.mark.parametrize("fmt,tiled", [("fp8g16", True), ("gptq", False)])
def test_layer_pre_matches_oracle(C, dev, fmt, tiled):
    from mdx import layout
    g = torch.Generator().manual_seed(50)
    args, dicts = _mats(g, [(8192, 4096), (1024, 4096), (1024, 4096)], fmt, dev, tiled)
    h = layout.regular_hadamard()
    nw = (1 + torch.randn(4096, generator=g) * 0.05).bfloat16()
    for R in (1, 8, 16):
        print(f"case layer_pre fmt={fmt} R={R}", flush=True)
        x = torch.randn(R, 4096, generator=g).bfloat16()
        outs = C.layer_pre(x.to(dev), nw.to(dev), 1e-6, h.to(dev), args, 0, tiled)
        xn, want = ref.layer_pre(bits(x), bits(nw), 1e-6, "h256", bits(h), dicts)
        assert_bits_equal(bits(outs[0]), xn, "xn")
        for i, w in enumerate(want):
            assert_bits_equal(bits(outs[1 + i]), w, f"out {i}")


@pytest.mark.parametrize("gated,compact", [(True, False), (False, False), (True, True)])
def test_layer_post_matches_oracle(C, dev, gated, compact):
    from mdx import layout
    g = torch.Generator().manual_seed(51 + 2 * gated + compact)
    args, dicts = _mats(g, [(4096, 4096), (12288, 4096), (12288, 4096), (4096, 12288)], "fp8g16", dev, True)
    h = layout.regular_hadamard()
    sig = torch.sigmoid(layout.bf16_all()).contiguous()
    lut = layout.silu_lut()
    nw = (1 + torch.randn(4096, generator=g) * 0.05).bfloat16()
    hd = h.to(dev)
    if compact:
        hd = torch.stack((hd[:16, :16], -hd[:16, :16])).contiguous()
    for R in (1, 8, 16):
        print(f"case layer_post gated={gated} compact={compact} R={R}", flush=True)
        x = torch.randn(R, 4096, generator=g).bfloat16()
        y = torch.randn(R, 4096, generator=g).bfloat16()
        qout = torch.randn(R, 8192, generator=g).bfloat16() if gated else None
        xd = x.to(dev)
        fn = C.layer_post_h16 if compact else C.layer_post
        out = fn(xd, y.to(dev), None if qout is None else qout.to(dev), sig.to(dev), *args[:4], nw.to(dev), 1e-6, hd,
                 lut.to(dev), *args[4:], 0, 6, True)
        assert out.data_ptr() == xd.data_ptr()
        gate = None if qout is None else ref.interleaved_gate(bits(qout))
        want, _ = ref.layer_post(bits(x), bits(y), gate, bits(sig), dicts[0], bits(nw), 1e-6, "h256", bits(h),
                                 bits(lut), *dicts[1:])
        assert_bits_equal(bits(xd), want, f"x R={R}")


@pytest.mark.parametrize("widths", [(4, 3), ()])
def test_layer_gdn_matches_oracle(C, dev, widths):
    from mdx import layout
    print(f"case layer_gdn widths={widths}", flush=True)
    g = torch.Generator().manual_seed(52 + len(widths))
    HK, HV, DH = 16, 32, 128
    NCH = 2 * HK * DH + HV * DH
    shapes = [(NCH, 4096), (4096, 4096), (4096, 4096), (12288, 4096), (12288, 4096), (4096, 12288)]
    args, dicts = _mats(g, shapes, "gptq", dev, True)
    h = layout.regular_hadamard()
    lut = layout.silu_lut()
    rng = np.random.default_rng(52)
    bfn = lambda a: ref.bf16_to_f32(ref.f32_to_bf16(np.asarray(a, np.float32)))
    wa = (torch.randn(HV, 4096, generator=g) * 0.02).bfloat16()
    wb = (torch.randn(HV, 4096, generator=g) * 0.02).bfloat16()
    conv_w = bfn(rng.standard_normal((NCH, 4)) * 0.5)
    dt_bias = rng.uniform(-1, 1, HV).astype(np.float32)
    g_decay = (-np.exp(rng.uniform(-1, 0.5, HV))).astype(np.float32)
    gnw = bfn(1 + rng.standard_normal(DH) * 0.1)
    nin = (1 + torch.randn(4096, generator=g) * 0.05).bfloat16()
    npo = (1 + torch.randn(4096, generator=g) * 0.05).bfloat16()
    slots, R = 8, 1 + sum(widths)
    parents = ref.tree_from_spec(ref.spec_of_widths(widths), slots)[0][:R]
    ctl = ([0, 0] + [0] * slots + parents + [-1] * (slots - R) + ref.verify_program(parents, R)
           + [0] * (slots - R))
    st = dict(conv_state=bfn(rng.standard_normal((NCH, 3))), pb=np.zeros((2, slots, NCH), np.float32),
              qb=np.zeros((2, slots, NCH), np.float32), rec=(rng.standard_normal((HV, DH, DH)) * 0.1).astype(np.float32),
              gates=np.zeros((2, slots, HV, 2), np.float32), sums=np.zeros((2, slots, HK, 2), np.float32))
    st32 = {k: v.copy() for k, v in st.items()}
    T = lambda a, dt=torch.bfloat16: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dt).to(dev)
    dst = {k: T(v, torch.bfloat16 if k in ("conv_state", "pb", "qb") else torch.float32) for k, v in st.items()}
    x = torch.randn(R, 4096, generator=g).bfloat16()
    xd = x.to(dev)
    C.layer_gdn(xd, nin.to(dev), 1e-6, h.to(dev), args, wa.to(dev), wb.to(dev), T(conv_w), dst["conv_state"], dst["pb"],
                dst["qb"], torch.tensor(ctl, dtype=torch.int32, device=dev), T(dt_bias, torch.float32),
                T(g_decay, torch.float32), dst["rec"], dst["gates"], dst["sums"], T(gnw), 1e-6, DH ** -0.5, HK,
                npo.to(dev), 1e-6, lut.to(dev), 0, 11, True)
    # pre part (exact), then the GDN core (float64 bound)
    xn, (proj, z) = ref.layer_pre(bits(x), bits(nin), 1e-6, "h256", bits(h), dicts[:2])
    rest = (conv_w, dt_bias, g_decay, gnw, 1e-6, DH ** -0.5, np.array(ctl), R, HK, slots)
    c64 = ref.gdn_step(st, ref.bf16_to_f32(proj), ref.bf16_to_f32(z), *ref.gdn_ab(xn, bits(wa), bits(wb)), *rest)
    c32 = ref.gdn_step(st32, ref.bf16_to_f32(proj), ref.bf16_to_f32(z), *ref.gdn_ab(xn, bits(wa), bits(wb), np.float32),
                       *rest, dtype=np.float32)
    core = C.layer_gdn_core(xd, R).float().cpu().numpy()
    e_ref, err = np.abs(c32 - c64), np.abs(core - c64)
    assert err.max() <= 1.5 * e_ref.max() + 1e-3 and err.mean() <= 1.5 * e_ref.mean() + 1e-5
    # post part from the GPU's own core (exact)
    want, _ = ref.layer_post(bits(x), bits(C.layer_gdn_core(xd, R)), None, None, dicts[2], bits(npo), 1e-6, "h256",
                             bits(h), bits(lut), *dicts[3:])
    assert_bits_equal(bits(xd), want, "x after the layer")
