"""Pins of the CPU oracle (oracle/ref.py) against independent implementations, closed forms and
exact arithmetic, plus the host-side layout / packing helpers. CPU only."""
import numpy as np
import pytest
import torch

from oracle import ref


def test_bf16_rounding_matches_torch():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(200000, generator=g) * torch.exp(torch.randn(200000, generator=g) * 6)
    x[:7] = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), 1e-40, -3e-39, 3.4e38])
    want = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ref.f32_to_bf16(x.numpy()), want)
    # round trip of every bf16 pattern except NaNs
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = ref.bf16_to_f32(allb)
    ok = ~np.isnan(f)
    assert np.array_equal(ref.f32_to_bf16(f)[ok], allb[ok])
    assert (ref.f32_to_bf16(f[~ok]) == 0x7FC0).all()


def test_fp8_and_fp16_decode_match_torch():
    allb = np.arange(256, dtype=np.uint8)
    f = ref.fp8e4m3_to_f32(allb)
    tf = torch.from_numpy(allb).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(f), np.isnan(tf)) and np.array_equal(f[~np.isnan(f)], tf[~np.isnan(tf)])
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    a = ref.scales_to_f32(h, "f16")
    b = torch.from_numpy(h.view(np.int16)).view(torch.float16).float().numpy()
    assert np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)])


def _packed(codes):
    codes = np.asarray(codes, dtype=np.int64)
    return (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8).view(np.int8)


def test_decode_closed_forms():
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 16, size=(32, 256))
    # integral scales, default codebook: w8 = (code - 8) * s exactly
    s = rng.integers(-15, 16, size=(32, 2)).astype(np.float32)
    w8 = ref.decode_w8(_packed(codes), s, None, 128)
    assert np.array_equal(w8, (codes - 8) * np.repeat(s, 128, axis=1).astype(np.int64))
    # half-even ties: (code - 8) * 0.5
    half = np.full((1, 1), 0.5, np.float32)
    c = np.array([[8 + 1, 8 + 3, 8 - 1, 8 - 3, 8 + 5, 8 - 5, 8 + 7, 8]])
    c = np.tile(c, (1, 16))
    got = ref.decode_w8(_packed(c), half, None, 128)[0, :8]
    assert got.tolist() == [0, 2, 0, -2, 2, -2, 4, 0]
    # clamp at +-127, NaN -> 0, inf * 0 = NaN -> 0
    big = np.full((1, 1), 100.0, np.float32)
    c2 = np.tile(np.array([[15, 0, 9, 8]]), (1, 32))
    assert ref.decode_w8(_packed(c2), big, None, 128)[0, :4].tolist() == [127, -127, 100, 0]
    nan = np.full((1, 1), np.nan, np.float32)
    assert (ref.decode_w8(_packed(c2), nan, None, 128) == 0).all()
    inf = np.full((1, 1), np.inf, np.float32)
    assert ref.decode_w8(_packed(c2), inf, None, 128)[0, :4].tolist() == [127, -127, 127, 0]
    # a general codebook, G16: one float32 product, then rint
    cb = rng.standard_normal(16).astype(np.float32)
    s16 = (rng.random((32, 16)) * 20).astype(np.float32)
    w8 = ref.decode_w8(_packed(codes), s16, cb, 16)
    brute = np.array([[np.clip(np.rint(np.float32(cb[codes[n, k]]) * np.float32(s16[n, k // 16])), -127, 127)
                       for k in range(256)] for n in range(4)])
    assert np.array_equal(w8[:4], brute)


def test_int32_accumulator_float64_path_is_exact():
    rng = np.random.default_rng(2)
    x = rng.integers(-128, 128, size=(8, 12288))
    w8 = rng.integers(-127, 128, size=(64, 12288))
    assert np.array_equal(ref.w4a8_acc(x, w8), ref.w4a8_acc_int64(x, w8))
    # wrap-around modulo 2^32
    assert ref.int32_wrap(2 ** 31) == -2 ** 31 and ref.int32_wrap(-2 ** 31 - 1) == 2 ** 31 - 1


def test_epilogue_matches_torch_ops():
    rng = np.random.default_rng(3)
    acc = rng.integers(-2 ** 24, 2 ** 24, size=(4, 512))
    xs = (rng.random(4) * 0.05 + 1e-3).astype(np.float32)
    sch = (rng.random(512) * 1e-3 + 1e-4).astype(np.float32)
    f = (torch.from_numpy(acc).float() * torch.from_numpy(xs)[:, None]) * torch.from_numpy(sch)[None, :]
    assert np.array_equal(ref.scaleback(acc, xs, sch), f.numpy())
    want = f.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ref.f32_to_bf16(ref.scaleback(acc, xs, sch)), want)


def _kron256():
    h = ref.H4
    for _ in range(3):
        h = np.kron(h, ref.H4)
    return h


def test_fwht_equals_exact_kronecker_product():
    rng = np.random.default_rng(4)
    # bf16 values scaled to integers: the fp64 transform must be exact
    x = ref.bfround(rng.standard_normal((4, 256)).astype(np.float32) * 3)
    xi = (x.astype(np.float64) * 2 ** 20).astype(np.int64)
    assert np.array_equal(xi.astype(np.float64), x.astype(np.float64) * 2 ** 20)
    exact = xi @ _kron256()
    got = ref.fwht256_f64(x.astype(np.float64)) * 2 ** 20
    assert np.array_equal(got, exact.astype(np.float64))
    h = _kron256()
    assert np.array_equal(h @ h, 256 * np.eye(256, dtype=np.int64))  # H256 / 16 is orthogonal


def test_rotation_modes_agree():
    rng = np.random.default_rng(5)
    x = ref.bfround(rng.standard_normal((3, 1024)).astype(np.float32))
    hb = ref.f32_to_bf16((_kron256() / 16).astype(np.float32))
    assert np.array_equal(ref.rotate_rows(x, "h256"), ref.rotate_rows(x, "matrix", hb))
    eye = ref.f32_to_bf16(np.eye(256, dtype=np.float32))
    assert np.array_equal(ref.rotate_rows(x, "matrix", eye), ref.rotate_rows(x, "none"))


def test_quantize_matches_torch_restatement():
    g = torch.Generator().manual_seed(6)
    for kind in ("normal", "outlier", "wide", "tiny", "zero"):
        x = torch.randn(5, 4096, generator=g)
        if kind == "outlier":
            x[:, torch.randint(0, 4096, (8,), generator=g)] *= 300
        if kind == "wide":
            x = x * torch.exp(torch.randn(5, 4096, generator=g) * 3)
        if kind == "tiny":
            x = x * 1e-36
        if kind == "zero":
            x = x * 0
        xr = x.to(torch.bfloat16).float()
        amax = xr.abs().amax(dim=1)
        scale = torch.clamp(amax / 127.0, min=1e-30)
        sb = scale.to(torch.bfloat16)
        sb = torch.where(sb == 0, torch.tensor(2.0 ** -126).to(torch.bfloat16), sb).float()
        q = torch.clamp(torch.round((xr / sb[:, None]).to(torch.bfloat16).float()), -128, 127).to(torch.int8)
        gq, gs = ref.quantize_rows(xr.numpy())
        assert np.array_equal(gq, q.numpy()), kind
        assert np.array_equal(gs, scale.numpy()), kind


def test_rmsnorm_within_fp64_tolerance():
    rng = np.random.default_rng(7)
    x = ref.f32_to_bf16(rng.standard_normal((4, 4096)).astype(np.float32))
    w = ref.f32_to_bf16((1 + rng.standard_normal(4096) * 0.02).astype(np.float32))
    got = ref.bf16_to_f32(ref.rmsnorm(x, w, 1e-6)).astype(np.float64)
    xf = ref.bf16_to_f32(x).astype(np.float64)
    want = xf / np.sqrt((xf * xf).mean(axis=1, keepdims=True) + 1e-6) * ref.bf16_to_f32(w)
    rel = np.abs(got - want) / np.maximum(np.abs(want), 1e-3)
    assert rel.max() <= 1e-2


def test_silu_table_close_to_float64():
    from mdx.layout import silu_lut
    lut = silu_lut().view(torch.int16).numpy().view(np.uint16)
    got = ref.bf16_to_f32(lut).astype(np.float64)
    want = ref.silu_lut_f64()
    fin = np.isfinite(want) & (np.abs(want) > 1e-30)
    assert (np.abs(got[fin] - want[fin]) <= np.abs(want[fin]) * 2 ** -7).all()


def test_tile_major_layout_invariants():
    from mdx import layout
    g = torch.Generator().manual_seed(8)
    q = torch.randint(-128, 128, (64, 512), generator=g, dtype=torch.int8)
    t = layout.tile_major_codes(q)
    assert t.shape == q.shape
    assert torch.equal(layout.row_major_codes(t), q)
    codes = layout.unpack_codes(q)  # [64, 1024] in k order
    # tile 1, chunk 2: piece (kq, c) holds column 16 + c's codes of k = 256 + 32 kq + [0, 32), each
    # 4-byte word w (k = 8 w + [0, 8)) with k 0..3 in its low nibbles and k 4..7 in its high nibbles
    nc = 1024 // 128
    blk = t.flatten().view(torch.uint8)[(1 * nc + 2) * 1024:(1 * nc + 3) * 1024].view(4, 16, 4, 4).to(torch.int32)
    for kq in range(4):
        for c in range(16):
            for w in range(4):
                k = 256 + 32 * kq + 8 * w
                want = codes[16 + c, k:k + 8]
                got = torch.cat([blk[kq, c, w] & 15, blk[kq, c, w] >> 4])
                assert torch.equal(got, want), (kq, c, w)


def test_gptq_packer_error_bound():
    from mdx import layout
    g = torch.Generator().manual_seed(9)
    N, K, G = 64, 1024, 128
    q = torch.randint(-8, 8, (N, K), generator=g)
    s = (torch.rand(N, K // G, generator=g) * 0.015 + 0.005).half()
    w_true = q.double() * s.double().repeat_interleave(G, dim=1)
    for integral in (True, False):
        packed, s_rel, sch, cb = layout.gptq_pack(q, s, G, integral=integral)
        w8 = ref.decode_w8(packed.numpy(), s_rel.float().numpy(), None, G)
        assert np.abs(w8).max() <= 127
        w = torch.from_numpy(w8).double() * sch.double()[:, None]
        if integral:
            assert torch.equal(s_rel.float(), torch.round(s_rel.float()))
            assert np.array_equal(w8, (q.numpy()) * np.repeat(s_rel.float().numpy(), G, axis=1).astype(np.int64))
            # group-scale error: |s_rel * sch - s_g| <= sch / 2 (round to nearest)
            bound = 0.5 * sch.double()[:, None] * q.abs().double() + 1e-9
        else:
            bound = 0.5 * sch.double()[:, None] + 1e-3 * w_true.abs() + 1e-9
        assert ((w - w_true).abs() <= bound).all(), integral
