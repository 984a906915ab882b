"""W4A8 linear, rot_quant and the fused MLP on the GPU against the CPU oracle: int8 / int32-derived
outputs bit for bit (bf16 outputs are bf16 roundings of bit-exact fp32 epilogues, so they are
compared bit for bit too). Reference tests mirrored: tests/test_w4a8_linear.py,
tests/test_rot_quant.py, tests/test_mono_mlp.py."""
import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits
from oracle import ref

pytestmark = pytest.mark.gpu


def random_w4(N, K, g, fmt):
    """Packed W4 weights in one of the scale formats:
    fp8g16   -- the reference checkpoint format (tests/test_w4a8_linear.py:9-16): random bytes,
                fp8 e4m3 G16 scale bytes 0x18..0x57, codebook i - 8
    gptq     -- GPTQ int4 / fp16 G128 scales ~U(0.005, 0.02) through the integral packer
    gptq_rint-- the same through the non-integral packer (per-weight rint decode)
    f32g32   -- float32 G32 scales with a random codebook (general decode)"""
    from mdx import layout
    if fmt == "fp8g16":
        q = torch.randint(-128, 128, (N, K // 2), generator=g, dtype=torch.int8)
        s = torch.randint(0x18, 0x58, (N, K // 16), generator=g, dtype=torch.uint8).view(torch.float8_e4m3fn)
        c = torch.rand(N, generator=g) * 1e-3 + 1e-4
        cb = torch.arange(-8, 8, dtype=torch.float32)
        return q, s, c, cb, 16
    if fmt in ("gptq", "gptq_rint"):
        qi = torch.randint(-8, 8, (N, K), generator=g)
        sg = (torch.rand(N, K // 128, generator=g) * 0.015 + 0.005).half()
        packed, s_rel, sch, _ = layout.gptq_pack(qi, sg, 128, integral=fmt == "gptq")
        return packed, s_rel, sch, None, 128
    if fmt == "f32g32":
        q = torch.randint(-128, 128, (N, K // 2), generator=g, dtype=torch.int8)
        s = torch.rand(N, K // 32, generator=g) * 30
        c = torch.rand(N, generator=g) * 1e-3 + 1e-4
        cb = torch.randn(16, generator=g)
        return q, s, c, cb, 32
    raise ValueError(fmt)


def s_f32(s):
    if s.dtype == torch.float8_e4m3fn:
        return ref.fp8e4m3_to_f32(s.view(torch.uint8).numpy())
    return s.float().numpy()


def oracle_linear(x, xs, w, residual=None, out="bf16"):
    q, s, c, cb, G = w
    return ref.w4a8_linear(x.numpy(), xs.numpy(), q.numpy(), s_f32(s), c.numpy(),
                           None if cb is None else cb.numpy(), G,
                           None if residual is None else bits(residual), out)


@pytest.mark.parametrize("N,K", [(4096, 4096), (12288, 4096), (4096, 12288)])
@pytest.mark.parametrize("fmt", ["fp8g16", "gptq", "gptq_rint", "f32g32"])
def test_w4a8_decode_linear_matches_oracle(C, dev, N, K, fmt):
    g = torch.Generator().manual_seed(N + K + len(fmt))
    w = random_w4(N, K, g, fmt)
    wd = [t.to(dev) if t is not None else None for t in w[:4]]
    for M in (1, 2, 3, 8, 16):
        print(f"case N={N} K={K} fmt={fmt} M={M}", flush=True)
        x = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
        xs = torch.rand(M, generator=g) * 0.05 + 1e-3
        out = C.w4a8_decode_linear(x.to(dev), xs.to(dev), *wd, None, w[4], 2, 0, False)
        assert_bits_equal(bits(out), oracle_linear(x, xs, w), f"{fmt} M={M}")


@pytest.mark.parametrize("fmt", ["fp8g16", "gptq", "gptq_rint"])
def test_w4a8_residual_and_f32_out(C, dev, fmt):
    g = torch.Generator().manual_seed(11)
    N, K = 1024, 4096
    w = random_w4(N, K, g, fmt)
    wd = [t.to(dev) if t is not None else None for t in w[:4]]
    for M in (1, 5):
        x = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
        xs = torch.rand(M, generator=g) * 0.05 + 1e-3
        res = torch.randn(M, N, generator=g).to(torch.bfloat16)
        out = C.w4a8_decode_linear(x.to(dev), xs.to(dev), *wd, res.to(dev), w[4], 2, 0, False)
        assert_bits_equal(bits(out), oracle_linear(x, xs, w, res), "bf16 residual")
        out32 = C.w4a8_decode_linear(x.to(dev), xs.to(dev), *wd, None, w[4], 0, 0, False)
        assert_bits_equal(bits(out32), oracle_linear(x, xs, w, None, "f32").view(np.uint32), "f32 out")


@pytest.mark.parametrize("fmt", ["gptq", "gptq_rint"])
@pytest.mark.parametrize("tpw,ks", [(3, 4), (5, 2), (6, 1)])
def test_w4a8_geometry_with_idle_tile_slots(C, dev, tpw, ks, monkeypatch, fmt):
    """Work-group geometries whose last work-group has tile slots past the matrix (256 tiles in
    groups of 3, 5, 6): the idle slots read inside the matrix and add nothing; every output equals
    the oracle's. (Regression: the idle slots once formed their weight addresses past the end.)"""
    g = torch.Generator().manual_seed(29 + tpw)
    N, K = 4096, 4096
    w = random_w4(N, K, g, fmt)
    wd = [t.to(dev) if t is not None else None for t in w[:4]]
    monkeypatch.setenv("MDX_GEMV_TPW", str(tpw))
    monkeypatch.setenv("MDX_GEMV_KS", str(ks))
    for M in (1, 8):
        print(f"case idle slots fmt={fmt} tpw={tpw} ks={ks} M={M}", flush=True)
        x = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
        xs = torch.rand(M, generator=g) * 0.05 + 1e-3
        out = C.w4a8_decode_linear(x.to(dev), xs.to(dev), *wd, None, w[4], 2, 0, False)
        assert_bits_equal(bits(out), oracle_linear(x, xs, w), f"tpw={tpw} ks={ks} M={M}")


def test_w4a8_rejects_bad_contracts(C, dev):
    x = torch.zeros(1, 4096, dtype=torch.int8, device=dev)
    xs = torch.ones(1, device=dev)
    q = torch.zeros(64, 2048, dtype=torch.int8, device=dev)
    s = torch.ones(64, 256, device=dev)
    c = torch.ones(64, device=dev)
    with pytest.raises(RuntimeError):
        C.w4a8_decode_linear(torch.zeros(17, 4096, dtype=torch.int8, device=dev), xs, q, s, c, None, None, 16)
    with pytest.raises(RuntimeError):
        C.w4a8_decode_linear(x, xs, q, s, c, None, None, 32)  # group size disagrees with the scales
    with pytest.raises(RuntimeError):
        C.w4a8_decode_linear(x, xs, q[:, :1000], s, c, None, None, 16)


def _rows(kind, M, K, g):
    x = torch.randn(M, K, generator=g)
    if kind == "outlier":
        x[:, torch.randint(0, K, (8,), generator=g)] *= 300
    if kind == "wide":
        x = x * torch.exp(torch.randn(M, K, generator=g) * 3)
    if kind == "tiny":
        x = x * 1e-36
    if kind == "zero":
        x = x * 0
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("K", [4096, 12288])
@pytest.mark.parametrize("rot", ["h256", "none", "matrix"])
def test_rot_quant_matches_oracle(C, dev, K, rot):
    from mdx import layout
    g = torch.Generator().manual_seed(K + len(rot))
    if rot == "h256":
        h = layout.regular_hadamard()
    elif rot == "none":
        h = torch.eye(256).to(torch.bfloat16)
    else:
        h = (torch.randn(256, 256, generator=g) / 16).to(torch.bfloat16)
    hd = h.to(dev)
    for M in (1, 3, 8):
        for kind in ("normal", "outlier", "wide", "tiny", "zero"):
            print(f"case K={K} rot={rot} M={M} kind={kind}", flush=True)
            x = _rows(kind, M, K, g)
            q, s = C.rot_quant(x.to(dev), hd, 3)
            wq, ws = ref.rot_quant(bits(x), "none" if rot == "none" else rot, bits(h))
            assert_bits_equal(bits(q), wq, f"q {kind}")
            assert_bits_equal(bits(s.view(-1)), ws.view(np.uint32), f"scale {kind}")


def _mlp_weights(g, fmt, dev, tiled):
    from mdx import layout
    ws = [random_w4(12288, 4096, g, fmt), random_w4(12288, 4096, g, fmt), random_w4(4096, 12288, g, fmt)]
    cb = ws[0][3]
    ws = [(q, s, c, cb, G) for q, s, c, _, G in ws]
    args = []
    for q, s, c, cbv, G in ws:
        if tiled:
            q = layout.tile_major_codes(q)
        cbt = cbv if cbv is not None else torch.arange(-8, 8, dtype=torch.float32)
        args += [q.to(dev), s.to(dev), c.to(dev), cbt.to(dev)]
    return ws, args


def _oracle_dicts(ws):
    return [dict(packed=q.numpy(), s=s_f32(s), sch=c.numpy(), cb=None if cb is None else cb.numpy(), G=G)
            for q, s, c, cb, G in ws]


@pytest.mark.parametrize("fmt,tiled,rot", [("gptq", True, "none"), ("gptq", False, "h256"),
                                           ("fp8g16", True, "h256"), ("fp8g16", False, "none")])
def test_mono_mlp_matches_oracle(C, dev, fmt, tiled, rot):
    from mdx import layout
    g = torch.Generator().manual_seed(21)
    ws, args = _mlp_weights(g, fmt, dev, tiled)
    h = layout.regular_hadamard() if rot == "h256" else torch.eye(256).to(torch.bfloat16)
    lut = layout.silu_lut()
    d = _oracle_dicts(ws)
    for M in (1, 2, 3, 8, 16):  # without rotation 1 and 2 rows take the in-prologue quantisations
        print(f"case mlp fmt={fmt} tiled={tiled} rot={rot} M={M}", flush=True)
        xn = torch.randn(M, 4096, generator=g).to(torch.bfloat16)
        out = C.mono_mlp(xn.to(dev), h.to(dev), lut.to(dev), *args, 0, 4, tiled)
        want = ref.mono_mlp(bits(xn), rot, bits(h), bits(lut), *d)
        assert_bits_equal(bits(out), want, f"M={M}")


@pytest.mark.parametrize("tiled,rot", [(True, "none"), (False, "none"), (True, "h256"), (False, "h256")])
def test_mono_mlp_faithful_scales_matches_oracle(C, dev, tiled, rot):
    """The MLP block on the config's own weight format (GPTQ int4, fp16 G128 group scales kept as fp16 ratios
    to the channel scale, decoded per weight by rint: reference csrc/w4a8_decode.sycl:35-45), 1, 2, 4, 8 and
    16 rows, tile-major and row-major codes, with and without the rotation of h, against the oracle bit for
    bit (reference tests/test_mono_mlp.py:14-50). Checks the kernels taken: the table-only MFMA variants,
    at one row without rotation the gate/up with the row prep in its prologue and the down quantising h in
    its prologue (16-byte tables), at eight rows the gate/up on 8-byte tables."""
    from mdx import _lib, layout
    g = torch.Generator().manual_seed(23)
    ws, args = _mlp_weights(g, "gptq_rint", dev, tiled)
    h = layout.regular_hadamard() if rot == "h256" else torch.eye(256).to(torch.bfloat16)
    lut = layout.silu_lut()
    d = _oracle_dicts(ws)
    for M in (1, 2, 4, 8, 16):
        print(f"case faithful mlp tiled={tiled} rot={rot} M={M}", flush=True)
        xn = torch.randn(M, 4096, generator=g).to(torch.bfloat16)
        _lib.gemv_trace()
        out = C.mono_mlp(xn.to(dev), h.to(dev), lut.to(dev), *args, 0, 4, tiled)
        tr = _lib.gemv_trace()
        want = ref.mono_mlp(bits(xn), rot, bits(h), bits(lut), *d)
        assert_bits_equal(bits(out), want, f"M={M}")
        assert tr and all(t["mfma"] and t["decode"] in ("table16", "table8") for t in tr), tr
        if M == 1 and rot == "none":
            assert [(t["src"], t["decode"]) for t in tr] == [(_lib.SRC_XP, "table16"), (_lib.SRC_HR, "table16")], tr
        if M == 8:  # the gate/up pair: 16-byte tables with the partials in the table region
            assert tr[0]["decode"] == "table16" and tr[0]["tpw"] == 2 and tr[0]["red_alias"], tr


def test_mono_mlp_faithful_scales_8_byte_tables(C, dev, monkeypatch):
    """The 8-byte table tier (the default codebook's eight magnitudes, expanded per chunk), forced by
    MDX_GEMV_TBL=8 where it applies: the MLP block on fp16-ratio scales at 1, 8 and 16 rows, bit for bit."""
    from mdx import _lib, layout
    monkeypatch.setenv("MDX_GEMV_TBL", "8")
    g = torch.Generator().manual_seed(27)
    ws, args = _mlp_weights(g, "gptq_rint", dev, True)
    h = torch.eye(256).to(torch.bfloat16)
    lut = layout.silu_lut()
    d = _oracle_dicts(ws)
    for M in (1, 8, 16):
        print(f"case faithful mlp table8 M={M}", flush=True)
        xn = torch.randn(M, 4096, generator=g).to(torch.bfloat16)
        _lib.gemv_trace()
        out = C.mono_mlp(xn.to(dev), h.to(dev), lut.to(dev), *args, 0, 4, True)
        tr = _lib.gemv_trace()
        assert_bits_equal(bits(out), ref.mono_mlp(bits(xn), "none", bits(h), bits(lut), *d), f"M={M}")
        assert tr and all(t["decode"] == "table8" for t in tr), tr


@pytest.mark.parametrize("K", [4096, 12288])
def test_rms_rot_quant_matches_oracle(C, dev, K):
    from mdx import _lib, layout
    g = torch.Generator().manual_seed(K + 5)
    w = (1 + torch.randn(K, generator=g) * 0.02).to(torch.bfloat16)
    for M in (1, 3, 8):
        for kind in ("normal", "outlier", "wide", "zero"):
            print(f"case rms K={K} M={M} kind={kind}", flush=True)
            x = _rows(kind, M, K, g)
            xn = torch.empty(M, K, dtype=torch.bfloat16, device=dev)
            for rot, name in ((_lib.ROT_NONE, "none"), (_lib.ROT_H256, "h256")):
                h = layout.regular_hadamard(dev)
                q, s = C.rms_rot_quant(x.to(dev), w.to(dev), 1e-6, rot, h, xn)
                wxn = ref.rmsnorm(bits(x), bits(w), 1e-6)
                assert_bits_equal(bits(xn), wxn, f"xn {kind}")
                wq, ws = ref.rot_quant(wxn, name)
                assert_bits_equal(bits(q), wq, f"q {kind} {name}")
                assert_bits_equal(bits(s), ws.view(np.uint32), f"scale {kind} {name}")


@pytest.mark.parametrize("fmt", ["gptq", "gptq_rint"])
def test_mlp_with_norm_matches_oracle(C, dev, fmt):
    from mdx import _lib, layout
    g = torch.Generator().manual_seed(33)
    ws, _ = _mlp_weights(g, fmt, dev, True)
    handles = [layout.W4(layout.tile_major_codes(q).to(dev), s.to(dev), c.to(dev), None, _lib.LAYOUT_TILE)
               for q, s, c, _, _ in ws]
    lut = layout.silu_lut()
    nw = (1 + torch.randn(4096, generator=g) * 0.02).to(torch.bfloat16)
    d = _oracle_dicts(ws)
    for M in (1, 2, 4, 8, 16):
        print(f"case norm-mlp fmt={fmt} M={M}", flush=True)
        x = torch.randn(M, 4096, generator=g).to(torch.bfloat16)
        out = C.mono_mlp_w4(x.to(dev), _lib.ROT_NONE, None, lut.to(dev), *handles, norm_w=nw.to(dev), eps=1e-6)
        xn = ref.rmsnorm(bits(x), bits(nw), 1e-6)
        want = ref.mono_mlp(xn, "none", None, bits(lut), *d)
        assert_bits_equal(bits(out), want, f"M={M}")


def _mlp_handles(g, dev, fmt="gptq"):
    from mdx import _lib, layout
    ws, _ = _mlp_weights(g, fmt, dev, True)
    cb = ws[0][3]
    cbt = None if cb is None else cb.to(dev)
    handles = [layout.W4(layout.tile_major_codes(q).to(dev), s.to(dev), c.to(dev), cbt, _lib.LAYOUT_TILE)
               for q, s, c, _, _ in ws]
    return ws, handles


@pytest.mark.parametrize("fmt", ["gptq", "gptq_rint"])
@pytest.mark.parametrize("rot", ["none", "h256"])
def test_mlp_with_residual_matches_oracle(C, dev, rot, fmt):
    """The MLP block with RMSNorm in front and a residual, for every row count class (one row, two,
    up to eight, sixteen), with and without the rotation of h, on integral and fp16-ratio group scales,
    against the oracle bit for bit."""
    from mdx import _lib, layout
    g = torch.Generator().manual_seed(41)
    ws, handles = _mlp_handles(g, dev, fmt)
    lut = layout.silu_lut(dev)
    nw = (1 + torch.randn(4096, generator=g) * 0.02).to(torch.bfloat16)
    code = _lib.ROT_H256 if rot == "h256" else _lib.ROT_NONE
    h = layout.regular_hadamard(dev) if rot == "h256" else None
    d = _oracle_dicts(ws)
    for M in (1, 2, 4, 5, 8, 16):
        print(f"case mlp-residual rot={rot} fmt={fmt} M={M}", flush=True)
        x = torch.randn(M, 4096, generator=g).to(torch.bfloat16)
        res = torch.randn(M, 4096, generator=g).to(torch.bfloat16)
        out = C.mono_mlp_w4(x.to(dev), code, h, lut, *handles, norm_w=nw.to(dev), eps=1e-6, residual=res.to(dev))
        xn = ref.rmsnorm(bits(x), bits(nw), 1e-6)
        want = ref.add_bf16(bits(res), ref.mono_mlp(xn, rot, None if h is None else bits(h.cpu()), bits(lut.cpu()), *d))
        assert_bits_equal(bits(out), want, f"M={M}")


@pytest.mark.parametrize("fmt", ["gptq", "gptq_rint"])
def test_mlp_down_quantises_h_equals_row_prep(C, dev, monkeypatch, fmt):
    """Without a rotation, at one or two rows, the down GEMV quantises h itself from gate/up's |h|
    maxima, and at one row the gate/up GEMV also prepares x itself (RMSNorm or none): the same
    outputs, bit for bit, as the row prep launches (MDX_MLP_HPREP=1), and as the oracle; with a
    residual, one to eight rows, over calls that reuse the workspace."""
    from mdx import _lib, layout
    g = torch.Generator().manual_seed(47)
    ws, handles = _mlp_handles(g, dev, fmt)
    lut = layout.silu_lut(dev)
    nw = (1 + torch.randn(4096, generator=g) * 0.02).to(torch.bfloat16)
    d = _oracle_dicts(ws)
    for M, norm in ((1, True), (1, False), (2, True), (5, True), (8, True), (3, True)):
        print(f"case mlp-hr fmt={fmt} M={M} norm={norm}", flush=True)
        x = torch.randn(M, 4096, generator=g).to(torch.bfloat16)
        res = torch.randn(M, 4096, generator=g).to(torch.bfloat16)
        nwd = nw.to(dev) if norm else None
        outs = []
        for hp in ("0", "1"):
            monkeypatch.setenv("MDX_MLP_HPREP", hp)
            outs.append(C.mono_mlp_w4(x.to(dev), _lib.ROT_NONE, None, lut, *handles, norm_w=nwd, eps=1e-6,
                                      residual=res.to(dev)))
        torch.cuda.synchronize()
        assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), f"M={M}"
        xn = ref.rmsnorm(bits(x), bits(nw), 1e-6) if norm else bits(x)
        want = ref.add_bf16(bits(res), ref.mono_mlp(xn, "none", None, bits(lut.cpu()), *d))
        assert_bits_equal(bits(outs[0]), want, f"M={M} norm={norm}")


@pytest.mark.parametrize("fmt", ["gptq", "gptq_rint"])
@pytest.mark.parametrize("rot", ["none", "h256"])
def test_mlp_graph_replays(C, dev, rot, fmt):
    """The MLP block captured once, replayed with new inputs between eager calls of the same block:
    every replay equals the eager result (no launch keeps state between calls)."""
    from mdx import _lib, layout
    g = torch.Generator().manual_seed(43)
    _, handles = _mlp_handles(g, dev, fmt)
    lut = layout.silu_lut(dev)
    code = _lib.ROT_H256 if rot == "h256" else _lib.ROT_NONE
    hd = layout.regular_hadamard(dev) if rot == "h256" else None
    nw = (1 + torch.randn(4096, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    for M in (1, 2, 8):
        print(f"case mlp graph rot={rot} fmt={fmt} M={M}", flush=True)
        x = torch.randn(M, 4096, generator=g).to(torch.bfloat16).to(dev)
        out = torch.empty(M, 4096, dtype=torch.bfloat16, device=dev)
        C.mono_mlp_w4(x, code, hd, lut, *handles, norm_w=nw, eps=1e-6, out=out)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            C.mono_mlp_w4(x, code, hd, lut, *handles, norm_w=nw, eps=1e-6, out=out)
        for rep in range(4):
            x.copy_(torch.randn(M, 4096, generator=g).to(torch.bfloat16).to(dev))
            graph.replay()
            torch.cuda.synchronize()
            got = out.clone()
            want = C.mono_mlp_w4(x, code, hd, lut, *handles, norm_w=nw, eps=1e-6)
            torch.cuda.synchronize()
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"M={M} replay {rep}"


def test_integral_decode_mode_matches_oracle(C, dev):
    """MDX_DECODE_INTEGRAL (the caller asserts integral scales; no per-launch check) gives the
    oracle's bits, as MDX_DECODE_AUTO does: the MLP at 1, 2 and 8 rows (the row-prep, bf16-row and
    int8-row sources) and a single linear at 1 and 8 rows."""
    from mdx import _lib, layout
    g = torch.Generator().manual_seed(61)
    ws, _ = _mlp_weights(g, "gptq", dev, True)
    handles = [layout.W4(layout.tile_major_codes(q).to(dev), s.to(dev), c.to(dev), None, _lib.LAYOUT_TILE,
                         _lib.DECODE_INTEGRAL) for q, s, c, _, _ in ws]
    lut = layout.silu_lut()
    nw = (1 + torch.randn(4096, generator=g) * 0.02).to(torch.bfloat16)
    d = _oracle_dicts(ws)
    for M in (1, 2, 8):
        print(f"case integral-mlp M={M}", flush=True)
        x = torch.randn(M, 4096, generator=g).to(torch.bfloat16)
        out = C.mono_mlp_w4(x.to(dev), _lib.ROT_NONE, None, lut.to(dev), *handles, norm_w=nw.to(dev), eps=1e-6)
        want = ref.mono_mlp(ref.rmsnorm(bits(x), bits(nw), 1e-6), "none", None, bits(lut), *d)
        assert_bits_equal(bits(out), want, f"M={M}")
    w = random_w4(4096, 4096, g, "gptq")
    h = layout.W4(layout.tile_major_codes(w[0]).to(dev), w[1].to(dev), w[2].to(dev), None, _lib.LAYOUT_TILE,
                  _lib.DECODE_INTEGRAL)
    for M in (1, 8):
        print(f"case integral-linear M={M}", flush=True)
        x = torch.randint(-127, 128, (M, 4096), generator=g, dtype=torch.int8)
        xs = torch.rand(M, generator=g) * 0.01 + 1e-3
        out = torch.empty(M, 4096, dtype=torch.bfloat16, device=dev)
        C.stream_gemv(x.to(dev), xs.to(dev), [h], [out])
        assert_bits_equal(bits(out), oracle_linear(x, xs, w), f"M={M}")
