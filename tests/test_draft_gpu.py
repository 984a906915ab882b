"""The fused draft-head ops and the bf16 row ops on the GPU: every output bit for bit against the
oracle's restatement (the library's fixed order), and against float64 within the reference's tolerance
(tests/test_draft_fused.py: 1e-2 relative L2, 2e-2 for the dequantised int8 row); in-place semantics
as the reference's (x updated only when h is given). Reference: csrc/draft_fused.sycl:76-287."""
import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits
from oracle import ref

pytestmark = pytest.mark.gpu

H, I = 4096, 12288


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300)


def _rms64(x, w, eps):
    x = np.asarray(x, np.float64)
    return x * w / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def _f(t):
    return t.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("rows", [1, 3])
def test_embed_norm_cat(C, dev, rows):
    from mdx import layout
    print(f"case draft_embed_norm_cat rows={rows}", flush=True)
    g = torch.Generator().manual_seed(rows)
    V = 1000
    q = torch.randint(-127, 128, (V, H), generator=g, dtype=torch.int8)
    s = torch.rand(V, generator=g) * 1e-3 + 1e-4
    hm = layout.regular_hadamard(None, torch.float32)
    hidden = torch.randn(rows, H, generator=g).bfloat16()
    we, wh = (torch.rand(H, generator=g) + 0.5).bfloat16(), (torch.rand(H, generator=g) + 0.5).bfloat16()
    tok = torch.tensor([123, 999, 5000][:rows])
    out = torch.empty(rows, 2 * H, dtype=torch.bfloat16, device=dev)
    e = torch.empty(0, device=dev)
    C.draft_embed_norm_cat(tok.to(dev), q.to(dev), s.to(dev), hm.to(dev), e, hidden.to(dev), we.to(dev), wh.to(dev),
                           1e-6, 1e-6, out)
    want = ref.draft_embed_norm_cat(bits(hidden), bits(we), bits(wh), 1e-6, 1e-6, q=q.numpy(), s=s.numpy(),
                                    token=tok.numpy(), unrotate=True)
    assert_bits_equal(bits(out), want, "embed_norm_cat (gather)")
    t = tok.clamp(max=V - 1)
    row = (q[t].double() * s[t, None].double()).view(rows, -1, 256) @ hm.double()
    emb = row.reshape(rows, H).bfloat16()
    w64 = np.concatenate([_rms64(_f(emb), _f(we), 1e-6), _rms64(_f(hidden), _f(wh), 1e-6)], 1)
    assert _rel(_f(out), w64) < 1e-2
    # a given bf16 embedding row instead of the gather
    out2 = torch.empty_like(out)
    C.draft_embed_norm_cat(e, e, e, e, emb.to(dev), hidden.to(dev), we.to(dev), wh.to(dev), 1e-6, 1e-6, out2)
    want2 = ref.draft_embed_norm_cat(bits(hidden), bits(we), bits(wh), 1e-6, 1e-6, emb_bits=bits(emb))
    assert_bits_equal(bits(out2), want2, "embed_norm_cat (row)")
    # the row gathered from a bf16 table at the token (tokens past the table clamp to its last row)
    table = torch.randn(V, H, generator=g).bfloat16()
    table[t] = emb
    out3 = torch.empty_like(out)
    C.draft_embed_norm_cat(tok.to(dev), e, e, e, table.to(dev), hidden.to(dev), we.to(dev), wh.to(dev), 1e-6, 1e-6,
                           out3)
    assert_bits_equal(bits(out3), want2, "embed_norm_cat (bf16 table)")


def test_add_rmsnorm_in_place(C, dev):
    print("case draft_add_rmsnorm", flush=True)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(H, generator=g).bfloat16()
    h = torch.randn(H, generator=g).bfloat16()
    w = (torch.rand(H, generator=g) + 0.5).bfloat16()
    xd = x.to(dev)
    out = torch.empty(H, dtype=torch.bfloat16, device=dev)
    C.draft_add_rmsnorm(xd, h.to(dev), w.to(dev), 1e-6, out)
    xn, want = ref.draft_add_rmsnorm(bits(x), bits(h), bits(w), 1e-6)
    assert_bits_equal(bits(xd).reshape(1, -1), xn, "x += h")
    assert_bits_equal(bits(out).reshape(1, -1), want, "RMSNorm")
    assert torch.equal(xd.cpu(), x + h)  # torch.add in bf16
    assert _rel(_f(out), _rms64(_f(x + h), _f(w), 1e-6)) < 1e-2
    before = xd.clone()
    out_n = torch.empty_like(out)
    C.draft_add_rmsnorm(xd, torch.empty(0, device=dev), w.to(dev), 1e-6, out_n)  # norm only
    assert torch.equal(xd, before)
    assert_bits_equal(bits(out_n), bits(out), "norm only")


def test_sigmoid_and_silu_mul(C, dev):
    from mdx import layout
    print("case draft_sigmoid_mul / draft_silu_mul", flush=True)
    g = torch.Generator().manual_seed(2)
    a = torch.randn(H, generator=g).bfloat16()
    qg = torch.randn(2 * H, generator=g).bfloat16()
    gated = torch.empty(H, dtype=torch.bfloat16, device=dev)
    C.draft_sigmoid_mul(a.to(dev), qg.to(dev), 256, gated)
    sig = bits(layout.sigmoid_lut())
    assert_bits_equal(bits(gated), ref.draft_sigmoid_mul(bits(a)[None], bits(qg)[None], 256, sig)[0], "sigmoid_mul")
    gate = qg.view(16, 512)[:, 256:].reshape(-1)
    assert _rel(_f(gated), _f(a) / (1 + np.exp(-_f(gate)))) < 1e-2
    # rows of a fused q | k | v projection (q part strided)
    R = 3
    qkv = torch.randn(R, 2 * H + 2048, generator=g).bfloat16()
    a3 = torch.randn(R, H, generator=g).bfloat16()
    qkv_d = qkv.to(dev)
    out3 = torch.empty(R, H, dtype=torch.bfloat16, device=dev)
    C.draft_sigmoid_mul(a3.to(dev), qkv_d[:, :2 * H], 256, out3)
    assert_bits_equal(bits(out3), ref.draft_sigmoid_mul(bits(a3), bits(qkv)[:, :2 * H], 256, sig), "strided rows")
    gu = torch.randn(2, 2 * I, generator=g).bfloat16()
    act = torch.empty(2, I, dtype=torch.bfloat16, device=dev)
    C.draft_silu_mul(gu.to(dev), act)
    silu = bits(layout.silu_lut())
    assert_bits_equal(bits(act), ref.draft_silu_mul(bits(gu), silu), "silu_mul")
    g64, u64 = _f(gu[:, :I]), _f(gu[:, I:])
    assert _rel(_f(act), g64 / (1 + np.exp(-g64)) * u64) < 1e-2


@pytest.mark.parametrize("rotate,quant", [(True, True), (False, False)])
def test_norm_rot_quant(C, dev, rotate, quant):
    from mdx import layout
    print(f"case draft_norm_rot_quant rotate={rotate} quant={quant}", flush=True)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(H, generator=g).bfloat16()
    d = torch.randn(H, generator=g).bfloat16()
    w = (torch.rand(H, generator=g) + 0.5).bfloat16()
    hm = layout.regular_hadamard(dev, torch.float32) if rotate else torch.empty(0, device=dev)
    xd = x.to(dev)
    xr = torch.empty(H, dtype=torch.bfloat16, device=dev)
    qx = torch.empty(H if quant else 0, dtype=torch.int8, device=dev)
    sx = torch.empty(1 if quant else 0, dtype=torch.float32, device=dev)
    C.draft_norm_rot_quant(xd, d.to(dev), w.to(dev), 1e-6, hm, xr, qx, sx)
    xn, wxr, wq, ws = ref.draft_norm_rot_quant(bits(x), bits(d), bits(w), 1e-6, "h256" if rotate else "none")
    assert_bits_equal(bits(xd)[None], xn, "x += d")
    assert_bits_equal(bits(xr)[None], wxr, "xr")
    n = _rms64(_f(x + d), _f(w), 1e-6)
    if rotate:
        n = (n.reshape(-1, 256) @ layout.regular_hadamard(None, torch.float64).numpy()).reshape(-1)
    assert _rel(_f(xr), n) < 1e-2
    if quant:
        assert_bits_equal(bits(qx)[None], wq, "qx")
        assert_bits_equal(bits(sx), ws.view(np.uint32), "sx")
        assert _rel(qx.float().cpu().numpy() * sx.item(), n) < 2e-2


def test_rmsnorm_and_silu_mul_rows(C, dev):
    """mdx_rmsnorm (the final norms) and mdx_silu_mul, bit for bit against the oracle."""
    from mdx import layout
    print("case rmsnorm / silu_mul", flush=True)
    g = torch.Generator().manual_seed(4)
    for R, K in ((1, 4096), (8, 4096), (3, 8192)):
        x = torch.randn(R, K, generator=g).bfloat16() * 3
        w = (1 + torch.randn(K, generator=g) * 0.1).bfloat16()
        out = C.rmsnorm(x.to(dev), w.to(dev), 1e-6)
        assert_bits_equal(bits(out), ref.rmsnorm(bits(x), bits(w), 1e-6), f"rmsnorm R={R} K={K}")
    lut = layout.silu_lut()
    gg, uu = torch.randn(5000, generator=g).bfloat16() * 4, torch.randn(5000, generator=g).bfloat16()
    out = C.silu_mul(gg.to(dev), uu.to(dev), lut.to(dev))
    assert_bits_equal(bits(out), ref.silu_mul(gg.float().numpy(), uu.float().numpy(), bits(lut)), "silu_mul")


def test_contract_errors_raise_before_launch(C, dev):
    x = torch.zeros(100, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError):
        C.draft_add_rmsnorm(x, torch.empty(0, device=dev), x, 1e-6, x)  # H not a multiple of 256
    hm = torch.eye(256, device=dev)
    xr = torch.empty(H, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError):  # a rotation other than the regular H256
        C.draft_norm_rot_quant(torch.zeros(H, dtype=torch.bfloat16, device=dev), torch.empty(0, device=dev),
                               torch.ones(H, dtype=torch.bfloat16, device=dev), 1e-6, hm, xr,
                               torch.empty(0, device=dev), torch.empty(0, device=dev))
