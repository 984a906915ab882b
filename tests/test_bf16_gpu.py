"""bf16 decode linear (lm_head and draft-block GEMMs) on the GPU against float64: bf16 outputs within
2^-8 relative plus the fp32 accumulation bound (2^-16 x sum |x||w|); the tile-major and row-major
layouts give identical bits (same products, same order)."""
import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits
from oracle import ref

pytestmark = pytest.mark.gpu


def _check(got, x, w, cols=None, res=None):
    xb, wb = bits(x), bits(w)
    if cols is not None:
        wb = wb[cols]
        got = got[:, cols]
    want, scale = ref.bf16_linear_f64(xb, wb)
    acc = np.abs(want)
    if res is not None:  # out = bf16(res + bf16(acc)): the product's own rounding adds 2^-9 |acc|
        r = ref.bf16_to_f32(bits(res)).astype(np.float64)
        want = want + (r if cols is None else r[:, cols])
    g = got.float().cpu().numpy().astype(np.float64)
    err = np.abs(g - want)
    bound = np.abs(want) * 2 ** -8 + (acc * 2 ** -8 if res is not None else 0) + scale * 2 ** -16 + 1e-30
    assert (err <= bound).all(), (err / bound).max()


@pytest.mark.parametrize("N,K", [(4096, 4096), (12288, 4096), (4096, 12288), (1024, 8192), (48, 64)])
@pytest.mark.parametrize("rows", [1, 3, 8, 16])
def test_bf16_linear_matches_f64(C, dev, N, K, rows):
    from mdx import layout
    g = torch.Generator().manual_seed(N + K + rows)
    x = torch.randn(rows, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    xd, wd = x.to(dev), w.to(dev)
    out_t = C.bf16_linear(xd, layout.tile_major_bf16(wd), tiled=True)
    out_r = C.bf16_linear(xd, wd, tiled=False)
    assert_bits_equal(bits(out_t), bits(out_r), "tile vs row layout")
    _check(out_t.cpu(), x, w)
    res = torch.randn(rows, N, generator=g).bfloat16()
    out_res = C.bf16_linear(xd, wd, tiled=False, residual=res.to(dev))
    _check(out_res.cpu(), x, w, res=res)


@pytest.mark.parametrize("rows", [1, 8])
def test_lm_head_151936(C, dev, rows):
    """The bf16 lm_head of the hybrid stack (vocab 151936, hidden 4096), checked on 4096 sampled
    vocabulary rows, plus the top-20 of the logits against the oracle's exact rank order."""
    from mdx import layout
    g = torch.Generator(device=dev).manual_seed(5)
    V, H = 151936, 4096
    w = (torch.randn(V, H, generator=g, device=dev) * 0.02).bfloat16()
    x = torch.randn(rows, H, generator=g, device=dev).bfloat16()
    wt = layout.tile_major_bf16(w)
    logits = C.bf16_linear(x, wt, tiled=True)
    # the streaming kernel (tile-major, many tiles) against the split-K kernel that reads row-major
    assert_bits_equal(bits(logits), bits(C.bf16_linear(x, w, tiled=False)), "tile vs row layout")
    cols = np.random.default_rng(0).choice(V, 4096, replace=False)
    _check(logits.cpu(), x.cpu(), w.cpu(), cols=cols)
    v, i = C.topk_rows(logits, 20)
    wv, wi = ref.topk_rows(bits(logits), 20)
    assert np.array_equal(i.cpu().numpy(), wi)


def test_bf16_rounding_matches_integer_rne_everywhere(C, dev):
    """The library rounds fp32 to bf16 with the hardware conversion; mdx_check_bf16_round compares it on
    the device with the integer round-to-nearest-even formulation over all 2^32 fp32 patterns
    (subnormals, infinities, ties; NaN -> 0x7FC0 for stored bits, any NaN for in-register values)."""
    from mdx import _lib
    n = torch.zeros(1, dtype=torch.int64, device=dev)
    first = torch.full((1,), -1, dtype=torch.int32, device=dev)
    _lib.call("mdx_check_bf16_round", _lib.ptr(n), _lib.ptr(first), _lib.stream_of(n))
    torch.cuda.synchronize()
    assert int(n.item()) == 0, f"{int(n.item())} patterns disagree, first 0x{int(first.item()) & 0xFFFFFFFF:08x}"


@pytest.mark.parametrize("rows", [1, 5, 16])
def test_many_tiles_partial_last_wave(C, dev, rows):
    """8195 tiles (more than one resident grid of single-tile waves: two tiles per wave in the
    streaming kernel, the last wave one): tile-major against row-major bits, with and without a
    residual, and within the float64 bound on sampled rows."""
    from mdx import layout
    g = torch.Generator(device=dev).manual_seed(11 + rows)
    N, K = 16 * 8195, 4096
    w = (torch.randn(N, K, generator=g, device=dev) * 0.02).bfloat16()
    x = torch.randn(rows, K, generator=g, device=dev).bfloat16()
    res = torch.randn(rows, N, generator=g, device=dev).bfloat16()
    wt = layout.tile_major_bf16(w)
    for r in (None, res):
        print(f"case many tiles rows={rows} residual={r is not None}", flush=True)
        got = C.bf16_linear(x, wt, tiled=True, residual=r)
        assert_bits_equal(bits(got), bits(C.bf16_linear(x, w, tiled=False, residual=r)), "tile vs row layout")
    cols = np.concatenate([np.arange(N - 64, N), np.random.default_rng(1).choice(N - 64, 960, replace=False)])
    _check(C.bf16_linear(x, wt, tiled=True).cpu(), x.cpu(), w.cpu(), cols=cols)
