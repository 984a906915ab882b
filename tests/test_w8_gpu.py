"""The W8A8 linear of the int8 ConvRot lm_head (mdx_int8_linear, omni's int8_linear_prequantized as the
reference's draft head calls it, comfy_mono_decode_xpu/draft_head.py:228) against the oracle's exact int8
logits (oracle/ref.py int8_head_logits: int64 dot, two fp32 products, bf16), bit for bit: 1..16 rows, the
vocabulary-sized head, small and long K, both weight layouts, extreme codes; the contract errors."""
import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits
from oracle import ref

pytestmark = pytest.mark.gpu


def _case(g, rows, N, K, extreme=False):
    if extreme:
        w = torch.full((N, K), -127, dtype=torch.int8)
        w[1::2] = 127
        x = torch.full((rows, K), -128, dtype=torch.int8)
    else:
        w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
        x = torch.randint(-128, 128, (rows, K), generator=g, dtype=torch.int8)
    xs = torch.rand(rows, generator=g) * 0.05 + 0.01
    ws = torch.rand(N, generator=g) * 1e-3 + 1e-4
    return x, xs, w, ws


def _want(x, xs, w, ws, cols=None):
    wn = w.numpy() if cols is None else w.numpy()[cols]
    sw = ws.numpy() if cols is None else ws.numpy()[cols]
    return np.stack([ref.int8_head_logits(x[r].numpy(), xs[r:r + 1].numpy(), wn, sw) for r in range(x.shape[0])])


@pytest.mark.parametrize("rows,N,K", [(1, 4096, 4096), (2, 1024, 12288), (5, 256, 64), (8, 4096, 4096),
                                      (16, 512, 4096), (3, 1024, 16384)])
@pytest.mark.parametrize("tiled", [True, False])
def test_int8_linear_matches_oracle(C, dev, rows, N, K, tiled):
    from mdx import layout
    print(f"case int8_linear rows={rows} N={N} K={K} tiled={tiled}", flush=True)
    g = torch.Generator().manual_seed(rows * 7 + K)
    x, xs, w, ws = _case(g, rows, N, K)
    wd = (layout.tile_major_i8(w) if tiled else w).to(dev)
    out = C.int8_linear_prequantized(x.to(dev), xs.to(dev), wd, ws.to(dev), tiled=tiled)
    assert_bits_equal(bits(out), _want(x, xs, w, ws), f"rows={rows} N={N} K={K}")


def test_int8_linear_vocabulary_head(C, dev):
    """The lm_head shape (151936 x 4096) at 1 and 8 rows: every logit of sampled columns and the top-20."""
    from mdx import layout
    g = torch.Generator().manual_seed(9)
    N, K = 151936, 4096
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    ws = torch.rand(N, generator=g) * 1e-3 + 1e-4
    wd, wsd = layout.tile_major_i8(w.to(dev)), ws.to(dev)
    cols = np.random.default_rng(1).choice(N, 4096, replace=False)
    for rows in (1, 8):
        print(f"case int8_linear vocabulary rows={rows}", flush=True)
        x = torch.randint(-128, 128, (rows, K), generator=g, dtype=torch.int8)
        xs = torch.rand(rows, generator=g) * 0.05 + 0.01
        out = C.int8_linear_prequantized(x.to(dev), xs.to(dev), wd, wsd, tiled=True)
        got = bits(out)
        assert_bits_equal(got[:, cols], _want(x, xs, w, ws, cols), f"sampled columns rows={rows}")
        # row 0 in full, in blocks of 16384 weight rows (the oracle's int64 dot of one block at a time)
        full = np.concatenate([ref.int8_head_logits(x[0].numpy(), xs[:1].numpy(), w[n0:n0 + 16384].numpy(),
                                                    ws[n0:n0 + 16384].numpy()) for n0 in range(0, N, 16384)])
        assert_bits_equal(got[0], full, "row 0 in full")


def test_int8_linear_extreme_codes(C, dev):
    """-128 activations against +-127 weights over K = 65536: |acc| = 2^23 * 127 stays exact in int32."""
    print("case int8_linear extreme codes", flush=True)
    g = torch.Generator().manual_seed(4)
    x, xs, w, ws = _case(g, 2, 32, 65536, extreme=True)
    out = C.int8_linear_prequantized(x.to(dev), xs.to(dev), w.to(dev), ws.to(dev))
    assert_bits_equal(bits(out), _want(x, xs, w, ws), "extreme")


def test_int8_linear_contract_errors(C, dev):
    g = torch.Generator().manual_seed(5)
    x, xs, w, ws = [t.to(dev) for t in _case(g, 17, 64, 128)]
    with pytest.raises(RuntimeError, match="rows"):
        C.int8_linear_prequantized(x, xs, w, ws)
    with pytest.raises(RuntimeError, match="N % 16"):
        C.int8_linear_prequantized(x[:2], xs[:2], w[:40], ws[:40].contiguous())
    with pytest.raises(RuntimeError, match="K % 64"):
        C.int8_linear_prequantized(x[:2, :96].contiguous(), xs[:2], w[:, :96].contiguous(), ws)
    with pytest.raises(RuntimeError, match="bias"):
        C.int8_linear_prequantized(x[:2], xs[:2], w, ws, bias=ws)
