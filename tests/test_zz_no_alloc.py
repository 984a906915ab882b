"""mdx_topk_rows_noalloc (the library's static device scratch instead of a workspace) against
mdx_topk_rows (a caller workspace) through the C ABI: identical values and indices, bit for bit, on two
calls in a row, the second smaller (fewer rows, shorter rows, smaller k), so the second call finds the
first one's contents in the shared scratch; rows above the scratch's 16 are rejected before any launch."""
import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits
from oracle import ref

pytestmark = pytest.mark.gpu


def _noalloc(x, k):
    from mdx import _lib
    R, N = x.shape
    values = torch.empty(R, k, dtype=torch.float32, device=x.device)
    indices = torch.empty(R, k, dtype=torch.int64, device=x.device)
    dt = _lib.DT_F32 if x.dtype == torch.float32 else _lib.DT_BF16
    _lib.call("mdx_topk_rows_noalloc", _lib.ptr(x), dt, R, N, k, _lib.ptr(values), _lib.ptr(indices), _lib.stream_of(x))
    return values, indices


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_topk_rows_matches_workspace_entry(C, dev, dtype):
    g = torch.Generator().manual_seed(11)
    for R, N, k in ((16, 151936, 20), (3, 40000, 7)):
        print(f"case noalloc topk_rows dtype={dtype} R={R} N={N} k={k}", flush=True)
        x = torch.randint(0, 50, (R, N), generator=g).to(dtype)  # tie-heavy rows
        x[0, 1000:1100] = float("inf") if R > 3 else 7.0
        xd = x.to(dev)
        v0, i0 = C.topk_rows(xd, k)
        v1, i1 = _noalloc(xd, k)
        torch.cuda.synchronize()
        assert_bits_equal(bits(i1), bits(i0), f"indices R={R}")
        assert_bits_equal(bits(v1), bits(v0), f"values R={R}")
        if R <= 3:
            wv, wi = ref.topk_rows(x.float().numpy() if dtype == torch.float32 else bits(x), k)
            assert_bits_equal(bits(i1), wi, "indices vs oracle")


def test_noalloc_rejects_rows_beyond_the_scratch(C, dev):
    from mdx import _lib
    x = torch.zeros(17, 4096, device=dev)
    v = torch.empty(17, 4, device=dev)
    i = torch.empty(17, 4, dtype=torch.int64, device=dev)
    with pytest.raises(RuntimeError, match="static top-k scratch"):
        _lib.call("mdx_topk_rows_noalloc", _lib.ptr(x), _lib.DT_F32, 17, 4096, 4, _lib.ptr(v), _lib.ptr(i),
                  _lib.stream_of(x))
