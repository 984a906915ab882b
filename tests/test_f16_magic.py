"""The per-weight decode tables of fp16 group scales are built on the device with packed half-precision
FMAs: q(k s) = the low byte of fl16(k s + 1536), k = 1..8 (one rounding of the exact k s + 1536; in
[1024, 2048) the half-precision spacing is 1, so the rounding is rint to nearest even, and 1536 is even).
This pins that identity against the reference's own decode, w8 = rint(fl32(cb[c] * s)) with no clamp
needed (csrc/w4a8_decode.sycl:4-11,35-45), for every fp16 scale the fast path accepts (|s| <= 127 / 8,
no NaN): exhaustively, all 38,882 bit patterns (both signs)."""
import numpy as np


FAST_MAX_BITS = 0x4BF0  # fp16 127 / 8 = 15.875: the largest |s| the fast path takes


def test_magic_number_rounding_equals_rint_for_every_fast_scale():
    bits = np.arange(0, FAST_MAX_BITS + 1, dtype=np.uint16)
    bits = np.concatenate([bits, bits | 0x8000])
    s = bits.view(np.float16).astype(np.float64)
    assert np.float16(15.875).view(np.uint16) == FAST_MAX_BITS
    for k in range(1, 9):
        exact = k * s + 1536.0                       # exact in float64 (k s has at most 14 significant bits)
        r16 = exact.astype(np.float16)               # one IEEE round-to-nearest-even to half precision
        low = (r16.view(np.uint16) & 0xFF).astype(np.uint8).view(np.int8)
        ref = np.rint((np.float32(k) * s.astype(np.float32))).astype(np.int64)  # the reference's fp32 rint
        assert np.abs(ref).max() <= 127
        assert np.array_equal(low.astype(np.int64), ref), k
    # the range bound matters: just above it, 8 s rounds past 127 (the clamp the fast path would miss)
    s_over = np.float16(15.9375).astype(np.float64)
    assert np.rint(8 * s_over) == 128
