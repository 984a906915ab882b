"""The activation quantisation's quotient (comfy-mono-decode-xpu_amd/csrc/mdx_gemv.hip, quant_rcp):
the code of a bf16 value v under the bf16 scale sb is rint(bf16(v / sb)) (the quotient rounded to
fp32, then to bf16). The kernels compute bf16(v * fl32(1 / sb)) instead; this checks, on the CPU, that
the two agree for every finite bf16 v against a spread of scales (the smallest normal binade, the
binade of 1.0, random ones), wherever the quotient survives the int8 clamp."""
import numpy as np


def _bf16(bits):
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def _bfround(x):
    u = x.view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), np.float32(np.nan), r)


def test_reciprocal_product_rounds_like_the_quotient():
    v = _bf16(np.arange(0, 0x7F80, dtype=np.uint32))  # every finite non-negative bf16 (the sign is symmetric)
    rng = np.random.default_rng(7)
    scales = list(range(0x0080, 0x0100)) + list(range(0x3F80, 0x4000)) + list(rng.integers(0x0080, 0x7F80, 200))
    with np.errstate(over="ignore"):
        for sbb in scales:
            sb = _bf16([sbb])[0]
            exact = _bfround((v.astype(np.float64) / np.float64(sb)).astype(np.float32))
            fast = _bfround(v * np.float32(np.float32(1.0) / sb))
            keep = np.abs(exact.astype(np.float64)) <= 256  # beyond, both clamp to +-127
            assert np.array_equal(exact[keep], fast[keep]), f"scale bits {sbb:#06x}"
