"""Host-side weight layouts (CPU)."""
import torch


def test_tile_major_bf16_layout():
    from mdx import layout
    w = torch.arange(32 * 64, dtype=torch.float32).reshape(32, 64).bfloat16()
    t = layout.tile_major_bf16(w).view(-1)
    # block (0, 0): lane 16 g + c holds row c, k in [8 g, 8 g + 8)
    for lane in (0, 1, 17, 63):
        g_, c = lane >> 4, lane & 15
        assert torch.equal(t[lane * 8:lane * 8 + 8], w[c, 8 * g_:8 * g_ + 8])
    assert torch.equal(torch.sort(t.float()).values, torch.sort(w.float().view(-1)).values)


def test_compact_h_expands_to_h256():
    from mdx import _C, layout
    h = layout.regular_hadamard()
    assert torch.equal(_C.expand_compact_h(torch.stack((h[:16, :16], -h[:16, :16]))).view(torch.int16), h.view(torch.int16))
