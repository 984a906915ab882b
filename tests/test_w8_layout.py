"""The int8 ConvRot lm_head's host side on the CPU: the tile-major int8 order (a permutation whose first
KiB is rows 0..15 x k 0..63 in lane order, inverted by row_major_i8), the ConvRot rotation (orthogonal:
(x H)(w H)^T = x w^T; H256 = kron(H4, H4, H4, H4) / 16 against an explicit Kronecker product) and the
per-row int8 quantisation of the rotated rows (|q s - w H| <= s / 2, the row maximum reaching 127)."""
import numpy as np
import torch

from oracle import ref


def test_tile_major_i8_order_and_inverse():
    from mdx import layout
    N, K = 48, 192
    w = torch.randint(-128, 128, (N, K), dtype=torch.int8, generator=torch.Generator().manual_seed(1))
    t = layout.tile_major_i8(w)
    assert t.shape == w.shape and torch.equal(layout.row_major_i8(t), w)
    flat = t.reshape(-1)
    for tile in (0, 2):
        for j in (0, 2):
            blk = flat[(tile * (K // 64) + j) * 1024:(tile * (K // 64) + j + 1) * 1024].reshape(64, 16)
            for lane in (0, 5, 17, 63):
                g, c = lane // 16, lane % 16
                assert torch.equal(blk[lane], w[16 * tile + c, 64 * j + 16 * g:64 * j + 16 * g + 16])
    assert torch.equal(torch.sort(flat)[0], torch.sort(w.reshape(-1))[0])


def test_convrot_rotation_is_the_kronecker_hadamard_and_orthogonal():
    from mdx import layout
    h = layout.regular_hadamard(dtype=torch.float64)
    h4 = torch.tensor(ref.H4, dtype=torch.float64)
    k = torch.kron(torch.kron(h4, h4), torch.kron(h4, h4)) / 16
    assert torch.equal(h, k)
    assert torch.allclose(h @ h.T, torch.eye(256, dtype=torch.float64), atol=1e-15)
    g = torch.Generator().manual_seed(2)
    w = torch.randn(32, 512, generator=g).bfloat16()
    x = torch.randn(3, 512, generator=g).bfloat16()
    wr = layout.convrot_rotate(w).double()
    xr = (x.double().reshape(3, 2, 256) @ h).reshape(3, 512)
    assert torch.allclose(xr @ wr.T, x.double() @ w.double().T, rtol=1e-5, atol=1e-5)


def test_int8_convrot_head_quantisation_bounds():
    from mdx import layout
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(40, 768, generator=g) * 0.02).bfloat16()
    w[7] = 0  # an all-zero row keeps the tiny scale
    q, s = layout.int8_convrot_head(w)
    r = layout.convrot_rotate(w)
    assert q.dtype == torch.int8 and s.dtype == torch.float32 and q.shape == w.shape
    err = (q.float() * s[:, None] - r).abs()
    assert (err <= s[:, None] * 0.5 * (1 + 1e-6)).all()
    live = torch.arange(40) != 7
    assert (q[live].abs().amax(1) == 127).all() and (q[7] == 0).all() and s[7] == 1e-30
