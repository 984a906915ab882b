"""Pin of the attention oracle against torch's float64 scaled_dot_product_attention with an explicit
boolean mask (an independent implementation), including the empty-prefix and draft cases. CPU only."""
import numpy as np
import torch

from oracle import ref


def test_attention_oracle_matches_torch_sdpa():
    g = torch.Generator().manual_seed(30)
    for H, Hk, S, D, L, parents in ((4, 2, 5, 64, 37, [-1, 0, 1, 1, 0]), (2, 1, 1, 128, 50, None),
                                    (4, 1, 3, 32, 0, [-1, 0, 0]), (8, 2, 8, 16, 9, [-1, 0, 1, 2, 3, 4, 5, 6])):
        cap = L + 7
        q = torch.randn(H, S, D, generator=g, dtype=torch.float64)
        k = torch.randn(Hk, cap, D, generator=g, dtype=torch.float64)
        v = torch.randn(Hk, cap, D, generator=g, dtype=torch.float64)
        xk = torch.randn(Hk, S, D, generator=g, dtype=torch.float64)
        xv = torch.randn(Hk, S, D, generator=g, dtype=torch.float64)
        mask = None if parents is None else ref.tree_mask(parents)
        got = ref.attention_f64(q.numpy(), k.numpy(), v.numpy(), L, xk.numpy(), xv.numpy(), mask)
        for h in range(H):
            kh = h // (H // Hk)
            K = torch.cat([k[kh, :L], xk[kh]])
            V = torch.cat([v[kh, :L], xv[kh]])
            allow = torch.zeros(S, L + S, dtype=torch.bool)
            allow[:, :L] = True
            for s in range(S):
                for t in range(S):
                    allow[s, L + t] = mask is not None and bool((mask[s] >> t) & 1)
            want = torch.nn.functional.scaled_dot_product_attention(q[h][None], K[None], V[None],
                                                                    attn_mask=allow[None])[0]
            assert np.allclose(got[:, h], want.numpy(), rtol=1e-12, atol=1e-12), (H, S, D, L)
    assert ref.tree_mask([-1, 0, 1, 1, 0]) == [1, 3, 7, 11, 17]
