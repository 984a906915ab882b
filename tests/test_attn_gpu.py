"""Decode attention on the GPU against the float64 oracle, with the bound of the reference's test
(tests/test_attn_dpas.py:70-74): max error <= 1.5 x e_ref.max + 1e-3, mean <= 1.5 x e_ref.mean + 1e-5,
where e_ref is the error of a float32 chain on the same bf16 inputs, rounded to bf16 like a kernel's
output (the Kitchen kernel the reference measures against is unavailable); with no cached prefix,
max <= 1.6e-2."""
import numpy as np
import pytest
import torch

from conftest import bits
from oracle import ref

pytestmark = pytest.mark.gpu


def _case(C, dev, H, Hk, D, L, cap, parents, seed):
    g = torch.Generator().manual_seed(seed)
    S = 1 if parents is None else len(parents)
    q = (torch.randn(1, H, S, D, generator=g) * 2).bfloat16()
    k = (torch.randn(1, Hk, cap, D, generator=g) * 1.5).bfloat16()
    v = torch.randn(1, Hk, cap, D, generator=g).bfloat16()
    xk = (torch.randn(1, Hk, S, D, generator=g) * 1.5).bfloat16()
    xv = torch.randn(1, Hk, S, D, generator=g).bfloat16()
    mask = None if parents is None else ref.tree_mask(parents)
    f = [t.float().numpy()[0] for t in (q, k, v, xk, xv)]
    want = ref.attention_f64(*f[:3], L, *f[3:], mask)
    chain = ref.bf16_to_f32(ref.f32_to_bf16(ref.attention_f64(*f[:3], L, *f[3:], mask, dtype=np.float32)))
    e_ref = np.abs(chain.astype(np.float64) - want)
    sl = torch.tensor([L], dtype=torch.int32, device=dev)
    mt = torch.empty(0, dtype=torch.int32, device=dev) if mask is None else torch.tensor(mask, dtype=torch.int32,
                                                                                        device=dev)
    out = C.attn_dpas(q.to(dev), k.to(dev), v.to(dev), sl, xk.to(dev), xv.to(dev), mt, 0)
    assert out.shape == (1, S, H * D)
    got = out.float().cpu().numpy().reshape(S, H, D).astype(np.float64)
    err = np.abs(got - want)
    assert np.isfinite(got).all()
    if L > 0:
        assert err.max() <= 1.5 * e_ref.max() + 1e-3, (err.max(), e_ref.max())
        assert err.mean() <= 1.5 * e_ref.mean() + 1e-5, (err.mean(), e_ref.mean())
    else:
        assert err.max() <= 1.6e-2
    return out


@pytest.mark.parametrize("L,cap,parents", [
    (0, 512, [-1, 0, 1]),
    (63, 4096, [-1, 0, 1, 2, 3, 4, 5, 6]),
    (777, 4096, [-1, 0, 0, 0, 0, 1, 1, 1]),
    (3500, 11400, [-1, 0, 1, 2, 3, 4, 5, 6]),
    (4096, 12416, [-1, 0, 1, 2, 3, 4, 5]),
    (11392, 11400, [-1, 0, 0, 1, 1]),
    (11400, 11400, [-1, 0, 1, 2, 3, 4, 5, 6]),
    (1000, 4096, None),
    (8000, 11400, None),
])
def test_attn_reference_shapes(C, dev, L, cap, parents):
    """The reference model's attention: 16 q / 4 kv heads, head_dim 256."""
    _case(C, dev, 16, 4, 256, L, cap, parents, L + cap)


@pytest.mark.parametrize("L", [2048, 8192, 1, 31, 500])
def test_attn_hybrid_verify_16_rows(C, dev, L):
    """32 q / 8 kv heads, head_dim 128, 16 tree rows (64 query rows per kv head)."""
    parents = [-1, 0, 1, 2, 3, 4, 5, 6, 0, 8, 1, 10, 2, 12, 3, 14]
    _case(C, dev, 32, 8, 128, L, L + 16 + 64, parents, 3 + L)


@pytest.mark.parametrize("H,Hk,D,L,parents", [(8, 8, 64, 300, [-1, 0, 1]), (32, 8, 128, 4000, None),
                                              (4, 1, 128, 0, [-1, 0, 1, 1, 2, 2, 3, 3, 4, 4, 5, 5, 6, 6, 7, 7]),
                                              (12, 1, 64, 700, [-1, 0, 1, 2]),
                                              (16, 8, 64, 2000, [-1, 0, 1, 1, 2, 2, 3, 3]),
                                              (32, 4, 128, 5000, [-1, 0, 1, 2]),
                                              (32, 8, 128, 1, [-1, 0, 1, 2, 3, 4, 5, 6]),
                                              (64, 8, 64, 9000, [-1, 0])])
def test_attn_other_shapes(C, dev, H, Hk, D, L, parents):
    _case(C, dev, H, Hk, D, L, max(L, 1) + 64, parents, 7 + L)


def test_attn_graph_replay_follows_device_seqlen(C, dev):
    """One captured launch replayed for several context lengths written into seqlen between replays."""
    g = torch.Generator().manual_seed(11)
    H, Hk, D, cap = 32, 8, 128, 4096
    parents = [-1, 0, 1, 2, 0, 4, 1, 6]
    S = len(parents)
    q = (torch.randn(1, H, S, D, generator=g) * 2).bfloat16()
    k = (torch.randn(1, Hk, cap, D, generator=g) * 1.5).bfloat16()
    v = torch.randn(1, Hk, cap, D, generator=g).bfloat16()
    xk = (torch.randn(1, Hk, S, D, generator=g) * 1.5).bfloat16()
    xv = torch.randn(1, Hk, S, D, generator=g).bfloat16()
    mask = ref.tree_mask(parents)
    dq, dk, dv, dxk, dxv = (t.to(dev) for t in (q, k, v, xk, xv))
    sl = torch.tensor([100], dtype=torch.int32, device=dev)
    mt = torch.tensor(mask, dtype=torch.int32, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        C.attn_dpas(dq, dk, dv, sl, dxk, dxv, mt, 0)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = C.attn_dpas(dq, dk, dv, sl, dxk, dxv, mt, 0)
    f = [t.float().numpy()[0] for t in (q, k, v, xk, xv)]
    for L in (100, 4000, 0, 2500):
        sl.fill_(L)
        graph.replay()
        torch.cuda.synchronize()
        want = ref.attention_f64(*f[:3], L, *f[3:], mask)
        got = out.float().cpu().numpy().reshape(S, H, D)
        assert np.abs(got - want).max() <= 2e-2, L
