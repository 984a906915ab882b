"""The tree-verify attention with the Q/K norm, RoPE and KV write in its own launch
(qk_norm_rope_attn) against the two calls it replaces (qk_norm_rope_kv + attn_dpas), bit for bit: the
attention output, the rows' q and k, and both caches in full. The q and k rows are also checked against
the oracle's rope_kv. Shapes of the hybrid's verify (32 q / 8 kv heads, head_dim 128; 8 and 16 tree
rows) and the prefill's 16-row chunks, every rotary size the fused form takes, with and without the
norm, gated (strided) q rows, empty and long prefixes, and a row whose position lies past the cache."""
import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits
from oracle import ref

pytestmark = pytest.mark.gpu

H, HK, D = 32, 8, 128


def _inputs(g, S, rd, cap, L, gated, scale=1.0):
    qg = (torch.randn(1, S, H, 2 * D, generator=g) * scale).bfloat16()
    q = qg[..., :D] if gated else qg[..., :D].contiguous()
    k = (torch.randn(1, S, HK, D, generator=g) * 3 * scale).bfloat16()
    v = torch.randn(1, S, HK, D, generator=g).bfloat16()
    wq = (1 + torch.randn(D, generator=g) * .3).bfloat16()
    wk = (1 + torch.randn(D, generator=g) * .3).bfloat16()
    f = torch.randn(S, rd // 2, 2, 2, generator=g)
    key = torch.randn(1, HK, cap, D, generator=g).bfloat16()
    val = torch.randn(1, HK, cap, D, generator=g).bfloat16()
    pos = torch.arange(L, L + S, dtype=torch.int64)
    return qg, q, k, v, wq, wk, f, key, val, pos


def _parents(S, g):
    # a random tree: each row's parent an earlier row (row 0 the root)
    return [-1] + [int(torch.randint(0, r, (1,), generator=g)) for r in range(1, S)]


@pytest.mark.parametrize("S,rd,norm,gated,L,cap", [
    (8, 64, True, True, 1024, 4096),
    (8, 64, True, False, 0, 64),
    (8, 32, False, True, 37, 512),
    (16, 128, True, True, 2047, 4096),
    (16, 64, True, False, 8000, 8192),
    (8, 128, False, False, 500, 1024),
    (16, 32, True, True, 1, 64),
    (8, 64, True, True, 4090, 4096),  # the last two rows' positions lie past the cache
])
def test_fused_rope_attention_equals_two_calls(C, dev, S, rd, norm, gated, L, cap):
    g = torch.Generator().manual_seed(S * 1000 + rd + L)
    qg, q, k, v, wq, wk, f, key, val, pos = _inputs(g, S, rd, cap, L, gated)
    mask = torch.tensor(ref.tree_mask(_parents(S, g)), dtype=torch.int32, device=dev)
    seq = torch.tensor([L], dtype=torch.int32, device=dev)
    qd = qg.to(dev)[..., :D] if gated else q.to(dev)
    kd_, vd_ = k.to(dev), v.to(dev)
    wqd, wkd = (wq.to(dev), wk.to(dev)) if norm else (None, None)
    fd, posd = f.to(dev), pos.to(dev)

    # the two calls
    key_a, val_a = key.to(dev), val.to(dev)
    if norm:
        qa, ka = C.qk_norm_rope_kv(qd, kd_, vd_, wqd, wkd, fd, key_a, val_a, posd, 1e-6, 2e-5, rd)
    else:
        qa, ka = C.rope_kv(qd, kd_, vd_, fd, key_a, val_a, posd, rd)
    out_a = C.attn_dpas(qa, key_a, val_a, seq, ka, vd_.transpose(1, 2), mask, 0)

    # the fused launch
    assert C.rope_attn_fits(H, HK, S, D, rd)
    key_b, val_b = key.to(dev), val.to(dev)
    kb = torch.empty(1, HK, S, D, dtype=torch.bfloat16, device=dev)
    qb = torch.empty(1, H, S, D, dtype=torch.bfloat16, device=dev)
    print(f"case S={S} rd={rd} norm={norm} gated={gated} L={L} cap={cap}", flush=True)
    out_b = C.qk_norm_rope_attn(qd, kd_, vd_, wqd, wkd, fd, key_b, val_b, posd, 1e-6 if norm else 1.0,
                                2e-5 if norm else 1.0, rd, seq, mask, kb, q_out=qb)
    torch.cuda.synchronize()
    assert_bits_equal(bits(out_b), bits(out_a), "attention output")
    assert_bits_equal(bits(qb), bits(qa), "q rows")
    assert_bits_equal(bits(kb), bits(ka), "k rows")
    assert_bits_equal(bits(key_b), bits(key_a), "key cache")
    assert_bits_equal(bits(val_b), bits(val_a), "value cache")

    # and the rows against the oracle's RoPE/KV restatement (its caches S rows longer: a position past the
    # cache writes into that margin, which is cut off, as the kernels write nothing there)
    pad = lambda c: np.concatenate([bits(c)[0], np.zeros((HK, S, D), np.uint16)], 1)
    args = (bits(q)[0], bits(k)[0], bits(v)[0], f.numpy(), pad(key), pad(val), pos.numpy(), rd)
    if norm:
        args = args + (bits(wq), bits(wk), 1e-6, 2e-5)
    wq_, wk_, ek, ev = ref.rope_kv(*args)
    assert_bits_equal(bits(qb)[0], wq_, "q rows vs oracle")
    assert_bits_equal(bits(kb)[0], wk_, "k rows vs oracle")
    assert_bits_equal(bits(key_b)[0], ek[:, :cap], "key cache vs oracle")
    assert_bits_equal(bits(val_b)[0], ev[:, :cap], "value cache vs oracle")


def test_fused_rope_attention_graph_replays(C, dev):
    """Captured once, replayed with new rows and a longer prefix: every replay equals the two calls."""
    S, rd, cap = 8, 64, 4096
    g = torch.Generator().manual_seed(5)
    qg, q, k, v, wq, wk, f, key, val, pos = _inputs(g, S, rd, cap, 100, False)
    mask = torch.tensor(ref.tree_mask(_parents(S, g)), dtype=torch.int32, device=dev)
    seq = torch.tensor([100], dtype=torch.int32, device=dev)
    qd, kd_, vd_, wqd, wkd, fd = q.to(dev), k.to(dev), v.to(dev), wq.to(dev), wk.to(dev), f.to(dev)
    posd = pos.to(dev)
    key_b, val_b = key.to(dev), val.to(dev)
    kb = torch.empty(1, HK, S, D, dtype=torch.bfloat16, device=dev)
    out_b = torch.empty(1, S, H * D, dtype=torch.bfloat16, device=dev)
    C.qk_norm_rope_attn(qd, kd_, vd_, wqd, wkd, fd, key_b, val_b, posd, 1e-6, 2e-5, rd, seq, mask, kb, out=out_b)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            C.qk_norm_rope_attn(qd, kd_, vd_, wqd, wkd, fd, key_b, val_b, posd, 1e-6, 2e-5, rd, seq, mask, kb,
                                out=out_b)
    for rep, L in enumerate((300, 1500, 3000)):
        qd.copy_(torch.randn(q.shape, generator=g).bfloat16().to(dev))
        kd_.copy_(torch.randn(k.shape, generator=g).bfloat16().to(dev))
        seq.fill_(L)
        posd.copy_(torch.arange(L, L + S, dtype=torch.int64).to(dev))
        key_a, val_a = key_b.clone(), val_b.clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        qa, ka = C.qk_norm_rope_kv(qd, kd_, vd_, wqd, wkd, fd, key_a, val_a, posd, 1e-6, 2e-5, rd)
        out_a = C.attn_dpas(qa, key_a, val_a, seq, ka, vd_.transpose(1, 2), mask, 0)
        torch.cuda.synchronize()
        assert_bits_equal(bits(out_b), bits(out_a), f"replay {rep} output")
        assert_bits_equal(bits(kb), bits(ka), f"replay {rep} k rows")
        assert_bits_equal(bits(key_b), bits(key_a), f"replay {rep} key cache")
        assert_bits_equal(bits(val_b), bits(val_a), f"replay {rep} value cache")


def test_fused_rope_attention_rejects(C, dev):
    """Shapes outside the fused form raise before any launch (the caller keeps the two calls)."""
    assert not C.rope_attn_fits(H, HK, 4, D, 64)     # 16 query rows per kv head
    assert not C.rope_attn_fits(H, HK, 8, 256, 64)   # head_dim 256
    assert not C.rope_attn_fits(H, HK, 8, D, 96)     # rotary 96
    S = 4
    z = torch.zeros(1, S, H, D, dtype=torch.bfloat16, device=dev)
    zk = torch.zeros(1, S, HK, D, dtype=torch.bfloat16, device=dev)
    cache = torch.zeros(1, HK, 64, D, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError):
        C.qk_norm_rope_attn(z, zk, zk, None, None, torch.zeros(S, 32, 2, 2, device=dev), cache, cache.clone(),
                            torch.arange(S, device=dev), 1.0, 1.0, 64, torch.zeros(1, dtype=torch.int32, device=dev),
                            torch.ones(S, dtype=torch.int32, device=dev),
                            torch.empty(1, HK, S, D, dtype=torch.bfloat16, device=dev))
