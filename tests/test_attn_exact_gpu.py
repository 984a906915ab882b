"""The exact attention (mdx_attn_exact) on the GPU against its restatement (oracle/ref.py attention_exact)
bit for bit: tree rows with masks, the draft row without a mask, an empty prefix, head dims 64 / 128 / 256,
GQA groups; the A/B switch routing attn_dpas through it; the fast kernel within the float64 bound of the
exact one's inputs; a decode with exact attention."""
import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits
from oracle import ref

pytestmark = pytest.mark.gpu


def _inputs(g, H, Hk, S, D, cap, dev):
    r = lambda *sh: torch.randn(*sh, generator=g).bfloat16()
    return r(1, H, S, D), r(1, Hk, cap, D), r(1, Hk, cap, D), r(1, Hk, S, D), r(1, Hk, S, D)


@pytest.mark.parametrize("H,Hk,S,D,L,cap,tree", [(32, 8, 8, 128, 300, 320, True), (32, 8, 1, 128, 257, 260, False),
                                                 (8, 2, 16, 256, 100, 130, True), (4, 4, 4, 64, 0, 16, True),
                                                 (16, 4, 3, 64, 1000, 1024, True)])
def test_exact_attention_bit_for_bit(C, dev, H, Hk, S, D, L, cap, tree):
    print(f"case attn_exact H={H} Hk={Hk} S={S} D={D} L={L}", flush=True)
    g = torch.Generator().manual_seed(H * S + D + L)
    q, k, v, xk, xv = _inputs(g, H, Hk, S, D, cap, dev)
    parents = [-1] + [int(torch.randint(0, r, (1,), generator=g)) for r in range(1, S)]
    mask = ref.tree_mask(parents) if tree else None
    md = torch.tensor(mask if tree else [], dtype=torch.int32, device=dev)
    seq = torch.tensor([L], dtype=torch.int32, device=dev)
    out = C.attn_exact(q.to(dev), k.to(dev), v.to(dev), seq, xk.to(dev), xv.to(dev), md)
    want = ref.attention_exact(bits(q)[0], bits(k)[0], bits(v)[0], L, bits(xk)[0], bits(xv)[0], mask,
                               np.float32(1.0 / np.sqrt(D)))
    assert_bits_equal(bits(out)[0], want, "exact attention")
    # the fast kernel: the float64 bound on the same inputs
    fast = C.attn_dpas(q.to(dev), k.to(dev), v.to(dev), seq, xk.to(dev), xv.to(dev), md, 0)
    f = lambda t: ref.bf16_to_f32(bits(t)[0])
    w64 = ref.attention_f64(f(q), f(k), f(v), L, f(xk), f(xv), mask).reshape(S, -1)
    for o in (out, fast):
        err = np.abs(ref.bf16_to_f32(bits(o)[0]).astype(np.float64) - w64)
        assert err.max() <= 2 ** -7 * np.abs(w64).max() + 1e-6


def test_switch_routes_attn_dpas(C, dev):
    g = torch.Generator().manual_seed(7)
    q, k, v, xk, xv = [t.to(dev) for t in _inputs(g, 32, 8, 4, 128, 200, dev)]
    md = torch.tensor(ref.tree_mask([-1, 0, 1, 0]), dtype=torch.int32, device=dev)
    seq = torch.tensor([150], dtype=torch.int32, device=dev)
    exact = C.attn_exact(q, k, v, seq, xk, xv, md)
    try:
        C.set_attention("exact")
        routed = C.attn_dpas(q, k, v, seq, xk, xv, md, 0)
    finally:
        C.set_attention("fast")
    assert torch.equal(routed, exact)
    assert not torch.equal(C.attn_dpas(q, k, v, seq, xk, xv, md, 0), exact)  # the fast kernel again
    with pytest.raises(RuntimeError):
        C.set_attention("port")


def test_decode_with_exact_attention(dev):
    from mdx import hybrid
    cfg = hybrid.HybridConfig(layers=4, inter=4096, vocab=32768, cap=256, greedy=True, attn="exact")
    m = hybrid.HybridModel(cfg, dev, seed=5)
    m.prefill(torch.randint(0, cfg.vocab, (37,), generator=torch.Generator().manual_seed(1)))
    for _ in range(3):
        st0 = m.st[0].item()
        m.step(m.parity)
        m.parity ^= 1
        torch.cuda.synchronize()
        assert torch.isfinite(m.logits.float()).all() and m.st[0].item() == st0 + m.result[0].item()
    m.capture()
    m.replay(2)
    torch.cuda.synchronize()


def test_attn_core_is_the_reference_name_of_the_exact_attention(C, dev):
    """_C.attn_core with the reference's positional arguments (q, key, value, seqlen, xk, xv, mask, nwg), as
    comfy_mono_decode_xpu/layer.py:428 calls it: the exact attention, bit for bit against the oracle, for a
    tree-verify call and a draft row (empty mask)."""
    g = torch.Generator().manual_seed(11)
    for H, Hk, S, D, L, cap, tree in ((32, 8, 8, 128, 400, 420, True), (32, 8, 1, 128, 99, 128, False)):
        print(f"case attn_core H={H} S={S} L={L}", flush=True)
        q, k, v, xk, xv = _inputs(g, H, Hk, S, D, cap, dev)
        mask = ref.tree_mask([-1] + list(range(S - 1))) if tree else None
        md = torch.tensor(mask if tree else [], dtype=torch.int32, device=dev)
        seq = torch.tensor([L], dtype=torch.int32, device=dev)
        out = C.attn_core(q.to(dev), k.to(dev), v.to(dev), seq, xk.to(dev), xv.to(dev), md, 0)
        assert out.shape == (1, S, H * D) and out.dtype == torch.bfloat16
        want = ref.attention_exact(bits(q)[0], bits(k)[0], bits(v)[0], L, bits(xk)[0], bits(xv)[0], mask,
                                   np.float32(1.0 / np.sqrt(D)))
        assert_bits_equal(bits(out)[0], want, "attn_core")
