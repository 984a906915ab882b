"""The exact attention's restatement (oracle/ref.py exp_c, attention_exact) pinned on the CPU: exp_c
against float64 exp over its whole input range (within 2 units of 2^-24) and at its special points; the
attention against the float64 reference within the float32 chain's own error, a uniform-weight case in
closed form (q = 0: the mean of the admitted value rows), and the tree-row / empty-row rules."""
import numpy as np
import pytest

from oracle import ref


def test_exp_c_against_float64():
    x = -np.linspace(0, 79.99, 400001).astype(np.float32)
    y = ref.exp_c(x).astype(np.float64)
    t = np.exp(x.astype(np.float64))
    assert (np.abs(y - t) / t).max() < 2 * 2 ** -24
    assert ref.exp_c(np.float32(0)) == 1.0
    assert ref.exp_c(np.float32(-80.5)) == 0 and ref.exp_c(np.float32(-np.inf)) == 0
    assert ref.exp_c(np.float32(np.nan)) == 0


def _case(seed, H=4, Hk=2, S=4, D=64, L=70, cap=80):
    g = np.random.default_rng(seed)
    bf = lambda *sh: ref.f32_to_bf16(g.standard_normal(sh).astype(np.float32))
    return bf(H, S, D), bf(Hk, cap, D), bf(Hk, cap, D), bf(Hk, S, D), bf(Hk, S, D)


@pytest.mark.parametrize("L,mask", [(70, [1, 3, 5, 9]), (70, None), (0, [1, 3, 5, 9]), (1, [1, 2, 4, 8])])
def test_attention_exact_against_float64(L, mask):
    q, k, v, xk, xv = _case(1)
    S = 4 if mask is not None else 1
    q, xk, xv = q[:, :S], xk[:, :S], xv[:, :S]
    scale = np.float32(1 / np.sqrt(64))
    got = ref.bf16_to_f32(ref.attention_exact(q, k, v, L, xk, xv, mask, scale)).astype(np.float64)
    f = ref.bf16_to_f32
    want = ref.attention_f64(f(q), f(k), f(v), L, f(xk), f(xv), mask).reshape(S, -1)
    assert np.abs(got - want).max() <= 2 ** -7 * np.abs(want).max() + 1e-6


def test_uniform_weights_give_the_mean():
    q, k, v, xk, xv = _case(2)
    q = np.zeros_like(q)  # every score 0: weights 1, the output the mean of the admitted rows
    mask = [1, 3, 5, 9]
    got = ref.bf16_to_f32(ref.attention_exact(q, k, v, 70, xk, xv, mask, np.float32(0.125))).reshape(4, 4, 64)
    f = ref.bf16_to_f32
    for s in range(4):
        rows = [t for t in range(4) if (mask[s] >> t) & 1]
        for h in range(4):
            V = np.concatenate([f(v)[h // 2, :70], f(xv)[h // 2, rows]]).astype(np.float64)
            assert np.allclose(got[s, h], V.mean(0), atol=2 ** -7 * np.abs(V.mean(0)).max() + 1e-3)


def test_no_tokens_give_zero():
    q, k, v, xk, xv = _case(3)
    out = ref.attention_exact(q[:, :1], k, v, 0, xk[:, :1], xv[:, :1], None, np.float32(0.125))
    assert (out == 0).all()
