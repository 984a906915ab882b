"""Pins of the RoPE / head-norm / accept-walk oracle (oracle/ref.py) by closed forms, float64 and
hand-worked trees. CPU only."""
import numpy as np

from oracle import ref


def _bits(rng, shape, scale=1.0):
    return ref.f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def test_rope_index_placement():
    """Each of f00, f01, f10, f11 lands on its own term: one-hot matrices move whole halves."""
    rng = np.random.default_rng(10)
    S, H, D, rd = 3, 2, 128, 64
    t = _bits(rng, (S, H, D))
    x = ref.bf16_to_f32(t)
    h = rd // 2
    for (i, j), want_lo, want_hi in (((0, 0), x[..., :h], 0 * x[..., :h]),
                                     ((0, 1), x[..., h:rd], 0 * x[..., :h]),
                                     ((1, 0), 0 * x[..., :h], x[..., :h]),
                                     ((1, 1), 0 * x[..., :h], x[..., h:rd])):
        f = np.zeros((S, h, 2, 2), np.float32)
        f[..., i, j] = 1
        o = ref.bf16_to_f32(ref.rope_rows(t, f, rd))
        assert np.array_equal(o[..., :h], want_lo + 0) and np.array_equal(o[..., h:rd], want_hi + 0), (i, j)
        assert np.array_equal(ref.rope_rows(t, f, rd)[..., rd:], t[..., rd:])  # pass-through lanes


def test_rope_rotation_matches_complex_multiply():
    """f = [[cos, -sin], [sin, cos]]: o = rotation of (t[j], t[j+h]) by theta, checked in float64
    within the bf16 output rounding (plus the two fp32 product roundings)."""
    rng = np.random.default_rng(11)
    S, H, D, rd = 4, 3, 256, 128
    t = _bits(rng, (S, H, D), 3)
    th = rng.random((S, rd // 2)) * 2 * np.pi
    f = np.stack([np.stack([np.cos(th), -np.sin(th)], -1), np.stack([np.sin(th), np.cos(th)], -1)], -2).astype(np.float32)
    o = ref.bf16_to_f32(ref.rope_rows(t, f, rd)).astype(np.float64)
    x = ref.bf16_to_f32(t).astype(np.float64)
    f64 = f.astype(np.float64)[:, None]
    lo, hi = x[..., :rd // 2], x[..., rd // 2:rd]
    w0 = lo * f64[..., 0, 0] + hi * f64[..., 0, 1]
    w1 = hi * f64[..., 1, 1] + lo * f64[..., 1, 0]
    for got, want in ((o[..., :rd // 2], w0), (o[..., rd // 2:rd], w1)):
        tol = np.abs(want) * 2 ** -8 + (np.abs(lo) + np.abs(hi)) * 2 ** -23
        assert (np.abs(got - want) <= tol).all()


def test_rope_products_round_separately():
    """a*fa + b*fb with a cancellation where an FMA would keep the low bits of a*fa: the oracle
    rounds both products to fp32 first."""
    a = np.float32(1 + 2 ** -7)  # bf16-representable
    fa = np.float32(1 + 2 ** -20)
    b = np.float32(-1)
    fb = np.float32(1 + 2 ** -7)
    t = ref.f32_to_bf16(np.array([[[a, b]]], np.float32))
    f = np.array([[[[fa, fb], [0, 0]]]], np.float32)
    o = ref.bf16_to_f32(ref.rope_rows(t, f, 2))[0, 0, 0]
    prod = np.float32(a * fa)
    want = np.float32(prod + np.float32(b * fb))
    assert o == ref.bfround(want)
    fused = np.float32(float(a) * float(fa) + float(b) * float(fb))  # what an FMA would give
    assert ref.bfround(fused) != o or fused != want


def test_head_rmsnorm_close_to_float64():
    rng = np.random.default_rng(12)
    for D in (128, 256):
        for scale in (1.0, 1e-4, 30.0):
            x = _bits(rng, (5, 4, D), scale)
            w = ref.f32_to_bf16((1 + rng.standard_normal(D) * 0.3).astype(np.float32))
            got = ref.bf16_to_f32(ref.head_rmsnorm(x, w, 1e-6)).astype(np.float64)
            xf = ref.bf16_to_f32(x).astype(np.float64)
            want = xf / np.sqrt((xf * xf).mean(-1, keepdims=True) + 1e-6) * ref.bf16_to_f32(w)
            assert (np.abs(got - want) <= np.abs(want) * 2 ** -7 + 1e-30).all(), (D, scale)
    z = np.zeros((1, 1, 128), np.uint16)
    z[..., ::2] = 0x8000  # -0.0
    assert (ref.bf16_to_f32(ref.head_rmsnorm(z, np.full(128, 0x3F80, np.uint16), 1e-6)) == 0).all()


def test_accept_walk_hand_cases():
    # tree (4, 3): chain 0-1-2, siblings 3, 4, 5 at depth 1 and 6, 7 at depth 2 (tree order)
    parent, children, depth, chain = ref.tree_from_spec(ref.spec_of_widths((4, 3)), 8)
    assert children[0] == [1, 5, 6, 7] and children[1] == [2, 3, 4] and chain == 2
    assert parent == [-1, 0, 1, 1, 1, 0, 0, 0] and depth == [0, 1, 2, 2, 2, 1, 1, 1]
    toks = [10, 11, 12, 13, 14, 15, 16, 17]
    # all chain drafts match -> full chain, on chain
    dr = [0, 10, 11, 0, 0, 0, 0, 0]
    path, commit, ranks, row, on_chain, kept = ref.accept_walk(children, toks, dr, chain)
    assert path == [0, 1, 2] and commit == [10, 11, 12] and row == 2 and on_chain and kept == 2
    # the root's first matching child is a sibling -> off chain, then a dead end
    dr = [0, 99, 0, 0, 0, 10, 10, 0]
    path, commit, ranks, row, on_chain, kept = ref.accept_walk(children, toks, dr, chain)
    assert path == [0, 5] and commit == [10, 15] and row == 5 and not on_chain and kept == 1
    # on chain at depth 1, then the depth-2 sibling 4
    dr = [0, 10, 98, 97, 11, 0, 0, 0]
    cand = list(range(100, 149))
    cand[7 * 0 + 3] = 10
    path, commit, ranks, row, on_chain, kept = ref.accept_walk(children, toks, dr, chain, cand)
    assert path == [0, 1, 4] and commit == [10, 11, 14] and not on_chain and kept == 2
    assert ranks == [3, 7]  # node 0: rank 3; node 1: not among its candidates
    rec = ref.accept_record(8, path, commit, ranks, row, on_chain, kept, 33)
    assert len(rec) == 21 and rec[:4] == [3, 10, 11, 14] and rec[9:12] == [4, 0, 2] and rec[19:] == [33, 2]


def test_commit_path_moves_in_order():
    cache = np.arange(2 * 10 * 1).reshape(2, 10, 1)
    # path [0, 2, 3]: slot 5+1 <- slot 5+2 (read before k=2 overwrites it), then slot 5+2 <- slot 5+3
    out = ref.commit_path(cache, [0, 2, 3], False, 5)
    assert out[0, :, 0].tolist() == [0, 1, 2, 3, 4, 5, 7, 8, 8, 9]
    # wrap-around of the ring
    out = ref.commit_path(cache, [0, 2], False, 9)
    assert out[0, 0, 0] == 1 and out[0, 1, 0] == 1
    assert np.array_equal(ref.commit_path(cache, [0, 1, 2], True, 5), cache)
