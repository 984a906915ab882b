"""Pins of the top-k oracle: the gather order against an explicit enumeration of the sweep, the radix
keys against value order over every bf16 pattern and special fp32 values, argmax and top-k against
brute force. CPU only."""
import numpy as np
import torch

from oracle import ref


def _enumerate_sweep(n, loads, width):
    """The element indices in the order a sweep of 1024 threads x `loads` vector loads of `width` visits
    them, written as the nested loops of the sweep itself."""
    order = []
    for it in range((n + 32767) // 32768):
        for thread in range(1024):
            for load in range(loads):
                for lane in range(width):
                    i = it * 32768 + load * 1024 * width + thread * width + lane
                    if i < n:
                        order.append(i)
    return np.array(order)


def test_gather_order_matches_sweep_enumeration():
    for loads, width in ((4, 8), (8, 4)):
        seq = _enumerate_sweep(70000, loads, width)
        assert sorted(seq.tolist()) == list(range(70000))
        pos = ref.gather_pos(seq, loads, width)
        assert (np.diff(pos) > 0).all()  # the visit order is the increasing gather position


def test_bf16_key_orders_like_values():
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = ref.bf16_to_f32(allb).astype(np.float64)
    key = ref.key_bf16(allb)
    fin = ~np.isnan(f)
    o = np.argsort(key[fin], kind="stable")
    fv = f[fin][o]
    assert (np.diff(fv) >= 0).all()  # non-decreasing values along increasing keys
    assert len(np.unique(key[fin])) == fin.sum()  # distinct (so -0 and +0 differ)
    assert ref.key_bf16(np.uint16(0x8000)) < ref.key_bf16(np.uint16(0x0000))
    assert (key[~fin] == 0xFFFF).all() and (key[fin] < 0xFFFF).all() and (key[fin] > 0).all()


def test_f32_key_orders_like_values():
    rng = np.random.default_rng(20)
    v = np.concatenate([rng.standard_normal(5000).astype(np.float32) * 1e3,
                        np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 3.4e38, -3.4e38], np.float32)])
    u = v.view(np.uint32)
    k = ref.key_f32(u)
    o = np.argsort(k)
    assert (np.diff(v[o].astype(np.float64)) >= 0).all()
    assert ref.key_f32(np.float32(-0.0).view(np.uint32)) < ref.key_f32(np.float32(0.0).view(np.uint32))
    assert ref.key_f32(np.uint32(0x7FC00000)) > ref.key_f32(np.float32(np.inf).view(np.uint32))
    assert ref.key_f32(np.uint32(0xFFC00000)) < ref.key_f32(np.float32(-np.inf).view(np.uint32))


def test_argmax_brute_force():
    rng = np.random.default_rng(21)
    for trial in range(200):
        n = 40
        x = ref.f32_to_bf16(np.round(rng.standard_normal(n) * 2).astype(np.float32))
        if trial % 3 == 0:
            x[rng.integers(0, n, 3)] = 0x8000  # -0
        if trial % 5 == 0:
            x[rng.integers(0, n)] = 0x7FC0
        f = ref.bf16_to_f32(x)
        nans = np.flatnonzero(np.isnan(f))
        if nans.size:
            want = int(nans[0])
        else:
            best = max(f)  # -0 == +0 under float comparison
            want = int(np.flatnonzero(f == best)[0])
        assert ref.argmax_bf16(x) == want


def test_topk_distinct_values_match_sort():
    rng = np.random.default_rng(22)
    x = rng.permutation(np.arange(40000, dtype=np.float32) - 20000) / 8
    xb = ref.f32_to_bf16(x)  # rounding to bf16 makes ties; the values are compared, not the indices
    f = ref.bf16_to_f32(xb)
    vals, idx = ref.fast_topk(xb, 8)
    want = np.sort(f)[::-1][:8]
    assert np.array_equal(ref.bf16_to_f32(vals), want)
    xf = rng.standard_normal((3, 50000)).astype(np.float32)
    v, i = ref.topk_rows(xf, 20)
    assert np.array_equal(v, -np.sort(-xf, axis=1)[:, :20])
    assert np.array_equal(np.take_along_axis(xf, i, 1), v)


def test_topk_ties_follow_gather_order():
    n = 70000
    seq4x8, seq8x4 = _enumerate_sweep(n, 4, 8), _enumerate_sweep(n, 8, 4)
    ones = ref.f32_to_bf16(np.ones(n, np.float32))
    assert ref.fast_topk(ones, 8)[1].tolist() == seq4x8[:8].tolist()
    assert ref.topk_rows(np.ones((1, n), np.float32), 64)[1][0].tolist() == seq8x4[:64].tolist()
    # ties at the top value plus a few larger ones
    x = np.zeros(n, np.float32)
    x[[5, 40000, 69999]] = 2
    x[seq8x4[100:200]] = 1
    v, i = ref.topk_rows(x[None], 10)
    assert i[0, :3].tolist() == [5, 40000, 69999] and i[0, 3:].tolist() == seq8x4[100:107].tolist()


def test_topk_matches_torch_on_distinct_rows():
    # torch-CPU topk has its own tie order, so it is compared only on rows without ties
    g = torch.Generator().manual_seed(23)
    x = torch.randperm(151936, generator=g).float().view(1, -1) / 3
    v, i = ref.topk_rows(x.numpy(), 20)
    tv, ti = torch.topk(x, 20)
    assert np.array_equal(i, ti.numpy()) and np.array_equal(v, tv.numpy())


def test_splitmix64_known_answers():
    """The sampling uniforms' mixer is SplitMix64's: the generator seeded with 0 (state += gamma, then the
    output function) gives 0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4, 0x06c45d188009454f."""
    state, outs = 0, []
    for _ in range(3):
        state = (state + ref.SPLITMIX_GAMMA) & ((1 << 64) - 1)
        outs.append(ref.splitmix64_mix(state))
    assert outs == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    # seeded_uniform(seed, counter, r, j) is the (n + 1)-th output of the generator seeded with `seed`
    seed = 12345
    for n in (0, 1, 1023, 4096 + 64 * 3 + 5):
        z = ref.splitmix64_mix((seed + (n + 1) * ref.SPLITMIX_GAMMA) & ((1 << 64) - 1))
        u = ref.seeded_uniform(seed, n // 1024, (n % 1024) // 64, n % 64)
        assert u == np.float32(((z >> 41) + 0.5) / 2 ** 23) and 0.0 < u < 1.0


def test_seeded_uniforms_spread():
    """The uniforms of consecutive rows, slots and counters fill (0, 1) evenly (a mixing or indexing
    mistake that repeats whole runs of values or leaves a bias shows here)."""
    u = np.array([ref.seeded_uniform(7, c, r, j) for c in range(8) for r in range(4) for j in range(64)])
    assert len(np.unique(u)) >= u.size - 2  # 23-bit values: a birthday collision or two is expected
    hist = np.histogram(u, bins=8, range=(0.0, 1.0))[0]
    assert abs(u.mean() - 0.5) < 0.03 and hist.min() > 0.8 * u.size / 8
