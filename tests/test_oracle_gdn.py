"""Pins of the oracle's Gated-DeltaNet step (oracle/ref.py: gdn_conv, gdn_gates, gdn_delta, gdn_step)
against independent restatements, in float64 (no bf16 rounding anywhere):

- the delta rule of one entry against the textbook matrix form on the transposed state
  M = S^T [d_v, d_k]: M' = a M (I - b k k^T) + b v k^T, o = M' q;
- b = 0 gives S' = a S; a non-committing entry leaves the state as it is;
- the causal conv of a chain against np.convolve over (history, rows);
- decay / beta against math.exp / math.log1p closed forms (both softplus branches);
- a whole tree step, every row, against a plain sequential GDN evaluated over that row's ancestor
  path (conv over the path, gates, L2 norms, recurrence, gated RMSNorm), and the deferred replay of an
  accepted prefix on the next step against the same sequential run continued;
- an invalid accepted slot: the persistent state and the outputs are left alone.

Reference: csrc/mono_gdn.sycl:313-374 (conv), :441-450 (gates), :464-498 (sums, norms), :526-571
(entries), :568 (the commit of the replayed state), :574-607 (gated RMSNorm)."""
import math

import numpy as np
import pytest

from oracle import ref

DH = 128


def _silu(y):
    return y / (1.0 + np.exp(-y))


def _gates_closed(a, b, dt, g):
    x = a + dt
    sp = x if x > 20 else math.log1p(math.exp(x))
    return math.exp(g * sp), 1.0 / (1.0 + math.exp(-b))


def seq_gdn(hist, rows, conv_w, S0, a, b, z, dt, g, gw, eps, qscale, HK):
    """A plain GDN over a token sequence (no tree, no deferral), float64. hist [C, 3] (oldest first),
    rows [T, C] projections, S0 [HV, d_k, d_v] (the library's storage), a/b [T, HV], z [T, HV * DH].
    Returns outputs [T, HV * DH] and the final state in the same storage."""
    T, C = rows.shape
    HV = S0.shape[0]
    KD = HK * DH
    full = np.concatenate([hist.T, rows])  # [3 + T, C]
    conv = np.empty((T, C))
    for c in range(C):
        conv[:, c] = np.convolve(full[:, c], conv_w[c, ::-1])[3:3 + T]
    conv = _silu(conv)
    M = np.array([S0[h].T for h in range(HV)])  # [HV, d_v, d_k]
    out = np.zeros((T, HV * DH))
    for t in range(T):
        for h in range(HV):
            kh = h // (HV // HK)
            q = conv[t, kh * DH:(kh + 1) * DH]
            k = conv[t, KD + kh * DH:KD + (kh + 1) * DH]
            v = conv[t, 2 * KD + h * DH:2 * KD + (h + 1) * DH]
            kn = k / max(np.linalg.norm(k), 1e-12)
            qn = q * qscale / max(np.linalg.norm(q), 1e-12)
            al, be = _gates_closed(a[t, h], b[t, h], dt[h], g[h])
            M[h] = al * M[h] @ (np.eye(DH) - be * np.outer(kn, kn)) + be * np.outer(v, kn)
            o = M[h] @ qn
            zz = z[t, h * DH:(h + 1) * DH]
            out[t, h * DH:(h + 1) * DH] = o * gw / np.sqrt(np.mean(o * o) + eps) * _silu(zz)
    return out, np.array([M[h].T for h in range(HV)])


def _case(rng, HK=1, HV=2):
    C = 2 * HK * DH + HV * DH
    return dict(HK=HK, HV=HV, C=C, conv_w=rng.standard_normal((C, 4)) * 0.5, dt=rng.uniform(-1, 1, HV),
                g=-np.exp(rng.uniform(-1, 0.5, HV)), gw=1 + rng.standard_normal(DH) * 0.1,
                hist=rng.standard_normal((C, 3)), S0=rng.standard_normal((HV, DH, DH)) * 0.1)


def _state(cs, slots):
    return dict(conv_state=cs["hist"].copy(), pb=np.zeros((2, slots, cs["C"])), qb=np.zeros((2, slots, cs["C"])),
                rec=cs["S0"].copy(), gates=np.zeros((2, slots, cs["HV"], 2)), sums=np.zeros((2, slots, cs["HK"], 2)))


def test_delta_entry_matches_matrix_form():
    rng = np.random.default_rng(0)
    for _ in range(5):
        S = rng.standard_normal((DH, DH))
        k = rng.standard_normal(DH)
        k /= np.linalg.norm(k)
        v, q = rng.standard_normal(DH), rng.standard_normal(DH)
        al, be = rng.uniform(0.2, 1.0), rng.uniform(0, 1)
        got = ref.gdn_delta(S, k, v, al, be)
        M = S.T
        want = (al * M @ (np.eye(DH) - be * np.outer(k, k)) + be * np.outer(v, k)).T
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(q @ got, (want.T @ q), rtol=1e-12, atol=1e-12)
        # beta = 0: pure decay
        np.testing.assert_allclose(ref.gdn_delta(S, k, v, al, 0.0), al * S, rtol=0, atol=0)
        # beta = 1, decay = 1 with a unit key: the key's memory becomes exactly v
        np.testing.assert_allclose(k @ ref.gdn_delta(S, k, v, 1.0, 1.0), v, rtol=1e-12, atol=1e-12)


def test_gates_closed_forms():
    a = np.array([[-3.0, 0.5, 19.0, 25.0]])
    b = np.array([[-4.0, 0.0, 2.0, 30.0]])
    dt = np.array([0.25, -0.5, 0.9, 0.0])
    g = np.array([-0.7, -1.3, -0.2, -2.0])
    dec, bet = ref.gdn_gates(a, b, dt, g)
    for h in range(4):
        wd, wb = _gates_closed(a[0, h], b[0, h], dt[h], g[h])
        assert dec[0, h] == pytest.approx(wd, rel=1e-14)
        assert bet[0, h] == pytest.approx(wb, rel=1e-14)
    assert dec[0, 3] == pytest.approx(math.exp(-2.0 * 25.0), rel=1e-14)  # the softplus(x) = x branch


def test_chain_conv_matches_np_convolve():
    rng = np.random.default_rng(1)
    cs = _case(rng)
    slots, R = 8, 6
    st = _state(cs, slots)
    proj = rng.standard_normal((R, cs["C"]))
    ctl = [0, 0] + [0] * slots + list(range(-1, R - 1)) + [-1] * (slots - R) + [0] * slots
    got = ref.gdn_conv(st, proj, cs["conv_w"], np.array(ctl), R, slots)
    full = np.concatenate([cs["hist"].T, proj])
    for c in range(cs["C"]):
        y = np.convolve(full[:, c], cs["conv_w"][c, ::-1])[3:3 + R]
        np.testing.assert_allclose(got[:R, c], _silu(y), rtol=1e-12, atol=1e-13)
    assert not got[R:].any()


def _tree(widths, slots):
    parents = ref.tree_from_spec(ref.spec_of_widths(widths), slots)[0]
    R = 1 + sum(widths)
    return parents[:R], R


def _path(parents, r):
    p = [r]
    while parents[p[-1]] >= 0:
        p.append(parents[p[-1]])
    return p[::-1]


@pytest.mark.parametrize("widths", [(4, 3), (1, 1, 1), (2, 2, 2, 1)])
def test_tree_step_and_replay_match_sequential(widths):
    rng = np.random.default_rng(2 + len(widths))
    cs = _case(rng)
    HK, HV, C = cs["HK"], cs["HV"], cs["C"]
    slots = 8
    parents, R = _tree(widths, slots)
    prog = ref.verify_program(parents, R)
    st = _state(cs, slots)
    eps, qs = 1e-6, DH ** -0.5
    steps = []
    accepted, pending = [0] * slots, 0
    hist, S = cs["hist"].copy(), cs["S0"].copy()
    for step in range(2):
        p = step % 2
        proj = rng.standard_normal((R, C))
        z = rng.standard_normal((R, HV * DH))
        a = rng.standard_normal((R, HV))
        b = rng.standard_normal((R, HV))
        ctl = np.array([pending, p] + accepted + parents + [-1] * (slots - R) + prog + [0] * (slots - R))
        core = ref.gdn_step(st, proj, z, a, b, cs["conv_w"], cs["dt"], cs["g"], cs["gw"], eps, qs, ctl, R, HK, slots)
        if step == 1:
            # the deferred replay of the accepted prefix committed exactly the sequential state
            np.testing.assert_allclose(st["rec"], S, rtol=1e-10, atol=1e-12)
            np.testing.assert_allclose(st["conv_state"], hist, rtol=0, atol=0)
        for r in range(R):
            path = _path(parents, r)
            o, _ = seq_gdn(hist, proj[path], cs["conv_w"], S, a[path], b[path], z[path], cs["dt"], cs["g"], cs["gw"],
                           eps, qs, HK)
            np.testing.assert_allclose(core[r], o[-1], rtol=1e-9, atol=1e-11, err_msg=f"step {step} row {r}")
        # accept a prefix of the chain; the sequential run continues over it
        chain = _path(parents, max(range(R), key=lambda r: len(_path(parents, r))))
        n = int(rng.integers(1, len(chain) + 1))
        _, S = seq_gdn(hist, proj[chain[:n]], cs["conv_w"], S, a[chain[:n]], b[chain[:n]], z[chain[:n]], cs["dt"],
                       cs["g"], cs["gw"], eps, qs, HK)
        hist = np.concatenate([hist.T, proj[chain[:n]]])[-3:].T
        accepted, pending = chain[:n] + [0] * (slots - n), n
        steps.append(n)


def test_no_pending_rows_leave_state():
    rng = np.random.default_rng(7)
    cs = _case(rng)
    slots = 8
    parents, R = _tree((2, 2), slots)
    st = _state(cs, slots)
    ctl = np.array([0, 0] + [0] * slots + parents + [-1] * (slots - R) + ref.verify_program(parents, R)
                   + [0] * (slots - R))
    ref.gdn_step(st, rng.standard_normal((R, cs["C"])), rng.standard_normal((R, cs["HV"] * DH)),
                 rng.standard_normal((R, cs["HV"])), rng.standard_normal((R, cs["HV"])), cs["conv_w"], cs["dt"],
                 cs["g"], cs["gw"], 1e-6, DH ** -0.5, ctl, R, cs["HK"], slots)
    np.testing.assert_array_equal(st["rec"], cs["S0"])


@pytest.mark.parametrize("bad", [-1, 8, 13])
def test_invalid_accepted_slot_replays_nothing(bad):
    rng = np.random.default_rng(8)
    cs = _case(rng)
    slots = 8
    parents, R = _tree((4, 3), slots)
    st = _state(cs, slots)
    st["qb"][1] = rng.standard_normal((slots, cs["C"]))
    st["gates"][1] = rng.uniform(0.1, 0.9, (slots, cs["HV"], 2))
    st["sums"][1] = rng.uniform(0.5, 2.0, (slots, cs["HK"], 2))
    ctl = np.array([3, 0] + [0, bad, 2] + [0] * (slots - 3) + parents + [-1] * (slots - R)
                   + ref.verify_program(parents, R) + [0] * (slots - R))
    core = ref.gdn_step(st, rng.standard_normal((R, cs["C"])), rng.standard_normal((R, cs["HV"] * DH)),
                        rng.standard_normal((R, cs["HV"])), rng.standard_normal((R, cs["HV"])), cs["conv_w"], cs["dt"],
                        cs["g"], cs["gw"], 1e-6, DH ** -0.5, ctl, R, cs["HK"], slots)
    np.testing.assert_array_equal(st["rec"], cs["S0"])
    assert not core.any()
