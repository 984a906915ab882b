"""Pins of the oracle's fused draft-head ops (oracle/ref.py: draft_*) against float64 restatements of
the eager ops they replace, within the reference's tolerance (tests/test_draft_fused.py:10-12: relative
L2 error below 1e-2; 2e-2 for the dequantised int8 row), and the gate / up index placement against a
one-hot construction."""
import numpy as np

from oracle import ref

H = 4096


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300)


def _bf(x):
    return ref.f32_to_bf16(np.asarray(x, np.float32))


def _rms64(x, w, eps):
    x = np.asarray(x, np.float64)
    return x * w / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def _h256():
    h = ref.H4.astype(np.float64)
    m = h
    for _ in range(3):
        m = np.kron(m, h)
    return m / 16


def test_embed_norm_cat_matches_f64():
    rng = np.random.default_rng(0)
    V = 50
    q = rng.integers(-127, 128, (V, H)).astype(np.int8)
    s = (rng.random(V) * 1e-3 + 1e-4).astype(np.float32)
    hid = _bf(rng.standard_normal((2, H)))
    we, wh = _bf(rng.random(H) + 0.5), _bf(rng.random(H) + 0.5)
    tok = np.array([7, 123])  # 123 is clamped to V - 1
    got = ref.draft_embed_norm_cat(hid, we, wh, 1e-6, 1e-6, q=q, s=s, token=tok, unrotate=True)
    t = np.array([7, V - 1])
    row = (q[t].astype(np.float64) * s[t][:, None].astype(np.float64)).reshape(2, -1, 256) @ _h256()
    emb = ref.bf16_to_f32(_bf(row.reshape(2, H)))
    want = np.concatenate([_rms64(emb, ref.bf16_to_f32(we), 1e-6), _rms64(ref.bf16_to_f32(hid), ref.bf16_to_f32(wh), 1e-6)], 1)
    assert _rel(ref.bf16_to_f32(got), want) < 1e-2
    # a given embedding row instead of the gather
    got2 = ref.draft_embed_norm_cat(hid, we, wh, 1e-6, 1e-6, emb_bits=_bf(emb))
    assert _rel(ref.bf16_to_f32(got2), want) < 1e-2


def test_add_rmsnorm_sigmoid_silu_match_f64():
    rng = np.random.default_rng(1)
    x, h = _bf(rng.standard_normal((1, H))), _bf(rng.standard_normal((1, H)))
    w = _bf(rng.random(H) + 0.5)
    xn, out = ref.draft_add_rmsnorm(x, h, w, 1e-6)
    x64 = ref.bf16_to_f32(x).astype(np.float64) + ref.bf16_to_f32(h)
    assert np.array_equal(xn, _bf(x64))  # one fp32 add of bf16 values, one rounding
    assert _rel(ref.bf16_to_f32(out), _rms64(ref.bf16_to_f32(xn), ref.bf16_to_f32(w), 1e-6)) < 1e-2
    xn2, _ = ref.draft_add_rmsnorm(x, None, w, 1e-6)
    assert np.array_equal(xn2, x)
    import torch
    sig = torch.sigmoid(torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)).view(torch.int16)
    sig = sig.numpy().view(np.uint16)
    silu = torch.nn.functional.silu(torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16))
    silu = silu.view(torch.int16).numpy().view(np.uint16)
    a, qg = _bf(rng.standard_normal((1, H))), _bf(rng.standard_normal((1, 2 * H)))
    got = ref.draft_sigmoid_mul(a, qg, 256, sig)
    gate = ref.bf16_to_f32(qg).reshape(16, 512)[:, 256:].reshape(1, H).astype(np.float64)
    assert _rel(ref.bf16_to_f32(got), ref.bf16_to_f32(a) / (1 + np.exp(-gate))) < 1e-2
    gu = _bf(rng.standard_normal((1, 2 * 12288)))
    g64, u64 = ref.bf16_to_f32(gu[:, :12288]).astype(np.float64), ref.bf16_to_f32(gu[:, 12288:])
    assert _rel(ref.bf16_to_f32(ref.draft_silu_mul(gu, silu)), g64 / (1 + np.exp(-g64)) * u64) < 1e-2


def test_sigmoid_gate_index_one_hot():
    """Only the gate element of (head, d) drives output (head, d): a one-hot large gate at head 2, d 5
    of the second half opens exactly that output."""
    D, heads = 8, 4
    lut = ref.f32_to_bf16(1 / (1 + np.exp(-ref.bf16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16)).astype(np.float64))))
    a = _bf(np.ones((1, heads * D)))
    qg = np.full((1, heads * 2 * D), _bf(-30.0), np.uint16)
    qg[0, 2 * 2 * D + D + 5] = _bf(30.0)
    qg[0, 1 * 2 * D + 3] = _bf(30.0)  # a query-half element: no effect
    out = ref.bf16_to_f32(ref.draft_sigmoid_mul(a, qg, D, lut))[0]
    assert out[2 * D + 5] == 1.0 and np.count_nonzero(out > 0.5) == 1


def test_norm_rot_quant_matches_f64():
    rng = np.random.default_rng(2)
    x, d = _bf(rng.standard_normal((1, H))), _bf(rng.standard_normal((1, H)))
    w = _bf(rng.random(H) + 0.5)
    xn, xr, q, sc = ref.draft_norm_rot_quant(x, d, w, 1e-6)
    assert np.array_equal(xn, ref.add_bf16(x, d))
    n = _rms64(ref.bf16_to_f32(xn), ref.bf16_to_f32(w), 1e-6)
    rot = (n.reshape(1, -1, 256) @ _h256()).reshape(1, H)
    assert _rel(ref.bf16_to_f32(xr), rot) < 1e-2
    assert _rel(q.astype(np.float64) * sc[:, None], rot) < 2e-2
    assert np.abs(q).max() == 127
    # unrotated: xr is the normed row itself
    _, xr0, _, _ = ref.draft_norm_rot_quant(x, d, w, 1e-6, rot="none")
    assert _rel(ref.bf16_to_f32(xr0), n) < 1e-2
