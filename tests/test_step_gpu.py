"""One decode step of the hybrid stack against the oracle's composition of the reference step
(comfy_mono_decode_xpu/mtp_loop.py:326-390: drafts -> verify layers -> final norm -> lm_head -> top-k ->
pick -> accept; the draft block of comfy_mono_decode_xpu/draft_head.py:179-212), stage by stage.

A 2-layer model (one Gated-DeltaNet layer, one attention layer) at full width: hidden 4096, MLP 12288,
vocab 151936, tree (4, 3), greedy picks. The step runs eagerly with its trace on; each stage is then
checked against the oracle applied to that stage's own inputs (the GPU's output of the previous stage,
or the state snapshot taken before the step): bit for bit wherever the arithmetic is fixed (the fused
draft ops, norms, RoPE and KV writes, the W4A8 segments, top-k, the pick, the accept record, counters,
hidden row and KV slot moves), within the float64 bounds of the bf16 GEMMs, attention and the GDN core
elsewhere."""
import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits
from oracle import ref

pytestmark = pytest.mark.gpu


def _np(t):
    return bits(t)


def _w4(w):
    from mdx import layout
    return dict(packed=layout.row_major_codes(w.q).cpu().numpy(), s=w.s.float().cpu().numpy(), sch=w.sc.cpu().numpy(),
                cb=None, G=128)


def _rows(wt):
    """The row-major [N, K] view of a tile-major bf16 weight (the inverse of layout.tile_major_bf16)."""
    N, K = wt.shape
    return wt.reshape(N // 16, K // 32, 4, 16, 8).permute(0, 3, 1, 2, 4).contiguous().reshape(N, K)


def _bf16_bound(got_bits, x_bits, w_bits, what):
    """bf16(x . W^T) within 2^-8 relative + the fp32 accumulation bound (2^-16 sum |x||w|)."""
    want, scale = ref.bf16_linear_f64(x_bits, w_bits)
    got = ref.bf16_to_f32(got_bits).astype(np.float64)
    err = np.abs(got - want)
    bound = np.abs(want) * 2 ** -8 + scale * 2 ** -16 + 1e-30
    assert (err <= bound).all(), (what, float((err / bound).max()))


def _attn_bound(got, q, k, v, L, xk, xv, mask, what):
    want = ref.attention_f64(q, k, v, L, xk, xv, mask)
    chain = ref.bf16_to_f32(ref.f32_to_bf16(ref.attention_f64(q, k, v, L, xk, xv, mask, dtype=np.float32)))
    e_ref = np.abs(chain.astype(np.float64) - want)
    err = np.abs(got - want)
    assert err.max() <= 1.5 * e_ref.max() + 1e-3, (what, err.max(), e_ref.max())
    assert err.mean() <= 1.5 * e_ref.mean() + 1e-5, (what, err.mean(), e_ref.mean())


@pytest.mark.parametrize("head,scales", [("bf16", "faithful"), ("int8", "faithful"), ("bf16", "integral")])
def test_decode_step_matches_oracle(C, dev, head, scales):
    from mdx import hybrid, layout
    cfg = hybrid.HybridConfig(layers=2, attn_every=2, cap=128, greedy=True, head=head, scales=scales)
    m = hybrid.HybridModel(cfg, dev, seed=11)
    m.prefill(torch.randint(0, cfg.vocab, (24,), generator=torch.Generator().manual_seed(3)))
    torch.cuda.synchronize()
    D, eps = cfg.head_dim, cfg.eps
    qd, kd = cfg.heads * D, cfg.kv_heads * D
    S, R, T = cfg.slots, m.R, m.tree
    snap = dict(st=m.st.cpu().numpy().copy(), ctl=m.ctl.cpu().numpy().copy(), nt=int(m.nt.item()),
                hbuf=_np(m.hbuf), mk=_np(m.mkv[0])[0], mv=_np(m.mkv[1])[0],
                key=_np(m.kv[1][0])[0], value=_np(m.kv[1][1])[0],
                gdn={k: v.float().cpu().numpy().copy() for k, v in m.gdn[0].items()})
    parity = m.parity
    m.trace = []
    m.step(parity)
    torch.cuda.synchronize()
    tr = {}
    for name, t in m.trace:
        tr.setdefault(name, []).append(t)
    M = m.mtp
    sig = _np(layout.sigmoid_lut())
    lut = _np(m.silu)
    ftab = m.ftab.cpu().numpy()
    rowmaj = _rows

    # ---- drafts -------------------------------------------------------------------------------------
    st0, st1 = int(snap["st"][0]), int(snap["st"][1])
    mk, mv = snap["mk"].copy(), snap["mv"].copy()
    tok, h = snap["nt"], snap["hbuf"]
    cols = np.random.default_rng(1).choice(cfg.vocab, 2048, replace=False)
    cols_d = torch.from_numpy(cols).to(dev)
    if head == "int8":
        q8 = layout.row_major_i8(m.lm8)[cols_d].cpu().numpy()
        s8 = m.lm8_s[cols_d].cpu().numpy()
    else:
        lm_cols = _np(rowmaj(m.lm_head)[cols_d])
    for k, width in enumerate(cfg.widths):
        print(f"case step draft {k}", flush=True)
        g = lambda n: _np(tr[f"mtp.{n}"][k])
        emb = _np(m.embed[tok:tok + 1])
        assert_bits_equal(g("cat"), ref.draft_embed_norm_cat(h, _np(M["norm_e"]), _np(M["norm_h"]), eps, eps, emb_bits=emb),
                          f"draft {k} cat")
        _bf16_bound(g("x_fc"), g("cat"), _np(rowmaj(M["fc"])), f"draft {k} fc")
        assert_bits_equal(g("xn_in"), ref.draft_add_rmsnorm(g("x_fc"), None, _np(M["norm_in"]), eps)[1], f"draft {k} norm_in")
        _bf16_bound(g("qkv"), g("xn_in"), _np(rowmaj(M["qkv"])), f"draft {k} qkv")
        qkv = g("qkv")
        q = qkv[:, :2 * qd].reshape(1, cfg.heads, 2 * D)[:, :, :D]
        kk = qkv[:, 2 * qd:2 * qd + kd].reshape(1, cfg.kv_heads, D)
        vv = qkv[:, 2 * qd + kd:].reshape(1, cfg.kv_heads, D)
        freqs = ftab[st0 + k][None]
        rq, rk, mk, mv = ref.rope_kv(q, kk, vv, freqs, mk, mv, [st1 + k], cfg.rotary, _np(M["qn"]), _np(M["kn"]), eps, eps)
        assert_bits_equal(g("qo")[0], rq, f"draft {k} rope q")
        assert_bits_equal(g("ko")[0], rk, f"draft {k} rope k")
        f32 = ref.bf16_to_f32
        _attn_bound(f32(g("y")).reshape(1, cfg.heads, D).astype(np.float64), f32(rq), f32(mk), f32(mv), st1 + k + 1,
                    f32(rk), f32(vv.transpose(1, 0, 2)), None, f"draft {k} attention")
        assert_bits_equal(g("gy"), ref.draft_sigmoid_mul(g("y").reshape(1, qd), qkv[:, :2 * qd], D, sig), f"draft {k} gate")
        _bf16_bound(g("o"), g("gy"), _np(rowmaj(M["o"])), f"draft {k} o_proj")
        xp, xnp = ref.draft_add_rmsnorm(g("x_fc"), g("o"), _np(M["norm_post"]), eps)
        assert_bits_equal(g("x_post"), xp, f"draft {k} x + o")
        assert_bits_equal(g("xn_post"), xnp, f"draft {k} norm_post")
        _bf16_bound(g("gu"), g("xn_post"), _np(rowmaj(M["gu"])), f"draft {k} gate|up")
        assert_bits_equal(g("act"), ref.draft_silu_mul(g("gu"), lut), f"draft {k} silu")
        _bf16_bound(g("d"), g("act"), _np(rowmaj(M["d"])), f"draft {k} down")
        xo, xr, qx, sx = ref.draft_norm_rot_quant(g("x_post"), g("d"), _np(M["norm_f"]), eps,
                                                  rot="h256" if head == "int8" else "none")
        assert_bits_equal(g("x_out"), xo, f"draft {k} x + down")
        assert_bits_equal(g("xf"), xr, f"draft {k} final norm")
        logits = _np(tr["draft.logits"][k])
        if head == "int8":
            assert_bits_equal(g("qx"), qx, f"draft {k} head activation")
            assert_bits_equal(g("sx"), sx.view(np.uint32), f"draft {k} head activation scale")
            assert_bits_equal(logits[0, cols], ref.int8_head_logits(qx[0], sx, q8, s8), f"draft {k} int8 lm_head")
        else:
            _bf16_bound(logits[:, cols], g("xf"), lm_cols, f"draft {k} lm_head")
        _, top = ref.fast_topk(logits[0], width)
        vt = m.vtok.cpu().numpy()[0]
        assert vt[T["fill_rows"][k]].tolist() == top.tolist(), f"draft {k} tree tokens"
        tok, h = int(top[0]), g("x_out")
    assert int(m.vtok[0, 0].item()) == snap["nt"]
    assert_bits_equal(_np(m.mkv[0])[0], mk, "MTP key cache")
    assert_bits_equal(_np(m.mkv[1])[0], mv, "MTP value cache")

    # ---- verify: layer 0 (Gated-DeltaNet), layer 1 (attention) ---------------------------------------
    vtok = _np(tr["verify.vtok"][0])[0]
    x0 = _np(tr["L0.in"][0])
    assert_bits_equal(x0, _np(m.embed[torch.from_numpy(vtok).to(dev)]), "embedding rows")
    L0 = m.layers[0]
    print("case step verify GDN layer", flush=True)
    xn, (proj, z) = ref.layer_pre(x0, _np(L0["norm_in"]), eps, "none", None, [_w4(L0["qkv"]), _w4(L0["z"])])
    assert_bits_equal(_np(tr["L0.proj"][0]), proj, "GDN qkv projection")
    assert_bits_equal(_np(tr["L0.z"][0]), z, "GDN z projection")
    ctl = np.concatenate([[snap["ctl"][0], parity], snap["ctl"][2:2 + S], T["parents"] + [-1] * (S - R),
                          T["prog"] + [0] * (S - R)]).astype(np.int64)
    gn = snap["gdn"]
    conv_w, gnw = ref.bf16_to_f32(_np(L0["conv_w"])), ref.bf16_to_f32(_np(L0["gnorm"]))
    dt_bias, g_decay = L0["dt_bias"].cpu().numpy(), L0["g_decay"].cpu().numpy()
    hk = cfg.gdn_key_heads
    res = []
    for dt in (np.float64, np.float32):
        st = dict(conv_state=gn["conv"].copy(), pb=gn["pb"].copy(), qb=gn["qb"].copy(), rec=gn["rec"].copy(),
                  gates=gn["gates"].copy(), sums=gn["sums"].copy())
        ab = ref.gdn_ab(xn, _np(L0["wa"]), _np(L0["wb"]), dt)
        res.append((ref.gdn_step(st, ref.bf16_to_f32(proj), ref.bf16_to_f32(z), *ab, conv_w, dt_bias, g_decay, gnw, eps,
                                 D ** -0.5, ctl, R, hk, S, dtype=dt), st))
    (c64, st64), (c32, _) = res
    core = ref.bf16_to_f32(_np(tr["L0.core"][0])).astype(np.float64)
    e_ref, err = np.abs(c32 - c64), np.abs(core - c64)
    assert err.max() <= 1.5 * e_ref.max() + 1e-3 and err.mean() <= 1.5 * e_ref.mean() + 1e-5, "GDN core"
    assert_bits_equal(_np(m.gdn[0]["conv"]), ref.f32_to_bf16(st64["conv_state"]), "GDN conv history")
    want, _ = ref.layer_post(x0, _np(tr["L0.core"][0]), None, None, _w4(L0["o"]), _np(L0["norm_post"]), eps, "none", None,
                             lut, _w4(L0["g"]), _w4(L0["u"]), _w4(L0["d"]))
    assert_bits_equal(_np(tr["L0.out"][0]), want, "GDN layer output")
    print("case step verify attention layer", flush=True)
    L1 = m.layers[1]
    x1 = _np(tr["L1.in"][0])
    assert_bits_equal(x1, _np(tr["L0.out"][0]), "layer hand-over")
    _, (q, kk, vv) = ref.layer_pre(x1, _np(L1["norm_in"]), eps, "none", None, [_w4(L1["q"]), _w4(L1["k"]), _w4(L1["v"])])
    for nm, w in (("q", q), ("k", kk), ("v", vv)):
        assert_bits_equal(_np(tr[f"L1.{nm}"][0]), w, f"attention {nm} projection")
    vpos = (np.asarray(T["tree_pos"].cpu()) + st0)
    apos = np.arange(R) + st0
    rq, rk, key, value = ref.rope_kv(q.reshape(R, cfg.heads, D), kk.reshape(R, cfg.kv_heads, D),
                                     vv.reshape(R, cfg.kv_heads, D), ftab[vpos], snap["key"], snap["value"], apos,
                                     cfg.rotary, _np(L1["qn"]), _np(L1["kn"]), eps, eps)
    assert_bits_equal(_np(tr["L1.qo"][0])[0], rq, "attention rope q")
    assert_bits_equal(_np(tr["L1.ko"][0])[0], rk, "attention rope k")
    f32 = ref.bf16_to_f32
    y = f32(_np(tr["L1.y"][0])).reshape(R, cfg.heads, D).astype(np.float64)
    _attn_bound(y, f32(rq), f32(snap["key"]), f32(snap["value"]), st0, f32(rk),
                f32(vv.reshape(R, cfg.kv_heads, D).transpose(1, 0, 2)), ref.tree_mask(T["parents"]), "verify attention")
    assert_bits_equal(_np(tr["L1.key_pre_accept"][0])[0], key, "KV cache rows written by the verify")
    assert_bits_equal(_np(tr["L1.value_pre_accept"][0])[0], value, "V cache rows written by the verify")
    want, _ = ref.layer_post(x1, _np(tr["L1.y"][0]).reshape(R, qd), None, None, _w4(L1["o"]), _np(L1["norm_post"]), eps,
                             "none", None, lut, _w4(L1["g"]), _w4(L1["u"]), _w4(L1["d"]))
    assert_bits_equal(_np(tr["L1.out"][0]), want, "attention layer output")

    # ---- head, pick, accept ---------------------------------------------------------------------------
    print("case step head and accept", flush=True)
    xf = ref.rmsnorm(_np(tr["L1.out"][0]), _np(m.final_norm), eps)
    logits = _np(tr["verify.logits"][0])
    if head == "int8":
        q, s = ref.rot_quant(xf, "h256")
        assert_bits_equal(_np(tr["verify.q"][0]), q, "verify head activation")
        assert_bits_equal(_np(tr["verify.s"][0]), s.view(np.uint32), "verify head activation scales")
        for r in range(R):
            assert_bits_equal(logits[r, cols], ref.int8_head_logits(q[r], s[r:r + 1], q8, s8), f"verify int8 lm_head row {r}")
    else:
        assert_bits_equal(_np(tr["verify.xf"][0]), xf, "final norm")
        _bf16_bound(logits[:, cols], xf, lm_cols, "verify lm_head")
    wv, wi = ref.topk_rows(logits, cfg.top_k)
    assert np.array_equal(_np(tr["verify.idx"][0]), wi), "top-20 indices"
    assert_bits_equal(_np(tr["verify.vals"][0]), wv.view(np.uint32), "top-20 values")
    toks = wi[:, 0]
    assert np.array_equal(_np(tr["verify.toks"][0])[0], toks), "greedy picks"
    path, commit, ranks, row, on_chain, kept = ref.accept_walk([list(c) for c in ref.tree_from_spec(
        ref.spec_of_widths(cfg.widths), S)[1]], toks.tolist(), vtok.tolist(), T["depth"])
    rec = ref.accept_record(S, path, commit, [], row, on_chain, kept, st0)
    assert m.result.cpu().tolist()[:len(rec)] == rec, "accept record"
    st = m.st.cpu().numpy()
    assert st[0] == st0 + len(path) and st[1] == st1 + kept, "counters"
    assert int(m.nt.item()) == toks[row], "next token"
    assert m.ctl[0].item() == len(path) and m.ctl[2:2 + len(path)].cpu().tolist() == path, "GDN replay control"
    assert_bits_equal(_np(m.hbuf)[0], _np(tr["L1.out"][0])[row], "hidden row of the accepted node")
    assert_bits_equal(_np(m.kv[1][0])[0], ref.commit_path(key, path, on_chain, st0), "K cache after the slot moves")
    assert_bits_equal(_np(m.kv[1][1])[0], ref.commit_path(value, path, on_chain, st0), "V cache after the slot moves")
