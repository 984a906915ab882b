"""The reference's `_C` operator surface (comfy_mono_decode_xpu/_C, csrc/bindings.cpp:71-104) on
MI355X: same function names, positional order, defaults and return shapes, taking torch tensors on
the ROCm device and forwarding raw pointers to libmdx's C ABI on torch's current stream.

Contract violations raise RuntimeError before anything is written (as TORCH_CHECK does in the
reference), so pure operators stay replayable by a caller's fallback. Arguments the reference
uses only to steer its Intel launch geometry (cols, nwg, fast) are accepted and ignored: libmdx
plans its own launches. There is no CPU path: without libmdx.so every call raises.
"""
from __future__ import annotations

import ctypes
import math
import os
import weakref

import torch

from . import _lib
from .layout import W4, classify_rotation

_OUT_DT = {0: (torch.float32, _lib.DT_F32), 2: (torch.bfloat16, _lib.DT_BF16)}


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _dev(t, what):
    _check(isinstance(t, torch.Tensor) and t.is_cuda, f"{what} must be a tensor on the ROCm device")


_CB_SEEN = {}  # id(codebook tensor) -> (weak reference to it, its _version, holds code - 8)
_CB_DEFAULT = torch.arange(-8, 8, dtype=torch.float32)


def _codebook(cb):
    """cb, or None when it holds the default codebook code - 8: libmdx then knows the table's symmetry (the
    8-byte magnitude tables, the integral form). The values are read once per tensor object and version
    (a host sync); while a graph is being captured an unseen tensor is passed as it is."""
    if cb is None:
        return None
    hit = _CB_SEEN.get(id(cb))
    if hit is None or hit[0]() is not cb or hit[1] != cb._version:
        if cb.is_cuda and torch.cuda.is_current_stream_capturing():
            return cb
        if len(_CB_SEEN) > 4096:
            _CB_SEEN.clear()
        hit = (weakref.ref(cb), cb._version, bool(torch.equal(cb.detach().cpu(), _CB_DEFAULT)))
        _CB_SEEN[id(cb)] = hit
    return None if hit[2] else cb


def _w4(q, s, sc, cb, tiled=False) -> W4:
    _dev(q, "packed W4")
    _check(q.dtype in (torch.int8, torch.uint8) and q.dim() == 2 and q.is_contiguous(),
           "packed must be contiguous int8 [N, K/2]")
    _check(s.dtype in (torch.float32, torch.float16, torch.float8_e4m3fn) and s.is_contiguous() and s.dim() == 2
           and s.shape[0] == q.shape[0], "s_rel must be contiguous fp32/fp16/fp8 [N, K/G]")
    _check((q.shape[1] * 2) % s.shape[1] == 0, "K must be a multiple of the group count")
    _check(sc.dtype == torch.float32 and sc.is_contiguous() and sc.numel() == q.shape[0], "s_channel f32 [N]")
    if cb is not None:
        _check(cb.dtype == torch.float32 and cb.numel() == 16 and cb.is_contiguous(), "codebook f32 [16]")
    return W4(q, s, sc, _codebook(cb), _lib.LAYOUT_TILE if tiled else _lib.LAYOUT_ROW, _lib.DECODE_AUTO)


def w4a8_decode_linear(x, x_scale, packed, s_rel, s_channel, codebook=None, residual=None, group_size=16,
                       out_dtype_code=2, cols=0, fast=False):
    """Reference csrc/w4a8_decode.sycl:325-370: one fused small-M W4A8 linear (row-major weights)."""
    _dev(x, "x")
    _check(x.dtype == torch.int8 and x.dim() == 2 and x.is_contiguous(), "x must be contiguous int8 [M, K]")
    M, K = x.shape
    _check(1 <= M <= 16, "1 <= M <= 16")
    _check(x.data_ptr() % 16 == 0, "x must be 16-byte aligned")
    w = _w4(packed, s_rel, s_channel, codebook)
    _check(w.k == K, "packed must be [N, K/2]")
    _check(w.group_size == group_size, f"s_rel has {s_rel.shape[1]} groups, not K / group_size")
    _check(x_scale.dtype == torch.float32 and x_scale.is_contiguous() and x_scale.numel() == M, "x_scale f32 [M]")
    _check(out_dtype_code in _OUT_DT, "out dtype fp32 or bf16")
    dt, code = _OUT_DT[out_dtype_code]
    out = torch.empty(M, w.n, dtype=dt, device=x.device)
    if residual is not None:
        _check(residual.dtype == dt and residual.is_contiguous() and residual.numel() == M * w.n,
               "residual must match output")
    _lib.call("mdx_w4a8_decode_linear", _lib.ptr(x), _lib.ptr(x_scale), w.struct(), _lib.ptr(residual), _lib.ptr(out),
              code, M, _lib.stream_of(x))
    return out


def rot_quant(x, h, order=0):
    """Reference csrc/act_prep.sycl:201-214: (int8 [..., K], f32 scale [..., 1])."""
    _dev(x, "x")
    _check(x.dtype == torch.bfloat16 and x.is_contiguous(), "x bf16 contiguous")
    _check(h.dtype == torch.bfloat16 and h.is_contiguous() and h.numel() == 65536, "H bf16 [256,256]")
    K = x.shape[-1]
    rows = x.numel() // K if K else 0
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    scale = torch.empty(tuple(x.shape[:-1]) + (1,), dtype=torch.float32, device=x.device)
    _lib.call("mdx_rot_quant", _lib.ptr(x), _lib.ptr(h), classify_rotation(h), _lib.ptr(q), _lib.ptr(scale), rows, K,
              _lib.stream_of(x))
    return q, scale


def quant_rows(x):
    """Per-token absmax int8 quantisation without rotation (rot_quant with the identity)."""
    K = x.shape[-1]
    rows = x.numel() // K
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    scale = torch.empty(tuple(x.shape[:-1]) + (1,), dtype=torch.float32, device=x.device)
    _lib.call("mdx_rot_quant", _lib.ptr(x), None, _lib.ROT_NONE, _lib.ptr(q), _lib.ptr(scale), rows, K,
              _lib.stream_of(x))
    return q, scale


_MLP_WS = {}


def _mlp_workspace(dev):
    """The per-device mono_mlp workspace (zero-filled once; every call leaves its control words and
    accumulators zero), sized for 16 rows, hidden 4096, intermediate 16384."""
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _MLP_WS.get(key)
    if ws is None:
        ws = _MLP_WS[key] = torch.zeros(_lib.lib().mdx_mono_mlp_workspace(16, 4096, 16384), dtype=torch.uint8,
                                        device=dev)
    return ws


def mlp_error(dev):
    """1 if an in-kernel wait of a mono_mlp call on this device's workspace gave up (else 0)."""
    off = _lib.lib().mdx_mono_mlp_error_offset()
    return int(_mlp_workspace(dev)[off:off + 4].view(torch.int32).item())


def mono_mlp_w4(xn, rot, h, silu_lut, gate: W4, up: W4, down: W4, norm_w=None, eps=1e-6, out=None, ws=None,
                residual=None):
    """mono_mlp on prepared W4 handles (the library's own callers); norm_w: RMSNorm the input first;
    residual: out = bf16(residual + bf16(down))."""
    K1 = xn.shape[-1]
    rows = xn.numel() // K1
    if out is None:
        out = torch.empty(rows, down.n, dtype=torch.bfloat16, device=xn.device)
    ws_bytes = _lib.lib().mdx_mono_mlp_workspace(rows, K1, gate.n)
    if ws is None:
        ws = _mlp_workspace(xn.device)
    _check(ws.numel() >= ws_bytes, "mono_mlp workspace too small")
    _lib.call("mdx_mono_mlp", _lib.ptr(xn), _lib.ptr(norm_w), float(eps), _lib.ptr(h), rot, _lib.ptr(silu_lut),
              gate.struct(), up.struct(), down.struct(), _lib.ptr(residual), _lib.ptr(out), rows, _lib.ptr(ws),
              ws.numel(), _lib.stream_of(xn))
    return out


def stream_gemv(x, x_scale, mats, outs, gate_up=False, residuals=None, out_dtype=torch.bfloat16, silu_lut=None):
    """One engine launch over 1..3 W4 handles sharing K (or a gate/up pair -> outs[0])."""
    rows = x.shape[0]
    arr = (_lib.W4P * len(mats))(*[ctypes.pointer(m.struct()) for m in mats])
    o = (ctypes.c_void_p * len(outs))(*[t.data_ptr() for t in outs])
    r = None
    if residuals is not None:
        r = (ctypes.c_void_p * len(residuals))(*[None if t is None else t.data_ptr() for t in residuals])
    code = _lib.DT_BF16 if out_dtype == torch.bfloat16 else _lib.DT_F32
    _lib.call("mdx_stream_gemv", _lib.ptr(x), _lib.ptr(x_scale), arr, len(mats), int(gate_up), o, r, code,
              _lib.ptr(silu_lut), rows, _lib.stream_of(x))


def rms_rot_quant(x, norm_w, eps, rot=_lib.ROT_NONE, h=None, xn_out=None):
    K = x.shape[-1]
    rows = x.numel() // K
    q = torch.empty(rows, K, dtype=torch.int8, device=x.device)
    scale = torch.empty(rows, dtype=torch.float32, device=x.device)
    _lib.call("mdx_rms_rot_quant", _lib.ptr(x), _lib.ptr(norm_w), float(eps), _lib.ptr(xn_out), _lib.ptr(h), rot,
              _lib.ptr(q), _lib.ptr(scale), rows, K, _lib.stream_of(x))
    return q, scale


def mono_mlp(xn, hadamard, silu_lut, gq, gs, gsc, gcb, uq, us, usc, ucb, dq, ds, dsc, dcb, nwg=0, stop=4, tiled=True):
    """Reference csrc/mono_mlp.sycl:34-180: the whole MLP block for 1..16 decode rows.

    Weights are the reference's tensors in either layout (tiled=True: the tile-major copies made
    by layout.tile_major_codes / tile_major_scales); group size is read off the scale shape."""
    _dev(xn, "xn")
    _check(xn.dtype == torch.bfloat16 and xn.is_contiguous(), "xn bf16")
    _check(stop == 4, "only the full block (stop=4) is supported")
    K1 = xn.shape[-1]
    rows = xn.numel() // K1
    _check(1 <= rows <= 16, "1..16 rows")
    g, u, d = _w4(gq, gs, gsc, gcb, tiled), _w4(uq, us, usc, ucb, tiled), _w4(dq, ds, dsc, dcb, tiled)
    _check(torch.equal(gcb, ucb) and torch.equal(gcb, dcb), "the three projections must share one codebook")
    u.cb = d.cb = g.cb  # one codebook buffer (libmdx requires the shared pointer)
    _check(g.k == K1 and u.k == K1 and d.k == g.n and u.n == g.n, "weight shapes")
    _check(silu_lut.dtype == torch.bfloat16 and silu_lut.numel() == 65536, "silu_lut bf16 [65536]")
    out = mono_mlp_w4(xn.reshape(rows, K1), classify_rotation(hadamard), hadamard, silu_lut, g, u, d)
    return out.reshape(*xn.shape[:-1], d.n)


def _bf16_heads(t, what):
    _dev(t, what)
    _check(t.dtype == torch.bfloat16 and t.stride(-1) == 1, f"{what}: bf16 with a contiguous last dim")


def _rope(qn, kn, vn, wq, wk, freqs, key, value, position, epsq, epsk, rd, outs=None):
    # q/k/v as [S, H, D] or [1, S, H, D] views (a gated q is the query half of [.., H, 2 D])
    qn, kn, vn = (t[0] if t.dim() == 4 else t for t in (qn, kn, vn))
    for t, n in ((qn, "q"), (kn, "k"), (vn, "v")):
        _bf16_heads(t, n)
        _check(t.dim() == 3, f"{n}: [S, H, D] or [1, S, H, D]")
    S, Hq, D = qn.shape
    Hk = kn.shape[1]
    _check(kn.shape == (S, Hk, D) and vn.shape == (S, Hk, D), "k/v shapes")
    _check(key.dtype == torch.bfloat16 and value.dtype == torch.bfloat16 and key.is_contiguous()
           and value.is_contiguous() and key.dim() == 4 and key.shape[0] == 1 and key.shape[1] == Hk
           and key.shape[3] == D and value.shape == key.shape, "bf16 [1, Hk, cap, D] cache")
    _check(freqs.dtype == torch.float32 and freqs.shape[-1] == 2 and freqs.shape[-2] == 2
           and freqs.shape[-3] == rd // 2 and freqs.stride(-1) == 1 and freqs.stride(-2) == 2
           and freqs.stride(-3) == 4 and freqs.numel() // (rd // 2 * 4) == S, "freqs [.., S, rd/2, 2, 2] f32")
    _check(position.dtype == torch.int64 and position.is_contiguous() and position.numel() >= S,
           "int64 positions [>= S]")
    fs = freqs.stride(-4) if freqs.dim() >= 4 else rd // 2 * 4
    if wq is not None:
        for w, n in ((wq, "weight_q"), (wk, "weight_k")):
            _check(w.dtype == torch.bfloat16 and w.is_contiguous() and w.numel() == D, f"{n}: bf16 [D]")
    if outs is None:
        q = torch.empty(1, Hq, S, D, dtype=torch.bfloat16, device=qn.device)
        k = torch.empty(1, Hk, S, D, dtype=torch.bfloat16, device=qn.device)
    else:
        q, k = outs
        _check(q.is_contiguous() and k.is_contiguous() and q.numel() == Hq * S * D and k.numel() == Hk * S * D,
               "outputs [1, Hq, S, D], [1, Hk, S, D]")
    _lib.call("mdx_qk_norm_rope_kv", _lib.ptr(qn), qn.stride(0), qn.stride(1), _lib.ptr(kn), kn.stride(0),
              kn.stride(1), _lib.ptr(vn), vn.stride(0), vn.stride(1), _lib.ptr(wq), _lib.ptr(wk), float(epsq),
              float(epsk), _lib.ptr(freqs), fs, _lib.ptr(key), _lib.ptr(value), _lib.ptr(position), _lib.ptr(q),
              _lib.ptr(k), S, Hq, Hk, D, key.shape[2], rd, _lib.stream_of(qn))
    return [q, k]


def rope_kv(qn, kn, vn, freqs, key, value, position, rd):
    """Reference csrc/rope_kv.sycl:58-114: partial split-half RoPE on q and k + the KV cache write.
    Returns [q [1, Hq, S, D], k [1, Hk, S, D]]."""
    return _rope(qn, kn, vn, None, None, freqs, key, value, position, 1.0, 1.0, rd)


def qk_norm_rope_kv(rawq, rawk, vn, weightq, weightk, freqs, key, value, position, epsq, epsk, rd, outs=None):
    """Reference csrc/rope_kv.sycl:120-245: per-head Q/K RMSNorm, then rope_kv. The norm's reduction
    order is the library's own (per-lane partials in element order, then a 64-lane halving tree)."""
    _check(weightq is not None and weightk is not None, "norm weights")
    _check(epsq > 0 and epsk > 0, "positive eps")
    return _rope(rawq, rawk, vn, weightq, weightk, freqs, key, value, position, epsq, epsk, rd, outs)


def _i64(t, what):
    _dev(t, what)
    _check(t.dtype == torch.int64 and t.is_contiguous(), f"{what}: contiguous int64 device tensor")


def mtp_prep_draft(st, k, ftab, freqs, mpos, mseq):
    """Reference csrc/mtp_loop.sycl:29-53: draft k's rope row and MTP KV positions from st."""
    _i64(st, "st")
    _i64(mpos, "mtp position")
    _check(mseq.dtype == torch.int32 and mseq.numel() >= 1, "mtp seqlen int32")
    _check(ftab.dtype == torch.float32 and ftab.is_contiguous() and freqs.dtype == torch.float32
           and freqs.is_contiguous() and ftab.dim() >= 3 and freqs.dim() == ftab.dim() and freqs.shape[2] == 1,
           "rope table [.., .., cap, ...] / row [.., .., 1, ...] float")
    n, cap = freqs.numel(), ftab.shape[2]
    _check(ftab.numel() == cap * n, "rope table row size")
    _lib.call("mdx_mtp_prep_draft", _lib.ptr(st), int(k), _lib.ptr(ftab), cap, n, _lib.ptr(freqs), _lib.ptr(mpos),
              mpos.numel(), _lib.ptr(mseq), _lib.stream_of(st))


def _slots_of(ctl):
    _check(ctl.dtype == torch.int32 and ctl.is_contiguous() and (ctl.numel() - 2) % 3 == 0, "ctl int32 [2 + 3 slots]")
    slots = (ctl.numel() - 2) // 3
    _check(slots in (8, 16), "8 or 16 slots")
    return slots


def mtp_prep_verify(st, apos, aseq, vpos, tree_pos, ctl, tree_ctl, parity, rope_offset):
    """Reference csrc/mtp_loop.sycl:55-84: verify positions, ctl parity and the tree program."""
    for t, n in ((st, "st"), (apos, "attention position"), (vpos, "verify positions"), (tree_pos, "tree positions")):
        _i64(t, n)
    _check(aseq.dtype == torch.int32, "attention seqlen int32")
    slots = _slots_of(ctl)
    _check(tree_ctl.dtype == torch.int32 and tree_ctl.numel() == 2 * slots and tree_ctl.is_contiguous(),
           "tree program int32 [2 slots]")
    rows = vpos.numel()
    _check(tree_pos.numel() == rows and 1 <= rows <= slots and apos.numel() <= 64, "rows")
    _lib.call("mdx_mtp_prep_verify", _lib.ptr(st), _lib.ptr(apos), apos.numel(), _lib.ptr(aseq), _lib.ptr(vpos),
              _lib.ptr(tree_pos), rows, _lib.ptr(ctl), _lib.ptr(tree_ctl), slots, int(parity), int(rope_offset),
              _lib.stream_of(st))


def mtp_prep_verify_rows(st, apos, aseq, vpos, tree_pos, ctl, tree_ctl, parity, rope_offset, nt, vtok, embed, ftab, x,
                         vfreqs):
    """mtp_prep_verify plus the verify rows' inputs in one launch (mdx_mtp_prep_verify_rows): vtok[0] = nt,
    x[r] = embed[vtok[r]], vfreqs[r] = ftab[vpos[r]]."""
    for t, n in ((st, "st"), (apos, "attention position"), (vpos, "verify positions"), (tree_pos, "tree positions"),
                 (nt, "next token"), (vtok, "verify tokens")):
        _i64(t, n)
    _check(aseq.dtype == torch.int32, "attention seqlen int32")
    slots = _slots_of(ctl)
    _check(tree_ctl.dtype == torch.int32 and tree_ctl.numel() == 2 * slots and tree_ctl.is_contiguous(),
           "tree program int32 [2 slots]")
    rows = vpos.numel()
    _check(tree_pos.numel() == rows and 1 <= rows <= slots and apos.numel() <= 64 and vtok.numel() >= rows, "rows")
    _check(embed.dtype == torch.bfloat16 and embed.dim() == 2 and embed.is_contiguous(), "embedding bf16 [vocab, H]")
    _check(ftab.dtype == torch.float32 and ftab.is_contiguous() and ftab.dim() >= 2, "RoPE table f32 [positions, ...]")
    fcols = ftab[0].numel()
    _check(x.dtype == torch.bfloat16 and x.is_contiguous() and x.numel() == rows * embed.shape[1], "x bf16 [rows, H]")
    _check(vfreqs.dtype == torch.float32 and vfreqs.is_contiguous() and vfreqs.numel() == rows * fcols, "vfreqs f32")
    _lib.call("mdx_mtp_prep_verify_rows", _lib.ptr(st), _lib.ptr(apos), apos.numel(), _lib.ptr(aseq), _lib.ptr(vpos),
              _lib.ptr(tree_pos), rows, _lib.ptr(ctl), _lib.ptr(tree_ctl), slots, int(parity), int(rope_offset),
              _lib.ptr(nt), _lib.ptr(vtok), _lib.ptr(embed), embed.shape[0], embed.shape[1], _lib.ptr(ftab),
              ftab.shape[0], fcols, _lib.ptr(x), _lib.ptr(vfreqs), _lib.stream_of(st))


def mtp_accept(st, toks, vtok, cand, children, rows, depth, x, nt_buf, h_buf, ctl, kv_ptrs, kv_heads, kv_cap,
               head_dim, result):
    """Reference csrc/mtp_loop.sycl:86-196: the accept walk, record, counters, ctl, next token and
    hidden row, and the KV slot moves of an off-chain path."""
    for t, n in ((st, "st"), (result, "result"), (nt_buf, "next token"), (vtok, "verify tokens")):
        _i64(t, n)
    slots = _slots_of(ctl)
    _check(toks.dtype == torch.int64 and toks.numel() >= rows and toks.stride(-1) == 1 and toks.is_contiguous(),
           "sampled tokens int64 [1, rows]")
    _check(1 <= rows <= slots and 0 <= depth < rows, "rows / depth")
    _check(children.dtype == torch.int32 and children.numel() == slots * slots and children.is_contiguous(),
           "children int32 [slots][slots]")
    has_cand = cand is not None and cand.numel() > 0
    _check(not has_cand or (cand.dtype == torch.int64 and cand.is_contiguous() and cand.numel() >= 7 * max(depth, 7)),
           "auto candidates int64 [max(depth, 7), 7]")
    _check(x.is_contiguous() and h_buf.is_contiguous() and x.dtype == torch.bfloat16 and h_buf.dtype == torch.bfloat16
           and x.numel() >= rows * h_buf.numel(), "hidden rows bf16")
    _check(kv_ptrs.dtype == torch.int64 and kv_ptrs.is_contiguous(), "kv pointer table")
    _check(result.numel() >= slots + 24, "result slot")
    _lib.call("mdx_mtp_accept", _lib.ptr(st), _lib.ptr(toks), _lib.ptr(vtok), _lib.ptr(cand) if has_cand else None,
              _lib.ptr(children), int(rows), int(depth), slots, _lib.ptr(x), h_buf.numel(), _lib.ptr(nt_buf),
              _lib.ptr(h_buf), _lib.ptr(ctl), _lib.ptr(kv_ptrs), kv_ptrs.numel(), int(kv_heads), int(kv_cap),
              int(head_dim), _lib.ptr(result), _lib.stream_of(st))


_TOPK_WS = {}


def _topk_ws(dev):
    """The per-device top-k workspace (zeroed once; the kernels leave their counters at zero)."""
    key = (dev.index if dev.index is not None else torch.cuda.current_device())
    ws = _TOPK_WS.get(key)
    if ws is None:
        ws = torch.zeros(_lib.lib().mdx_topk_workspace(16), dtype=torch.uint8, device=dev)
        _TOPK_WS[key] = ws
    return ws


def _bf16_row(x):
    _dev(x, "x")
    _check(x.dtype == torch.bfloat16 and x.is_contiguous(), "bf16 contiguous")
    V = x.shape[-1]
    _check(x.numel() == V and 32768 <= V < 2 ** 31, "one long row")
    return V


def fast_topk(x, k, argmax_order=False):
    """Reference csrc/fast_topk.sycl:164-170: exact top-k (k <= 8) of one bf16 row in torch XPU order,
    or its argmax (argmax_order, k = 1). Returns [values bf16 [1, k], indices int64 [1, k]]."""
    V = _bf16_row(x)
    _check(1 <= k <= 8, "1 <= k <= 8")
    values = torch.empty(1, k, dtype=torch.bfloat16, device=x.device)
    indices = torch.empty(1, k, dtype=torch.int64, device=x.device)
    ws = _topk_ws(x.device)
    _lib.call("mdx_fast_topk", _lib.ptr(x), V, int(k), int(bool(argmax_order)), _lib.ptr(values), _lib.ptr(indices),
              _lib.ptr(ws), ws.numel(), _lib.stream_of(x))
    return [values, indices]


def fast_pick(x, k):
    """Reference csrc/fast_topk.sycl:172-175: top-k (topk order) and the argmax of the same row in one
    launch. Returns [values [1, k], indices [1, k], argmax int64 [1]]."""
    V = _bf16_row(x)
    _check(1 <= k <= 8, "1 <= k <= 8")
    values = torch.empty(1, k, dtype=torch.bfloat16, device=x.device)
    indices = torch.empty(1, k, dtype=torch.int64, device=x.device)
    am = torch.empty(1, dtype=torch.int64, device=x.device)
    ws = _topk_ws(x.device)
    _lib.call("mdx_fast_pick", _lib.ptr(x), V, int(k), _lib.ptr(values), _lib.ptr(indices), _lib.ptr(am),
              _lib.ptr(ws), ws.numel(), _lib.stream_of(x))
    return [values, indices, am]


def topk_rows(x, k):
    """Reference csrc/topk_rows.sycl:223-246: exact top-k (k <= 64) of 1..16 fp32 or bf16 rows in torch
    XPU fp32 order. Returns [values f32 [R, k], indices int64 [R, k]]."""
    _dev(x, "x")
    _check(x.dtype in (torch.float32, torch.bfloat16) and x.is_contiguous() and x.dim() == 2,
           "x: contiguous fp32 / bf16 [R, N]")
    R, N = x.shape
    _check(1 <= R <= 16, "1 <= rows <= 16")
    _check(1 <= k <= 64 and 4096 <= N < 2 ** 31, "1 <= k <= 64, 4096 <= N")
    values = torch.empty(R, k, dtype=torch.float32, device=x.device)
    indices = torch.empty(R, k, dtype=torch.int64, device=x.device)
    ws = _topk_ws(x.device)
    _lib.call("mdx_topk_rows", _lib.ptr(x), _lib.DT_F32 if x.dtype == torch.float32 else _lib.DT_BF16, R, N, int(k),
              _lib.ptr(values), _lib.ptr(indices), _lib.ptr(ws), ws.numel(), _lib.stream_of(x))
    return [values, indices]


def topk_sample(values, indices, uniform, temperature, out=None):
    """Gumbel-max pick over the rows' top k (the decode loop's sampling, one launch): out[r] =
    indices[r, argmax_j(values[r, j] / temperature - log(-log(clamp(uniform[r, j], 1e-20, 1))))]."""
    _dev(values, "values")
    R, k = values.shape
    _check(values.dtype == torch.float32 and indices.dtype == torch.int64 and uniform.dtype == torch.float32
           and values.is_contiguous() and indices.is_contiguous() and uniform.is_contiguous()
           and indices.shape == values.shape and uniform.shape == values.shape, "values f32 / indices int64 / uniform f32 [R, k]")
    if out is None:
        out = torch.empty(R, dtype=torch.int64, device=values.device)
    _check(out.dtype == torch.int64 and out.is_contiguous() and out.numel() == R, "out int64 [R]")
    _lib.call("mdx_topk_sample", _lib.ptr(values), _lib.ptr(indices), _lib.ptr(uniform), float(temperature), R, k,
              _lib.ptr(out), _lib.stream_of(values))
    return out


def topk_sample_seeded(values, indices, seed, counter, temperature, out=None):
    """topk_sample with uniforms drawn on the device (mdx_topk_sample_seeded): SplitMix64 of (seed,
    counter[0], row, slot); counter int64 on the device (the step's committed position)."""
    _dev(values, "values")
    R, k = values.shape
    _check(values.dtype == torch.float32 and indices.dtype == torch.int64 and values.is_contiguous()
           and indices.is_contiguous() and indices.shape == values.shape, "values f32 / indices int64 [R, k]")
    _i64(counter, "counter")
    if out is None:
        out = torch.empty(R, dtype=torch.int64, device=values.device)
    _check(out.dtype == torch.int64 and out.is_contiguous() and out.numel() == R, "out int64 [R]")
    _lib.call("mdx_topk_sample_seeded", _lib.ptr(values), _lib.ptr(indices), int(seed) & ((1 << 64) - 1), _lib.ptr(counter),
              float(temperature), R, k, _lib.ptr(out), _lib.stream_of(values))
    return out


_ATTN_WS = {}
_ATTN_WS_RETIRED = []


def _attn_ws(dev, nbytes):
    """Per-device attention workspace, grown on demand (zeroed when allocated; launches keep their
    counters at zero). Growing happens outside graph capture: warm up once per shape before capturing.
    A workspace that is outgrown stays allocated for the life of the process: a graph captured
    earlier still holds its address."""
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _ATTN_WS.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _ATTN_WS_RETIRED.append(ws)
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _ATTN_WS[key] = ws
    return ws


# MDX_ATTN=exact routes attn_dpas through the exact attention (the A/B switch of the reference's
# MONO_DECODE_XPU_ATTN, comfy_mono_decode_xpu/layer.py:43); set_attention changes it at run time
_ATTN_MODE = [os.environ.get("MDX_ATTN", "fast")]


def set_attention(mode):
    """"fast" (flash decoding on MFMA, tolerance parity) or "exact" (one canonical fp32 order)."""
    _check(mode in ("fast", "exact"), "attention mode: 'fast' or 'exact'")
    _ATTN_MODE[0] = mode


def attn_exact(q, key, value, seqlen, xk, xv, mask, out=None):
    """The exact attention (mdx_attn_exact): attn_dpas's operands and output, one canonical fp32 order."""
    for t, n in ((q, "q"), (key, "key"), (value, "value"), (xk, "xk"), (xv, "xv")):
        _dev(t, n)
        _check(t.dtype == torch.bfloat16 and t.dim() == 4 and t.shape[0] == 1 and t.stride(3) == 1, f"{n}: bf16 [1, ., ., D]")
    _, H, S, D = q.shape
    _check(key.is_contiguous() and value.is_contiguous() and key.shape == value.shape and key.shape[3] == D,
           "cache bf16 [1, Hk, cap, D]")
    Hk, cap = key.shape[1], key.shape[2]
    _check(seqlen.dtype == torch.int32 and seqlen.numel() >= 1, "int32 seqlen")
    _check(mask.dtype == torch.int32 and mask.is_contiguous(), "int32 mask")
    merge = mask.numel() > 0
    _check(1 <= S <= 16 and H % Hk == 0 and (mask.numel() == S if merge else S == 1), "batch 1, 1..16 rows")
    _check(xk.shape == xv.shape and xk.shape[1] == Hk and xk.shape[2] == S and xk.shape[3] == D,
           "xk / xv [1, Hk, S, D]")
    if out is None:
        out = torch.empty(1, S, H * D, dtype=torch.bfloat16, device=q.device)
    _check(out.dtype == torch.bfloat16 and out.is_contiguous() and out.numel() == S * H * D, "out bf16 [1, S, H * D]")
    _lib.call("mdx_attn_exact", _lib.ptr(q), q.stride(1), q.stride(2), _lib.ptr(key), _lib.ptr(value), _lib.ptr(seqlen),
              _lib.ptr(xk), xk.stride(1), xk.stride(2), _lib.ptr(xv), xv.stride(1), xv.stride(2),
              _lib.ptr(mask) if merge else None, _lib.ptr(out), H, Hk, S, D, cap, float(1.0 / math.sqrt(D)),
              _lib.stream_of(q))
    return out


def attn_core(q, key, value, seqlen, xk, xv, mask, nwg=0, out=None):
    """Reference csrc/attn_port.sycl:355-365 (exported as _C.attn_core, csrc/bindings.cpp:81): the attention
    that comfy_mono_decode_xpu/layer.py:428 calls when its fused attention path is switched off
    (MONO_DECODE_XPU_ATTN_DPAS=0), the result that its tests compare bit for bit. Here it is the exact
    attention (mdx_attn_exact: one canonical fp32 order), with attn_dpas's operands and its bf16
    [1, S, H * D] output. nwg steers the reference's launch geometry (negative: its phase clocks) and is
    accepted and ignored."""
    return attn_exact(q, key, value, seqlen, xk, xv, mask, out)


def attn_dpas(q, key, value, seqlen, xk, xv, mask, chunks_hint=0, out=None):
    """Reference csrc/attn_dpas.sycl:269-342: decode attention of the tree-verify rows (mask int32 [S])
    or the draft row (empty mask, S = 1) over the cache prefix [0, seqlen[0]) and the admitted tree rows.
    q bf16 [1, H, S, D]; key/value bf16 [1, Hk, cap, D]; xk/xv bf16 [1, Hk, S, D]. Returns bf16
    [1, S, H * D]. chunks_hint: 0 plans the context split; n > 0 caps it at n chunks per kv head."""
    if _ATTN_MODE[0] == "exact":
        return attn_exact(q, key, value, seqlen, xk, xv, mask, out)
    for t, n in ((q, "q"), (key, "key"), (value, "value"), (xk, "xk"), (xv, "xv")):
        _dev(t, n)
        _check(t.dtype == torch.bfloat16 and t.dim() == 4 and t.shape[0] == 1 and t.stride(3) == 1, f"{n}: bf16 [1, ., ., D]")
    _, H, S, D = q.shape
    _check(key.is_contiguous() and value.is_contiguous() and key.shape == value.shape and key.shape[3] == D,
           "cache bf16 [1, Hk, cap, D]")
    Hk, cap = key.shape[1], key.shape[2]
    _check(seqlen.dtype == torch.int32 and seqlen.numel() >= 1, "int32 seqlen")
    _check(mask.dtype == torch.int32 and mask.is_contiguous(), "int32 mask")
    merge = mask.numel() > 0
    _check(1 <= S <= 16 and H % Hk == 0 and (mask.numel() == S if merge else S == 1), "batch 1, 1..16 rows")
    _check(xk.shape == xv.shape and xk.shape[1] == Hk and xk.shape[2] == S and xk.shape[3] == D,
           "xk / xv [1, Hk, S, D]")
    _check((H // Hk) * S <= 64, "at most 64 query rows per kv head")
    if out is None:
        out = torch.empty(1, S, H * D, dtype=torch.bfloat16, device=q.device)
    _check(out.dtype == torch.bfloat16 and out.is_contiguous() and out.numel() == S * H * D, "out bf16 [1, S, H * D]")
    need = _lib.lib().mdx_attn_workspace(H, Hk, S, D, cap, int(chunks_hint))
    ws = _attn_ws(q.device, need)
    _lib.call("mdx_attn_decode", _lib.ptr(q), q.stride(1), q.stride(2), _lib.ptr(key), _lib.ptr(value), _lib.ptr(seqlen),
              _lib.ptr(xk), xk.stride(1), xk.stride(2), _lib.ptr(xv), xv.stride(1), xv.stride(2),
              _lib.ptr(mask) if merge else None, _lib.ptr(out),
              H, Hk, S, D, cap, int(chunks_hint), _lib.ptr(ws), ws.numel(), _lib.stream_of(q))
    return out


def rope_attn_fits(H, Hk, S, D, rd):
    """Whether qk_norm_rope_attn takes these tree-verify rows (head_dim 128, rd 32 / 64 / 128, 17..64 query
    rows per kv head, the streaming attention form). MDX_ROPE_ATTN=0 turns the fused form off (A/B)."""
    return (_ATTN_MODE[0] != "exact" and D == 128 and rd in (32, 64, 128) and H % Hk == 0
            and 16 < (H // Hk) * S <= 64 and os.environ.get("MDX_ATTN_V1", "0") != "1"
            and os.environ.get("MDX_ROPE_ATTN", "1") != "0")


def qk_norm_rope_attn(rawq, rawk, vn, weightq, weightk, freqs, key, value, position, epsq, epsk, rd, seqlen, mask,
                      k_out, out=None, q_out=None, chunks_hint=0):
    """qk_norm_rope_kv followed by attn_dpas over the tree rows (mask int32 [S]), in one launch plus the merge
    (this library's own fusion; the reference runs csrc/rope_kv.sycl:120-245 and csrc/attn_dpas.sycl:269-342
    as two calls). Bit-identical to the pair: the rows' k land in k_out [1, Hk, S, D] and the cache at
    `position` (past the attended prefix), their q in q_out [1, H, S, D] when given. Returns bf16 [1, S, H * D].
    rope_attn_fits says which shapes it takes."""
    qn, kn, vn = (t[0] if t.dim() == 4 else t for t in (rawq, rawk, vn))
    for t, n in ((qn, "q"), (kn, "k"), (vn, "v")):
        _bf16_heads(t, n)
        _check(t.dim() == 3, f"{n}: [S, H, D] or [1, S, H, D]")
    S, H, D = qn.shape
    Hk = kn.shape[1]
    _check(kn.shape == (S, Hk, D) and vn.shape == (S, Hk, D), "k/v shapes")
    _check(rope_attn_fits(H, Hk, S, D, rd), "shape outside the fused form (use qk_norm_rope_kv + attn_dpas)")
    _check(key.dtype == torch.bfloat16 and value.dtype == torch.bfloat16 and key.is_contiguous()
           and value.is_contiguous() and key.dim() == 4 and key.shape[0] == 1 and key.shape[1] == Hk
           and key.shape[3] == D and value.shape == key.shape, "bf16 [1, Hk, cap, D] cache")
    _check(freqs.dtype == torch.float32 and freqs.shape[-1] == 2 and freqs.shape[-2] == 2
           and freqs.shape[-3] == rd // 2 and freqs.stride(-1) == 1 and freqs.stride(-2) == 2
           and freqs.stride(-3) == 4 and freqs.numel() // (rd // 2 * 4) == S, "freqs [.., S, rd/2, 2, 2] f32")
    fs = freqs.stride(-4) if freqs.dim() >= 4 else rd // 2 * 4
    _check(position.dtype == torch.int64 and position.is_contiguous() and position.numel() >= S,
           "int64 positions [>= S]")
    _check((weightq is None) == (weightk is None), "norm weights: both or neither")
    if weightq is not None:
        _check(epsq > 0 and epsk > 0, "positive eps")
        for w, n in ((weightq, "weight_q"), (weightk, "weight_k")):
            _check(w.dtype == torch.bfloat16 and w.is_contiguous() and w.numel() == D, f"{n}: bf16 [D]")
    _check(seqlen.dtype == torch.int32 and seqlen.numel() >= 1, "int32 seqlen")
    _check(mask.dtype == torch.int32 and mask.is_contiguous() and mask.numel() == S, "int32 mask [S]")
    _check(k_out.dtype == torch.bfloat16 and k_out.is_contiguous() and k_out.numel() == Hk * S * D, "k_out bf16 [1, Hk, S, D]")
    if q_out is not None:
        _check(q_out.dtype == torch.bfloat16 and q_out.is_contiguous() and q_out.numel() == H * S * D,
               "q_out bf16 [1, H, S, D]")
    if out is None:
        out = torch.empty(1, S, H * D, dtype=torch.bfloat16, device=qn.device)
    _check(out.dtype == torch.bfloat16 and out.is_contiguous() and out.numel() == S * H * D, "out bf16 [1, S, H * D]")
    cap = key.shape[2]
    ws = _attn_ws(qn.device, _lib.lib().mdx_attn_workspace(H, Hk, S, D, cap, int(chunks_hint)))
    _lib.call("mdx_attn_decode_rope", _lib.ptr(qn), qn.stride(0), qn.stride(1), _lib.ptr(kn), kn.stride(0), kn.stride(1),
              _lib.ptr(vn), vn.stride(0), vn.stride(1), _lib.ptr(weightq), _lib.ptr(weightk), float(epsq), float(epsk),
              _lib.ptr(freqs), fs, int(rd), _lib.ptr(key), _lib.ptr(value), _lib.ptr(position), _lib.ptr(seqlen),
              _lib.ptr(mask), _lib.ptr(k_out), _lib.ptr(q_out), _lib.ptr(out), H, Hk, S, D, cap, int(chunks_hint),
              _lib.ptr(ws), ws.numel(), _lib.stream_of(qn))
    return out


def bf16_linear(x, w, tiled=True, residual=None, out=None):
    """bf16 decode linear (lm_head / draft block GEMMs; the reference's F.linear at
    comfy_mono_decode_xpu/mtp_loop.py:221-225): bf16(x . W^T) with fp32 accumulation, 1..16 rows.
    w: [N, K] bf16, tile-major (layout.tile_major_bf16) when tiled, else row-major."""
    _dev(x, "x")
    _check(x.dtype == torch.bfloat16 and x.is_contiguous() and x.dim() == 2, "x: contiguous bf16 [rows, K]")
    _check(w.dtype == torch.bfloat16 and w.is_contiguous() and w.dim() == 2 and w.shape[1] == x.shape[1],
           "w: contiguous bf16 [N, K]")
    rows, N = x.shape[0], w.shape[0]
    if out is None:
        out = torch.empty(rows, N, dtype=torch.bfloat16, device=x.device)
    _check(out.dtype == torch.bfloat16 and out.is_contiguous() and out.shape == (rows, N), "out bf16 [rows, N]")
    if residual is not None:
        _check(residual.dtype == torch.bfloat16 and residual.is_contiguous() and residual.shape == (rows, N),
               "residual bf16 [rows, N]")
    _lib.call("mdx_bf16_linear", _lib.ptr(x), _lib.ptr(w), _lib.LAYOUT_TILE if tiled else _lib.LAYOUT_ROW,
              _lib.ptr(residual), _lib.ptr(out), rows, N, x.shape[1], _lib.stream_of(x))
    return out


def int8_linear_prequantized(x, x_scale, w, w_scale, bias=None, out_dtype=2, tiled=False, out=None):
    """W8A8 linear of the int8 ConvRot lm_head (omni_xpu_kernel's int8_linear_prequantized, called at
    comfy_mono_decode_xpu/draft_head.py:228): bf16((float(acc) * x_scale[m]) * w_scale[n]) with acc the exact
    int32 dot of the int8 rows. x int8 [rows, K] (1..16 rows), x_scale f32 [rows] (or [rows, 1]), w int8
    [N, K] (tile-major, layout.tile_major_i8, when tiled), w_scale f32 [N]. Only bf16 out (out_dtype 2)
    and no bias, the forms the reference's head uses."""
    _dev(x, "x")
    _check(bias is None, "bias is not supported (the int8 head has none)")
    _check(out_dtype == 2, "out_dtype 2 (bf16) only")
    _check(x.dtype == torch.int8 and x.is_contiguous() and x.dim() == 2, "x: contiguous int8 [rows, K]")
    rows, K = x.shape
    _check(x_scale.dtype == torch.float32 and x_scale.is_contiguous() and x_scale.numel() == rows, "x_scale f32 [rows]")
    _check(w.dtype == torch.int8 and w.is_contiguous() and w.dim() == 2 and w.shape[1] == K, "w: contiguous int8 [N, K]")
    N = w.shape[0]
    _check(w_scale.dtype == torch.float32 and w_scale.is_contiguous() and w_scale.numel() == N, "w_scale f32 [N]")
    if out is None:
        out = torch.empty(rows, N, dtype=torch.bfloat16, device=x.device)
    _check(out.dtype == torch.bfloat16 and out.is_contiguous() and out.numel() == rows * N, "out bf16 [rows, N]")
    _lib.call("mdx_int8_linear", _lib.ptr(x), _lib.ptr(x_scale), _lib.ptr(w), _lib.ptr(w_scale),
              _lib.LAYOUT_TILE if tiled else _lib.LAYOUT_ROW, _lib.ptr(out), rows, N, K, _lib.stream_of(x))
    return out


def gdn_core(proj, z, xn, wa, wb, conv_w, conv_state, proj_buf, qkv_buf, ctl, dt_bias, g_decay, rec_state, gates_buf,
             sums_buf, gnorm_w, gnorm_eps, qscale, hk, core=None, raw=False):
    """The Gated-DeltaNet core of csrc/mono_gdn.sycl:313-607 (layer_gdn phases P3-P5; layer_gdn_core's
    output): deferred conv, gates, sums, replay + verify delta rule, gated RMSNorm. Buffers are updated
    in place; returns core bf16 [R, HV * 128]. raw=True leaves out the gated RMSNorm (core holds the
    delta rule's bf16 outputs; gnorm_rot_quant applies it later)."""
    for t, n in ((proj, "proj"), (z, "z"), (xn, "xn"), (wa, "wa"), (wb, "wb"), (conv_w, "conv_w"), (conv_state, "conv_state"),
                 (proj_buf, "proj_buf"), (qkv_buf, "qkv_buf"), (gnorm_w, "gnorm_w")):
        _dev(t, n)
        _check(t.dtype == torch.bfloat16 and t.is_contiguous(), f"{n}: contiguous bf16")
    for t, n in ((dt_bias, "dt_bias"), (g_decay, "g_decay"), (rec_state, "rec_state"), (gates_buf, "gates"),
                 (sums_buf, "sums")):
        _check(t.dtype == torch.float32 and t.is_contiguous(), f"{n}: contiguous f32")
    slots = _slots_of(ctl)
    R, C = proj.shape[-2], proj.shape[-1]
    HV = rec_state.shape[-3]
    _check(rec_state.shape[-2:] == (128, 128) and C == 2 * hk * 128 + HV * 128, "GDN shapes")
    _check(xn.numel() == R * xn.shape[-1] and wa.shape == (HV, xn.shape[-1]) and wb.shape == wa.shape,
           "xn [R, K], wa / wb [HV, K]")
    _check(z.shape[-1] == HV * 128 and conv_w.numel() == C * 4
           and conv_state.numel() == C * 3, "GDN operand shapes")
    _check(proj_buf.numel() == 2 * slots * C and qkv_buf.numel() == 2 * slots * C, "proj / qkv buffers [2, slots, C]")
    _check(gates_buf.numel() == 2 * slots * HV * 2 and sums_buf.numel() == 2 * slots * hk * 2, "gates / sums buffers")
    if core is None:
        core = torch.empty(R, HV * 128, dtype=torch.bfloat16, device=proj.device)
    if raw:
        _lib.call("mdx_gdn_core_raw", _lib.ptr(proj), _lib.ptr(xn), _lib.ptr(wa), _lib.ptr(wb), xn.shape[-1],
                  _lib.ptr(conv_w), _lib.ptr(conv_state), _lib.ptr(proj_buf), _lib.ptr(qkv_buf), _lib.ptr(ctl),
                  _lib.ptr(dt_bias), _lib.ptr(g_decay), _lib.ptr(rec_state), _lib.ptr(gates_buf), _lib.ptr(sums_buf),
                  float(qscale), _lib.ptr(core), R, int(hk), HV, slots, _lib.stream_of(proj))
        return core
    _lib.call("mdx_gdn_core", _lib.ptr(proj), _lib.ptr(z), _lib.ptr(xn), _lib.ptr(wa), _lib.ptr(wb), xn.shape[-1],
              _lib.ptr(conv_w), _lib.ptr(conv_state),
              _lib.ptr(proj_buf), _lib.ptr(qkv_buf), _lib.ptr(ctl), _lib.ptr(dt_bias), _lib.ptr(g_decay),
              _lib.ptr(rec_state), _lib.ptr(gates_buf), _lib.ptr(sums_buf), _lib.ptr(gnorm_w), float(gnorm_eps),
              float(qscale), _lib.ptr(core), R, int(hk), HV, slots, _lib.stream_of(proj))
    return core


def gdn_proj(q, s, w_qkv, w_z, proj, z, xn, wa, wb, conv_w, conv_state, proj_buf, qkv_buf, ctl, dt_bias, g_decay,
             gates_buf, hk, z_gate=None, x_row=None, norm_w=None, eps=0.0):
    """The GDN input projections with the deferred conv and the gates in one launch (mdx_gdn_proj):
    [proj | z] = W4A8 GEMV of the int8 rows q / s over the W4 handles w_qkv, w_z; the conv runs in the
    epilogue of the tiles that produce each qkv channel (conv_state, proj_buf, qkv_buf updated as
    gdn_core's conv phase), and extra work-groups compute the gates (decay, beta) from xn, wa, wb. The
    in_proj GEMMs + deltanet_conv_step_deferred + the gates of gated_delta_decode_deferred
    (comfy_mono_decode_xpu/layer.py:216-228, 593). z_gate (optional, like z) receives the gated RMSNorm's
    gate factors bf16(silu(z)) for gnorm_linear(z_gated=True). x_row (one bf16 row [1, K]) with norm_w /
    eps: the row prep (RMSNorm + quantisation, no rotation) runs in the launch; q, s and xn are then
    unused (None). Follow with gdn_delta."""
    R = proj.shape[0]
    HV = wa.shape[0]
    K = wa.shape[1]
    slots = _slots_of(ctl)
    for t, n in ((proj, "proj"), (z, "z"), (wa, "wa"), (wb, "wb"), (conv_w, "conv_w"),
                 (conv_state, "conv_state"), (proj_buf, "proj_buf"), (qkv_buf, "qkv_buf")):
        _dev(t, n)
        _check(t.dtype == torch.bfloat16 and t.is_contiguous(), f"{n}: contiguous bf16")
    for t, n in ((dt_bias, "dt_bias"), (g_decay, "g_decay"), (gates_buf, "gates")):
        _check(t.dtype == torch.float32 and t.is_contiguous(), f"{n}: contiguous f32")
    C = w_qkv.n
    if x_row is None:
        _check(q.dtype == torch.int8 and q.is_contiguous() and q.shape[0] == R and s.numel() >= R, "q int8 [R, K], s f32 [R]")
        _check(xn.dtype == torch.bfloat16 and xn.numel() == R * K, "xn bf16 [R, K]")
    else:
        _check(R == 1 and x_row.dtype == torch.bfloat16 and x_row.numel() == K and norm_w is not None
               and norm_w.dtype == torch.bfloat16 and norm_w.numel() == K, "x_row bf16 [1, K] with norm_w bf16 [K]")
    _check(proj.numel() == R * C and z.numel() == R * w_z.n and wb.shape == wa.shape, "GDN projection shapes")
    _check(conv_w.numel() == C * 4 and conv_state.numel() == C * 3 and proj_buf.numel() == 2 * slots * C
           and qkv_buf.numel() == 2 * slots * C and gates_buf.numel() == 2 * slots * HV * 2, "GDN buffers")
    _check(z_gate is None or (z_gate.dtype == torch.bfloat16 and z_gate.is_contiguous() and z_gate.numel() == z.numel()),
           "z_gate bf16 like z")
    _lib.call("mdx_gdn_proj", _lib.ptr(q), _lib.ptr(s), ctypes.pointer(w_qkv.struct()), ctypes.pointer(w_z.struct()),
              _lib.ptr(proj), _lib.ptr(z), _lib.ptr(xn), _lib.ptr(wa), _lib.ptr(wb), _lib.ptr(conv_w),
              _lib.ptr(conv_state), _lib.ptr(proj_buf), _lib.ptr(qkv_buf), _lib.ptr(ctl), _lib.ptr(dt_bias),
              _lib.ptr(g_decay), _lib.ptr(gates_buf), _lib.ptr(z_gate), _lib.ptr(x_row), _lib.ptr(norm_w), float(eps),
              R, int(hk), HV, slots, _lib.stream_of(proj))


def gdn_delta(qkv_buf, ctl, rec_state, gates_buf, qscale, hk, core):
    """The delta rule after gdn_proj (mdx_gdn_delta): replay + verify entries over rec_state from the
    conv outputs in qkv_buf and the gates; core [R, HV * 128] receives the raw bf16 outputs (gated
    RMSNorm not applied)."""
    slots = _slots_of(ctl)
    HV = rec_state.shape[-3]
    R = core.shape[0]
    _check(qkv_buf.dtype == torch.bfloat16 and core.dtype == torch.bfloat16 and core.is_contiguous()
           and core.shape[-1] == HV * 128, "qkv_buf bf16, core bf16 [R, HV * 128]")
    _check(rec_state.dtype == torch.float32 and rec_state.shape[-2:] == (128, 128) and gates_buf.dtype == torch.float32,
           "rec_state f32 [HV, 128, 128], gates f32")
    _check(qkv_buf.numel() == 2 * slots * (2 * hk + HV) * 128 and gates_buf.numel() == 2 * slots * HV * 2, "GDN buffers")
    _lib.call("mdx_gdn_delta", _lib.ptr(qkv_buf), _lib.ptr(ctl), _lib.ptr(rec_state), _lib.ptr(gates_buf),
              float(qscale), _lib.ptr(core), R, int(hk), HV, slots, _lib.stream_of(core))
    return core


# ---------------------------------------------------------------------------------------------------
# decoder-layer segments (csrc/mono_layer.sycl, csrc/mono_gdn.sycl)
# ---------------------------------------------------------------------------------------------------
_SCRATCH = {}


def _scratch(dev):
    """Per-device buffers of the layer segments (stable addresses for graph capture), 16 rows."""
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    sc = _SCRATCH.get(key)
    if sc is None:
        bf = dict(dtype=torch.bfloat16, device=dev)
        sc = _SCRATCH[key] = dict(
            q1=torch.empty(16, 16384, dtype=torch.int8, device=dev), s=torch.empty(64, dtype=torch.float32, device=dev),
            xn=torch.empty(16, 4096, **bf), x1=torch.empty(16, 4096, **bf), proj=torch.empty(16, 16384, **bf),
            z=torch.empty(16, 8192, **bf), ab=torch.empty(16, 256, **bf), core=torch.empty(16, 8192, **bf),
            core_n=torch.empty(16, 8192, **bf), zg=torch.empty(16, 8192, **bf),
            mlp_ws=_mlp_workspace(dev),
            wab={})
    return sc


def _buf(t, R, N):
    """A contiguous [R, N] view at the start of a scratch buffer."""
    return t.view(-1)[:R * N].view(R, N)


def _w4_list(mats, tiled):
    _check(len(mats) % 4 == 0 and len(mats) >= 4, "W4 matrices as (q, s, sc, cb) groups")
    ws = [_w4(mats[i], mats[i + 1], mats[i + 2], mats[i + 3], tiled) for i in range(0, len(mats), 4)]
    for w in ws[1:]:
        w.cb = ws[0].cb if (w.cb is not None and ws[0].cb is not None and torch.equal(w.cb, ws[0].cb)) else w.cb
    return ws


def _rows_of(x):
    _dev(x, "x")
    _check(x.dtype == torch.bfloat16 and x.is_contiguous() and x.shape[-1] == 4096, "x bf16 [..., 4096]")
    R = x.numel() // 4096
    _check(1 <= R <= 16, "1..16 rows")
    return R


def gate_rot_quant(y, gate, sig_lut, hadamard, q=None, scale=None):
    """bf16(y * sig_lut[gate]) -> rot_quant (layer_post's first phase, csrc/mono_layer.sycl:243-256).
    gate: [R, 2 K] interleaved per 256-head ([query | gate]) or [R, K]."""
    K = y.shape[-1]
    R = y.numel() // K
    inter = gate.numel() == 2 * R * K
    _check(gate.dtype == torch.bfloat16 and gate.is_contiguous() and (inter or gate.numel() == R * K), "gate bf16")
    if q is None:
        q = torch.empty(R, K, dtype=torch.int8, device=y.device)
        scale = torch.empty(R, dtype=torch.float32, device=y.device)
    g = (2 * K, 256, 512, 256) if inter else (K, K, K, 0)
    _lib.call("mdx_gate_rot_quant", _lib.ptr(y), _lib.ptr(gate), *g, _lib.ptr(sig_lut), _lib.ptr(hadamard),
              classify_rotation(hadamard), _lib.ptr(q), _lib.ptr(scale), R, K, _lib.stream_of(y))
    return q, scale


def layer_pre(x, norm_w, eps, hadamard, mats, nwg=0, tiled=True):
    """Reference csrc/mono_layer.sycl:69-155: xn = RMSNorm(x), q = rot_quant(xn), then 1..3 W4
    projections of q in one engine launch. Returns [xn, out_0, ...] (bf16)."""
    R = _rows_of(x)
    _check(norm_w.dtype == torch.bfloat16 and norm_w.numel() == 4096, "norm weight bf16 [4096]")
    ws = _w4_list(mats, tiled)
    _check(len(ws) <= 3 and all(w.k == 4096 for w in ws), "1..3 W4 matrices with K = hidden")
    xn = torch.empty(R, 4096, dtype=torch.bfloat16, device=x.device)
    q, s = rms_rot_quant(x.reshape(R, 4096), norm_w, eps, classify_rotation(hadamard), hadamard, xn_out=xn)
    outs = [torch.empty(R, w.n, dtype=torch.bfloat16, device=x.device) for w in ws]
    stream_gemv(q, s, ws, outs)
    return [xn] + outs


def gnorm_linear(y, z, gnorm_w, eps, w, out, residual=None, y_out=None, q=None, scale=None, z_gated=False):
    """out = [residual +] W4A8 GEMV of w over the gated RMSNorm of y (per 128-element head; z the gate input,
    or with z_gated its gate factors as gdn_proj's z_gate), the rows quantised without rotation
    (mdx_gnorm_linear): one launch at one or two rows, else the row prep into q / scale (int8 [R, K], f32
    [R]) then the GEMV. y_out receives the normalised rows."""
    R, K = y.shape[0], y.shape[-1]
    for t, n in ((y, "y"), (z, "z"), (gnorm_w, "gnorm_w"), (out, "out")):
        _dev(t, n)
        _check(t.dtype == torch.bfloat16 and t.is_contiguous(), f"{n}: contiguous bf16")
    _check(z.numel() == R * K and w.k == K and out.numel() == R * w.n and gnorm_w.numel() == 128, "gated-norm linear shapes")
    _check(residual is None or (residual.dtype == torch.bfloat16 and residual.numel() == R * w.n), "residual bf16 [R, N]")
    _lib.call("mdx_gnorm_linear", _lib.ptr(y), _lib.ptr(z), int(bool(z_gated)), _lib.ptr(gnorm_w), float(eps),
              _lib.ptr(y_out),
              ctypes.pointer(w.struct()), _lib.ptr(residual), _lib.ptr(out), _lib.ptr(q), _lib.ptr(scale), R,
              _lib.stream_of(y))
    return out


def _layer_post(x, y, gate, sig_lut, O, norm_w, eps, hadamard, silu_lut, G, U, D, stop, gnorm=None, gnorm_out=None):
    """gnorm = (z, weight, eps[, z_gated]): y holds a Gated-DeltaNet's raw outputs, gated-RMSNormed (into
    gnorm_out, or in place) before the out_proj; z_gated: z holds the gate factors (gdn_proj's z_gate; only
    without rotation)."""
    R = _rows_of(x)
    _check(stop >= 6, "only the full post block (stop >= 6) is supported")
    _check(y.dtype == torch.bfloat16 and y.is_contiguous() and y.numel() == R * 4096, "y bf16 [R, 4096]")
    sc = _scratch(x.device)
    x2 = x.view(R, 4096)
    rot = classify_rotation(hadamard)
    q, s = _buf(sc["q1"], R, 4096), sc["s"][:R]
    x1 = _buf(sc["x1"], R, 4096)
    if gnorm is not None and rot == _lib.ROT_NONE and gnorm_out is not None:
        # the gated RMSNorm + quantisation in the out_proj's launch where the shape allows (mdx_gnorm_linear)
        z, gw, geps = gnorm[:3]
        gnorm_linear(y.view(R, 4096), z, gw, geps, O, x1, residual=x2, y_out=gnorm_out, q=q, scale=s,
                     z_gated=len(gnorm) > 3 and gnorm[3])
        mono_mlp_w4(x1, rot, hadamard, silu_lut, G, U, D, norm_w=norm_w, eps=eps, out=x2, ws=sc["mlp_ws"], residual=x1)
        return x
    if gnorm is not None:
        # y holds the Gated-DeltaNet's raw outputs: the per-head gated RMSNorm (z, weight, eps), written
        # into gnorm_out (or back into y), then the rotation + quantisation
        z, gw, geps = gnorm[:3]
        _check(len(gnorm) == 3 or not gnorm[3], "gate factors in place of z need no rotation")
        _lib.call("mdx_gnorm_rot_quant", _lib.ptr(y), _lib.ptr(z), _lib.ptr(gw), float(geps),
                  _lib.ptr(y if gnorm_out is None else gnorm_out), _lib.ptr(hadamard), rot, _lib.ptr(q), _lib.ptr(s), R,
                  4096, _lib.stream_of(y))
    elif gate is not None:
        gate_rot_quant(y.view(R, 4096), gate, sig_lut, hadamard, q, s)
    else:
        _lib.call("mdx_rot_quant", _lib.ptr(y), _lib.ptr(hadamard), rot, _lib.ptr(q), _lib.ptr(s), R, 4096,
                  _lib.stream_of(y))
    stream_gemv(q, s, [O], [x1], residuals=[x2])
    mono_mlp_w4(x1, rot, hadamard, silu_lut, G, U, D, norm_w=norm_w, eps=eps, out=x2, ws=sc["mlp_ws"], residual=x1)
    return x


def layer_post(x, y, gate, sig_lut, oq, os_, osc, ocb, norm_w, eps, hadamard, silu_lut, gq, gs, gsc, gcb, uq, us, usc,
               ucb, dq, ds, dsc, dcb, nwg=0, stop=6, tiled=True):
    """Reference csrc/mono_layer.sycl:157-318: y' = bf16(y * sigmoid(gate)) (optional), x1 = x +
    o_proj(rot_quant(y')), x = x1 + mlp(RMSNorm(x1)); x is updated in place and returned."""
    O, G, U, D = (_w4(*w, tiled) for w in ((oq, os_, osc, ocb), (gq, gs, gsc, gcb), (uq, us, usc, ucb),
                                           (dq, ds, dsc, dcb)))
    U.cb = D.cb = G.cb
    return _layer_post(x, y, gate, sig_lut, O, norm_w, eps, hadamard, silu_lut, G, U, D, stop)


def expand_compact_h(h16):
    """The full H256 from layer_post_h16's [2, 16, 16] (+H16, -H16): block (kb, cb) is -H16 when the
    base-4 digits of kb ^ cb hold an odd number of 3s (comfy_mono_decode_xpu/layer.py:74-90)."""
    b = torch.arange(16, device=h16.device)
    d = b[:, None] ^ b[None, :]
    d = d & (d >> 1) & 5
    neg = ((d & 1) ^ (d >> 2)).bool()
    return torch.where(neg[:, None, :, None], h16[1][None, :, None, :], h16[0][None, :, None, :]).reshape(256, 256)


def layer_post_h16(x, y, gate, sig_lut, oq, os_, osc, ocb, norm_w, eps, hadamard, *rest):
    """Reference layer_post_h16 (csrc/mono_layer.sycl:157-318 with CompactH): the rotation given as its
    [2, 16, 16] compact form."""
    _check(hadamard.dim() == 3 and tuple(hadamard.shape) == (2, 16, 16), "compact Hadamard [2, 16, 16]")
    sc = _scratch(x.device)
    key = ("h16", hadamard.data_ptr(), hadamard._version)
    full = sc["wab"].get(key)
    if full is None or full[0] is not hadamard:
        full = sc["wab"][key] = (hadamard, expand_compact_h(hadamard).contiguous())
    return layer_post(x, y, gate, sig_lut, oq, os_, osc, ocb, norm_w, eps, full[1], *rest)


def layer_gdn(x, norm_in, eps_in, hadamard, w4, wa, wb, conv_w, conv_state, proj_buf, qkv_buf, ctl, dt_bias, g_decay,
              rec_state, gates_buf, sums_buf, gnorm_w, gnorm_eps, qscale, hk, norm_post, eps_post, silu_lut, nwg=0,
              stop=11, tiled=True):
    """Reference csrc/mono_gdn.sycl:87-699: x += out_proj(GDN(RMSNorm(x))); x += mlp(RMSNorm(x)) for
    1..16 tree-verify rows, in place. w4: qkv, z, out, gate, up, down as (q, s, sc, cb) groups (24
    tensors). stop 5: only the GDN core (read it with layer_gdn_core); stop >= 6: the whole layer."""
    R = _rows_of(x)
    _check(len(w4) == 24, "W4: qkv, z, out, gate, up, down (q, s, sc, cb each)")
    QKV, Z, O, G, U, D = _w4_list(w4, tiled)
    HV = rec_state.shape[-3]
    _check(wa.dtype == torch.bfloat16 and wa.shape == (HV, 4096) and wb.shape == wa.shape, "w_a / w_b bf16 [HV, 4096]")
    sc = _scratch(x.device)
    x2 = x.view(R, 4096)
    rot = classify_rotation(hadamard)
    xn, q, s = _buf(sc["xn"], R, 4096), _buf(sc["q1"], R, 4096), sc["s"][:R]
    # one row without rotation: the row prep runs in the projection launch
    xrow = R == 1 and rot == _lib.ROT_NONE and QKV.s.dtype == torch.float16
    if not xrow:
        _lib.call("mdx_rms_rot_quant", _lib.ptr(x2), _lib.ptr(norm_in), float(eps_in), _lib.ptr(xn), _lib.ptr(hadamard),
                  rot, _lib.ptr(q), _lib.ptr(s), R, 4096, _lib.stream_of(x))
    proj, z = _buf(sc["proj"], R, QKV.n), _buf(sc["z"], R, Z.n)
    # the projections with the conv and the gates (one launch), then the delta rule; sums_buf is the
    # reference's, unused here (the norms come from qkv_buf)
    zg = _buf(sc["zg"], R, Z.n) if rot == _lib.ROT_NONE and stop >= 6 else None
    gdn_proj(q, s, QKV, Z, proj, z, xn, wa, wb, conv_w, conv_state, proj_buf, qkv_buf, ctl, dt_bias, g_decay,
             gates_buf, hk, z_gate=zg, x_row=x2 if xrow else None, norm_w=norm_in, eps=eps_in)
    core = gdn_delta(qkv_buf, ctl, rec_state, gates_buf, qscale, hk, _buf(sc["core"], R, HV * 128))
    # the gated RMSNorm writes the layer's core output (layer_gdn_core) into core_n: in the out_proj's
    # launch or its activation prep (stop >= 6), else on its own
    core_n = _buf(sc["core_n"], R, HV * 128)
    if stop < 6:
        _lib.call("mdx_gnorm_rot_quant", _lib.ptr(core), _lib.ptr(z), _lib.ptr(gnorm_w), float(gnorm_eps),
                  _lib.ptr(core_n), None, _lib.ROT_NONE, None, None, R, HV * 128, _lib.stream_of(core))
    else:
        U.cb = D.cb = G.cb
        _layer_post(x, core, None, None, O, norm_post, eps_post, hadamard, silu_lut, G, U, D, 6,
                    gnorm=(z, gnorm_w, gnorm_eps) if zg is None else (zg, gnorm_w, gnorm_eps, True), gnorm_out=core_n)
    return x


def layer_gdn_core(like, rows):
    """Reference csrc/mono_gdn.sycl:702-704: the GDN core output of the last layer_gdn on this device
    (rows 0..rows-1), valid until the next call."""
    return _buf(_scratch(like.device)["core_n"], rows, 4096)


def rmsnorm(x, w, eps, out=None):
    """bf16 RMSNorm of rows in the library's fixed order (the draft block's norms)."""
    K = x.shape[-1]
    rows = x.numel() // K
    _check(x.dtype == torch.bfloat16 and x.is_contiguous() and w.numel() == K, "x bf16 [.., K], w bf16 [K]")
    if out is None:
        out = torch.empty_like(x)
    _lib.call("mdx_rmsnorm", _lib.ptr(x), _lib.ptr(w), float(eps), _lib.ptr(out), rows, K, _lib.stream_of(x))
    return out


def silu_mul(g, u, silu_lut, out=None):
    """bf16(silu_lut[g] * u) elementwise (the draft block's SwiGLU)."""
    _check(g.dtype == torch.bfloat16 and u.dtype == torch.bfloat16 and g.numel() == u.numel(), "bf16 g / u")
    if out is None:
        out = torch.empty_like(g)
    _lib.call("mdx_silu_mul", _lib.ptr(g), _lib.ptr(u), _lib.ptr(silu_lut), _lib.ptr(out), g.numel(), _lib.stream_of(g))
    return out


# ---------------------------------------------------------------------------------------------------
# fused draft-head ops (csrc/draft_fused.sycl, called from comfy_mono_decode_xpu/draft_head.py:179-211)
# ---------------------------------------------------------------------------------------------------
_LUTS = {}


def _luts(dev):
    """torch's sigmoid and SiLU of every bf16 value on this device (the draft ops' activations)."""
    from . import layout
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    t = _LUTS.get(key)
    if t is None:
        t = _LUTS[key] = (layout.sigmoid_lut(dev), layout.silu_lut(dev))
    return t


def _present(t):
    return t is not None and t.numel() > 0


def _bf16c(t, what):
    _dev(t, what)
    _check(t.dtype == torch.bfloat16 and t.is_contiguous(), f"{what}: contiguous bf16")


_HROT = {}


def _regular_h(hmat, what="hadamard"):
    """True for the regular ConvRot H256 in fp32 [256, 256] (the only rotation the reference's draft ops
    apply: csrc/draft_fused.sycl:46-73 runs the fixed transform whenever a matrix is passed)."""
    from . import layout
    _dev(hmat, what)
    _check(hmat.dtype == torch.float32 and hmat.is_contiguous() and hmat.numel() == 65536, f"{what}: f32 [256, 256]")
    key = (hmat.data_ptr(), hmat._version)
    hit = _HROT.get(key)
    if hit is None or hit[0] is not hmat:
        ok = torch.equal(hmat.reshape(256, 256), layout.regular_hadamard(hmat.device, torch.float32))
        if len(_HROT) >= 8:
            _HROT.pop(next(iter(_HROT)))
        hit = _HROT[key] = (hmat, ok)
    _check(hit[1], f"{what}: only the regular ConvRot H256 (kron(H4, H4, H4, H4) / 16) is supported")
    return True


def draft_embed_norm_cat(token, q, s, hmat, emb, hidden, we, wh, eps_e, eps_h, out):
    """Reference csrc/draft_fused.sycl:76-151: out = cat(RMSNorm_e(emb), RMSNorm_h(hidden)), the embedding
    row gathered from an int8 ConvRot table (q [V, H] int8, s [V] f32, un-rotated by H256 when hmat is
    given) at token, or given as the bf16 row emb (q empty), or, with q empty and token given, gathered
    from the bf16 table emb [V, H] at token (tokens clamped into [0, V) in both gathers). Rows: hidden
    [rows, H] (the reference: one)."""
    _bf16c(hidden, "hidden")
    _bf16c(we, "we")
    _bf16c(wh, "wh")
    H = we.numel()
    _check(wh.numel() == H and H >= 256 and H % 256 == 0 and hidden.numel() % H == 0, "hidden size")
    rows = hidden.numel() // H
    _bf16c(out, "out")
    _check(out.numel() == 2 * rows * H, "out bf16 [rows, 2 H]")
    gather = _present(q)
    if gather:
        _dev(q, "q")
        _check(q.dtype == torch.int8 and q.dim() == 2 and q.shape[1] == H and q.is_contiguous(), "q int8 [V, H]")
        _check(s.dtype == torch.float32 and s.is_contiguous() and s.numel() == q.shape[0], "s float [V]")
        _check(token.dtype == torch.int64 and token.is_contiguous() and token.numel() == rows, "token int64 [rows]")
        unrot = _present(hmat) and _regular_h(hmat)
        _lib.call("mdx_draft_embed_norm_cat", _lib.ptr(token), _lib.ptr(q), _lib.ptr(s), q.shape[0], int(unrot), None,
                  _lib.ptr(hidden), _lib.ptr(we), _lib.ptr(wh), float(eps_e), float(eps_h), _lib.ptr(out), rows, H,
                  _lib.stream_of(hidden))
    elif _present(token):
        _dev(token, "token")
        _bf16c(emb, "emb")
        _check(emb.dim() == 2 and emb.shape[1] == H, "emb bf16 table [V, H]")
        _check(token.dtype == torch.int64 and token.is_contiguous() and token.numel() == rows, "token int64 [rows]")
        _lib.call("mdx_draft_embed_norm_cat", _lib.ptr(token), None, None, emb.shape[0], 0, _lib.ptr(emb),
                  _lib.ptr(hidden), _lib.ptr(we), _lib.ptr(wh), float(eps_e), float(eps_h), _lib.ptr(out), rows, H,
                  _lib.stream_of(hidden))
    else:
        _bf16c(emb, "emb")
        _check(emb.numel() == rows * H, "emb bf16 [rows, H]")
        _lib.call("mdx_draft_embed_norm_cat", None, None, None, 0, 0, _lib.ptr(emb), _lib.ptr(hidden), _lib.ptr(we),
                  _lib.ptr(wh), float(eps_e), float(eps_h), _lib.ptr(out), rows, H, _lib.stream_of(hidden))


def draft_add_rmsnorm(x, h, w, eps, out):
    """Reference csrc/draft_fused.sycl:153-184: x = bf16(x + h) in place (h empty: x unchanged), out =
    RMSNorm(x). x / h / out [rows, H] bf16 (the reference: one row)."""
    _bf16c(x, "x")
    _bf16c(w, "w")
    _bf16c(out, "out")
    H = w.numel()
    _check(H >= 256 and H % 256 == 0 and x.numel() % H == 0 and out.numel() == x.numel(), "bf16 [rows, H] rows")
    if _present(h):
        _bf16c(h, "h")
        _check(h.numel() == x.numel(), "h bf16 like x")
    _lib.call("mdx_draft_add_rmsnorm", _lib.ptr(x), _lib.ptr(h) if _present(h) else None, _lib.ptr(w), float(eps),
              _lib.ptr(out), x.numel() // H, H, _lib.stream_of(x))


def draft_sigmoid_mul(a, qg, head_dim, out):
    """Reference csrc/draft_fused.sycl:186-203: out = bf16(a * bf16(sigmoid(gate))), the gate being the second
    half of each 2 head_dim block of the q projection qg (contiguous, or rows [rows, >= 2 n] with a row
    stride: the q part of a fused q|k|v projection)."""
    _bf16c(a, "a")
    _bf16c(out, "out")
    _dev(qg, "qg")
    _check(qg.dtype == torch.bfloat16 and qg.stride(-1) == 1, "q projection bf16")
    D = int(head_dim)
    if qg.is_contiguous():
        rows, row_stride = 1, qg.numel()
        n = a.numel()
    else:
        _check(qg.dim() == 2, "q projection: contiguous, or [rows, 2 n] rows")
        rows, row_stride = qg.shape[0], qg.stride(0)
        _check(a.numel() % rows == 0, "a [rows, n]")
        n = a.numel() // rows
        _check(qg.shape[1] >= 2 * n, "q projection [rows, 2 n]")
    _check(D >= 1 and n % D == 0 and (qg.numel() >= 2 * n if rows == 1 else True) and out.numel() == a.numel(),
           "q projection bf16 [heads x 2 head_dim]")
    sig, _ = _luts(a.device)
    _lib.call("mdx_draft_sigmoid_mul", _lib.ptr(a), _lib.ptr(qg), row_stride, D, _lib.ptr(sig), _lib.ptr(out), rows, n,
              _lib.stream_of(a))


def draft_silu_mul(gu, out):
    """Reference csrc/draft_fused.sycl:205-218: out = bf16(bf16(silu(gate)) * up) over the concatenated
    gate | up rows gu [rows, 2 I] (the reference: one row)."""
    _bf16c(gu, "gu")
    _bf16c(out, "out")
    I = out.shape[-1]
    _check(gu.numel() == 2 * out.numel() and out.numel() % I == 0, "gate | up bf16 [2I], out bf16 [I]")
    rows = out.numel() // I
    _, silu = _luts(gu.device)
    _lib.call("mdx_draft_silu_mul", _lib.ptr(gu), 2 * I, _lib.ptr(silu), _lib.ptr(out), rows, I, _lib.stream_of(gu))


def draft_norm_rot_quant(x, h, w, eps, hmat, xr, qx, sx):
    """Reference csrc/draft_fused.sycl:220-287: x = bf16(x + h) in place (optional), xr = bf16(H256 rotation of
    RMSNorm(x)), rowwise int8 quantisation of xr into qx / sx (scale = max(amax / 127, 1e-30), q = rint(xr /
    bf16(scale))). An empty hmat (the reference requires one) leaves xr unrotated; empty qx / sx skip the
    quantisation (a bf16 lm_head reads xr)."""
    _bf16c(x, "x")
    _bf16c(w, "w")
    _bf16c(xr, "xr")
    H = w.numel()
    _check(H >= 256 and H % 256 == 0 and x.numel() % H == 0 and xr.numel() == x.numel(), "x / w / xr bf16 [rows, H]")
    rows = x.numel() // H
    rot = _lib.ROT_H256 if (_present(hmat) and _regular_h(hmat)) else _lib.ROT_NONE
    if _present(h):
        _bf16c(h, "h")
        _check(h.numel() == x.numel(), "h bf16 like x")
    quant = _present(qx)
    if quant:
        _dev(qx, "qx")
        _check(qx.dtype == torch.int8 and qx.is_contiguous() and qx.numel() == x.numel(), "qx int8 [rows, H]")
        _check(sx.dtype == torch.float32 and sx.is_contiguous() and sx.numel() == rows, "sx float [rows]")
    _lib.call("mdx_draft_norm_rot_quant", _lib.ptr(x), _lib.ptr(h) if _present(h) else None, _lib.ptr(w), float(eps),
              rot, _lib.ptr(xr), _lib.ptr(qx) if quant else None, _lib.ptr(sx) if quant else None, rows, H,
              _lib.stream_of(x))


# ---------------------------------------------------------------------------------------------------
# two-stage draft lm_head (csrc/draft_lmhead.sycl, comfy_mono_decode_xpu/draft_lmhead.py)
# ---------------------------------------------------------------------------------------------------
_PICK_WS = {}


def _pick_ws(dev):
    """The per-device draft-pick workspace (zeroed once; every call leaves its counter at zero)."""
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _PICK_WS.get(key)
    if ws is None:
        ws = _PICK_WS[key] = torch.zeros(_lib.lib().mdx_draft_pick_workspace(), dtype=torch.uint8, device=dev)
    return ws


def _pick_outputs(top, ranks_row, token, vtok, children, calls, nout):
    for t, n in ((token, "token"), (vtok, "vtok")):
        _dev(t, n)
        _check(t.dtype == torch.int64 and t.is_contiguous(), f"{n}: contiguous int64")
    _check(token.numel() == 1, "token: one int64")
    for t, n in ((top, "top"), (ranks_row, "ranks row")):
        if _present(t):
            _check(t.dtype == torch.int64 and t.is_contiguous() and t.numel() >= nout, f"{n}: int64 [>= nout]")
    ch = [int(c) for c in children]
    _check(1 <= len(ch) <= 8 and len(ch) <= nout, "children: 1..min(8, nout) rows")
    _check(all(0 <= c < vtok.numel() for c in ch), "child row")
    if calls is not None:
        _check(calls.dtype == torch.int64 and calls.numel() >= 1, "calls counter int64")
    return (ctypes.c_int64 * len(ch))(*ch), len(ch)


def draft_pick(approx, qx, sx, w, sw, nout, argmax_first, top, ranks_row, token, vtok, children, calls):
    """Reference csrc/draft_lmhead.sycl:82-291: from approximate scores approx bf16 [N], the exact int8 logits
    of candidates (the 32 best scores of each of 32 segments), their top-nout in torch topk order and the
    argmax; writes top / ranks_row[:nout] (either may be empty), token, vtok[children] and calls += 1. An
    empty w: the scores are the logits (qx, sx, sw ignored)."""
    _dev(approx, "approx")
    _check(approx.dtype == torch.bfloat16 and approx.is_contiguous(), "approx: bf16 row")
    N = approx.numel()
    exact = w.numel() == 0
    K = 0
    if not exact:
        _check(w.dtype == torch.int8 and w.is_contiguous() and w.dim() == 2 and w.shape[0] == N, "w: int8 [N, K]")
        K = w.shape[1]
        _check(qx.dtype == torch.int8 and qx.is_contiguous() and qx.numel() == K, "qx: int8 [K]")
        _check(sx.dtype == torch.float32 and sx.numel() == 1, "sx: one float")
        _check(sw.dtype == torch.float32 and sw.is_contiguous() and sw.numel() == N, "sw: float [N]")
    _check(1 <= int(nout) <= 8, "1 <= nout <= 8")
    ch, nch = _pick_outputs(top, ranks_row, token, vtok, children, calls, int(nout))
    ws = _pick_ws(approx.device)
    _lib.call("mdx_draft_pick", _lib.ptr(approx), N, None if exact else _lib.ptr(qx), None if exact else _lib.ptr(sx),
              None if exact else _lib.ptr(w), None if exact else _lib.ptr(sw), K, int(nout), int(bool(argmax_first)),
              _lib.ptr(top) if _present(top) else None, _lib.ptr(ranks_row) if _present(ranks_row) else None,
              _lib.ptr(token), _lib.ptr(vtok), vtok.numel(), ch, nch, _lib.ptr(calls), _lib.ptr(ws), ws.numel(),
              _lib.stream_of(approx))


def draft_pick_bf16(approx, x, w, nout, argmax_first, top, top_values, token, vtok, children, calls=None, tiled=True):
    """The draft pick of a bf16 lm_head (this library's own): as draft_pick, with the candidates' exact logits
    those bf16_linear(x, w) gives (recomputed with its MFMA chain), 16 candidates per segment; top_values
    (bf16, may be None) receives the top-nout logits. Equals bf16_linear + fast_topk whenever their top-nout
    lies within the candidates."""
    _dev(approx, "approx")
    _check(approx.dtype == torch.bfloat16 and approx.is_contiguous(), "approx: bf16 row")
    N = approx.numel()
    _check(w.dtype == torch.bfloat16 and w.is_contiguous() and w.dim() == 2 and w.shape[0] == N, "w: bf16 [N, K]")
    K = w.shape[1]
    _check(x.dtype == torch.bfloat16 and x.is_contiguous() and x.numel() == K, "x: bf16 [K]")
    _check(1 <= int(nout) <= 8, "1 <= nout <= 8")
    if top_values is not None:
        _check(top_values.dtype == torch.bfloat16 and top_values.numel() >= nout, "top values bf16 [>= nout]")
    ch, nch = _pick_outputs(top, None, token, vtok, children, calls, int(nout))
    ws = _pick_ws(approx.device)
    _lib.call("mdx_draft_pick_bf16", _lib.ptr(approx), _lib.ptr(x), _lib.ptr(w), _lib.LAYOUT_TILE if tiled else _lib.LAYOUT_ROW,
              N, K, int(nout), int(bool(argmax_first)), _lib.ptr(top) if _present(top) else None,
              _lib.ptr(top_values), _lib.ptr(token), _lib.ptr(vtok), vtok.numel(), ch, nch, _lib.ptr(calls), _lib.ptr(ws),
              ws.numel(), _lib.stream_of(approx))
