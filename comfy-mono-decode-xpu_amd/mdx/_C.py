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

import torch

from . import _lib
from .layout import W4, classify_rotation

_OUT_DT = {0: (torch.float32, _lib.DT_F32), 2: (torch.bfloat16, _lib.DT_BF16)}


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _dev(t, what):
    _check(isinstance(t, torch.Tensor) and t.is_cuda, f"{what} must be a tensor on the ROCm device")


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
    return W4(q, s, sc, cb, _lib.LAYOUT_TILE if tiled else _lib.LAYOUT_ROW, _lib.DECODE_AUTO)


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


def mono_mlp_w4(xn, rot, h, silu_lut, gate: W4, up: W4, down: W4, norm_w=None, eps=1e-6, out=None, ws=None):
    """mono_mlp on prepared W4 handles (the library's own callers); norm_w: RMSNorm the input first."""
    K1 = xn.shape[-1]
    rows = xn.numel() // K1
    if out is None:
        out = torch.empty(rows, down.n, dtype=torch.bfloat16, device=xn.device)
    ws_bytes = _lib.lib().mdx_mono_mlp_workspace(rows, K1, gate.n)
    if ws is None:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=xn.device)
    _lib.call("mdx_mono_mlp", _lib.ptr(xn), _lib.ptr(norm_w), float(eps), _lib.ptr(h), rot, _lib.ptr(silu_lut),
              gate.struct(), up.struct(), down.struct(), _lib.ptr(out), rows, _lib.ptr(ws), ws.numel(),
              _lib.stream_of(xn))
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
