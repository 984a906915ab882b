"""ctypes binding of libmdx.so (the C ABI declared in include/mdx.h).

torch is imported first on purpose: torch ships its own HIP runtime (soname libamdhip64.so.7), and
loading it before libmdx makes the dynamic loader bind libmdx to that same runtime, so torch's
streams and device pointers are valid inside libmdx.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see above)

HERE = os.path.dirname(os.path.abspath(__file__))
# MDX_LIB: another build of the library to load (side-by-side A/B timing of two builds in one run)
LIB_PATH = os.environ.get("MDX_LIB") or os.path.join(HERE, "libmdx.so")

MDX_OK, MDX_EINVAL, MDX_EHIP = 0, 1, 2
DT_F32, DT_F16, DT_FP8E4M3, DT_BF16 = 0, 1, 2, 3
LAYOUT_ROW, LAYOUT_TILE = 0, 1
DECODE_EXACT, DECODE_AUTO, DECODE_INTEGRAL = 0, 1, 2
ROT_NONE, ROT_H256, ROT_MATRIX = 0, 1, 2

c_void_p, c_int32, c_int64, c_size_t = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t


class MdxW4(ctypes.Structure):
    _fields_ = [("q", c_void_p), ("s_rel", c_void_p), ("s_channel", c_void_p), ("codebook", c_void_p),
                ("n", c_int64), ("k", c_int64), ("group_size", c_int64),
                ("s_dtype", c_int32), ("layout", c_int32), ("decode", c_int32), ("reserved", c_int32)]


W4P = ctypes.POINTER(MdxW4)

# name -> (restype, argtypes); every symbol declared in include/mdx.h
SIGNATURES = {
    "mdx_last_error": (ctypes.c_char_p, []),
    "mdx_version": (ctypes.c_int, []),
    "mdx_w4a8_decode_linear": (ctypes.c_int, [c_void_p, c_void_p, W4P, c_void_p, c_void_p, c_int32, c_int64, c_void_p]),
    "mdx_rot_quant": (ctypes.c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "mdx_mono_mlp_workspace": (c_size_t, [c_int64, c_int64, c_int64]),
    "mdx_mono_mlp_error_offset": (c_size_t, []),
    "mdx_mono_mlp": (ctypes.c_int, [c_void_p, c_void_p, ctypes.c_float, c_void_p, c_int32, c_void_p, W4P, W4P, W4P,
                                    c_void_p, c_void_p, c_int64, c_void_p, c_size_t, c_void_p]),
    "mdx_gate_rot_quant": (ctypes.c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p,
                                          c_int32, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "mdx_stream_gemv": (ctypes.c_int, [c_void_p, c_void_p, ctypes.POINTER(W4P), c_int32, c_int32,
                                       ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p), c_int32, c_void_p, c_int64,
                                       c_void_p]),
    "mdx_rms_rot_quant": (ctypes.c_int, [c_void_p, c_void_p, ctypes.c_float, c_void_p, c_void_p, c_int32, c_void_p,
                                         c_void_p, c_int64, c_int64, c_void_p]),
    "mdx_qk_norm_rope_kv": (ctypes.c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int64,
                                           c_int64, c_void_p, c_void_p, ctypes.c_float, ctypes.c_float, c_void_p,
                                           c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64,
                                           c_int64, c_int64, c_int64, c_int64, c_void_p]),
    "mdx_mtp_prep_draft": (ctypes.c_int, [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                                          c_void_p, c_void_p]),
    "mdx_mtp_prep_verify": (ctypes.c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int64,
                                           c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p]),
    "mdx_mtp_prep_verify_rows": (ctypes.c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int64,
                                                c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p,
                                                c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p,
                                                c_void_p, c_void_p]),
    "mdx_mtp_accept": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64,
                                      c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64,
                                      c_int64, c_int64, c_void_p, c_void_p]),
    "mdx_topk_workspace": (c_size_t, [c_int64]),
    "mdx_fast_topk": (ctypes.c_int, [c_void_p, c_int64, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_size_t,
                                     c_void_p]),
    "mdx_fast_pick": (ctypes.c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                     c_void_p]),
    "mdx_topk_rows": (ctypes.c_int, [c_void_p, c_int32, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p,
                                     c_size_t, c_void_p]),
    "mdx_attn_workspace": (c_size_t, [c_int64, c_int64, c_int64, c_int64, c_int64, c_int64]),
    "mdx_attn_decode": (ctypes.c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                       c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64,
                                       c_int64, c_int64, c_int64, c_int64, c_void_p, c_size_t, c_void_p]),
    "mdx_attn_decode_rope": (ctypes.c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int64,
                                            c_int64, c_void_p, c_void_p, ctypes.c_float, ctypes.c_float, c_void_p,
                                            c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                            c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64,
                                            c_int64, c_void_p, c_size_t, c_void_p]),
    "mdx_bf16_linear": (ctypes.c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_int64, c_int64, c_int64,
                                       c_void_p]),
    "mdx_attn_exact": (ctypes.c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                      c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64,
                                      c_int64, c_int64, c_int64, ctypes.c_float, c_void_p]),
    "mdx_int8_linear": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_int64,
                                       c_int64, c_void_p]),
    "mdx_gdn_core": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p,
                                    c_void_p, c_void_p, c_void_p,
                                    c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_float,
                                    ctypes.c_float, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p]),
    "mdx_gdn_core_raw": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p,
                                        c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                        ctypes.c_float, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p]),
    "mdx_gdn_proj": (ctypes.c_int, [c_void_p, c_void_p, W4P, W4P, c_void_p, c_void_p,
                                    c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                    c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_float,
                                    c_int64, c_int64, c_int64, c_int64, c_void_p]),
    "mdx_gdn_delta": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_float, c_void_p, c_int64, c_int64,
                                     c_int64, c_int64, c_void_p]),
    "mdx_gnorm_linear": (ctypes.c_int, [c_void_p, c_void_p, c_int32, c_void_p, ctypes.c_float, c_void_p, W4P,
                                        c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
    "mdx_gnorm_rot_quant": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, ctypes.c_float, c_void_p, c_void_p,
                                           ctypes.c_int32, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "mdx_topk_rows_noalloc": (ctypes.c_int, [c_void_p, c_int32, c_int64, c_int64, c_int64, c_void_p, c_void_p,
                                             c_void_p]),
    "mdx_topk_sample": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, ctypes.c_float, c_int64, c_int64, c_void_p,
                                       c_void_p]),
    "mdx_topk_sample_seeded": (ctypes.c_int, [c_void_p, c_void_p, ctypes.c_uint64, c_void_p, ctypes.c_float, c_int64,
                                              c_int64, c_void_p, c_void_p]),
    "mdx_rmsnorm": (ctypes.c_int, [c_void_p, c_void_p, ctypes.c_float, c_void_p, c_int64, c_int64, c_void_p]),
    "mdx_silu_mul": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
    "mdx_draft_embed_norm_cat": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p,
                                                c_void_p, c_void_p, ctypes.c_float, ctypes.c_float, c_void_p, c_int64,
                                                c_int64, c_void_p]),
    "mdx_draft_add_rmsnorm": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, ctypes.c_float, c_void_p, c_int64, c_int64,
                                             c_void_p]),
    "mdx_draft_sigmoid_mul": (ctypes.c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                                             c_int64, c_void_p]),
    "mdx_draft_silu_mul": (ctypes.c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "mdx_draft_norm_rot_quant": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, ctypes.c_float, c_int32, c_void_p,
                                                c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "mdx_stream_read": (ctypes.c_int, [c_void_p, c_int64, c_int32, c_void_p, c_void_p]),
    "mdx_gemv_trace": (c_int32, [c_void_p, c_int32]),
    "mdx_check_bf16_round": (ctypes.c_int, [c_void_p, c_void_p, c_void_p]),
    "mdx_draft_pick_workspace": (c_size_t, []),
    "mdx_draft_pick": (ctypes.c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int32,
                                      c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                      c_void_p, c_size_t, c_void_p]),
    "mdx_draft_pick_bf16": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_int32, c_int64, c_int64, c_int64, c_int32,
                                           c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                           c_void_p, c_size_t, c_void_p]),
}

_lib = None


class MdxError(RuntimeError):
    pass


def lib():
    """The loaded library (raises if it was not built: there is no fallback path)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MdxError(f"libmdx.so not built ({LIB_PATH}); run comfy-mono-decode-xpu_amd/build.py")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def call(name, *args):
    rc = getattr(lib(), name)(*args)
    if rc != MDX_OK:
        msg = lib().mdx_last_error().decode(errors="replace")
        raise MdxError(f"{name}: {msg}")
    return rc


SRC_Q8, SRC_HR, SRC_XP, SRC_GN = 0, 1, 2, 3
SRC_INT_ONLY, SRC_TBL, SRC_TBL8, SRC_GDN = 4, 8, 16, 32


def gemv_trace():
    """The GEMV kernel variants this thread launched since the previous call (mdx_gemv_trace): a list of
    dicts {mfma, src (SRC_Q8 / SRC_HR / SRC_XP), decode ("integral", "table16", "table8" or "generic"),
    s_dtype, rows, tpw, ks, red_alias, gdn (a Gated-DeltaNet projection: conv epilogue, gate work-groups)}."""
    buf = (c_int32 * (7 * 64))()
    n = lib().mdx_gemv_trace(buf, 64)
    out = []
    for i in range(min(n, 64)):
        mfma, src, sdt, rows, tpw, ks, alias = buf[7 * i:7 * i + 7]
        dec = ("integral" if src & SRC_INT_ONLY else "table16" if src & SRC_TBL else "table8" if src & SRC_TBL8
               else "generic")
        out.append(dict(mfma=bool(mfma), src=src & 3, decode=dec, s_dtype=sdt, rows=rows, tpw=tpw, ks=ks,
                        red_alias=bool(alias), gdn=bool(src & SRC_GDN)))
    return out


def stream_of(t: torch.Tensor):
    return c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def ptr(t):
    return None if t is None else c_void_p(t.data_ptr())
