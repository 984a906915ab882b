"""On-disk W4A8 checkpoints -> the packed-W4 contract in the GEMV engine's tile-major layout.

Two source forms of a quantized linear, each checked against the contract before anything is packed
(an ineligible linear is reported with a reason and left to the caller, as the reference's routing
falls back per module, comfy_mono_decode_xpu/mono.py:31-38):

- GPTQ (AutoGPTQ / GPTQModel tensors: qweight int32 [K/8, N] with code k = 8 i + j in bits 4 j..4 j + 3
  of row i, qzeros int32 [K/G, N/8] packed the same way along N, scales fp16 [K/G, N], g_idx int32 [K]):
  w[n, k] = scales[g_idx[k], n] * (code[k, n] - zero[g_idx[k], n]). Eligible: 4 bits, symmetric
  (every zero 8; the "gptq" v1 format stores zero - 1), groups in order (g_idx[k] = k // G), no bias,
  finite positive scales. Packed by layout.gptq_pack (q = code - 8 with the default codebook).
- comfy-kitchen's AsymW4A8Int8Layout (the reference kernel's own contract, csrc/w4a8_decode.sycl:4-11):
  codes int8 [N, K/2] (byte b: code 2 b low nibble, 2 b + 1 high), fp8 e4m3 group scales [N, K/16],
  s_channel [N], codebook f32 [16]. Eligible exactly when the reference's checks pass
  (comfy_mono_decode_xpu/mono.py:58-96: group size 16, ConvRot group 256, not mma-packed, not
  transposed, no correction, contiguous int8 codes, N % 16 == 0, K % 256 == 0, scale / codebook /
  s_channel sizes, no bias, fp8 scale bytes below 0x80). The tensors are kept bit for bit; only the
  codes are permuted tile-major (the reference's tiles.tile_major does the same for its own tile,
  comfy_mono_decode_xpu/tiles.py:45-48,304-354).

The int8 ConvRot lm_head (comfy-kitchen's TensorWiseINT8Layout with convrot, group 256) is taken under
the checks of comfy_mono_decode_xpu/draft_lmhead.py:33-46.

Safetensors files are read lazily (safe_open): a linear's tensors are loaded when it is packed. GPTQ
keys are the standard `<prefix>.qweight / .qzeros / .scales / .g_idx / .bias`. The reference reads live
QuantizedTensor objects, not files, and comfy-kitchen's serialiser is not part of it; for a W4A8 layout
stored in a file this module's key map is `<prefix>.weight` (codes), `.weight_scale`, `.s_channel`,
`.codebook` (and `.bias`), a parameter of the reader (`W4A8_KEYS`). Live objects with `_qdata` and
`_params` (what the reference's tiles.row_major reads) go through w4_from_quantized.
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field

import torch

from . import _lib, layout

W4A8_KEYS = dict(codes="weight", scale="weight_scale", s_channel="s_channel", codebook="codebook", bias="bias")


class Ineligible(Exception):
    """A linear that the packed-W4 contract does not cover; `reason` names the failed check."""

    def __init__(self, reason, detail=""):
        super().__init__(f"{reason}: {detail}" if detail else reason)
        self.reason = reason


def _need(cond, reason, detail=""):
    if not cond:
        raise Ineligible(reason, detail)


# ---------------------------------------------------------------------------------------------------
# GPTQ
# ---------------------------------------------------------------------------------------------------
def unpack_int32_nibbles(t: torch.Tensor, axis: int) -> torch.Tensor:
    """int32 words holding 8 4-bit codes (code j in bits 4 j..4 j + 3) -> int32 codes, the words' axis
    `axis` expanded eightfold (element 8 i + j from word i)."""
    shifts = torch.arange(0, 32, 4, dtype=torch.int32, device=t.device)
    if axis == 0:
        c = (t[:, None, :] >> shifts[None, :, None]) & 15
        return c.reshape(t.shape[0] * 8, t.shape[1])
    c = (t[:, :, None] >> shifts[None, None, :]) & 15
    return c.reshape(t.shape[0], t.shape[1] * 8)


def w4_from_gptq(qweight, qzeros, scales, g_idx=None, bias=None, *, bits=4, group_size=None, sym=True,
                 checkpoint_format="gptq", integral=False, device=None, tiled=True) -> layout.W4:
    """A GPTQ linear -> layout.W4 (tile-major unless tiled=False). integral=False (the default) keeps the
    fp16 group scales as fp16 ratios to the channel scale (per-weight rint decode, the reference's A1
    contract); integral=True re-quantises them to 4-bit integer multiples (the integral fast path, group
    scale error up to smax / 30)."""
    _need(bits == 4, "bits", f"{bits}-bit")
    _need(sym, "zeros", "asymmetric quantisation")
    _need(bias is None, "bias")
    _need(qweight.dtype == torch.int32 and qweight.dim() == 2, "qweight", "int32 [K/8, N]")
    K, N = qweight.shape[0] * 8, qweight.shape[1]
    _need(scales.dim() == 2 and scales.shape[1] == N and scales.dtype in (torch.float16, torch.bfloat16, torch.float32),
          "scales", "[K/G, N]")
    G = K // scales.shape[0] if scales.shape[0] else 0
    _need(G > 0 and G * scales.shape[0] == K, "shape", "group size does not divide K")
    _need(group_size in (None, -1, G), "shape", f"group size {group_size} against scales for {G}")
    _need(N % 16 == 0 and K % 256 == 0, "shape", f"N {N} % 16, K {K} % 256")
    _need(G >= 16 and G & (G - 1) == 0, "shape", f"group size {G}: a power of two >= 16")
    _need(qzeros.dtype == torch.int32 and qzeros.shape == (K // G, N // 8), "qzeros", "int32 [K/G, N/8]")
    zeros = unpack_int32_nibbles(qzeros, 1)
    zeros = zeros + 1 if checkpoint_format == "gptq" else zeros
    _need(bool((zeros == 8).all()), "zeros", "symmetric GPTQ stores zero 8 in every group")
    if g_idx is not None:
        _need(g_idx.numel() == K, "g_idx", "[K]")
        _need(torch.equal(g_idx.to(torch.int64).cpu(), torch.arange(K) // G), "g_idx",
              "act-order (desc_act) permutes the groups")
    s = scales.float()
    _need(bool(torch.isfinite(s).all()) and bool((s > 0).all()), "scales", "finite and positive")
    codes = unpack_int32_nibbles(qweight.to(device) if device is not None else qweight, 0)  # [K, N]
    q = (codes.t().contiguous() - 8).to(torch.int8)
    st = s.t().contiguous().to(q.device).to(torch.float16)
    packed, s_rel, sch, _ = layout.gptq_pack(q, st, G, integral=integral)
    decode = _lib.DECODE_INTEGRAL if integral else _lib.DECODE_AUTO
    if tiled:
        return layout.W4(layout.tile_major_codes(packed), s_rel, sch, None, _lib.LAYOUT_TILE, decode)
    return layout.W4(packed, s_rel, sch, None, _lib.LAYOUT_ROW, decode)


# ---------------------------------------------------------------------------------------------------
# comfy-kitchen AsymW4A8Int8Layout
# ---------------------------------------------------------------------------------------------------
def w4_from_asym_w4a8(codes, scale, s_channel, codebook, bias=None, *, group_size=16, convrot_groupsize=256,
                      mma_packed=False, transposed=False, correction=None, device=None, tiled=True) -> layout.W4:
    """The reference's W4A8 tensors -> layout.W4, under the checks of comfy_mono_decode_xpu/mono.py:58-96
    (_layout_ok and _static_ok). The tensors are kept bit for bit."""
    _need(not mma_packed and not transposed, "layout", "mma-packed or transposed codes")
    _need(group_size == 16 and convrot_groupsize == 256, "group", f"group {group_size}, ConvRot {convrot_groupsize}")
    _need(correction is None, "correction")
    _need(bias is None, "bias")
    _need(scale is not None and codebook is not None and s_channel is not None, "params", "scale, codebook, s_channel")
    _need(codes.dtype == torch.int8 and codes.dim() == 2 and codes.is_contiguous(), "codes", "contiguous int8 [N, K/2]")
    N, K = codes.shape[0], codes.shape[1] * 2
    _need(N > 0 and K > 0 and N % 16 == 0 and K % 256 == 0, "shape", f"N {N} % 16, K {K} % 256")
    _need(scale.dtype == torch.float8_e4m3fn and scale.is_contiguous() and scale.numel() == N * (K // 16), "scale",
          "fp8 e4m3 [N, K/16]")
    _need(codebook.numel() == 16 and s_channel.numel() == N, "params", "codebook [16], s_channel [N]")
    _need(int(scale.view(torch.uint8).max()) < 128, "scale", "fp8 scale bytes 0x00-0x7F (non-negative)")
    dev = device if device is not None else codes.device
    q = codes.to(dev).contiguous()
    s = scale.reshape(N, K // 16).to(dev).contiguous()
    sc = s_channel.reshape(-1).to(torch.float32).to(dev).contiguous()
    cb = codebook.reshape(-1).to(torch.float32).to(dev).contiguous()
    if tiled:
        return layout.W4(layout.tile_major_codes(q), s, sc, cb, _lib.LAYOUT_TILE, _lib.DECODE_AUTO)
    return layout.W4(q, s, sc, cb, _lib.LAYOUT_ROW, _lib.DECODE_AUTO)


def w4_from_quantized(w, bias=None, device=None, tiled=True) -> layout.W4:
    """A live comfy-kitchen QuantizedTensor (duck-typed: `_qdata` and `_params` with scale, s_channel,
    codebook, group_size, convrot_groupsize, mma_packed, transposed, correction) -> layout.W4."""
    p, q = getattr(w, "_params", None), getattr(w, "_qdata", None)
    _need(p is not None and q is not None, "layout", "not a quantized tensor")
    return w4_from_asym_w4a8(q, getattr(p, "scale", None), getattr(p, "s_channel", None), getattr(p, "codebook", None),
                             bias, group_size=getattr(p, "group_size", None),
                             convrot_groupsize=getattr(p, "convrot_groupsize", None),
                             mma_packed=getattr(p, "mma_packed", False), transposed=getattr(p, "transposed", False),
                             correction=getattr(p, "correction", None), device=device, tiled=tiled)


def int8_head_from_tensorwise(q, s, *, convrot=True, convrot_groupsize=256, transposed=False, group=128,
                              device=None, tiled=True):
    """An int8 ConvRot lm_head (TensorWiseINT8Layout: q int8 [N, K], per-row scale f32 [N]) -> (weights for
    the W8A8 linear, f32 scales [N]), under the checks of comfy_mono_decode_xpu/draft_lmhead.py:33-46."""
    _need(convrot and convrot_groupsize == 256 and not transposed, "layout", "ConvRot group 256, not transposed")
    _need(isinstance(s, torch.Tensor) and q.dtype == torch.int8 and q.dim() == 2 and q.is_contiguous(), "codes",
          "contiguous int8 [N, K]")
    N, K = q.shape
    _need(s.numel() == N and s.dtype == torch.float32, "scale", "f32 [N]")
    _need(K % group == 0 and K % 256 == 0 and N % 16 == 0, "shape", f"N {N} % 16, K {K} % 256")
    dev = device if device is not None else q.device
    qd = q.to(dev).contiguous()
    return (layout.tile_major_i8(qd) if tiled else qd), s.reshape(-1).to(dev).contiguous()


# ---------------------------------------------------------------------------------------------------
# safetensors files
# ---------------------------------------------------------------------------------------------------
@dataclass
class Report:
    """What a scan or a load found: the packed linears' prefixes and, per ineligible linear, its reason."""
    formats: dict = field(default_factory=dict)   # prefix -> "gptq" | "w4a8" | "dense"
    packed: list = field(default_factory=list)
    fallback: dict = field(default_factory=dict)  # prefix -> reason
    shapes: dict = field(default_factory=dict)    # prefix -> (N, K)

    def reasons(self):
        out = {}
        for r in self.fallback.values():
            out[r] = out.get(r, 0) + 1
        return out


class Checkpoint:
    """A safetensors file (or a list of shards) read lazily. GPTQ options come from the caller or the
    file's metadata (`quantize_config`-style keys: bits, group_size, sym, desc_act, checkpoint_format)."""

    def __init__(self, paths, keys=None, **gptq):
        from safetensors import safe_open
        self.paths = [paths] if isinstance(paths, str) else list(paths)
        self._files = [safe_open(p, framework="pt") for p in self.paths]
        self._where = {}
        meta = {}
        for f in self._files:
            meta.update(f.metadata() or {})
            for k in f.keys():
                self._where[k] = f
        self.keys = dict(W4A8_KEYS, **(keys or {}))
        self.gptq = dict(bits=int(meta.get("bits", 4)), group_size=int(meta.get("group_size", -1)),
                         sym=str(meta.get("sym", "true")).lower() == "true",
                         checkpoint_format=meta.get("checkpoint_format", "gptq"))
        self.gptq.update(gptq)

    def __contains__(self, k):
        return k in self._where

    def tensor(self, k):
        return self._where[k].get_tensor(k)

    def shape(self, k):
        return tuple(self._where[k].get_slice(k).get_shape())

    def _opt(self, k):
        return self.tensor(k) if k in self._where else None

    def linears(self):
        """prefix -> format of every linear weight in the file."""
        out = {}
        for k in self._where:
            if k.endswith(".qweight"):
                out[k[:-len(".qweight")]] = "gptq"
        wk, sk = "." + self.keys["codes"], "." + self.keys["scale"]
        for k in self._where:
            if k.endswith(wk):
                p = k[:-len(wk)]
                if p in out:
                    continue
                if p + sk in self._where and p + "." + self.keys["s_channel"] in self._where:
                    out[p] = "w4a8"
                elif len(self.shape(k)) == 2:
                    out[p] = "dense"
        return dict(sorted(out.items()))

    def out_in(self, prefix, fmt):
        """(N, K) of a linear."""
        if fmt == "gptq":
            k8, n = self.shape(prefix + ".qweight")
            return n, k8 * 8
        n, kb = self.shape(prefix + "." + self.keys["codes"])
        return n, kb * 2 if fmt == "w4a8" else kb

    def w4(self, prefix, fmt=None, device=None, tiled=True, integral=False) -> layout.W4:
        fmt = fmt or self.linears().get(prefix)
        if fmt == "gptq":
            return w4_from_gptq(self.tensor(prefix + ".qweight"), self.tensor(prefix + ".qzeros"),
                                self.tensor(prefix + ".scales"), self._opt(prefix + ".g_idx"),
                                self._opt(prefix + ".bias"), integral=integral, device=device, tiled=tiled,
                                **self.gptq)
        if fmt == "w4a8":
            k = self.keys
            return w4_from_asym_w4a8(self.tensor(prefix + "." + k["codes"]), self.tensor(prefix + "." + k["scale"]),
                                     self.tensor(prefix + "." + k["s_channel"]), self.tensor(prefix + "." + k["codebook"]),
                                     self._opt(prefix + "." + k["bias"]), device=device, tiled=tiled)
        raise Ineligible("format", f"{prefix}: not a packed W4 linear ({fmt})")

    def load(self, prefixes=None, device=None, tiled=True, integral=False):
        """Pack every eligible W4 linear (or those named). Returns ({prefix: W4}, Report)."""
        rep = Report(formats=self.linears())
        out = {}
        for p, fmt in rep.formats.items():
            if prefixes is not None and p not in prefixes:
                continue
            rep.shapes[p] = self.out_in(p, fmt)
            if fmt == "dense":
                continue
            try:
                out[p] = self.w4(p, fmt, device=device, tiled=tiled, integral=integral)
                rep.packed.append(p)
            except Ineligible as e:
                rep.fallback[p] = e.reason
        return out, rep


# ---------------------------------------------------------------------------------------------------
# the hybrid decoder's per-model contract
# ---------------------------------------------------------------------------------------------------
_LAYER = re.compile(r"(?:^|\.)layers\.(\d+)\.(.+)$")
_ROLES = {"mlp.gate_proj": "g", "mlp.up_proj": "u", "mlp.down_proj": "d",
          "self_attn.q_proj": "q", "self_attn.k_proj": "k", "self_attn.v_proj": "v", "self_attn.o_proj": "o",
          "linear_attn.in_proj_qkv": "qkv", "linear_attn.in_proj_z": "z", "linear_attn.out_proj": "o"}


def plan_hybrid(report: Report, cfg):
    """The W4 linears of a Qwen3.5-style hybrid decoder (block.mlp.{gate,up,down}_proj,
    block.self_attn.{q,k,v,o}_proj, block.linear_attn.{in_proj_qkv, in_proj_z, out_proj}; the modules
    comfy_mono_decode_xpu/layer.py:123-127 routes) checked against the shapes of `cfg` (a HybridConfig).
    Returns ({layer: {role: prefix}}, {prefix: reason}) -- a layer runs on the packed path only when every
    one of its linears is packed and has its expected shape (the reference routes a block whole,
    comfy_mono_decode_xpu/layer.py:119-160)."""
    H, I, D = cfg.hidden, cfg.inter, cfg.head_dim
    qd, kd = cfg.heads * D, cfg.kv_heads * D
    gdn_ch = 2 * cfg.gdn_key_heads * 128 + cfg.gdn_value_heads * 128
    hv = cfg.gdn_value_heads * 128
    want_attn = {"q": {(qd, H), (2 * qd, H)}, "k": {(kd, H)}, "v": {(kd, H)}, "o": {(H, qd)}}
    want_gdn = {"qkv": {(gdn_ch, H)}, "z": {(hv, H)}, "o": {(H, hv)}}
    want_mlp = {"g": {(I, H)}, "u": {(I, H)}, "d": {(H, I)}}
    layers, bad = {}, {}
    for p, fmt in report.formats.items():
        m = _LAYER.search(p)
        if not m or m.group(2) not in _ROLES:
            continue
        i, role = int(m.group(1)), _ROLES[m.group(2)]
        layers.setdefault(i, {})[role] = p
    plan = {}
    for i, roles in sorted(layers.items()):
        if i >= cfg.layers:
            for p in roles.values():
                bad[p] = "layer"
            continue
        want = dict(want_mlp, **(want_attn if cfg.attention(i) else want_gdn))
        ok = True
        for role, shapes in want.items():
            p = roles.get(role)
            if p is None:
                ok = False
                continue
            if p in report.fallback:
                bad[p] = report.fallback[p]
                ok = False
            elif p not in report.packed:
                bad[p] = "format"
                ok = False
            elif report.shapes.get(p) not in shapes:
                bad[p] = "shape"
                ok = False
        if ok:
            plan[i] = {r: roles[r] for r in want}
    return plan, bad
