"""Host-side weight preparation: the packed-W4 contract, its tile-major copy, GPTQ ingestion,
the ConvRot Hadamard and the activation lookup tables.

The packed-W4 contract is the reference's (comfy_mono_decode_xpu/mono.py:58-79,
csrc/w4a8_decode.sycl:4-11): codes [N, K/2] int8 (byte b = code of k = 2b in the low nibble,
2b + 1 in the high), relative group scales s_rel [N, K/G], fp32 channel scales [N], a 16-entry
fp32 codebook; w8 = isnan(r) ? 0 : clamp(r, -127, 127), r = rint(codebook[code] * s_rel).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from . import _lib

_SDT = {torch.float32: _lib.DT_F32, torch.float16: _lib.DT_F16, torch.float8_e4m3fn: _lib.DT_FP8E4M3}


def _split_nibbles(b: torch.Tensor) -> torch.Tensor:
    """Every 4-byte word of 8 codes in the packed order (byte i: code 2i low, 2i + 1 high) -> the
    split order: low nibbles of bytes 0..3 = codes 0..3, high nibbles = codes 4..7."""
    u = b.contiguous().view(torch.uint8).reshape(-1, 4)
    codes = torch.stack([u & 15, u >> 4], dim=-1).reshape(-1, 8)
    return (codes[:, :4] | (codes[:, 4:] << 4)).reshape(b.shape).view(torch.int8)


def _join_nibbles(b: torch.Tensor) -> torch.Tensor:
    """Inverse of _split_nibbles."""
    u = b.contiguous().view(torch.uint8).reshape(-1, 4)
    codes = torch.cat([u & 15, u >> 4], dim=-1)  # codes 0..7
    return (codes[:, 0::2] | (codes[:, 1::2] << 4)).reshape(b.shape).view(torch.int8)


def tile_major_codes(packed: torch.Tensor) -> torch.Tensor:
    """[N, K/2] codes -> the tile-major copy [N/16][K/128][4][16][16 B], kept as [N, K/2].

    Chunk (tile, k0) of 16 columns x 128 k becomes one contiguous KiB whose 16-byte piece
    (kq, c) is column c's codes of k0 + 32 kq + [0, 32): one coalesced load per wave. Within each
    4-byte word (8 consecutive k) the low nibbles hold k 0..3 and the high nibbles k 4..7, so a
    word's two nibble masks line up with two natural-order activation words (no byte shuffles)."""
    n, kb = packed.shape
    assert n % 16 == 0 and kb % 64 == 0, "N % 16 and K % 128"
    t = packed.reshape(n // 16, 16, kb // 64, 4, 16).permute(0, 2, 3, 1, 4).contiguous().reshape(n, kb)
    return _split_nibbles(t)


def row_major_codes(tiled: torch.Tensor) -> torch.Tensor:
    """Inverse of tile_major_codes."""
    n, kb = tiled.shape
    t = _join_nibbles(tiled)
    return t.reshape(n // 16, kb // 64, 4, 16, 16).permute(0, 3, 1, 2, 4).contiguous().reshape(n, kb)


def pack_codes(codes: torch.Tensor) -> torch.Tensor:
    """int codes [N, K] in 0..15 -> packed int8 [N, K/2] (k = 2b low nibble, 2b + 1 high)."""
    c = codes.to(torch.int32)
    return ((c[:, 0::2] & 15) | ((c[:, 1::2] & 15) << 4)).to(torch.uint8).view(torch.int8)


def unpack_codes(packed: torch.Tensor) -> torch.Tensor:
    b = packed.view(torch.uint8).to(torch.int32)
    out = torch.empty(packed.shape[0], packed.shape[1] * 2, dtype=torch.int32, device=packed.device)
    out[:, 0::2] = b & 15
    out[:, 1::2] = b >> 4
    return out


def gptq_pack(q: torch.Tensor, scales: torch.Tensor, group_size: int = 128, integral: bool = False):
    """GPTQ int4 symmetric weights (q in [-8, 7] as [N, K], fp16 group scales [N, K/G]) -> the
    packed-W4 contract (packed, s_rel fp16, s_channel fp32, codebook None = code - 8).

    integral=False (the default; the form checkpoint ingestion produces): s_channel[n] =
    max_g s_g * 8 / 127 and s_rel = fp16(s_g / s_channel) <= 127 / 8, decoded per weight by rint, the
    reference's W4 contract (csrc/w4a8_decode.sycl:4-11,35-45). integral=True (lossy, opt-in):
    s_channel[n] = max_g s_g / 15 and s_rel = round(s_g / s_channel) in 1..15, which re-quantises each
    group scale (up to smax / (30 s_g) relative error) so that w8 = q * s_rel exactly and libmdx can
    take its factorised integer path. In both, w8 * s_channel approximates q * s_g, |w8| <= 127 (no
    clamp)."""
    n, k = q.shape
    assert k % group_size == 0 and scales.shape == (n, k // group_size)
    s = scales.float()
    # the channel scales on the host: a GPU division by a scalar is a multiplication by its reciprocal,
    # so the same weights would pack differently on the two devices (the rest is elementwise IEEE)
    smax = s.abs().amax(dim=1).clamp_min(1e-30).cpu()
    sch = (smax / 15.0 if integral else smax * 8.0 / 127.0).to(s.device)
    if integral:
        s_rel = torch.round(s / sch[:, None]).clamp(1, 15)
    else:
        s_rel = (s / sch[:, None]).clamp(max=127.0 / 8.0)
    packed = pack_codes(q.to(torch.int32) + 8)
    return packed, s_rel.to(torch.float16).contiguous(), sch.float().contiguous(), None


@dataclass
class W4:
    """A packed W4A8 linear on the device: the four contract tensors plus how libmdx reads them."""
    q: torch.Tensor
    s: torch.Tensor
    sc: torch.Tensor
    cb: torch.Tensor | None
    layout: int = _lib.LAYOUT_ROW
    decode: int = _lib.DECODE_AUTO
    _struct: object = field(default=None, repr=False, compare=False)

    @property
    def n(self):
        return self.q.shape[0]

    @property
    def k(self):
        return self.q.shape[1] * 2

    @property
    def group_size(self):
        return self.k // self.s.shape[1]

    def struct(self):
        if self._struct is None:
            st = _lib.MdxW4()
            st.q, st.s_rel = self.q.data_ptr(), self.s.data_ptr()
            st.s_channel = self.sc.data_ptr()
            st.codebook = None if self.cb is None else self.cb.data_ptr()
            st.n, st.k, st.group_size = self.n, self.k, self.group_size
            st.s_dtype = _SDT[self.s.dtype]
            st.layout, st.decode = self.layout, self.decode
            self._struct = st
        return self._struct

    def tiled(self) -> "W4":
        """The tile-major copy (resident weights): codes permuted, scales unchanged."""
        assert self.layout == _lib.LAYOUT_ROW
        return W4(tile_major_codes(self.q), self.s, self.sc, self.cb, _lib.LAYOUT_TILE, self.decode)


def integral_ok(s_rel: torch.Tensor, codebook: torch.Tensor | None) -> bool:
    """True if w8 = (code - 8) * s_rel exactly for every weight: default codebook and integer
    scales in [-15, 15] (so |w8| <= 120 < 127 and rint is a no-op)."""
    if s_rel.dtype not in (torch.float16, torch.float32, torch.float8_e4m3fn):
        return False
    if codebook is not None:
        ref = torch.arange(-8, 8, dtype=torch.float32, device=codebook.device)
        if codebook.numel() != 16 or not torch.equal(codebook.reshape(-1).float(), ref):
            return False
    s = s_rel.float()
    return bool(torch.isfinite(s).all() and (s == torch.round(s)).all() and (s.abs() <= 15).all())


def w4_from(q, s, sc, cb, layout=_lib.LAYOUT_ROW, decode=_lib.DECODE_AUTO) -> W4:
    return W4(q, s, sc, cb, layout, decode)


# ---- ConvRot Hadamard -------------------------------------------------------------------------
H4 = ((1, 1, 1, -1), (1, 1, -1, 1), (1, -1, 1, 1), (-1, 1, 1, 1))


def regular_hadamard(device=None, dtype=torch.bfloat16) -> torch.Tensor:
    """kron(H4, H4, H4, H4) / 16 (comfy_kitchen's regular ConvRot H256; reference
    csrc/draft_fused.sycl:49-65, comfy_mono_decode_xpu/layer.py:74-90)."""
    h4 = torch.tensor(H4, dtype=torch.float64)
    h = h4
    for _ in range(3):
        h = torch.kron(h, h4)
    return (h / 16).to(dtype).to(device).contiguous()


_rot_cache: dict = {}


def classify_rotation(h: torch.Tensor | None) -> int:
    """MDX_ROT_* for a [256, 256] bf16 matrix: the regular H256 and the identity get their exact
    fast forms; anything else is applied as a generic matrix. Cached per (pointer, version); the
    cache holds the tensor itself, so a cached address cannot be reused by another tensor."""
    if h is None:
        return _lib.ROT_NONE
    key = (h.data_ptr(), h._version, tuple(h.shape), h.device)
    hit = _rot_cache.get(key)
    if hit is not None and hit[0] is h:
        return hit[1]
    kind = _lib.ROT_MATRIX
    if h.numel() == 65536:
        hb = h.reshape(256, 256)
        if torch.equal(hb.view(torch.int16), regular_hadamard(hb.device, hb.dtype).view(torch.int16)):
            kind = _lib.ROT_H256
        elif torch.equal(hb.float(), torch.eye(256, device=hb.device)):
            kind = _lib.ROT_NONE
    if len(_rot_cache) >= 16:
        _rot_cache.pop(next(iter(_rot_cache)))
    _rot_cache[key] = (h, kind)
    return kind


def bf16_all(device=None) -> torch.Tensor:
    return torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).to(device)


def silu_lut(device=None) -> torch.Tensor:
    """torch's own SiLU for every bf16 input (reference comfy_mono_decode_xpu/mono.py:44-45)."""
    return F.silu(bf16_all(device)).contiguous()


def sigmoid_lut(device=None) -> torch.Tensor:
    return torch.sigmoid(bf16_all(device)).contiguous()


def tile_major_bf16(w: torch.Tensor) -> torch.Tensor:
    """bf16 [N, K] -> the bf16 linear's tile-major order [N/16][K/32][64 lanes][8] (lane 16 g + c holds
    row 16 t + c, k in [32 j + 8 g, 32 j + 8 g + 8) of block (t, j)), returned as [N, K]."""
    N, K = w.shape
    assert N % 16 == 0 and K % 32 == 0
    return w.reshape(N // 16, 16, K // 32, 4, 8).permute(0, 2, 3, 1, 4).contiguous().reshape(N, K)


def tile_major_i8(w: torch.Tensor) -> torch.Tensor:
    """int8 [N, K] -> the W8A8 linear's tile-major order [N/16][K/64][64 lanes][16] (lane 16 g + c holds
    row 16 t + c, k in [64 j + 16 g, 64 j + 16 g + 16) of block (t, j)), returned as [N, K]."""
    N, K = w.shape
    assert w.dtype == torch.int8 and N % 16 == 0 and K % 64 == 0
    return w.reshape(N // 16, 16, K // 64, 4, 16).permute(0, 2, 3, 1, 4).contiguous().reshape(N, K)


def row_major_i8(t: torch.Tensor) -> torch.Tensor:
    """Inverse of tile_major_i8."""
    N, K = t.shape
    return t.reshape(N // 16, K // 64, 4, 16, 16).permute(0, 3, 1, 2, 4).contiguous().reshape(N, K)


def convrot_rotate(w: torch.Tensor) -> torch.Tensor:
    """w [N, K] (K % 256 == 0) -> float32 w . H256 per 256-column group, H256 = kron(H4, H4, H4, H4) / 16 (the
    ConvRot rotation, comfy_mono_decode_xpu/layer.py:74-90; orthogonal, so (x H)(w H)^T = x w^T), computed
    in float64 (exact for bf16 inputs up to one rounding to float32)."""
    N, K = w.shape
    assert K % 256 == 0
    h = regular_hadamard(w.device, torch.float64)
    out = torch.empty(N, K, dtype=torch.float32, device=w.device)
    for n0 in range(0, N, 8192):
        b = w[n0:n0 + 8192].to(torch.float64).reshape(-1, K // 256, 256)
        out[n0:n0 + 8192] = (b @ h).reshape(-1, K).float()
    return out


def int8_convrot_head(w: torch.Tensor):
    """An int8 ConvRot lm_head from a bf16 / float head [N, K]: the rows rotated by H256 per 256 group
    (convrot_rotate), then quantised per row, s = max(amax / 127, 1e-30) (f32), q = clamp(rint(w_rot / s),
    -127, 127) int8 -- the weight form comfy-kitchen's TensorWiseINT8Layout with convrot (group size 256)
    holds and draft_lmhead._plain accepts (comfy_mono_decode_xpu/draft_lmhead.py:33-46). Returns (q int8
    [N, K] row-major, s f32 [N])."""
    N, K = w.shape
    q = torch.empty(N, K, dtype=torch.int8, device=w.device)
    s = torch.empty(N, dtype=torch.float32, device=w.device)
    for n0 in range(0, N, 16384):
        r = convrot_rotate(w[n0:n0 + 16384])
        sc = (r.abs().amax(1) / 127.0).clamp_min(1e-30)
        q[n0:n0 + 16384] = torch.round(r / sc[:, None]).clamp(-127, 127).to(torch.int8)
        s[n0:n0 + 16384] = sc
    return q, s


def int4_scoring_copy(w: torch.Tensor, group_size: int = 128) -> W4:
    """An int4 copy of a bf16 or int8 head [N, K] for the first stage of the two-stage draft lm_head
    (comfy_mono_decode_xpu/draft_lmhead.py:80-95 makes the same kind of copy of its int8 head): per group of
    `group_size` along K, symmetric codes q = clamp(rint(w / s_g), -8, 7) with s_g = amax_g / 7, packed by
    the integral GPTQ packer and laid out tile-major. Its products are scores for choosing candidates,
    never logits. Built in row blocks (bounded temporary memory)."""
    N, K = w.shape
    assert K % group_size == 0
    codes, scales = [], []
    for n0 in range(0, N, 16384):
        b = w[n0:n0 + 16384].float().view(-1, K // group_size, group_size)
        sg = (b.abs().amax(-1) / 7.0).clamp_min(1e-30)
        codes.append((b / sg[..., None]).round().clamp(-8, 7).to(torch.int8).view(-1, K))
        scales.append(sg)
    q = torch.cat(codes)
    sg = torch.cat(scales).clamp(max=65504.0).to(torch.float16)
    packed, s_rel, sch, _ = gptq_pack(q, sg, group_size, integral=True)
    del q
    return W4(tile_major_codes(packed), s_rel, sch, None, _lib.LAYOUT_TILE, _lib.DECODE_INTEGRAL)
