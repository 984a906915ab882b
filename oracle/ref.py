"""CPU oracle: a numpy restatement of the reference operator chain of the W4A8 decode path.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as what results are compared against / the timed CPU baseline -- never as a product path.

Every function cites the reference file:line it restates (comfy-mono-decode-xpu). Floating-point
steps are single IEEE operations on numpy float32 / float64 scalars or arrays (round to nearest
even, no fused multiply-add), bf16 is the round-to-nearest-even of the top 16 bits with NaN ->
0x7FC0. Where the reference's own order is not portable (Intel DPAS accumulation, the EU rsqrt),
the library's canonical order is restated instead; each such place says so.

Pinning (tests/test_oracle.py): bf16 / fp16 / fp8 conversions against torch's independent
conversions; the int8-grid decode against its closed forms (integral scales, half-even ties,
clamp, NaN); the int32 dot against an exact float64 matmul; the rotation against exact rational
arithmetic on the Kronecker matrix; RMSNorm against float64; top-k rank keys against brute-force
sorts; the accept walk against an independent tree walk.
"""
from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------------------------
# scalar formats
# ---------------------------------------------------------------------------------------------


def bf16_to_f32(b):
    """bf16 bit patterns (uint16) -> float32 (exact)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f):
    """float32 -> bf16 bits, round to nearest even; NaN -> 0x7FC0 (library convention)."""
    u = np.asarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, np.uint16(0x7FC0), r).astype(np.uint16)


def bfround(f):
    return bf16_to_f32(f32_to_bf16(f))


def fp8e4m3_to_f32(b):
    """OCP float8 e4m3fn bytes -> float32 (bias 7, subnormals m * 2^-9, 0x7F/0xFF NaN)."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int64)
    s = np.where(b >> 7, -1.0, 1.0)
    e = (b >> 3) & 15
    m = b & 7
    v = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return (s * v).astype(np.float32)


def scales_to_f32(s, dtype):
    """s_rel storage (raw numpy array of the given dtype name) -> float32."""
    if dtype == "f32":
        return np.asarray(s, dtype=np.float32)
    if dtype == "f16":
        return np.asarray(s).view(np.float16).astype(np.float32)
    if dtype == "fp8":
        return fp8e4m3_to_f32(np.asarray(s).view(np.uint8))
    raise ValueError(dtype)


# ---------------------------------------------------------------------------------------------
# A1: W4A8 decode linear -- csrc/w4a8_decode.sycl:4-11 (contract), :33-45 (decode4), :139-166
# ---------------------------------------------------------------------------------------------


def unpack_codes(packed):
    """packed [N, K/2] -> codes [N, K]: byte b holds k = 2b (low nibble), 2b + 1 (high)
    (csrc/w4a8_decode.sycl:33-45: code i of a word is bits 4i..4i+3)."""
    b = np.asarray(packed).view(np.uint8)
    out = np.empty((b.shape[0], b.shape[1] * 2), dtype=np.int64)
    out[:, 0::2] = b & 15
    out[:, 1::2] = b >> 4
    return out


def decode_w8(packed, s_rel_f32, codebook=None, group_size=128):
    """w8[n, k] = isnan(r) ? 0 : clamp(r, -127, 127), r = rint(float(cb[code]) * s_rel[n, k / G])
    in float32 (csrc/w4a8_decode.sycl:35-45; default codebook i - 8, :82). Returns int8 [N, K]."""
    packed = np.asarray(packed)
    s_rel_f32 = np.asarray(s_rel_f32, dtype=np.float32)
    cb = (np.arange(16, dtype=np.float32) - 8) if codebook is None else np.asarray(codebook, dtype=np.float32)
    n = packed.shape[0]
    out = np.empty((n, packed.shape[1] * 2), dtype=np.int8)
    for r0 in range(0, n, 1024):  # row blocks bound the temporaries
        codes = unpack_codes(packed[r0:r0 + 1024])
        sc = np.repeat(s_rel_f32[r0:r0 + 1024], group_size, axis=1)
        with np.errstate(invalid="ignore", over="ignore"):
            r = np.rint(cb[codes] * sc)  # float32 product (one rounding), then round-half-even
            r = np.where(np.isnan(r), 0.0, np.clip(r, -127, 127))
        out[r0:r0 + 1024] = r.astype(np.int8)
    return out


def int32_wrap(a):
    return ((np.asarray(a, dtype=np.int64) + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(np.int64)


def w4a8_acc(x, w8):
    """acc[m, n] = sum_k x[m, k] * w8[n, k] modulo 2^32 (csrc/w4a8_decode.sycl:8-9, 130-133).
    Computed as float64 matmuls of the integer values: exact, since |x| <= 128, |w8| <= 127 and
    K <= 2^20 keep every partial sum below 2^53 (checked)."""
    x = np.asarray(x, dtype=np.int64)
    assert x.shape[1] <= 1 << 20
    xf = x.astype(np.float64)
    w8 = np.asarray(w8)
    acc = np.empty((x.shape[0], w8.shape[0]), dtype=np.int64)
    for r0 in range(0, w8.shape[0], 2048):
        acc[:, r0:r0 + 2048] = (xf @ w8[r0:r0 + 2048].astype(np.float64).T).astype(np.int64)
    return int32_wrap(acc)


def w4a8_acc_int64(x, w8):
    """The same sum in int64 arithmetic (the bit-exact path, used to pin w4a8_acc)."""
    return int32_wrap(np.asarray(x, dtype=np.int64) @ np.asarray(w8, dtype=np.int64).T)


def scaleback(acc, xs, sch):
    """f = (float(acc) * xs[m]) * sch[n], each product rounded on its own
    (csrc/w4a8_decode.sycl:155-157; fused_scaleback, csrc/mono_common.hpp:510-516)."""
    f = np.asarray(acc, dtype=np.int64).astype(np.float32)
    f = (f * np.asarray(xs, dtype=np.float32).reshape(-1, 1)).astype(np.float32)
    return (f * np.asarray(sch, dtype=np.float32).reshape(1, -1)).astype(np.float32)


def w4a8_linear(x, xs, packed, s_rel_f32, sch, codebook=None, group_size=128, residual=None, out="bf16"):
    """The fused linear (csrc/w4a8_decode.sycl:139-166): bf16 bits or float32 out; with residual,
    cast(float(residual) + float(cast(f)))."""
    acc = w4a8_acc(x, decode_w8(packed, s_rel_f32, codebook, group_size))
    f = scaleback(acc, xs, sch)
    if out == "bf16":
        if residual is None:
            return f32_to_bf16(f)
        return f32_to_bf16(bf16_to_f32(residual) + bfround(f))
    if residual is None:
        return f
    return (np.asarray(residual, dtype=np.float32) + f).astype(np.float32)


# ---------------------------------------------------------------------------------------------
# A2: rot_quant -- csrc/act_prep.sycl:4-10, 70-91 (mono_common.hpp:419-441)
# ---------------------------------------------------------------------------------------------
H4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.int64)


def fwht256_f64(x):
    """x [..., 256] float64 -> x . kron(H4, H4, H4, H4) (no 1/16), as the library computes it:
    radix-4 stages along strides 1, 4, 16, 64, butterfly out = ((a0+a1)+a2)-a3,
    ((a0+a1)-a2)+a3, ((a0-a1)+a2)+a3, ((a1-a0)+a2)+a3 (H4 rows, csrc/draft_fused.sycl:59-64).
    Canonical order of this library: the reference's bf16 DPAS accumulation is not portable."""
    a = np.array(x, dtype=np.float64)
    for st in (1, 4, 16, 64):
        v = a.reshape(a.shape[:-1] + (256 // (4 * st), 4, st))
        a0, a1, a2, a3 = v[..., 0, :], v[..., 1, :], v[..., 2, :], v[..., 3, :]
        o = np.stack([((a0 + a1) + a2) - a3, ((a0 + a1) - a2) + a3, ((a0 - a1) + a2) + a3, ((a1 - a0) + a2) + a3],
                     axis=-2)
        a = o.reshape(a.shape)
    return a


def rotate_rows(xf, rot, h=None):
    """x_rot = bf16(x_group . H) per 256-group. rot: 'none' | 'h256' | 'matrix' (h: bf16 bits
    [256, 256]). fp64 sums (fixed order), one rounding to fp32, one to bf16."""
    xf = np.asarray(xf, dtype=np.float32)
    if rot == "none":
        return xf.copy()
    g = xf.reshape(xf.shape[0], -1, 256).astype(np.float64)
    if rot == "h256":
        r = fwht256_f64(g) * 0.0625
    else:
        hf = bf16_to_f32(h).reshape(256, 256).astype(np.float64)
        r = np.zeros_like(g)
        for k in range(256):  # sequential fp64 sum of exact products
            r = r + g[..., k:k + 1] * hf[k][None, None, :]
    return bfround(r.astype(np.float32).reshape(xf.shape))


def quantize_rows(xr):
    """scale = max(amax / 127, 1e-30) (f32), sb = bf16(scale) (0 -> 0x0080),
    q = int8(clamp(rint(float(bf16(xr / sb))), -128, 127)) (csrc/act_prep.sycl:70-91)."""
    xr = np.asarray(xr, dtype=np.float32)
    amax = np.fmax.reduce(np.abs(xr), axis=1, initial=np.float32(0)).astype(np.float32)
    scale = np.maximum((amax / np.float32(127.0)).astype(np.float32), np.float32(1e-30)).astype(np.float32)
    sb = f32_to_bf16(scale)
    sb = np.where((sb & 0x7FFF) == 0, np.uint16(0x0080), sb)
    sbf = bf16_to_f32(sb)
    with np.errstate(invalid="ignore", divide="ignore"):
        d = bfround((xr / sbf[:, None]).astype(np.float32))
        q = np.clip(np.rint(d), -128, 127)
    q = np.where(np.isnan(q), 0, q)
    return q.astype(np.int8), scale


def rot_quant(x_bits, rot="h256", h=None):
    """rot_quant(x, h) on bf16 bits [rows, K] -> (int8 [rows, K], f32 scale [rows])."""
    return quantize_rows(rotate_rows(bf16_to_f32(x_bits), rot, h))


# ---------------------------------------------------------------------------------------------
# A5: RMSNorm (library canonical order; the reference's OmniXPU tree + EU rsqrt,
# csrc/mono_common.hpp:452-505, is not portable)
# ---------------------------------------------------------------------------------------------


def rmsnorm_factor(xf, eps):
    """r = 1 / sqrt(ss / K + eps) for float32 rows [rows, K] (K a multiple of 256), all float32.
    ss in the library's canonical order: the row is cut into 256-element groups and each group
    into 64 runs of 4 elements (run l: elements 4 l .. 4 l + 3); a run's partial is
    ((sq0 + sq1) + sq2) + sq3, a group's sum is the halving tree over its 64 run partials
    (p[l] + p[l + 32], then + 16, ..., + 1), and ss adds the group sums in group order."""
    xf = np.asarray(xf, dtype=np.float32)
    rows, K = xf.shape
    assert K % 256 == 0
    sq = (xf * xf).astype(np.float32).reshape(rows, K // 256, 64, 4)
    p = sq[..., 0]
    for e in range(1, 4):
        p = (p + sq[..., e]).astype(np.float32)
    n = 64
    while n > 1:
        n //= 2
        p = (p[..., :n] + p[..., n:2 * n]).astype(np.float32)
    gs = p[..., 0]
    ss = gs[:, 0]
    for g in range(1, K // 256):
        ss = (ss + gs[:, g]).astype(np.float32)
    mean = (ss / np.float32(K)).astype(np.float32)
    return (np.float32(1.0) / np.sqrt((mean + np.float32(eps)).astype(np.float32))).astype(np.float32)


def rmsnorm(x_bits, w_bits, eps):
    """y = bf16((x * r) * w) (mono_common.hpp:497-502 form), r from rmsnorm_factor."""
    x = bf16_to_f32(x_bits).astype(np.float32)
    r = rmsnorm_factor(x, eps)
    w = bf16_to_f32(w_bits)
    return f32_to_bf16(((x * r[:, None]).astype(np.float32) * w[None, :]).astype(np.float32))


# ---------------------------------------------------------------------------------------------
# A4: mono_mlp -- csrc/mono_mlp.sycl:109-167
# ---------------------------------------------------------------------------------------------


def silu_mul(g_f32, u_f32, lut_bits):
    """h = bf16(float(lut[bf16(g)]) * float(bf16(u))) (csrc/mono_mlp.sycl:130-138)."""
    gb = f32_to_bf16(g_f32)
    act = bf16_to_f32(np.asarray(lut_bits, dtype=np.uint16)[gb])
    return f32_to_bf16((act * bfround(u_f32)).astype(np.float32))


def mono_mlp(xn_bits, rot, h, lut_bits, gate, up, down):
    """gate/up/down: dicts with packed, s (f32 array), sch, cb, G (row-major contract tensors);
    a dict may carry its decoded "w8" to skip the decode."""
    def w8(d):
        if "w8" not in d:
            d["w8"] = decode_w8(d["packed"], d["s"], d["cb"], d["G"])
        return d["w8"]
    q1, s1 = rot_quant(xn_bits, rot, h)
    accg = w4a8_acc(q1, w8(gate))
    accu = w4a8_acc(q1, w8(up))
    hb = silu_mul(scaleback(accg, s1, gate["sch"]), scaleback(accu, s1, up["sch"]), lut_bits)
    q2, s2 = rot_quant(hb, rot, h)
    accd = w4a8_acc(q2, w8(down))
    return f32_to_bf16(scaleback(accd, s2, down["sch"]))


def silu_lut_f64():
    """A float64 SiLU over every bf16 pattern (a pin for torch's table, not the table itself)."""
    x = bf16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16)).astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        return x / (1.0 + np.exp(-x))


# ---------------------------------------------------------------------------------------------
# RoPE + KV write (csrc/rope_kv.sycl)
# ---------------------------------------------------------------------------------------------


def head_rmsnorm(x_bits, w_bits, eps):
    """Per-head RMSNorm of qk_norm_rope_kv in the library's fixed order (the reference's Q tree of
    two 128-lane torch partials and its K tree with the EU rsqrt, csrc/rope_kv.sycl:193-219, are not
    portable): 64 lanes, lane l owns d = l + 64 j and sums x[d]^2 over j in order (fp32); the lanes are
    added by a halving tree (offsets 32, 16, .., 1); r = 1 / sqrt(ss / D + eps) with IEEE sqrt and
    divide; t = bf16((x * r) * w) (csrc/rope_kv.sycl:225-227). x_bits [..., D] bf16 bits."""
    x = bf16_to_f32(x_bits)
    D = x.shape[-1]
    lanes = x.reshape(x.shape[:-1] + (D // 64, 64))
    sq = (lanes * lanes).astype(np.float32)
    part = sq[..., 0, :]
    for j in range(1, D // 64):
        part = (part + sq[..., j, :]).astype(np.float32)
    off = 32
    while off >= 1:
        part = part.copy()
        part[..., :off] = (part[..., :off] + part[..., off:2 * off]).astype(np.float32)
        off //= 2
    ss = part[..., 0]
    r = (np.float32(1) / np.sqrt((ss / np.float32(D)).astype(np.float32) + np.float32(eps))).astype(np.float32)
    w = bf16_to_f32(w_bits)
    return f32_to_bf16(((x * r[..., None]).astype(np.float32) * w).astype(np.float32))


def rope_rows(t_bits, freqs, rd):
    """Partial split-half RoPE (csrc/rope_kv.sycl:5-11,44-52, tests/test_rope_kv.py:9-23).
    t_bits [S, H, D] bf16 bits; freqs f32 [S, rd/2, 2, 2]. For j < rd/2 with h = rd/2:
    o[j] = bf16(fl(t[j] * f00) + fl(t[j+h] * f01)), o[j+h] = bf16(fl(t[j+h] * f11) + fl(t[j] * f10))."""
    t = bf16_to_f32(t_bits)
    h = rd // 2
    f = np.asarray(freqs, dtype=np.float32)[:, None]  # [S, 1, h, 2, 2]
    lo, hi = t[..., :h], t[..., h:rd]
    o0 = (lo * f[..., 0, 0]).astype(np.float32) + (hi * f[..., 0, 1]).astype(np.float32)
    o1 = (hi * f[..., 1, 1]).astype(np.float32) + (lo * f[..., 1, 0]).astype(np.float32)
    out = np.array(t_bits, dtype=np.uint16, copy=True)
    out[..., :h] = f32_to_bf16(o0.astype(np.float32))
    out[..., h:rd] = f32_to_bf16(o1.astype(np.float32))
    return out


def rope_kv(q_bits, k_bits, v_bits, freqs, key_bits, value_bits, pos, rd, wq=None, wk=None, epsq=1e-6, epsk=1e-6):
    """rope_kv / qk_norm_rope_kv (csrc/rope_kv.sycl:58-114,120-245): returns q [Hq, S, D], k [Hk, S, D]
    and the updated caches key/value [Hk, cap, D] (rows pos[s] <- rotated k / v)."""
    if wq is not None:
        q_bits, k_bits = head_rmsnorm(q_bits, wq, epsq), head_rmsnorm(k_bits, wk, epsk)
    rq, rk = rope_rows(q_bits, freqs, rd), rope_rows(k_bits, freqs, rd)
    key, value = np.array(key_bits, copy=True), np.array(value_bits, copy=True)
    for s, p in enumerate(np.asarray(pos)):
        key[:, p] = rk[s]
        value[:, p] = v_bits[s]
    return rq.transpose(1, 0, 2).copy(), rk.transpose(1, 0, 2).copy(), key, value


# ---------------------------------------------------------------------------------------------
# MTP loop bookkeeping (csrc/mtp_loop.sycl, comfy_mono_decode_xpu/mtp_loop.py)
# ---------------------------------------------------------------------------------------------


def accept_walk(children, toks, dr, depth, cand=None):
    """The host accept walk (comfy_mono_decode_xpu/mtp_loop.py:117-136): from the root, step to the
    first child whose draft token equals the token the verify chose at the current node.
    children: list of child lists. Returns path, commit, ranks, row, on_chain, kept."""
    path = [0]
    while True:
        cur = path[-1]
        nxt = [c for c in children[cur] if dr[c] == toks[cur]]
        if not nxt:
            break
        path.append(nxt[0])
    ranks = []
    if cand is not None:
        for node in path:
            if node >= depth:
                break
            row7 = list(cand[7 * node:7 * node + 7])
            ranks.append(row7.index(toks[node]) if toks[node] in row7 else 7)
    commit = [dr[r] for r in path[1:]] + [toks[path[-1]]]
    row = path[-1]
    on_chain = row == len(path) - 1
    kept = min(len(path) if on_chain else len(path) - 1, depth)
    return path, commit, ranks, row, on_chain, kept


def accept_record(slots, path, commit, ranks, row, on_chain, kept, pos):
    """The int64 result record of mtp_accept (csrc/mtp_loop.sycl:143-161), slots generalised:
    [n, commit[slots] (-1 padded), row, on_chain, nranks, ranks[7], pos, kept]; at most 7 ranks are
    recorded (the first 7 chain nodes of a deeper 16-slot tree)."""
    ranks = ranks[:7]
    r = [len(path)] + commit + [-1] * (slots - len(commit)) + [row, int(on_chain), len(ranks)]
    r += ranks + [0] * (7 - len(ranks)) + [pos, kept]
    return r


def commit_path(cache, path, on_chain, pos):
    """FixedKVState.commit_path's slot moves (csrc/mtp_loop.sycl:177-192, tests/test_mtp_accept.py:95-102):
    for an off-chain path, slot (pos + k) % cap <- slot (pos + path[k]) % cap, k ascending, applied in
    sequence on cache [Hk, cap, D]."""
    out = np.array(cache, copy=True)
    cap = out.shape[1]
    if not on_chain:
        for k, src in enumerate(path[1:], 1):
            if src != k:
                out[:, (pos + k) % cap] = out[:, (pos + src) % cap]
    return out


def tree_from_spec(spec, rows):
    """VerifyTree parent / children / depth / chain of a nested child-list spec (qwen35 tree order:
    depth-first, first child is the chain; tests/test_mtp_accept.py:15-36)."""
    parent, children, depth = [], [], []

    def add(node, p):
        r = len(parent)
        parent.append(p)
        children.append([])
        depth.append(0 if p < 0 else depth[p] + 1)
        if p >= 0:
            children[p].append(r)
        for child in node:
            add(child, r)
    add(spec, -1)
    chain = 0
    while children[chain]:
        chain = children[chain][0]
    while len(parent) < rows:
        parent.append(-1)
        children.append([])
        depth.append(0)
    return parent, children, depth, chain


def spec_of_widths(widths):
    """qwen35.tree_spec: a chain with (width - 1) leaf siblings at each depth."""
    node = []
    for width in reversed(widths):
        node = [node] + [[] for _ in range(width - 1)]
    return node


# ---------------------------------------------------------------------------------------------
# exact top-k in torch's XPU order (csrc/fast_topk.sycl, csrc/topk_rows.sycl)
# ---------------------------------------------------------------------------------------------


def gather_pos(i, loads, width):
    """Position of element i in the gather order of torch XPU's topk sweep: per 32768-element iteration,
    1024 threads each issue `loads` vector loads of `width` elements; order (iteration, thread, load,
    lane) (csrc/fast_topk.sycl:4-9: loads 4 x width 8 for bf16; csrc/topk_rows.sycl:7-11: 8 x 4 for fp32)."""
    i = np.asarray(i, dtype=np.int64)
    it, off = i >> 15, i & 32767
    load, thread, lane = off // (1024 * width), (off % (1024 * width)) // width, off % width
    return (it << 15) + thread * (loads * width) + load * width + lane


def key_bf16(b):
    """bf16 radix key (csrc/fast_topk.sycl:22-26): NaN on top, -0 below +0, larger key first."""
    b = np.asarray(b, dtype=np.uint16).astype(np.int64)
    nan = (b & 0x7FFF) > 0x7F80
    return np.where(nan, 0xFFFF, np.where(b & 0x8000, b ^ 0xFFFF, b | 0x8000))


def key_f32(u):
    """fp32 radix key (csrc/topk_rows.sycl:33): sign-flipped bits, +NaN on top, -NaN at the bottom."""
    u = np.asarray(u, dtype=np.uint32).astype(np.int64)
    return np.where(u & 0x80000000, u ^ 0xFFFFFFFF, u | 0x80000000)


def key_argmax(b):
    """argmax rank key (csrc/fast_topk.sycl:31-40): NaN first, -0 == +0."""
    b = np.asarray(b, dtype=np.uint16).astype(np.int64)
    nan = (b & 0x7FFF) > 0x7F80
    b = np.where((b & 0x7FFF) == 0, 0, b)
    return np.where(nan, 0xFFFFFFFF, np.where(b & 0x8000, 0x7FFF - (b & 0x7FFF), 0x8000 + b))


def _topk_by(key, second, k):
    """Indices of the k best by (key desc, second asc)."""
    order = np.lexsort((second, -key))
    return order[:k]


def fast_topk(x_bits, k, argmax_order=False):
    """fast_topk (csrc/fast_topk.sycl:67-170): one bf16 row -> (values bits [k], indices [k])."""
    x_bits = np.asarray(x_bits, dtype=np.uint16).reshape(-1)
    i = np.arange(x_bits.size, dtype=np.int64)
    if argmax_order:
        idx = _topk_by(key_argmax(x_bits), i, k)
    else:
        idx = _topk_by(key_bf16(x_bits), gather_pos(i, 4, 8), k)
    return x_bits[idx], idx


def argmax_bf16(x_bits):
    return int(fast_topk(x_bits, 1, True)[1][0])


def topk_rows(x, k):
    """topk_rows (csrc/topk_rows.sycl:104-246): fp32 values [R, N] (or bf16 bits as uint16) ->
    (values f32 [R, k], indices [R, k]) in torch XPU fp32 order."""
    x = np.asarray(x)
    u = (x.astype(np.uint32) << 16) if x.dtype == np.uint16 else x.astype(np.float32).view(np.uint32)
    g = gather_pos(np.arange(u.shape[1], dtype=np.int64), 8, 4)
    idx = np.stack([_topk_by(key_f32(row), g, k) for row in u])
    return np.take_along_axis(u, idx, 1).view(np.float32), idx


# ---------------------------------------------------------------------------------------------
# tree-verify decode attention (csrc/attn_dpas.sycl; tests/test_attn_dpas.py:11-29)
# ---------------------------------------------------------------------------------------------


def tree_mask(parents):
    """Row s admits its ancestors and itself (tests/test_attn_dpas.py:11-15)."""
    m = []
    for r, p in enumerate(parents):
        m.append((m[p] if p >= 0 else 0) | (1 << r))
    return m


def attention_f64(q, k, v, L, xk, xv, mask, dtype=np.float64):
    """Softmax attention of each (head h, row s) over the cache prefix [0, L) and the tree rows its mask
    admits, in `dtype` (float64: the reference bound; float32: the fp32 chain whose error sets the
    tolerance). q [H, S, D], k/v [Hk, cap, D], xk/xv [Hk, S, D] as float arrays; mask list or None.
    Returns [S, H, D] in dtype (unrounded)."""
    H, S, D = q.shape
    Hk = k.shape[0]
    out = np.zeros((S, H, D), dtype=dtype)
    scale = dtype(1.0) / np.sqrt(dtype(D))
    for h in range(H):
        kh = h // (H // Hk)
        for s in range(S):
            rows = [t for t in range(S) if mask is not None and (mask[s] >> t) & 1]
            K = np.concatenate([k[kh, :L], xk[kh, rows]]).astype(dtype)
            V = np.concatenate([v[kh, :L], xv[kh, rows]]).astype(dtype)
            if K.shape[0] == 0:
                continue
            sc = (K @ q[h, s].astype(dtype)) * scale
            e = np.exp(sc - sc.max())
            out[s, h] = (e / e.sum()) @ V
    return out


# ---------------------------------------------------------------------------------------------
# bf16 linear (lm_head; comfy_mono_decode_xpu/mtp_loop.py:221-225)
# ---------------------------------------------------------------------------------------------


def bf16_linear_f64(x_bits, w_bits):
    """x . W^T in float64 of bf16 inputs (the tolerance reference), and sum |x| . |W|^T (the scale of
    the fp32 accumulation error)."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    w = bf16_to_f32(w_bits).astype(np.float64)
    return x @ w.T, np.abs(x) @ np.abs(w).T


# ---------------------------------------------------------------------------------------------
# Gated-DeltaNet decode step with deferred replay (csrc/mono_gdn.sycl:313-374,398-607)
# ---------------------------------------------------------------------------------------------
GDN_DH = 128
GDN_CW = 3


def _rnd(v, dtype, bf=True):
    """bf16 rounding in the float32 chain; identity in float64 (the exact reference)."""
    if dtype == np.float64 or not bf:
        return np.asarray(v, dtype=dtype)
    return bfround(np.asarray(v, dtype=np.float32))


def gdn_conv(state, proj, conv_w, ctl, R, slots, dtype=np.float64):
    """The deferred causal conv (kernel 4) over tree ancestors (csrc/mono_gdn.sycl:313-374).
    state: dict with conv_state [C, 3], pb [2, slots, C] (bf16 values as float). proj [R, C].
    ctl = [pending, parity, accepted[slots], parents[slots], prog[slots]].
    Updates conv_state (shifted by the previous step's accepted rows) and pb[parity]; returns the conv
    outputs qb [slots, C] (SiLU(bf16(sum)) rounded to bf16; rows >= R zero)."""
    pending, p = ctl[0], ctl[1]
    acc_slots = ctl[2:2 + slots]
    parents = ctl[2 + slots:2 + 2 * slots]
    C = proj.shape[1]
    old = state["conv_state"].astype(dtype)
    prev = state["pb"][1 - p].astype(dtype)
    hist = np.empty((C, GDN_CW), dtype=dtype)
    for r in range(GDN_CW):
        j = pending + r
        # an accepted slot outside [0, slots) is clamped into the range (the reference reads it
        # unchecked, mono_gdn.sycl:345-349; such a step replays nothing, see gdn_step)
        hist[:, r] = old[:, j] if j < GDN_CW else prev[min(max(int(acc_slots[j - GDN_CW]), 0), slots - 1)]
    w = conv_w.astype(dtype)
    out = np.zeros((slots, C), dtype=dtype)
    for ts in range(R):
        anc = [ts]
        miss = [0]
        for d in range(1, GDN_CW + 1):
            a = parents[anc[-1]] if anc[-1] >= 0 else -1
            a = -1 if a >= R else a  # a parent is an earlier row of this step
            anc.append(a)
            miss.append(miss[-1] + (a < 0))
        s = np.zeros(C, dtype=dtype)
        for d in range(GDN_CW + 1):
            v = proj[anc[d]].astype(dtype) if anc[d] >= 0 else hist[:, GDN_CW - miss[d]]
            s = s + v * w[:, GDN_CW - d] if dtype == np.float64 else (s + (v * w[:, GDN_CW - d]).astype(np.float32)).astype(np.float32)
        y = _rnd(s, dtype)
        out[ts] = _rnd(y / (1 + np.exp(-y)), dtype)
    state["conv_state"] = hist.astype(state["conv_state"].dtype)
    pbn = np.zeros((slots, C), dtype=state["pb"].dtype)
    pbn[:R] = proj
    state["pb"][p] = pbn
    return out


def gdn_ab(xn_bits, wa_bits, wb_bits, dtype=np.float64):
    """a = xn . wa^T, b = xn . wb^T (the in_proj_a / in_proj_b linears, csrc/mono_gdn.sycl:232-268):
    float64 unrounded (the reference bound), or the float32 dot rounded to bf16 (the chain)."""
    x = bf16_to_f32(xn_bits).astype(dtype)
    a = x @ bf16_to_f32(wa_bits).astype(dtype).T
    b = x @ bf16_to_f32(wb_bits).astype(dtype).T
    return _rnd(a, dtype), _rnd(b, dtype)


def gdn_gates(a, b, dt_bias, g_decay, dtype=np.float64):
    """decay = exp(g_decay * softplus(a + dt_bias)) (softplus(x) = x above 20), beta = bf16(sigmoid(b))
    (csrc/mono_gdn.sycl:441-450). a, b: [R, HV] bf16 values."""
    av = a.astype(dtype) + dt_bias.astype(dtype)
    sp = np.where(av > 20, av, np.log1p(np.exp(np.minimum(av, 20))))
    decay = np.exp(g_decay.astype(dtype) * sp)
    beta = _rnd(1 / (1 + np.exp(-b.astype(dtype))), dtype)
    return decay, beta


def gdn_delta(S, kn, v, decay, beta, dtype=np.float64):
    """One entry of the gated delta rule on a value head's state S [d_k rows, d_v columns] (stored
    as rec_state[(h * 128 + row) * 128 + col], csrc/mono_gdn.sycl:385,526-571): S <- S * decay,
    kv[c] = sum_r S[r, c] kn[r], delta = (v - kv) * beta, S[r, c] <- S[r, c] + kn[r] delta[c].
    Returns the updated state (the caller keeps it only for a committing entry)."""
    Sd = S * dtype(decay)
    kv = kn @ Sd
    delta = (v - kv) * dtype(beta)
    return Sd + np.outer(kn, delta)


def gdn_step(state, proj, z, a, b, conv_w, dt_bias, g_decay, gnorm_w, eps, qscale, ctl, R, HK, slots,
             dtype=np.float64):
    """One deferred GDN step. state: conv_state [C, 3], pb / qb [2, slots, C], rec [HV, 128, 128],
    gates [2, slots, HV, 2], sums [2, slots, HK, 2] (mutated). Returns core [R, HV * 128] (float;
    rows not produced by a verify entry are 0).
    Entries: first the previous step's accepted slots (parity 1 - p, always committed), then this
    step's verify program (prog & 15 = slot, prog & 32 = commit); the persistent state keeps only the
    replayed entries; verify entries update a working copy when they commit."""
    DH = GDN_DH
    pending, p = int(ctl[0]), int(ctl[1])
    HV = state["rec"].shape[0]
    KD = HK * DH
    qb = gdn_conv(state, proj, conv_w, ctl, R, slots, dtype)
    state["qb"][p] = qb.astype(state["qb"].dtype)
    decay, beta = gdn_gates(a, b, dt_bias, g_decay, dtype)
    gates = np.zeros((slots, HV, 2))
    gates[:R, :, 0] = decay
    gates[:R, :, 1] = beta
    state["gates"][p] = gates
    sums = np.zeros((slots, HK, 2))
    for ts in range(R):
        for kh in range(HK):
            for which in range(2):
                v = qb[ts, which * KD + kh * DH:which * KD + (kh + 1) * DH].astype(dtype)
                sums[ts, kh, which] = np.sum(v * v)
    state["sums"][p] = sums
    acc_slots = [int(s) for s in ctl[2:2 + slots]]
    prog = [int(s) for s in ctl[2 + 2 * slots:2 + 3 * slots]]
    E0 = 0
    while E0 < pending and 0 <= acc_slots[E0] < slots:
        E0 += 1
    replayed = E0 == pending
    E1 = 0
    if replayed:
        while E1 < R and prog[E1] >= 0 and (prog[E1] & 15) < R:
            E1 += 1
    core = np.zeros((R, HV * DH), dtype=np.float64)
    for h in range(HV):
        kh = h // (HV // HK)
        S = state["rec"][h].astype(dtype)
        raw = {}
        for e in range(E0 + E1):
            verify = e >= E0
            par = p if verify else 1 - p
            ts = (prog[e - E0] & 15) if verify else acc_slots[e]
            commit = (not verify) or bool(prog[e - E0] & 32)
            src = qb if verify else state["qb"][1 - p].astype(dtype)
            # the reference reads a replayed row's sums from the buffer its step stored them in
            # (csrc/mono_gdn.sycl:464-498); they are the sums of the same qb row, taken again here
            sq = sums[ts, kh] if verify else [np.sum(src[ts, w * KD + kh * DH:w * KD + (kh + 1) * DH].astype(dtype) ** 2)
                                              for w in (0, 1)]
            dec, bet = (state["gates"][par][ts, h] if not verify else gates[ts, h])
            q = src[ts, kh * DH:(kh + 1) * DH].astype(dtype)
            k = src[ts, KD + kh * DH:KD + (kh + 1) * DH].astype(dtype)
            v = src[ts, 2 * KD + h * DH:2 * KD + (h + 1) * DH].astype(dtype)
            kn = k / max(np.sqrt(sq[1]), 1e-12)
            qn = (q * qscale) / max(np.sqrt(sq[0]), 1e-12)
            Su = gdn_delta(S, kn, v, dec, bet, dtype)
            if verify:
                raw[ts] = _rnd(qn @ Su, dtype)
            if commit:
                S = Su
            # the persistent state keeps the replayed entries only, and only when every pending slot
            # was valid (csrc/mono_gdn.sycl:568)
            if e == E0 - 1 and replayed:
                state["rec"][h] = S.astype(state["rec"].dtype)
        for ts, rv in raw.items():
            ss = np.sum(rv.astype(dtype) ** 2)
            rsq = 1 / np.sqrt(ss / DH + eps)
            normed = _rnd(rv * gnorm_w.astype(dtype) * rsq, dtype)
            zz = z[ts, h * DH:(h + 1) * DH].astype(dtype)
            gz = _rnd(zz / (1 + np.exp(-zz)), dtype)
            core[ts, h * DH:(h + 1) * DH] = _rnd(normed * gz, dtype)
    return core


def verify_program(parents, R):
    """A verify program for a chain-with-leaf-siblings tree (qwen35 tree_spec shape): nodes in an order
    where each node sees the state after exactly its ancestors; chain nodes commit (bit 32), leaves do
    not. Returns prog [R]."""
    children = [[] for _ in range(R)]
    for r in range(R):
        if parents[r] >= 0:
            children[parents[r]].append(r)
    order, node = [], 0
    while True:
        order.append((node, True))
        kids = children[node]
        for leaf in kids[1:]:
            assert not children[leaf], "only the first child may have children"
            order.append((leaf, False))
        if not kids:
            break
        node = kids[0]
    order[-1] = (order[-1][0], False) if order[-1][1] else order[-1]
    assert len(order) == R
    return [n | (32 if c else 0) for n, c in order]


# ---------------------------------------------------------------------------------------------
# decoder-layer segments (csrc/mono_layer.sycl:69-318)
# ---------------------------------------------------------------------------------------------


def gate_mul(y_bits, gate_bits, sig_lut_bits):
    """y' = bf16(float(y) * float(sig[gate])) (csrc/mono_layer.sycl:243-252, bf16_mul)."""
    sig = bf16_to_f32(np.asarray(sig_lut_bits, dtype=np.uint16)[np.asarray(gate_bits, dtype=np.uint16)])
    return f32_to_bf16((bf16_to_f32(y_bits) * sig).astype(np.float32))


def interleaved_gate(q_out_bits, K=4096, head=256):
    """The gate half of q_proj's [head][query | gate] output rows (csrc/mono_layer.sycl:248)."""
    q = np.asarray(q_out_bits).reshape(q_out_bits.shape[0], K // head, 2 * head)
    return q[:, :, head:].reshape(q_out_bits.shape[0], K)


def add_bf16(res_bits, f_bits):
    """bf16(float(res) + float(f)) (the residual rule of every epilogue)."""
    return f32_to_bf16((bf16_to_f32(res_bits) + bf16_to_f32(f_bits)).astype(np.float32))


def layer_pre(x_bits, norm_w_bits, eps, rot, h, mats):
    """xn = RMSNorm(x); q = rot_quant(xn); outs = W4 linears (csrc/mono_layer.sycl:69-155).
    mats: dicts as for mono_mlp."""
    xn = rmsnorm(x_bits, norm_w_bits, eps)
    q, s = rot_quant(xn, rot, h)
    outs = [f32_to_bf16(scaleback(w4a8_acc(q, decode_w8(m["packed"], m["s"], m["cb"], m["G"])), s, m["sch"]))
            for m in mats]
    return xn, outs


def layer_post(x_bits, y_bits, gate_bits, sig_bits, o, norm_w_bits, eps, rot, h, lut_bits, g, u, d):
    """x1 = x + o_proj(rot_quant(gate_mul(y))); x = x1 + mlp(RMSNorm(x1)) (csrc/mono_layer.sycl:157-318)."""
    yy = y_bits if gate_bits is None else gate_mul(y_bits, gate_bits, sig_bits)
    q, s = rot_quant(yy, rot, h)
    x1 = f32_to_bf16(bf16_to_f32(x_bits) + bfround(scaleback(w4a8_acc(q, decode_w8(o["packed"], o["s"], o["cb"],
                                                                                      o["G"])), s, o["sch"])))
    mlp = mono_mlp(rmsnorm(x1, norm_w_bits, eps), rot, h, lut_bits, g, u, d)
    return add_bf16(x1, mlp), x1


# ---------------------------------------------------------------------------------------------
# fused draft-head ops (csrc/draft_fused.sycl:76-287; comfy_mono_decode_xpu/draft_head.py:179-211).
# The reference computes them in fp32 without a fixed order; the library's fixed order is restated
# (the rmsnorm above, the exact FWHT of rotate_rows), pinned to float64 within the reference's
# tolerance (tests/test_draft_fused.py:10-12: 1e-2 relative L2).
# ---------------------------------------------------------------------------------------------


def draft_embed_norm_cat(hidden_bits, we_bits, wh_bits, eps_e, eps_h, emb_bits=None, q=None, s=None, token=None,
                         unrotate=False):
    """[RMSNorm_e(e) | RMSNorm_h(hidden)] per row, e = emb_bits, or the int8 table row q[t] * s[t]
    (t = token clamped into [0, V)), un-rotated by H256 (exact sum, one rounding to fp32), then bf16
    (csrc/draft_fused.sycl:113-149)."""
    hidden_bits = np.asarray(hidden_bits, dtype=np.uint16).reshape(-1, np.asarray(we_bits).size)
    if q is not None:
        t = np.clip(np.asarray(token, dtype=np.int64).reshape(-1), 0, q.shape[0] - 1)
        row = (np.asarray(q, dtype=np.float32)[t] * np.asarray(s, dtype=np.float32)[t][:, None]).astype(np.float32)
        if unrotate:
            g = row.reshape(row.shape[0], -1, 256).astype(np.float64)
            row = (fwht256_f64(g) * 0.0625).astype(np.float32).reshape(row.shape)
        emb_bits = f32_to_bf16(row)
    emb_bits = np.asarray(emb_bits, dtype=np.uint16).reshape(hidden_bits.shape)
    return np.concatenate([rmsnorm(emb_bits, we_bits, eps_e), rmsnorm(hidden_bits, wh_bits, eps_h)], axis=1)


def draft_add_rmsnorm(x_bits, h_bits, w_bits, eps):
    """(x', out): x' = bf16(x + h) (x when h is None), out = RMSNorm(x') (csrc/draft_fused.sycl:164-182)."""
    x_bits = np.asarray(x_bits, dtype=np.uint16).reshape(-1, np.asarray(w_bits).size)
    xn = x_bits if h_bits is None else add_bf16(x_bits, np.asarray(h_bits, dtype=np.uint16).reshape(x_bits.shape))
    return xn, rmsnorm(xn, w_bits, eps)


def draft_sigmoid_mul(a_bits, qg_bits, head_dim, sig_lut_bits):
    """bf16(a * sig[gate]) with the gate the second half of each 2 head_dim block of the q projection row
    (csrc/draft_fused.sycl:196-201). a [rows, n], qg [rows, >= 2 n]."""
    a_bits = np.asarray(a_bits, dtype=np.uint16)
    rows, n = a_bits.shape
    qg = np.asarray(qg_bits, dtype=np.uint16)[:, :2 * n].reshape(rows, n // head_dim, 2, head_dim)
    return gate_mul(a_bits, qg[:, :, 1].reshape(rows, n), sig_lut_bits)


def draft_silu_mul(gu_bits, lut_bits):
    """bf16(silu[g] * u) over gate | up rows gu [rows, 2 I] (csrc/draft_fused.sycl:211-216)."""
    gu = np.asarray(gu_bits, dtype=np.uint16)
    I = gu.shape[1] // 2
    return silu_mul(bf16_to_f32(gu[:, :I]), bf16_to_f32(gu[:, I:]), lut_bits)


def draft_norm_rot_quant(x_bits, h_bits, w_bits, eps, rot="h256"):
    """(x', xr, q, scale): x' = bf16(x + h), xr = bf16(rotate(RMSNorm(x'))), scale = max(amax(xr) / 127,
    1e-30), q = clamp(rint(fl32(xr / bf16(scale))), -128, 127) (csrc/draft_fused.sycl:245-286)."""
    xn, n = draft_add_rmsnorm(x_bits, h_bits, w_bits, eps)
    xr = rotate_rows(bf16_to_f32(n), rot)
    amax = np.max(np.abs(xr), axis=1).astype(np.float32)
    scale = np.maximum((amax / np.float32(127)).astype(np.float32), np.float32(1e-30)).astype(np.float32)
    div = bfround(scale)
    q = np.clip(np.rint((xr / div[:, None]).astype(np.float32)), -128, 127).astype(np.int8)
    return xn, f32_to_bf16(xr), q, scale


# ---------------------------------------------------------------------------------------------
# two-stage draft lm_head, second stage (csrc/draft_lmhead.sycl:82-291)
# ---------------------------------------------------------------------------------------------


def int8_head_logits(qx, sx, w8, sw):
    """Exact int8 head logits bf16((float(acc) * sx) * sw[n]), acc the int32 dot of the int8 row with qx
    (csrc/draft_lmhead.sycl:217-220): int64 sums (exact), one rounding to fp32, two fp32 products."""
    acc = np.asarray(w8, dtype=np.int64) @ np.asarray(qx, dtype=np.int64).reshape(-1)
    f = (acc.astype(np.float32) * np.float32(np.asarray(sx, dtype=np.float32).reshape(-1)[0])).astype(np.float32)
    f = (f * np.asarray(sw, dtype=np.float32).reshape(-1)).astype(np.float32)
    return f32_to_bf16(f)


def draft_pick(logit_bits, nout, argmax_first, children, nvtok):
    """The draft's outputs from the exact logits (csrc/draft_lmhead.sycl:263-284): top-nout in torch topk
    order, the token (argmax, or top[0]), vtok[children[0]] = token, vtok[children[j]] = top[j]; vtok is
    returned with -1 elsewhere."""
    _, top = fast_topk(logit_bits, nout)
    tok = argmax_bf16(logit_bits) if argmax_first else int(top[0])
    vtok = np.full(nvtok, -1, dtype=np.int64)
    vtok[children[0]] = tok
    for j, c in enumerate(children[1:], 1):
        vtok[c] = top[j]
    return top, tok, vtok


# ---------------------------------------------------------------------------------------------
# exact attention (the exactness fallback beside attn_dpas; the reference's bit-identical port of its
# upstream attention, csrc/attn_port.sycl:1-12, has the same role): one canonical fp32 order
# ---------------------------------------------------------------------------------------------
_EXP_C = [np.float32(float.fromhex(h)) for h in ("0x1.a01a02p-13", "0x1.6c16c2p-10", "0x1.111112p-7",
                                                 "0x1.555556p-5", "0x1.555556p-3", "0x1.0p-1", "0x1.0p0", "0x1.0p0")]
_LOG2E = np.float32(float.fromhex("0x1.715476p+0"))
_LN2_HI = np.float32(float.fromhex("0x1.62e4p-1"))
_LN2_LO = np.float32(float.fromhex("0x1.7f7d1cp-20"))


def exp_c(x):
    """e^x (x <= 0) as the exact attention computes it: n = rint(fl(x log2e)), r = fl(fl(x - fl(n ln2_hi)) -
    fl(n ln2_lo)), Horner over the fp32 Taylor coefficients 1/7! .. 1/0!, times 2^n; 0 below -80 or for NaN."""
    f32 = np.float32
    x = np.asarray(x, dtype=f32)
    n = np.rint((x * _LOG2E).astype(f32)).astype(f32)
    r = ((x - (n * _LN2_HI).astype(f32)).astype(f32) - (n * _LN2_LO).astype(f32)).astype(f32)
    p = np.full_like(r, _EXP_C[0])
    for c in _EXP_C[1:]:
        p = ((p * r).astype(f32) + c).astype(f32)
    with np.errstate(invalid="ignore"):
        out = np.ldexp(p, np.where(x > -80, n, 0).astype(np.int32)).astype(f32)
    return np.where(x > -80, out, f32(0)).astype(f32)


def attention_exact(q_bits, key_bits, value_bits, L, xk_bits, xv_bits, mask, scale):
    """The exact attention's result bits [S, H * D] for q [H, S, D], caches [Hk, cap, D], tree rows xk / xv
    [Hk, S, D] (bf16 bits), L cached tokens, mask (list or None), scale (fp32). Tokens: the prefix [0, L),
    then the admitted tree rows ascending. score = fl(dot * scale), the dot in dimension order; weights
    e = exp_c(score - max); l = 64 lane partials (lane j: tokens j, j + 64, .. in order) reduced by a halving
    tree; o[d] in token order; out = bf16(o / l), 0 for no tokens."""
    f32 = np.float32
    qf, kf, vf = bf16_to_f32(q_bits), bf16_to_f32(key_bits), bf16_to_f32(value_bits)
    xkf, xvf = bf16_to_f32(xk_bits), bf16_to_f32(xv_bits)
    H, S, D = qf.shape
    Hk = kf.shape[0]
    scale = f32(scale)
    out = np.zeros((S, H, D), dtype=np.uint16)
    for h in range(H):
        kh = h // (H // Hk)
        for s in range(S):
            rows = [t for t in range(S) if mask is not None and (int(mask[s]) >> t) & 1]
            K = np.concatenate([kf[kh, :L], xkf[kh, rows]]).astype(f32)
            V = np.concatenate([vf[kh, :L], xvf[kh, rows]]).astype(f32)
            n = K.shape[0]
            if n == 0:
                continue
            acc = np.zeros(n, dtype=f32)
            for d in range(D):
                acc = (acc + (qf[h, s, d] * K[:, d]).astype(f32)).astype(f32)
            sc = (acc * scale).astype(f32)
            e = exp_c((sc - sc.max()).astype(f32))
            ep = np.zeros(-(-n // 64) * 64, dtype=f32)
            ep[:n] = e
            parts = np.zeros(64, dtype=f32)
            for i in range(ep.size // 64):
                parts = (parts + ep[64 * i:64 * i + 64]).astype(f32)
            for o in (32, 16, 8, 4, 2, 1):
                parts[:o] = (parts[:o] + parts[o:2 * o]).astype(f32)
            o = np.zeros(D, dtype=f32)
            for u in range(n):
                o = (o + (e[u] * V[u]).astype(f32)).astype(f32)
            out[s, h] = f32_to_bf16((o / parts[0]).astype(f32))
    return out.reshape(S, H * D)


# ---------------------------------------------------------------------------------------------
# Sampling uniforms drawn on the device (mdx_topk_sample_seeded; no counterpart in the reference,
# which draws them with torch's generator)
# ---------------------------------------------------------------------------------------------

_M64 = (1 << 64) - 1
SPLITMIX_GAMMA = 0x9E3779B97F4A7C15


def splitmix64_mix(z):
    """SplitMix64's output function (Steele, Lea and Flood 2014) of a 64-bit state z."""
    z &= _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def seeded_uniform(seed, counter, r, j):
    """(k + 0.5) * 2^-23 as float32, k the top 23 bits of splitmix64_mix(seed + (n + 1) * gamma),
    n = counter * 1024 + 64 r + j."""
    n = (int(counter) * 1024 + 64 * int(r) + int(j)) & _M64
    z = splitmix64_mix((int(seed) + (n + 1) * SPLITMIX_GAMMA) & _M64)
    return np.float32((float(z >> 41) + 0.5) * 2.0 ** -23)

