"""Host hooks: route a host program's decode calls to libmdx and fall back to the host's own code on
anything the contract does not cover (the reference's ComfyUI hook layer, comfy_mono_decode_xpu/
__init__.py:1-80 for the switches, patch.py:31-110 for the W4A8 linear, mono.py:147-194 for the MLP
block, layer.py:496-617 for the decoder block).

Three pieces, each installed on its own (one that fails to install is logged and the others load):

- "w4":    wraps the host's W4A8 linear entry (omni_xpu_kernel's `w4a8_linear_prequantized` signature:
           x_int8, x_scale, packed, relative_scale, channel_scale, codebook, bias, group_size, out_dtype);
           a call inside the kernel contract runs `mdx_w4a8_decode_linear`, bit-identical to the
           contract's mm -> scaleback -> cast; any other call runs the original.
- "mono":  wraps `MLP.forward(x, norm)` for 1..16 decode rows whose three projections are packed W4A8
           (comfy-kitchen's layout with a ConvRot group of 256): the host's norm, then one libmdx MLP block.
- "layer": wraps the hybrid decoder block's `forward(x, attention_mask, freqs_cis, optimized_attention,
           past_key_value)` for 1..16 decode rows: layer_pre -> Q/K norm + RoPE + KV write -> tree
           attention -> layer_post for attention blocks, layer_gdn for Gated-DeltaNet blocks.

Failures follow the breaker rule of mdx/guard.py (the reference's contract, comfy_mono_decode_xpu/guard.py:
30-43): an error before any state was modified switches the piece off and runs the original; an error
after a write (KV rows, the recurrent state, x in place) switches it off and re-raises, since replaying the
block would apply it twice. A sub-path that has already switched itself off raises SubpathError, which
leaves the piece on. stats() counts the calls each piece took and, per reason, those it left to the host.

Switches (environment): MDX_DECODE=0 turns every piece off; MDX_DECODE_<PIECE>=1/0 (W4, MONO, LAYER)
overrides it per piece.

The decoder block protocol (the host's modules, duck-typed as the reference reads them):
  block.layer_type ("linear_attention" for GDN), block.input_layernorm / post_attention_layernorm (weight or
  scale(), eps), block.mlp.{gate,up,down}_proj.weight (packed W4A8 tensors: `_qdata` + `_params`);
  attention: block.self_attn.{q,k,v,o}_proj, q_norm / k_norm, num_heads, num_kv_heads, head_dim,
  rotary_dim (q_proj gated: [query | gate] per head); past_key_value: key / value [1, Hk, cap, D],
  position int64 [S], seqlen int32 [1], mask int32 [S] (tree rows; empty for one row);
  GDN: block.linear_attn.{in_proj_qkv, in_proj_z, out_proj} (W4A8), in_proj_a / in_proj_b (bf16),
  conv1d.weight [C, 1, 4], norm.eps, key_head_dim, num_key_heads; past_key_value: decode_step(S),
  conv_state, proj_buf, qkv_buf, ctl, dt_bias, g_decay, recurrent_state, gates_buf, sumsq_buf, norm_weight
  (comfy_mono_decode_xpu/layer.py:576-580).
"""
from __future__ import annotations

import logging
import os
import threading
from typing import NamedTuple

import torch

from . import guard

CLAIM = "__mdx_hook__"
DEVICE_TYPE = "cuda"  # the device type whose tensors libmdx takes (ROCm devices are "cuda" in torch)
PIECES = ("W4", "MONO", "LAYER")
_lock = threading.Lock()
_stats = {p: {"fast": 0, "fallback": {}} for p in ("w4", "mono", "layer")}
_consts = {}
UNCOUNTED = ""  # a route's miss that stats() does not count (inputs that are plainly not a decode call)


class SubpathError(guard.PassThrough):
    """A sub-path failed after writing state and has switched itself off; the block is not replayed."""


def stats():
    with _lock:
        return {p: {"fast": d["fast"], "fallback": dict(d["fallback"])} for p, d in _stats.items()}


def reset_stats():
    with _lock:
        for d in _stats.values():
            d["fast"] = 0
            d["fallback"].clear()


def _count(piece, why=None):
    """One call of `piece` taken by the fast path (why None) or left to the host for `why`."""
    with _lock:
        d = _stats[piece]
        if why is None:
            d["fast"] += 1
        elif why != UNCOUNTED:
            d["fallback"][why] = d["fallback"].get(why, 0) + 1


def _lib_C():
    """libmdx's operator surface (raises when the library is missing: no CPU path)."""
    from . import _C, _lib
    _lib.lib()
    return _C


def _constants(device):
    c = _consts.get(device)
    if c is None:
        from . import layout
        h = layout.regular_hadamard(device)
        c = _consts[device] = (h, layout.silu_lut(device), layout.sigmoid_lut(device))
    return c


def _compiling():
    comp = getattr(torch, "compiler", None)
    return bool(comp is not None and getattr(comp, "is_compiling", lambda: False)())


def _dispatch(piece, why, fast, host):
    """host() when the piece is switched off or the route missed (`why`: the reason, or UNCOUNTED), else
    fast(progress) under the piece's breaker, counted when it answers."""
    if why is not None:
        _count(piece, why)
        return host()

    def counted(progress):
        out = fast(progress)
        _count(piece)
        return out

    return guard.shielded(piece, counted, host)


def _claim(wrapper, original):
    setattr(wrapper, CLAIM, True)
    wrapper.__wrapped__ = original
    return wrapper


# ---------------------------------------------------------------------------------------------------
# the W4A8 linear entry
# ---------------------------------------------------------------------------------------------------
class LinearCall(NamedTuple):
    """The arguments of the host's W4A8 linear entry, by name."""
    x: torch.Tensor
    x_scale: torch.Tensor
    packed: torch.Tensor
    s_rel: torch.Tensor
    s_channel: torch.Tensor
    codebook: torch.Tensor | None
    bias: torch.Tensor | None
    group_size: int
    out_dtype: torch.dtype

    @property
    def k(self):
        return self.x.shape[-1]

    @property
    def rows(self):
        return self.x.numel() // self.k if self.k else 0


_OUT_CODE = {torch.float32: 0, torch.bfloat16: 2}  # libmdx's output dtype codes


def _pow2(v):
    return v > 0 and v & (v - 1) == 0


# The linear contract as (reason, test that the call breaks it), checked in this order: the output the
# host asked for, the activation, the geometry, the weight tensors, then where the operands live
# (the reference's checks, comfy_mono_decode_xpu/patch.py:32-55, with this library's limits: 1..16 rows,
# K % 128, power-of-two groups of at least 16, fp32 / fp16 / fp8 group scales).
_LINEAR_RULES = (
    ("bias", lambda c: c.bias is not None),
    ("out_dtype", lambda c: c.out_dtype not in _OUT_CODE),
    ("x", lambda c: c.x.device.type != DEVICE_TYPE or c.x.dtype != torch.int8 or not c.x.is_contiguous()),
    ("rows", lambda c: not 1 <= c.rows <= 16),
    ("shape", lambda c: c.k % 128 or c.k > 65536 or c.group_size < 16 or not _pow2(c.group_size)
     or c.k % c.group_size),
    ("packed", lambda c: c.packed.dtype not in (torch.int8, torch.uint8) or c.packed.dim() != 2
     or not c.packed.is_contiguous() or c.packed.shape[1] * 2 != c.k or c.packed.shape[0] % 16),
    ("align", lambda c: c.packed.data_ptr() % 16 or c.x.data_ptr() % 16),
    ("s_rel", lambda c: c.s_rel.dtype not in (torch.float32, torch.float16, torch.float8_e4m3fn)
     or not c.s_rel.is_contiguous() or c.s_rel.numel() != c.packed.shape[0] * (c.k // c.group_size)),
    ("s_channel", lambda c: c.s_channel.numel() != c.packed.shape[0]),
    ("codebook", lambda c: c.codebook is not None and (c.codebook.dtype != torch.float32 or c.codebook.numel() != 16)),
    ("operands", lambda c: c.x_scale.numel() != c.rows
     or any(t is not None and t.device != c.x.device for t in (c.x_scale, c.packed, c.s_rel, c.s_channel, c.codebook))),
)


def linear_contract(*args):
    """None when libmdx's W4A8 linear takes the call (the host's positional arguments), else the first
    reason it does not."""
    call = LinearCall(*args)
    for why, breaks in _LINEAR_RULES:
        if breaks(call):
            return why
    return None


def _linear_fast(call):
    """The call through mdx_w4a8_decode_linear: rows flattened, the scales as contiguous f32 vectors."""
    C = _lib_C()
    out = C.w4a8_decode_linear(call.x.reshape(call.rows, call.k), call.x_scale.reshape(-1).float().contiguous(),
                               call.packed, call.s_rel, call.s_channel.reshape(-1).float().contiguous(),
                               call.codebook, None, call.group_size, _OUT_CODE[call.out_dtype])
    return out.view(*call.x.shape[:-1], call.packed.shape[0])


def wrap_linear(original):
    def w4a8_linear_prequantized(x_int8, x_scale, packed, relative_scale, channel_scale, codebook=None, bias=None,
                                 group_size=16, out_dtype=torch.bfloat16):
        call = LinearCall(x_int8, x_scale, packed, relative_scale, channel_scale, codebook, bias, group_size,
                          out_dtype)
        host = lambda: original(*call)  # noqa: E731
        if not guard.BOARD.allows("w4") or _compiling():
            return host()
        # a pure function of its inputs: on a failure the host's entry recomputes the call
        return _dispatch("w4", linear_contract(*call), lambda progress: _linear_fast(call), host)

    return _claim(w4a8_linear_prequantized, original)


def install_w4(module, name="w4a8_linear_prequantized"):
    original = getattr(module, name)
    if getattr(original, CLAIM, False):
        return False
    setattr(module, name, wrap_linear(original))
    return True


# ---------------------------------------------------------------------------------------------------
# packed weights of the host's modules
# ---------------------------------------------------------------------------------------------------
def _w4_of(lin):
    """(q, s, s_channel, codebook) of a packed W4A8 linear module, or None (checkpoint.w4_from_quantized's
    checks: the reference's _layout_ok / _static_ok)."""
    from . import checkpoint
    w = getattr(lin, "weight", None)
    if getattr(lin, "weight_function", None) or getattr(lin, "bias_function", None):
        return None
    try:
        W = checkpoint.w4_from_quantized(w, getattr(lin, "bias", None), tiled=False)
    except checkpoint.Ineligible:
        return None
    return [W.q, W.s, W.sc, W.cb]


def _cached(owner, attr, key, make):
    hit = getattr(owner, attr, None)
    if hit is not None and hit[0] == key:
        return hit[1]
    v = make()
    setattr(owner, attr, (key, v))
    return v


def _norm_weight(norm):
    w = norm.scale() if callable(getattr(norm, "scale", None)) else norm.weight
    return w.to(torch.bfloat16).contiguous()


# ---------------------------------------------------------------------------------------------------
# the MLP block
# ---------------------------------------------------------------------------------------------------
def _mlp_route(mod, x, norm):
    """(None, packed parts) when the MLP block takes the call, else (reason, None)."""
    if (norm is None or x.device.type != DEVICE_TYPE or x.dtype != torch.bfloat16 or x.shape[-1] != 4096
            or not 1 <= x.numel() // x.shape[-1] <= 16):
        return UNCOUNTED, None
    lins = (mod.gate_proj, mod.up_proj, mod.down_proj)
    parts = _cached(mod, "_mdx_mlp", tuple(id(getattr(l, "weight", None)) for l in lins),
                    lambda: [_w4_of(l) for l in lins])
    if any(p is None for p in parts):
        return "weights", None
    cb = parts[0][3]
    if not all(torch.equal(cb, p[3]) for p in parts[1:]):
        return "codebook", None  # the block decodes its three projections with one table
    return None, parts


def wrap_mlp(original):
    def forward(self, x, norm=None):
        host = lambda: original(self, x, norm=norm)  # noqa: E731
        if not guard.BOARD.allows("mono"):
            return host()
        why, parts = _mlp_route(self, x, norm)

        def fast(progress):  # writes nothing: the host's forward recomputes from x on a failure
            C = _lib_C()
            h, lut, _ = _constants(x.device)
            rows = norm(x).reshape(-1, x.shape[-1]).contiguous()
            out = C.mono_mlp(rows, h, lut, *parts[0], *parts[1], *parts[2], 0, 4, False)
            return out.reshape(*x.shape[:-1], out.shape[-1])

        return _dispatch("mono", why, fast, host)

    return _claim(forward, original)


def install_mono(MLP):
    if getattr(MLP.forward, CLAIM, False):
        return False
    MLP.forward = wrap_mlp(MLP.forward)
    return True


# ---------------------------------------------------------------------------------------------------
# the decoder block
# ---------------------------------------------------------------------------------------------------
def static_plan(block):
    """The block's packed weights and extras, or None when any linear is outside the contract (the block
    then always runs the host's forward; comfy_mono_decode_xpu/layer.py:119-160)."""
    gdn = getattr(block, "layer_type", None) == "linear_attention"
    mix = block.linear_attn if gdn else block.self_attn
    pre = [mix.in_proj_qkv, mix.in_proj_z] if gdn else [mix.q_proj, mix.k_proj, mix.v_proj]
    out = mix.out_proj if gdn else mix.o_proj
    mlp = block.mlp
    lins = pre + [out, mlp.gate_proj, mlp.up_proj, mlp.down_proj]
    parts = [_w4_of(l) for l in lins]
    if any(p is None for p in parts):
        return None
    if not all(torch.equal(parts[-3][3], p[3]) for p in parts[-2:]):
        return None
    plan = dict(gdn=gdn, pre=[t for p in parts[:len(pre)] for t in p], out=parts[len(pre)],
                mlp=[t for p in parts[-3:] for t in p],
                norm_in=(_norm_weight(block.input_layernorm), block.input_layernorm.eps),
                norm_post=(_norm_weight(block.post_attention_layernorm), block.post_attention_layernorm.eps))
    if gdn:
        conv = mix.conv1d
        if getattr(conv, "bias", None) is not None:
            return None
        plan["extra"] = dict(wa=mix.in_proj_a.weight.to(torch.bfloat16).contiguous(),
                             wb=mix.in_proj_b.weight.to(torch.bfloat16).contiguous(),
                             conv_w=conv.weight.reshape(conv.weight.shape[0], -1).to(torch.bfloat16).contiguous())
    else:
        H, Hk, D = mix.num_heads, mix.num_kv_heads, mix.head_dim
        if D not in (64, 128, 256) or H % Hk or parts[0][0].shape[0] not in (H * D, 2 * H * D):
            return None
        plan["gated"] = parts[0][0].shape[0] == 2 * H * D
    return plan


def attn_core(mix, q, k, v, freqs, kv):
    """Q/K RMSNorm + RoPE + the KV write at kv.position, then tree attention over the cache prefix and
    the block's own rows: y bf16 [S, heads * head_dim]. q [S, heads * head_dim (* 2 when gated)]."""
    C = _lib_C()
    S = q.shape[0]
    H, Hk, D = mix.num_heads, mix.num_kv_heads, mix.head_dim
    gated = q.shape[-1] == 2 * H * D
    rawq = q.view(1, S, H, 2 * D)[..., :D] if gated else q.view(1, S, H, D)
    rawk, vv = k.view(1, S, Hk, D), v.view(1, S, Hk, D)
    qo, ko = C.qk_norm_rope_kv(rawq, rawk, vv, _norm_weight(mix.q_norm), _norm_weight(mix.k_norm), freqs, kv.key,
                               kv.value, kv.position, mix.q_norm.eps, mix.k_norm.eps, mix.rotary_dim)
    return C.attn_dpas(qo, kv.key, kv.value, kv.seqlen, ko, vv.transpose(1, 2), kv.mask, 0).view(S, H * D)


def _run_gdn(block, plan, x2, kv, progress):
    C = _lib_C()
    h, silu, _ = _constants(x2.device)
    mix, ex = block.linear_attn, plan["extra"]
    (nin, ein), (npo, epo) = plan["norm_in"], plan["norm_post"]
    progress.wrote()  # the one launch writes x, the conv history and the recurrent state
    C.layer_gdn(x2, nin, ein, h, plan["pre"] + plan["out"] + plan["mlp"], ex["wa"], ex["wb"], ex["conv_w"],
                kv.conv_state, kv.proj_buf, kv.qkv_buf, kv.ctl, kv.dt_bias, kv.g_decay, kv.recurrent_state,
                kv.gates_buf, kv.sumsq_buf, kv.norm_weight, mix.norm.eps, mix.key_head_dim ** -0.5, mix.num_key_heads,
                npo, epo, silu, 0, 11, False)


def _run_attention(block, plan, x2, S, freqs_cis, kv, progress):
    C = _lib_C()
    h, silu, sig = _constants(x2.device)
    mix = block.self_attn
    (nin, ein), (npo, epo) = plan["norm_in"], plan["norm_post"]
    outs = C.layer_pre(x2, nin, ein, h, plan["pre"], 0, False)  # pure: nothing written yet
    progress.wrote()  # from here on KV rows, then x in place
    y = attn_core(mix, outs[1], outs[2], outs[3], freqs_cis, kv)
    gate = None
    if plan["gated"]:  # the gate half of each head's [query | gate] block, as a plain [S, heads * head_dim] gate
        gate = outs[1].view(S, mix.num_heads, 2, mix.head_dim)[:, :, 1].reshape(S, -1).contiguous()
    C.layer_post(x2, y.contiguous(), gate, sig, *plan["out"], npo, epo, h, silu, *plan["mlp"], 0, 6, False)


def _block_route(block, x, attention_mask, kv, max_rows):
    """(None, plan, rows) when the decoder block takes the call, else (reason, None, 0)."""
    miss = (UNCOUNTED, None, 0)
    if kv is None or x.device.type != DEVICE_TYPE or x.dtype != torch.bfloat16 or x.dim() != 3:
        return miss
    B, S = x.shape[0], x.shape[1]
    if B != 1 or not 1 <= S <= max_rows or x.shape[-1] != 4096 or not x.is_contiguous():
        return miss
    if getattr(block, "layer_type", None) == "linear_attention":
        if not kv.decode_step(S):  # the cache's own judgement: a prefill chunk is not a decode step
            return miss
    else:
        mix = block.self_attn
        if attention_mask is not None or (mix.num_heads // mix.num_kv_heads) * S > 64:
            return miss
    key = tuple(id(getattr(m, "weight", None)) for m in _block_linears(block))
    plan = _cached(block, "_mdx_plan", key, lambda: static_plan(block))
    if plan is None:
        return "weights", None, 0
    return None, plan, S


def wrap_block(original, max_rows=16):
    def forward(self, x, attention_mask=None, freqs_cis=None, optimized_attention=None, past_key_value=None):
        host = lambda: original(self, x, attention_mask, freqs_cis, optimized_attention, past_key_value)  # noqa: E731
        if not guard.BOARD.allows("layer"):
            return host()
        why, plan, S = _block_route(self, x, attention_mask, past_key_value, max_rows)

        def fast(progress):
            x2 = x.view(S, 4096)
            if plan["gdn"]:
                _run_gdn(self, plan, x2, past_key_value, progress)
            else:
                _run_attention(self, plan, x2, S, freqs_cis, past_key_value, progress)
            return x, past_key_value

        # a failure after a write re-raises (replaying the block would apply it twice); SubpathError
        # passes through: that sub-path is off already
        return _dispatch("layer", why, fast, host)

    return _claim(forward, original)


def _block_linears(block):
    gdn = getattr(block, "layer_type", None) == "linear_attention"
    mix = block.linear_attn if gdn else block.self_attn
    names = ("in_proj_qkv", "in_proj_z", "out_proj") if gdn else ("q_proj", "k_proj", "v_proj", "o_proj")
    return [getattr(mix, n) for n in names] + [block.mlp.gate_proj, block.mlp.up_proj, block.mlp.down_proj]


def install_layer(Block):
    if getattr(Block.forward, CLAIM, False):
        return False
    Block.forward = wrap_block(Block.forward)
    return True


# ---------------------------------------------------------------------------------------------------
# switches and installation
# ---------------------------------------------------------------------------------------------------
def enabled(piece, env=None):
    env = os.environ if env is None else env
    v = env.get(f"MDX_DECODE_{piece}")
    if v is not None:
        return v == "1"
    return env.get("MDX_DECODE", "1") == "1"


def install(w4_module=None, mlp_class=None, block_class=None, env=None):
    """Install every enabled piece whose host target is given. Returns {piece: installed (bool) or the
    error text}; a piece that fails to install is logged and leaves the others alone. Without libmdx
    nothing is installed (the host keeps its own paths)."""
    try:
        _lib_C()
    except Exception as e:
        logging.warning("[mdx] libmdx not loadable (%s): the host keeps its own decode paths", e)
        return {}
    out = {}
    for piece, target, fn in (("W4", w4_module, install_w4), ("MONO", mlp_class, install_mono),
                              ("LAYER", block_class, install_layer)):
        if target is None or not enabled(piece, env):
            continue
        try:
            out[piece] = fn(target)
            logging.info("[mdx] %s installed=%s", piece, out[piece])
        except Exception as e:  # never take the host down: that piece keeps the host's path
            logging.exception("[mdx] %s failed to install; it stays on the host's path", piece)
            out[piece] = f"{type(e).__name__}: {e}"
    return out


def install_comfy(w4_module=None, env=None):
    """Install into a ComfyUI process: its Qwen3.5 decoder block and MLP classes, and the W4A8 linear entry
    of `w4_module` when the host's quantisation backend exposes one (`w4a8_linear_prequantized`). Returns
    what install() returns, or {} when ComfyUI is not importable."""
    try:
        from comfy.text_encoders import llama, qwen35
    except Exception:
        return {}
    return install(w4_module, getattr(llama, "MLP", None), getattr(qwen35, "Qwen35TransformerBlock", None), env)
