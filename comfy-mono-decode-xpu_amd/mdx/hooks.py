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

Failures follow the reference's rule (guard.py): an error before any state was modified switches the
piece off and runs the original; an error after a write (KV rows, the recurrent state, x in place) switches
it off and re-raises, since replaying the block would apply it twice. A sub-path that has already
switched itself off raises SubpathError, which leaves the piece on. stats() counts the calls each piece
took and, per reason, those it left to the host.

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

import torch

from . import guard

CLAIM = "__mdx_hook__"
DEVICE_TYPE = "cuda"  # the device type whose tensors libmdx takes (ROCm devices are "cuda" in torch)
PIECES = ("W4", "MONO", "LAYER")
_lock = threading.Lock()
_stats = {p: {"fast": 0, "fallback": {}} for p in ("w4", "mono", "layer")}
_consts = {}


class SubpathError(RuntimeError):
    """A sub-path failed after writing state and has switched itself off; the block is not replayed."""


def stats():
    with _lock:
        return {p: {"fast": d["fast"], "fallback": dict(d["fallback"])} for p, d in _stats.items()}


def reset_stats():
    with _lock:
        for d in _stats.values():
            d["fast"] = 0
            d["fallback"].clear()


def _fast(piece):
    with _lock:
        _stats[piece]["fast"] += 1


def _fallback(piece, why):
    with _lock:
        f = _stats[piece]["fallback"]
        f[why] = f.get(why, 0) + 1


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


# ---------------------------------------------------------------------------------------------------
# the W4A8 linear entry
# ---------------------------------------------------------------------------------------------------
def linear_contract(x, x_scale, packed, s_rel, s_channel, codebook, bias, group_size, out_dtype):
    """None when libmdx's W4A8 linear takes the call, else the reason (the reference's checks,
    comfy_mono_decode_xpu/patch.py:32-55, with this library's limits: 1..16 rows, K % 128, power-of-two
    groups of at least 16, fp32 / fp16 / fp8 group scales)."""
    if bias is not None:
        return "bias"
    if out_dtype not in (torch.bfloat16, torch.float32):
        return "out_dtype"
    if x.device.type != DEVICE_TYPE or x.dtype != torch.int8 or not x.is_contiguous():
        return "x"
    k = x.shape[-1]
    rows = x.numel() // k if k else 0
    if not 1 <= rows <= 16:
        return "rows"
    if k % 128 or k > 65536 or group_size < 16 or group_size & (group_size - 1) or k % group_size:
        return "shape"
    if (packed.dtype not in (torch.int8, torch.uint8) or packed.dim() != 2 or not packed.is_contiguous()
            or packed.shape[1] * 2 != k or packed.shape[0] % 16):
        return "packed"
    if packed.data_ptr() % 16 or x.data_ptr() % 16:
        return "align"
    if (s_rel.dtype not in (torch.float32, torch.float16, torch.float8_e4m3fn) or not s_rel.is_contiguous()
            or s_rel.numel() != packed.shape[0] * (k // group_size)):
        return "s_rel"
    if s_channel.numel() != packed.shape[0]:
        return "s_channel"
    if codebook is not None and (codebook.dtype != torch.float32 or codebook.numel() != 16):
        return "codebook"
    if (x_scale.numel() != rows or any(t.device != x.device for t in (x_scale, packed, s_rel, s_channel))
            or (codebook is not None and codebook.device != x.device)):
        return "operands"
    return None


def wrap_linear(original):
    def w4a8_linear_prequantized(x_int8, x_scale, packed, relative_scale, channel_scale, codebook=None, bias=None,
                                 group_size=16, out_dtype=torch.bfloat16):
        args = (x_int8, x_scale, packed, relative_scale, channel_scale, codebook, bias, group_size, out_dtype)
        if guard.off("w4") or _compiling():
            return original(*args)
        why = linear_contract(*args)
        if why is not None:
            _fallback("w4", why)
            return original(*args)
        k = x_int8.shape[-1]
        try:
            C = _lib_C()
            x2 = x_int8.reshape(-1, k)
            xs = x_scale.reshape(-1).to(torch.float32).contiguous()
            sc = channel_scale.reshape(-1).to(torch.float32).contiguous()
            out = C.w4a8_decode_linear(x2, xs, packed, relative_scale, sc, codebook, None, group_size,
                                       0 if out_dtype == torch.float32 else 2)
        except Exception as e:  # a pure function of its inputs: the original recomputes it
            guard.failed("w4", e)
            return original(*args)
        _fast("w4")
        return out.reshape(*x_int8.shape[:-1], packed.shape[0])

    setattr(w4a8_linear_prequantized, CLAIM, True)
    w4a8_linear_prequantized.__wrapped__ = original
    return w4a8_linear_prequantized


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
def wrap_mlp(original):
    def forward(self, x, norm=None):
        if (guard.off("mono") or norm is None or x.device.type != DEVICE_TYPE or x.dtype != torch.bfloat16
                or x.shape[-1] != 4096 or not 1 <= x.numel() // x.shape[-1] <= 16):
            return original(self, x, norm=norm)
        lins = (self.gate_proj, self.up_proj, self.down_proj)
        key = tuple(id(getattr(l, "weight", None)) for l in lins)
        parts = _cached(self, "_mdx_mlp", key, lambda: [_w4_of(l) for l in lins])
        if any(p is None for p in parts):
            _fallback("mono", "weights")
            return original(self, x, norm=norm)
        if not (torch.equal(parts[0][3], parts[1][3]) and torch.equal(parts[0][3], parts[2][3])):
            _fallback("mono", "codebook")
            return original(self, x, norm=norm)
        try:
            C = _lib_C()
            h, lut, _ = _constants(x.device)
            xn = norm(x)
            out = C.mono_mlp(xn.reshape(-1, x.shape[-1]).contiguous(), h, lut, *parts[0], *parts[1], *parts[2], 0, 4,
                             False)
        except Exception as e:  # nothing was written: the original recomputes from x
            guard.failed("mono", e)
            return original(self, x, norm=norm)
        _fast("mono")
        return out.reshape(*x.shape[:-1], out.shape[-1])

    setattr(forward, CLAIM, True)
    forward.__wrapped__ = original
    return forward


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


def _run(block, plan, x, S, freqs_cis, kv, state):
    C = _lib_C()
    h, silu, sig = _constants(x.device)
    x2 = x.view(S, 4096)
    (nin, ein), (npo, epo) = plan["norm_in"], plan["norm_post"]
    if plan["gdn"]:
        mix, ex = block.linear_attn, plan["extra"]
        args = (x2, nin, ein, h, plan["pre"] + plan["out"] + plan["mlp"], ex["wa"], ex["wb"], ex["conv_w"],
                kv.conv_state, kv.proj_buf, kv.qkv_buf, kv.ctl, kv.dt_bias, kv.g_decay, kv.recurrent_state,
                kv.gates_buf, kv.sumsq_buf, kv.norm_weight, mix.norm.eps, mix.key_head_dim ** -0.5, mix.num_key_heads,
                npo, epo, silu, 0, 11, False)
        state["mutated"] = True  # marked before the launch: a failure does not prove that nothing ran
        C.layer_gdn(*args)
        return x, kv
    outs = C.layer_pre(x2, nin, ein, h, plan["pre"], 0, False)
    state["mutated"] = True  # the attention core writes KV rows before attending
    y = attn_core(block.self_attn, outs[1], outs[2], outs[3], freqs_cis, kv)
    # the gate half of each head's [query | gate] block, as a plain [S, heads * head_dim] gate
    mix = block.self_attn
    gate = (outs[1].view(S, mix.num_heads, 2, mix.head_dim)[:, :, 1].reshape(S, -1).contiguous()
            if plan["gated"] else None)
    C.layer_post(x2, y.contiguous(), gate, sig, *plan["out"], npo, epo, h, silu, *plan["mlp"], 0, 6, False)
    return x, kv


def wrap_block(original, max_rows=16):
    def forward(self, x, attention_mask=None, freqs_cis=None, optimized_attention=None, past_key_value=None):
        args = (self, x, attention_mask, freqs_cis, optimized_attention, past_key_value)
        B, S = (x.shape[0], x.shape[1]) if x.dim() == 3 else (0, 0)
        if (guard.off("layer") or past_key_value is None or x.device.type != DEVICE_TYPE or x.dtype != torch.bfloat16
                or B != 1 or not 1 <= S <= max_rows or x.shape[-1] != 4096 or not x.is_contiguous()):
            return original(*args)
        gdn = getattr(self, "layer_type", None) == "linear_attention"
        if gdn and not past_key_value.decode_step(S):
            return original(*args)
        if not gdn and (attention_mask is not None
                        or (self.self_attn.num_heads // self.self_attn.num_kv_heads) * S > 64):
            return original(*args)
        key = tuple(id(getattr(m, "weight", None)) for m in _block_linears(self))
        plan = _cached(self, "_mdx_plan", key, lambda: static_plan(self))
        if plan is None:
            _fallback("layer", "weights")
            return original(*args)
        state = {"mutated": False}
        try:
            out = _run(self, plan, x, S, freqs_cis, past_key_value, state)
        except SubpathError:
            raise  # that sub-path is already off; state may be written, so the block is not replayed
        except Exception as e:
            guard.failed("layer", e, can_fallback=not state["mutated"])
            if state["mutated"]:
                raise  # KV rows, the recurrent state or x already changed: replaying would apply them twice
            return original(*args)
        _fast("layer")
        return out

    setattr(forward, CLAIM, True)
    forward.__wrapped__ = original
    return forward


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
