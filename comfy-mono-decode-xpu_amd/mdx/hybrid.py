"""A synthetic Qwen3.5-style W4A8 hybrid model decoded with MTP tree verification on one MI355X.

Shape (defaults): 32 layers, every 4th full attention (32 q / 8 kv heads, head_dim 128, partial RoPE
theta 1e7, Q/K RMSNorm), the rest Gated-DeltaNet (16 key / 32 value heads of 128, conv 4); hidden
4096, SwiGLU MLP 12288; random GPTQ int4 weights (G128 fp16 scales, tile-major); a 1-layer bf16 MTP
draft block; a bf16 lm_head over vocab 151936; an 8-row draft tree (tree_spec (4, 3): two drafts per
step); top-k 20 sampling.

One decode step (comfy_mono_decode_xpu/mtp_loop.py:187-489, graph_step.py:62-127):
  drafts   for depth k: mtp_prep_draft -> MTP block (embed + hidden norms, fc, attention layer, MLP)
           -> final norm -> lm_head -> fast_topk(width_k): the tree's children at depth k + 1;
  verify   mtp_prep_verify -> 32 layers over the tree rows (layer_pre / qk_norm_rope_kv / attn_dpas /
           layer_post for attention layers, layer_gdn for GDN layers) -> final norm -> lm_head ->
           topk_rows(20) -> Gumbel-max sampling -> mtp_accept (counters, ctl, next token, hidden row,
           KV slot moves).
Every counter lives on the device, so a step is one captured HIP graph; two graphs alternate the
replay parity of the GDN buffers. The host only replays graphs.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _C, _lib, _tree, layout


@dataclass
class HybridConfig:
    layers: int = 32
    hidden: int = 4096
    inter: int = 12288
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    rotary: int = 64
    theta: float = 1e7
    gdn_key_heads: int = 16
    gdn_value_heads: int = 32
    vocab: int = 151936
    widths: tuple = (4, 3)
    slots: int = 16
    top_k: int = 20
    temperature: float = 1.0
    greedy: bool = False          # take the top-1 instead of sampling
    sample_seed: int = 0x5EED5EED  # the sampling uniforms' seed (SplitMix64 of seed, position, row, slot)
    two_stage: bool = False       # drafts: int4 scores + the draft pick instead of the full lm_head
    head: str = "bf16"            # "int8": the int8 ConvRot lm_head (W8A8) for the verify and the drafts
    eps: float = 1e-6
    cap: int = 2048
    attn_every: int = 4           # layer i is full attention iff i % attn_every == attn_every - 1
    auto: bool = False            # adaptive tree: drafts keep 7 candidates, the accept records their ranks
    attn: str = "fast"            # "exact": attention in one canonical fp32 order (mdx_attn_exact)
    rotate: bool = False          # W4 activations rotated by H256 before quantisation (ConvRot-packed weights)
    # W4 group scales of the random weights: "faithful" keeps each fp16 G128 group scale as an fp16 ratio to
    # the channel scale, decoded per weight by rint (the reference contract, what checkpoint ingestion
    # produces); "integral" re-quantises them to 4-bit integer multiples of the channel scale (lossy)
    scales: str = "faithful"
    # synthetic weights with a predictable next token (token t -> t + 1 mod vocab) for the verify and the
    # drafts: the lm_head row v is the embedding of v - 1, the layers' and the MTP block's output
    # projections are scaled down (the residual stream stays the embedding) and the MTP block's fc passes
    # the embedding half through. Every kernel does the same work on the same shapes; the drafts are
    # accepted, so a step commits len(widths) + 1 tokens.
    predictable: bool = False
    # GDN layers: the conv and the gates in the input projections' launch (mdx_gdn_proj + mdx_gdn_delta);
    # False: the projections, then the conv + gates and the delta rule as their own launches
    # (mdx_stream_gemv + mdx_gdn_core_raw). Both give the same bits.
    gdn_fold: bool = True

    def attention(self, i):
        return i % self.attn_every == self.attn_every - 1


def _gptq(N, K, gen, dev, integral=False):
    q = torch.randint(-8, 8, (N, K), generator=gen, device=dev, dtype=torch.int8)
    s = (torch.rand(N, K // 128, generator=gen, device=dev) * 0.015 + 0.005).half()
    packed, s_rel, sch, _ = layout.gptq_pack(q, s, 128, integral=integral)
    del q
    return layout.W4(layout.tile_major_codes(packed), s_rel, sch, None, _lib.LAYOUT_TILE,
                     _lib.DECODE_INTEGRAL if integral else _lib.DECODE_AUTO)


def _norm(n, gen, dev, spread=0.02):
    return (1 + spread * torch.randn(n, generator=gen, device=dev)).bfloat16()


def _bf16w(N, K, gen, dev, std):
    return layout.tile_major_bf16((torch.randn(N, K, generator=gen, device=dev) * std).bfloat16())


def tree_tensors(widths, slots, dev):
    """Parents, depths, verify program, ancestor masks, children table and, per depth, the rows that
    receive the draft's candidates (chain child first) of tree_spec(widths)."""
    parents, children, depth, chain = _tree.tree_from_spec(_tree.spec_of_widths(widths), slots)
    R = 1 + sum(widths)
    prog = _tree.verify_program(parents[:R], R)
    mask = []
    for r in range(R):
        p = parents[r]
        mask.append((mask[p] if p >= 0 else 0) | (1 << r))
    ch = torch.full((slots, slots), -1, dtype=torch.int32)
    for r, cs in enumerate(children[:slots]):
        for j, c in enumerate(cs):
            ch[r, j] = c
    chain_nodes = [0]
    while children[chain_nodes[-1]]:
        chain_nodes.append(children[chain_nodes[-1]][0])
    fill_rows = [list(children[chain_nodes[k]]) for k in range(len(widths))]
    fill = [torch.tensor(r, dtype=torch.int64, device=dev) for r in fill_rows]
    tree_ctl = torch.tensor(parents[:R] + [-1] * (slots - R) + prog + [0] * (slots - R), dtype=torch.int32, device=dev)
    return dict(R=R, depth=chain, parents=parents[:R], prog=prog,
                mask=torch.tensor(mask, dtype=torch.int32, device=dev), children=ch.reshape(-1).to(dev),
                tree_pos=torch.tensor(depth[:R], dtype=torch.int64, device=dev), tree_ctl=tree_ctl, fill=fill,
                fill_rows=fill_rows)


def rope_table(cfg, dev):
    """[cap, rd/2, 2, 2] rotation matrices [[cos, -sin], [sin, cos]] of each position."""
    half = cfg.rotary // 2
    inv = cfg.theta ** (-torch.arange(half, dtype=torch.float64) * 2 / cfg.rotary)
    ang = torch.arange(cfg.cap, dtype=torch.float64)[:, None] * inv[None, :]
    c, s = torch.cos(ang), torch.sin(ang)
    return torch.stack([torch.stack([c, -s], -1), torch.stack([s, c], -1)], -2).float().contiguous().to(dev)


class HybridModel:
    """Random-init weights of the hybrid stack and its decode state on one device."""

    def __init__(self, cfg: HybridConfig, device, seed=5):
        self.cfg = c = cfg
        dev = self.dev = torch.device(device)
        gen = torch.Generator(device=dev).manual_seed(seed)
        H, I = c.hidden, c.inter
        qd, kd = c.heads * c.head_dim, c.kv_heads * c.head_dim
        hk, hv = c.gdn_key_heads, c.gdn_value_heads
        self.gdn_ch = 2 * hk * 128 + hv * 128
        self.embed = (torch.randn(c.vocab, H, generator=gen, device=dev) * 0.5).bfloat16()
        head = (torch.randn(c.vocab, H, generator=gen, device=dev) * 0.02).bfloat16()
        if c.predictable:
            # logit of t + 1 at an embedding e_t: 0.015 |e_t|^2 / rms(e_t) ~ 31, the others ~ N(0, 0.5)
            head = (torch.roll(self.embed.float(), shifts=1, dims=0) * 0.015).bfloat16()
        if c.head not in ("bf16", "int8"):
            raise ValueError("head: 'bf16' or 'int8'")
        self.lm_head = self.lm_rows = self.lm8 = self.lm8_rows = self.lm8_s = None
        if c.head == "int8":
            # the int8 ConvRot head (rows rotated by H256 per 256 group, per-row scales), tile-major for the
            # W8A8 linear; the two-stage drafts score an int4 copy of it and the pick recomputes its
            # candidates from the row-major int8 rows (comfy_mono_decode_xpu/draft_lmhead.py:68-84)
            q8, self.lm8_s = layout.int8_convrot_head(head)
            del head
            self.lm8 = layout.tile_major_i8(q8)
            self.lm4 = layout.int4_scoring_copy(q8.float() * self.lm8_s[:, None]) if c.two_stage else None
            self.lm8_rows = q8 if c.two_stage else None
            del q8
        else:
            self.lm_head = layout.tile_major_bf16(head)
            # the two-stage draft head: an int4 copy of the lm_head scored by the W4A8 GEMV, and the row-major
            # head the draft pick reads its candidates from (8 KiB contiguous per row; the tile-major copy
            # serves the full-vocabulary passes)
            self.lm4 = layout.int4_scoring_copy(head) if c.two_stage else None
            self.lm_rows = head if c.two_stage else None
            del head
        self.final_norm = _norm(H, gen, dev)
        self.h256 = layout.regular_hadamard(dev)
        self.h256f = layout.regular_hadamard(dev, torch.float32)  # the draft ops take the f32 matrix
        # the W4 activation preps: plain absmax (GPTQ weights) or H256 first (ConvRot-packed weights)
        self.rot, self.hrot = (_lib.ROT_H256, self.h256) if c.rotate else (_lib.ROT_NONE, None)
        self.silu = layout.silu_lut(dev)
        self.sig = torch.sigmoid(layout.bf16_all(dev)).contiguous()
        self.layers = []
        if c.scales not in ("faithful", "integral"):
            raise ValueError(f"HybridConfig.scales: {c.scales!r} (faithful | integral)")
        integ = c.scales == "integral"
        for i in range(c.layers):
            L = dict(norm_in=_norm(H, gen, dev), norm_post=_norm(H, gen, dev), g=_gptq(I, H, gen, dev, integ),
                     u=_gptq(I, H, gen, dev, integ), d=_gptq(H, I, gen, dev, integ))
            L["u"].cb = L["d"].cb = L["g"].cb
            if c.attention(i):
                L.update(q=_gptq(qd, H, gen, dev, integ), k=_gptq(kd, H, gen, dev, integ), v=_gptq(kd, H, gen, dev, integ),
                         o=_gptq(H, qd, gen, dev, integ), qn=_norm(c.head_dim, gen, dev, 0.1), kn=_norm(c.head_dim, gen, dev, 0.1))
            else:
                L.update(qkv=_gptq(self.gdn_ch, H, gen, dev, integ), z=_gptq(hv * 128, H, gen, dev, integ), o=_gptq(H, hv * 128, gen, dev, integ),
                         wa=(torch.randn(hv, H, generator=gen, device=dev) * 0.02).bfloat16(),
                         wb=(torch.randn(hv, H, generator=gen, device=dev) * 0.02).bfloat16(),
                         conv_w=(torch.randn(self.gdn_ch, 4, generator=gen, device=dev) * 0.5).bfloat16(),
                         dt_bias=torch.rand(hv, generator=gen, device=dev) * 2 - 1,
                         g_decay=-torch.exp(torch.rand(hv, generator=gen, device=dev) * 1.5 - 1),
                         gnorm=_norm(128, gen, dev, 0.1))
            self.layers.append(L)
        # the MTP draft block (bf16; gated attention: the q projection holds [query | gate] per head)
        self.mtp = dict(norm_e=_norm(H, gen, dev), norm_h=_norm(H, gen, dev), fc=_bf16w(H, 2 * H, gen, dev, 0.02),
                        norm_in=_norm(H, gen, dev), qkv=_bf16w(2 * qd + 2 * kd, H, gen, dev, 0.02),
                        qn=_norm(c.head_dim, gen, dev, 0.1), kn=_norm(c.head_dim, gen, dev, 0.1),
                        o=_bf16w(H, qd, gen, dev, 0.02), norm_post=_norm(H, gen, dev),
                        gu=_bf16w(2 * I, H, gen, dev, 0.02), d=_bf16w(H, I, gen, dev, 0.02), norm_f=_norm(H, gen, dev))
        if c.predictable:
            for L in self.layers:
                for r in ("o", "d"):
                    L[r].sc.mul_(1e-6)  # (1e-3 is not enough: the GDN layers' outputs grow along the stack)
            M = self.mtp
            M["fc"] = layout.tile_major_bf16(torch.cat([torch.eye(H, device=dev), torch.zeros(H, H, device=dev)], 1).bfloat16())
            M["o"] = layout.tile_major_bf16((torch.randn(H, qd, generator=gen, device=dev) * 2e-5).bfloat16())
            M["d"] = layout.tile_major_bf16((torch.randn(H, I, generator=gen, device=dev) * 2e-5).bfloat16())
        self.ftab = rope_table(c, dev)
        self._state(gen)

    def load_w4(self, weights, plan):
        """Replace the W4 linears of the layers in `plan` ({layer: {role: prefix}}, as checkpoint.plan_hybrid
        returns) by packed checkpoint linears (`weights`: {prefix: layout.W4}). The layer's three MLP
        projections must share one codebook (the MLP block decodes them with one table); the attention
        q_proj must be ungated ([heads * head_dim, hidden]). Weights packed with a ConvRot rotation
        (comfy-kitchen's W4A8 layout) need cfg.rotate."""
        c = self.cfg
        qd = c.heads * c.head_dim
        for i, roles in plan.items():
            ws = {r: weights[p] for r, p in roles.items()}
            if "q" in ws and ws["q"].n != qd:
                raise ValueError(f"layer {i}: a gated q_proj ({ws['q'].n} rows) is not supported here")
            cbs = [ws[r].cb for r in ("g", "u", "d")]
            if not (all(cb is None for cb in cbs) or all(cb is not None and torch.equal(cb, cbs[0]) for cb in cbs)):
                raise ValueError(f"layer {i}: gate / up / down codebooks differ")
            self.layers[i].update(ws)

    # ---- decode state --------------------------------------------------------------------------
    def _state(self, gen):
        c, dev = self.cfg, self.dev
        S = c.slots
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.kv = [None] * c.layers
        self.gdn = [None] * c.layers
        for i in range(c.layers):
            if c.attention(i):
                self.kv[i] = (torch.zeros(1, c.kv_heads, c.cap, c.head_dim, **bf),
                              torch.zeros(1, c.kv_heads, c.cap, c.head_dim, **bf))
            else:
                hv, hk = c.gdn_value_heads, c.gdn_key_heads
                conv = torch.zeros(self.gdn_ch, 3, **bf)
                self.gdn[i] = dict(conv=conv, pb=torch.zeros(2, S, self.gdn_ch, **bf),
                                   qb=torch.zeros(2, S, self.gdn_ch, **bf),
                                   rec=torch.randn(hv, 128, 128, generator=gen, device=dev) * 0.1,
                                   gates=torch.zeros(2, S, hv, 2, device=dev), sums=torch.zeros(2, S, hk, 2, device=dev))
        self.mkv = (torch.zeros(1, c.kv_heads, c.cap, c.head_dim, **bf),
                    torch.zeros(1, c.kv_heads, c.cap, c.head_dim, **bf))
        ptrs = []
        for kv in self.kv:
            if kv is not None:
                ptrs += [kv[0].data_ptr(), kv[1].data_ptr()]
        self.kv_ptrs = torch.tensor([p - (1 << 64) if p >= (1 << 63) else p for p in ptrs], dtype=torch.int64, device=dev)
        i64 = dict(dtype=torch.int64, device=dev)
        self.st = torch.zeros(4, **i64)
        self.ctl = torch.zeros(2 + 3 * S, dtype=torch.int32, device=dev)
        self.result = torch.zeros(S + 24, **i64)
        self.nt = torch.zeros(1, 1, **i64)
        self.hbuf = torch.zeros(1, c.hidden, **bf)
        # the tree rows' buffers at the slot capacity; _set_tree takes views of the first R rows
        self._rows = dict(vtok=torch.zeros(1, S, **i64), toks=torch.zeros(1, S, **i64), apos=torch.zeros(S, **i64),
                          vpos=torch.zeros(1, S, **i64), vfreqs=torch.zeros(S, c.rotary // 2, 2, 2, device=dev),
                          x=torch.zeros(S, c.hidden, **bf), logits=torch.zeros(S, c.vocab, **bf))
        self.aseq = torch.zeros(1, dtype=torch.int32, device=dev)
        qd, kd = c.heads * c.head_dim, c.kv_heads * c.head_dim
        # MTP block buffers (up to `slots` rows: one per draft, a chain of rows in the prefill)
        self.dfreqs = torch.zeros(1, 1, 1, c.rotary // 2, 2, 2, device=dev)
        self.mpos = torch.zeros(S, **i64)
        self.mseq = torch.zeros(1, dtype=torch.int32, device=dev)
        self.dh = torch.zeros(S, c.hidden, **bf)
        self.dcat = torch.zeros(S, 2 * c.hidden, **bf)
        self.dx = torch.zeros(S, c.hidden, **bf)
        self.dxn = torch.zeros(S, c.hidden, **bf)
        self.dqkv = torch.zeros(S, 2 * qd + 2 * kd, **bf)
        self.dy = torch.zeros(S, qd, **bf)
        self.dgy = torch.zeros(S, qd, **bf)
        self.do = torch.zeros(S, c.hidden, **bf)
        self.dgu = torch.zeros(S, 2 * c.inter, **bf)
        self.dact = torch.zeros(S, c.inter, **bf)
        self.dd = torch.zeros(S, c.hidden, **bf)
        self.dxf = torch.zeros(S, c.hidden, **bf)
        self.dqx = torch.zeros(S, c.hidden, dtype=torch.int8, device=dev)
        self.dsx = torch.zeros(S, dtype=torch.float32, device=dev)
        self.pick_calls = torch.zeros(1, **i64)
        self.dlogits = torch.zeros(1, c.vocab, **bf)
        self.dtop = torch.zeros(7, 8, **i64)
        self.dtok = torch.zeros(7, 1, **i64)
        # auto: the 7 candidates of chain node k (the draft at depth k) at [7 k, 7 k + 7) for the accept's ranks
        self.cand = torch.zeros(7 * 7, **i64)
        # every tree's device tensors, kept for the model's lifetime: a captured graph holds their
        # addresses, and a tree may come back after another one (decode_auto, _set_tree)
        self._trees = {}
        self._set_tree(c.widths)
        self.empty_mask = torch.empty(0, dtype=torch.int32, device=dev)
        self.graphs = {}
        # host-side upper bound of the committed position st[0]: every KV write of a step lands at
        # most R - 1 past it, and each step commits at most len(widths) + 1 tokens
        self.pos_bound = None
        # a list to receive (name, copy) of the step's intermediates (eager steps only; None: off)
        self.trace = None

    def _set_tree(self, widths):
        """Use the tree tree_spec(widths) from the next step on (views of the first R tree-row buffers)."""
        c = self.cfg
        widths = tuple(int(w) for w in widths)
        if not (1 <= len(widths) <= 7 and all(1 <= w <= (7 if c.auto else 8) for w in widths)
                and 1 + sum(widths) <= c.slots):
            raise ValueError(f"widths {widths}: 1..7 depths of 1..{7 if c.auto else 8} candidates within "
                             f"{c.slots} slots")
        self.widths = widths
        if widths not in self._trees:
            self._trees[widths] = tree_tensors(widths, c.slots, self.dev)
        self.tree = self._trees[widths]
        R = self.R = self.tree["R"]
        b = self._rows
        self.vtok, self.toks, self.vpos = b["vtok"][:, :R], b["toks"][:, :R], b["vpos"][:, :R]
        self.apos, self.vfreqs, self.x, self.logits = b["apos"][:R], b["vfreqs"][:R], b["x"][:R], b["logits"][:R]

    def _attend(self, q, key, value, seq, xk, xv, mask, out):
        if self.cfg.attn == "exact":
            _C.attn_exact(q, key, value, seq, xk, xv, mask, out=out)
        else:
            _C.attn_dpas(q, key, value, seq, xk, xv, mask, 0, out=out)

    def _tracing(self):
        return self.trace is not None and not torch.cuda.is_current_stream_capturing()

    def _tr(self, name, t):
        if self._tracing():
            self.trace.append((name, t.detach().clone()))

    def _reserve(self, steps):
        """Raise before launching `steps` decode steps whose KV writes could pass the cache capacity."""
        if self.pos_bound is None:
            raise RuntimeError("prefill() first")
        per = len(self.widths) + 1
        need = self.pos_bound + steps * per + self.R
        if need > self.cfg.cap:
            raise RuntimeError(f"{steps} more decode steps may write KV position {need - 1}, past the cache capacity "
                               f"{self.cfg.cap}")
        self.pos_bound += steps * per

    # ---- the pieces of a step ------------------------------------------------------------------
    def _attn_layer(self, i, x, R, mask, seq, pos, freqs):
        c, L = self.cfg, self.layers[i]
        key, value = self.kv[i]
        xn = torch.empty(R, c.hidden, dtype=torch.bfloat16, device=self.dev)
        q, s = _C.rms_rot_quant(x, L["norm_in"], c.eps, self.rot, self.hrot, xn_out=xn)
        qd, kd = c.heads * c.head_dim, c.kv_heads * c.head_dim
        qkv = [torch.empty(R, n, dtype=torch.bfloat16, device=self.dev) for n in (qd, kd, kd)]
        _C.stream_gemv(q, s, [L["q"], L["k"], L["v"]], qkv)
        for nm, t in zip(("q", "k", "v"), qkv):
            self._tr(f"L{i}.{nm}", t)
        qv = qkv[0].view(1, R, c.heads, c.head_dim)
        kv_ = qkv[1].view(1, R, c.kv_heads, c.head_dim)
        vv = qkv[2].view(1, R, c.kv_heads, c.head_dim)
        qo = torch.empty(1, c.heads, R, c.head_dim, dtype=torch.bfloat16, device=self.dev)
        ko = torch.empty(1, c.kv_heads, R, c.head_dim, dtype=torch.bfloat16, device=self.dev)
        y = torch.empty(1, R, qd, dtype=torch.bfloat16, device=self.dev)
        if c.attn != "exact" and _C.rope_attn_fits(c.heads, c.kv_heads, R, c.head_dim, c.rotary):
            # the Q/K norm, RoPE and KV write inside the attention launch (the same bits as the two calls)
            _C.qk_norm_rope_attn(qv, kv_, vv, L["qn"], L["kn"], freqs, key, value, pos, c.eps, c.eps, c.rotary, seq,
                                 mask, ko, out=y, q_out=qo if self._tracing() else None)
        else:
            _C.qk_norm_rope_kv(qv, kv_, vv, L["qn"], L["kn"], freqs, key, value, pos, c.eps, c.eps, c.rotary, outs=(qo, ko))
            self._attend(qo, key, value, seq, ko, vv.transpose(1, 2), mask, y)
        self._tr(f"L{i}.qo", qo)
        self._tr(f"L{i}.ko", ko)
        self._tr(f"L{i}.y", y)
        _C._layer_post(x, y.view(R, qd), None, None, L["o"], L["norm_post"], c.eps, self.hrot, self.silu, L["g"], L["u"],
                       L["d"], 6)

    def _gdn_layer(self, i, x, R):
        c, L, G = self.cfg, self.layers[i], self.gdn[i]
        sc = _C._scratch(self.dev)
        xn, q, s = _C._buf(sc["xn"], R, c.hidden), _C._buf(sc["q1"], R, c.hidden), sc["s"][:R]
        # one row without rotation: the row prep runs in the projection launch (fp16 scales)
        xrow = c.gdn_fold and R == 1 and self.rot == _lib.ROT_NONE and L["qkv"].s.dtype == torch.float16
        if not xrow:
            _lib.call("mdx_rms_rot_quant", _lib.ptr(x), _lib.ptr(L["norm_in"]), float(c.eps), _lib.ptr(xn),
                      _lib.ptr(self.hrot), self.rot, _lib.ptr(q), _lib.ptr(s), R, c.hidden, _lib.stream_of(x))
        hv = c.gdn_value_heads
        proj, z = _C._buf(sc["proj"], R, self.gdn_ch), _C._buf(sc["z"], R, hv * 128)
        core = _C._buf(sc["core"], R, hv * 128)
        zg = _C._buf(sc["zg"], R, hv * 128) if c.gdn_fold and self.rot == _lib.ROT_NONE else None
        if c.gdn_fold:
            _C.gdn_proj(q, s, L["qkv"], L["z"], proj, z, xn, L["wa"], L["wb"], L["conv_w"], G["conv"], G["pb"], G["qb"],
                        self.ctl, L["dt_bias"], L["g_decay"], G["gates"], c.gdn_key_heads, z_gate=zg,
                        x_row=x.view(1, -1) if xrow else None, norm_w=L["norm_in"], eps=c.eps)
            _C.gdn_delta(G["qb"], self.ctl, G["rec"], G["gates"], 128 ** -0.5, c.gdn_key_heads, core)
        else:
            _C.stream_gemv(q, s, [L["qkv"], L["z"]], [proj, z])
            _C.gdn_core(proj, z, xn, L["wa"], L["wb"], L["conv_w"], G["conv"], G["pb"], G["qb"], self.ctl, L["dt_bias"],
                        L["g_decay"], G["rec"], G["gates"], G["sums"], L["gnorm"], c.eps, 128 ** -0.5, c.gdn_key_heads,
                        core=core, raw=True)
        self._tr(f"L{i}.proj", proj)
        self._tr(f"L{i}.z", z)
        self._tr(f"L{i}.core_raw", core)
        core_n = _C._buf(sc["core_n"], R, hv * 128)
        _C._layer_post(x, core, None, None, L["o"], L["norm_post"], c.eps, self.hrot, self.silu, L["g"], L["u"], L["d"], 6,
                       gnorm=(z, L["gnorm"], c.eps) if zg is None else (zg, L["gnorm"], c.eps, True), gnorm_out=core_n)
        self._tr(f"L{i}.core", core_n)

    def verify_layers(self, x, R, mask, seq, pos, freqs):
        for i in range(self.cfg.layers):
            self._tr(f"L{i}.in", x)
            if self.cfg.attention(i):
                self._attn_layer(i, x, R, mask, seq, pos, freqs)
            else:
                self._gdn_layer(i, x, R)
            self._tr(f"L{i}.out", x)

    def mtp_block(self, n, tok, h, freqs, kvpos, seq, mask):
        """The MTP block over n rows (tokens `tok` [n], hidden rows `h` [n, H]), in the fused-op structure
        of comfy_mono_decode_xpu/draft_head.py:179-212: cat(RMSNorm_e(embed[tok]), RMSNorm_h(h)) -> fc -> x;
        RMSNorm_in -> q|gate, k, v -> Q/K norm + RoPE + the MTP KV write at kvpos -> attention over the MTP
        cache prefix [0, seq) (and, with a mask, the block's own rows) -> times sigmoid(gate) -> o_proj;
        x += o, RMSNorm_post -> gate|up -> SiLU(gate) * up -> down; x += down, RMSNorm_f. Leaves the new
        hidden rows x in self.dh[:n] and their final norm (the lm_head input) in self.dxf[:n]."""
        c, M = self.cfg, self.mtp
        H, D = c.hidden, c.head_dim
        qd, kd = c.heads * D, c.kv_heads * D
        cat = _C._buf(self.dcat, n, 2 * H)
        _C.draft_embed_norm_cat(tok.view(-1), None, None, None, self.embed, h, M["norm_e"], M["norm_h"], c.eps, c.eps, cat)
        x = _C._buf(self.dh, n, H)
        xn = _C._buf(self.dxn, n, H)
        _C.bf16_linear(cat, M["fc"], out=x)
        self._tr("mtp.cat", cat)
        self._tr("mtp.x_fc", x)
        _C.draft_add_rmsnorm(x, None, M["norm_in"], c.eps, xn)
        self._tr("mtp.xn_in", xn)
        qkv = _C._buf(self.dqkv, n, 2 * qd + 2 * kd)
        _C.bf16_linear(xn, M["qkv"], out=qkv)
        self._tr("mtp.qkv", qkv)
        qg = qkv[:, :2 * qd]
        qv = qg.reshape(n, c.heads, 2 * D)[:, :, :D]
        kv_ = qkv[:, 2 * qd:2 * qd + kd].view(1, n, c.kv_heads, D)
        vv = qkv[:, 2 * qd + kd:].view(1, n, c.kv_heads, D)
        mk, mv = self.mkv
        qo = torch.empty(1, c.heads, n, D, dtype=torch.bfloat16, device=self.dev)
        ko = torch.empty(1, c.kv_heads, n, D, dtype=torch.bfloat16, device=self.dev)
        _C.qk_norm_rope_kv(qv, kv_, vv, M["qn"], M["kn"], freqs, mk, mv, kvpos, c.eps, c.eps, c.rotary, outs=(qo, ko))
        y = _C._buf(self.dy, n, qd)
        self._attend(qo, mk, mv, seq, ko, vv.transpose(1, 2), self.empty_mask if mask is None else mask,
                     y.view(1, n, qd))
        gy = _C._buf(self.dgy, n, qd)
        _C.draft_sigmoid_mul(y, qg if n > 1 else qg.view(-1), D, gy)
        self._tr("mtp.qo", qo)
        self._tr("mtp.ko", ko)
        self._tr("mtp.y", y)
        self._tr("mtp.gy", gy)
        o = _C._buf(self.do, n, H)
        _C.bf16_linear(gy, M["o"], out=o)
        self._tr("mtp.o", o)
        _C.draft_add_rmsnorm(x, o, M["norm_post"], c.eps, xn)
        self._tr("mtp.x_post", x)
        self._tr("mtp.xn_post", xn)
        gu = _C._buf(self.dgu, n, 2 * c.inter)
        _C.bf16_linear(xn, M["gu"], out=gu)
        act = _C._buf(self.dact, n, c.inter)
        _C.draft_silu_mul(gu, act)
        d = _C._buf(self.dd, n, H)
        _C.bf16_linear(act, M["d"], out=d)
        self._tr("mtp.gu", gu)
        self._tr("mtp.act", act)
        self._tr("mtp.d", d)
        if c.head == "int8":
            # the int8 head's input: the final norm rotated by H256 and quantised per row
            _C.draft_norm_rot_quant(x, d, M["norm_f"], c.eps, self.h256f, _C._buf(self.dxf, n, H), self.dqx[:n],
                                    self.dsx[:n])
            self._tr("mtp.qx", self.dqx[:n])
            self._tr("mtp.sx", self.dsx[:n])
        else:
            _C.draft_norm_rot_quant(x, d, M["norm_f"], c.eps, None, _C._buf(self.dxf, n, H), None, None)
        self._tr("mtp.x_out", x)
        self._tr("mtp.xf", _C._buf(self.dxf, n, H))

    def draft(self, k, tok, h, width):
        """Draft depth k: the MTP block on the chain token `tok` [1] and hidden row `h` [1, H] at the
        device positions of mtp_prep_draft, then the final norm, the lm_head and the top-`width`, written
        to the tree rows of depth k + 1 (chain child first). Returns the chain token [1].
        two_stage: the lm_head's int4 copy scores the vocabulary and the draft pick recomputes the exact
        logits of its candidates (the same result whenever the exact top-width is among them).
        auto: the draft keeps its 7 best candidates in self.cand[7 k, 7 k + 7) (the accept records the rank
        of the verify's token among them), the first `width` become tree rows."""
        c, T = self.cfg, self.tree
        nout = 7 if c.auto else width
        _C.mtp_prep_draft(self.st, k, self.ftab.view(1, 1, c.cap, c.rotary // 2, 2, 2), self.dfreqs, self.mpos, self.mseq)
        self.mtp_block(1, tok, h, self.dfreqs.view(1, c.rotary // 2, 2, 2), self.mpos[:1], self.mseq, None)
        xf = self.dxf[:1]
        picked = None
        if c.head == "int8":
            qx, sx = self.dqx[:1], self.dsx[:1]
            if c.two_stage:
                _C.stream_gemv(qx, sx, [self.lm4], [self.dlogits])
                _C.draft_pick(self.dlogits.view(-1), qx.view(-1), sx, self.lm8_rows, self.lm8_s, nout, False,
                              self.dtop[k], None, self.dtok[k], self.vtok.view(-1), T["fill_rows"][k], self.pick_calls)
                picked = self.dtop[k]
            else:
                _C.int8_linear_prequantized(qx, sx, self.lm8, self.lm8_s, tiled=True, out=self.dlogits)
        elif c.two_stage:
            q, s = _C.quant_rows(xf)
            _C.stream_gemv(q, s.view(-1), [self.lm4], [self.dlogits])
            _C.draft_pick_bf16(self.dlogits.view(-1), xf.view(-1), self.lm_rows, nout, False, self.dtop[k], None,
                               self.dtok[k], self.vtok.view(-1), T["fill_rows"][k], tiled=False)
            picked = self.dtop[k]
        else:
            _C.bf16_linear(xf, self.lm_head, out=self.dlogits)
        if picked is not None:
            if c.auto:
                self.cand[7 * k:7 * k + 7].copy_(picked[:7])
            return self.dtok[k]
        self._tr("draft.logits", self.dlogits)
        top = _C.fast_topk(self.dlogits, nout, False)[1].view(-1)
        self.vtok[0].index_copy_(0, T["fill"][k], top[:width])
        if c.auto:
            self.cand[7 * k:7 * k + 7].copy_(top)
        return top[:1]

    def draft_part(self):
        """The step's drafts: depth k proposes the children of chain node k."""
        tok, h = self.nt.view(-1), self.hbuf
        # (the root row's verify token is the next token, stored by the verify's prep launch)
        for k, w in enumerate(self.widths):
            tok, h = self.draft(k, tok, h, w), self.dh[:1]

    def step(self, parity):
        """One decode step on the device (drafts, verify, sampling, accept). An eager step checks the
        KV capacity itself; a captured one is checked when its graph is replayed."""
        if not torch.cuda.is_current_stream_capturing():
            self._reserve(1)
        self.draft_part()
        self.verify_part(parity)

    def verify_part(self, parity):
        """The step's verify: the tree rows through the layers, lm_head, top-k, sampling, accept."""
        c, T = self.cfg, self.tree
        R = self.R
        # verify
        # positions and control words, the root token, and the rows' embeddings and RoPE rows: one launch
        _C.mtp_prep_verify_rows(self.st, self.apos, self.aseq, self.vpos, T["tree_pos"], self.ctl, T["tree_ctl"], parity, 0,
                                self.nt.view(-1), self.vtok, self.embed, self.ftab, self.x, self.vfreqs)
        self._tr("verify.vtok", self.vtok)
        self.verify_layers(self.x, R, T["mask"], self.aseq, self.apos, self.vfreqs)
        if c.head == "int8":
            q, s = _C.rms_rot_quant(self.x, self.final_norm, c.eps, _lib.ROT_H256, self.h256)
            _C.int8_linear_prequantized(q, s, self.lm8, self.lm8_s, tiled=True, out=self.logits)
            self._tr("verify.q", q)
            self._tr("verify.s", s)
        else:
            xf = _C.rmsnorm(self.x, self.final_norm, c.eps)
            _C.bf16_linear(xf, self.lm_head, out=self.logits)
            self._tr("verify.xf", xf)
        self._tr("verify.logits", self.logits)
        vals, idx = _C.topk_rows(self.logits, c.top_k)
        self._tr("verify.vals", vals)
        self._tr("verify.idx", idx)
        if c.greedy:
            self.toks.copy_(idx[:, :1].reshape(1, R))
        else:
            # Gumbel-max over the top-k: a sample of softmax(vals / T) restricted to the top k
            # uniforms drawn on the device from the seed and the step's committed position (st[0])
            _C.topk_sample_seeded(vals, idx, c.sample_seed, self.st, c.temperature, out=self.toks.view(R))
        self._tr("verify.toks", self.toks)
        for i, kv in enumerate(self.kv):
            if kv is not None:
                self._tr(f"L{i}.key_pre_accept", kv[0])
                self._tr(f"L{i}.value_pre_accept", kv[1])
        _C.mtp_accept(self.st, self.toks, self.vtok, self.cand if c.auto else None, T["children"], R, T["depth"], self.x,
                      self.nt, self.hbuf.view(1, 1, -1), self.ctl, self.kv_ptrs, c.kv_heads, c.cap, c.head_dim,
                      self.result)

    # ---- prefill (not timed) -------------------------------------------------------------------
    def prefill(self, prompt):
        """Feed prompt[:-1] through the verify path as chains of up to `slots` rows, each committed in
        full (the next chain replays it), and the MTP block over the same chains (hidden row of
        position p with token p + 1). The last prompt token is the first decode step's root row."""
        c = self.cfg
        S = c.slots
        dev = self.dev
        prompt = prompt.to(dev)
        if prompt.numel() < 2 or prompt.numel() + self.R > c.cap:
            raise RuntimeError(f"prompt of {prompt.numel()} tokens: needs 2 <= tokens and tokens + {self.R} tree rows "
                               f"<= the cache capacity {c.cap}")
        body = prompt[:-1]
        n0, parity = 0, 0
        while n0 < body.numel():
            n = min(S, body.numel() - n0)
            chain_ctl = torch.tensor(list(range(-1, n - 1)) + [-1] * (S - n) + [r | 32 for r in range(n)] + [0] * (S - n),
                                     dtype=torch.int32, device=dev)
            tpos = torch.arange(n, dtype=torch.int64, device=dev)
            apos = torch.empty(n, dtype=torch.int64, device=dev)
            vpos = torch.empty(1, n, dtype=torch.int64, device=dev)
            _C.mtp_prep_verify(self.st, apos, self.aseq, vpos, tpos, self.ctl, chain_ctl, parity, 0)
            freqs = torch.index_select(self.ftab, 0, vpos.view(-1))
            x = torch.index_select(self.embed, 0, body[n0:n0 + n])
            mask = torch.tensor([(1 << (r + 1)) - 1 for r in range(n)], dtype=torch.int32, device=dev)
            self.verify_layers(x, n, mask, self.aseq, apos, freqs)
            # the MTP block over the chain: hidden of position p with token p + 1
            st1 = int(self.st[1].item())
            kvpos = torch.arange(st1, st1 + n, dtype=torch.int64, device=dev)
            seq = torch.tensor([st1], dtype=torch.int32, device=dev)
            self.mtp_block(n, prompt[n0 + 1:n0 + 1 + n], x, freqs, kvpos, seq, mask)
            self.st[1] += n
            # commit the whole chain: the next step replays it
            self.st[0] += n
            self.ctl[0] = n
            self.ctl[2:2 + S] = torch.arange(S, dtype=torch.int32, device=dev)
            parity ^= 1
            self.hbuf.copy_(x[n - 1:n])
            n0 += n
        self.nt.fill_(int(prompt[-1].item()))
        self.parity = parity
        self.pos_bound = body.numel()

    # ---- graphs ----------------------------------------------------------------------------------
    def _warm(self):
        """Two eager steps (one per parity) on a side stream: workspaces reach their sizes before capture.
        They are real decode steps of the current tree."""
        st = torch.cuda.Stream(self.dev)
        st.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(st):
            for p in (self.parity, self.parity ^ 1):
                self.step(p)
        torch.cuda.current_stream(self.dev).wait_stream(st)

    def capture(self):
        """Capture one whole step per parity for the current tree (after an eager warm-up of each)."""
        self._warm()
        for p in (0, 1):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.step(p)
            self.graphs[(self.widths, p)] = g

    def replay(self, steps):
        self._reserve(steps)
        for _ in range(steps):
            self.graphs[(self.widths, self.parity)].replay()
            self.parity ^= 1

    def capture_parts(self):
        """Capture the current tree's step as two graphs, the drafts and (per parity) the verify, so that
        device events between them time each part (the adaptive tree's inputs)."""
        self._warm()
        gd = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gd):
            self.draft_part()
        gv = {}
        for p in (0, 1):
            gv[p] = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gv[p]):
                self.verify_part(p)
        self.graphs[(self.widths, "parts")] = (gd, gv)

    def decode_auto(self, steps, fold_every=32):
        """`steps` decode steps with the adaptive tree (cfg.auto): each step replays the current tree's
        draft and verify graphs with HIP events around them and copies its accept record to the host;
        every `fold_every` steps the records' ranks and the events' times are folded in
        (autotree.Hits / Clock) and autotree.best_widths may change the tree (a new tree is captured on
        first use; its two warm-up steps are decode steps too). Returns {"steps", "tokens", "widths"
        (the tree of every step), "draft_ms", "verify_ms"}."""
        from . import autotree
        if not self.cfg.auto:
            raise RuntimeError("decode_auto needs HybridConfig(auto=True) (the drafts keep 7 candidates)")
        if not hasattr(self, "auto_hits"):
            self.auto_hits, self.auto_clock = autotree.Hits(), autotree.Clock()
        S = self.cfg.slots
        host = torch.zeros(fold_every, S + 24, dtype=torch.int64).pin_memory()
        out = {"steps": 0, "tokens": 0, "widths": []}
        pending = []

        def fold():
            torch.cuda.synchronize()
            for ev, slot, nd in pending:
                r = host[slot].tolist()
                n, nranks = int(r[0]), int(r[S + 3])
                self.auto_hits.add(r[S + 4:S + 4 + nranks])
                out["tokens"] += n
                self.auto_clock.add(ev[0].elapsed_time(ev[1]) / nd, ev[1].elapsed_time(ev[2]))
            pending.clear()
            if self.auto_clock.ready:
                best = autotree.best_widths(self.widths, self.auto_hits, self.auto_clock.draft_ms,
                                            self.auto_clock.verify_ms, S)
                if best != self.widths:
                    self._set_tree(best)

        done = 0
        while done < steps:
            if (self.widths, "parts") not in self.graphs:
                st0 = int(self.st[0].item())
                self.capture_parts()  # two eager steps of this tree
                torch.cuda.synchronize()
                out["tokens"] += int(self.st[0].item()) - st0
                out["widths"] += [self.widths] * 2
                done += 2
                continue
            gd, gv = self.graphs[(self.widths, "parts")]
            self._reserve(1)
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
            ev[0].record()
            gd.replay()
            ev[1].record()
            gv[self.parity].replay()
            ev[2].record()
            slot = len(pending)
            host[slot].copy_(self.result, non_blocking=True)
            pending.append((ev, slot, len(self.widths)))
            out["widths"].append(self.widths)
            self.parity ^= 1
            done += 1
            if len(pending) == fold_every:
                fold()
        if pending:
            fold()
        out["steps"] = done
        out["draft_ms"], out["verify_ms"] = self.auto_clock.draft_ms, self.auto_clock.verify_ms
        return out
