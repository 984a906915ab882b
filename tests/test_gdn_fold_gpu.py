"""The Gated-DeltaNet step with the conv and the gates in the projection launch (mdx_gdn_proj +
mdx_gdn_delta) against the same step as separate launches (mdx_stream_gemv + mdx_gdn_core_raw, whose
conv, gates and delta rule are checked against the float64 oracle in test_gdn_gpu.py), bit for bit:
the projections, the conv history, both step buffers, the gates (rows past R zeroed), the recurrent
state and the raw core rows, over three deferred steps (verify a tree, accept a path, replay it), for
1, 8 and 16 rows, faithful and integral weights, and a step whose pending list holds an invalid slot."""
import pytest
import torch

pytestmark = pytest.mark.gpu

HK, HV, DH, H = 16, 32, 128, 4096
NCH = 2 * HK * DH + HV * DH


def _state(gen, dev, slots):
    bf = lambda *s: torch.randn(*s, generator=gen, device=dev).bfloat16()
    return dict(conv=bf(NCH, 3), pb=bf(2, slots, NCH), qb=bf(2, slots, NCH),
                rec=torch.randn(HV, DH, DH, generator=gen, device=dev) * 0.1,
                gates=torch.rand(2, slots, HV, 2, generator=gen, device=dev),
                sums=torch.zeros(2, slots, HK, 2, device=dev))


@pytest.mark.parametrize("slots,widths,integral", [(8, (), False), (8, (), True), (8, (4, 3), False), (8, (1,) * 7, True),
                                                   (16, (4, 3, 2, 2, 2, 2), False), (16, (1,) * 15, True)])
def test_fold_matches_separate_launches(C, dev, slots, widths, integral):
    from mdx import _lib, hybrid
    from oracle import ref
    gen = torch.Generator(device=dev).manual_seed(7 + slots + len(widths))
    w_qkv = hybrid._gptq(NCH, H, gen, dev, integral)
    w_z = hybrid._gptq(HV * DH, H, gen, dev, integral)
    bf = lambda *s: torch.randn(*s, generator=gen, device=dev).bfloat16()
    wa, wb = bf(HV, H) * 0.02, bf(HV, H) * 0.02
    conv_w = bf(NCH, 4) * 0.5
    dt_bias = torch.rand(HV, generator=gen, device=dev) * 2 - 1
    g_decay = -torch.exp(torch.rand(HV, generator=gen, device=dev) * 1.5 - 1)
    nw = (1 + 0.02 * torch.randn(H, generator=gen, device=dev)).bfloat16()
    A = _state(gen, dev, slots)
    B = {k: v.clone() for k, v in A.items()}
    tree = ref.tree_from_spec(ref.spec_of_widths(widths), slots)
    R = 1 + sum(widths)
    parents = tree[0][:R] + [-1] * (slots - R)
    prog = ref.verify_program(tree[0][:R], R) + [0] * (slots - R)
    accepted, pending = [0] * slots, 0
    for step in range(4):
        p = step % 2
        if step == 3:  # an invalid pending list: nothing replayed or verified, the buffers still advance
            accepted, pending = [0, slots] + [0] * (slots - 2), 2
        print(f"case gdn fold slots={slots} R={R} integral={integral} step={step}", flush=True)
        ctl = torch.tensor([pending, p] + accepted + parents + prog, dtype=torch.int32, device=dev)
        x = bf(R, H)
        xn = torch.empty_like(x)
        q, s = C.rms_rot_quant(x, nw, 1e-6, _lib.ROT_NONE, None, xn_out=xn)
        outs = {}
        for name, st in (("fold", A), ("split", B)):
            proj, z = torch.empty(R, NCH, **dict(dtype=torch.bfloat16, device=dev)), torch.empty(R, HV * DH, dtype=torch.bfloat16, device=dev)
            core = torch.full((R, HV * DH), 7.0, dtype=torch.bfloat16, device=dev)
            if name == "fold":
                _lib.gemv_trace()
                zg = torch.empty_like(z)
                # one row: the row prep in the launch (x itself, no q / s / xn)
                C.gdn_proj(None if R == 1 else q, None if R == 1 else s, w_qkv, w_z, proj, z, None if R == 1 else xn, wa,
                           wb, conv_w, st["conv"], st["pb"], st["qb"], ctl, dt_bias, g_decay, st["gates"], HK, z_gate=zg,
                           x_row=x if R == 1 else None, norm_w=nw, eps=1e-6)
                tr = _lib.gemv_trace()
                assert len(tr) == 1 and tr[0]["gdn"] and tr[0]["decode"] == ("integral" if integral else "table16"), tr
                assert tr[0]["src"] == (_lib.SRC_XP if R == 1 else _lib.SRC_Q8), tr
                C.gdn_delta(st["qb"], ctl, st["rec"], st["gates"], DH ** -0.5, HK, core)
            else:
                C.stream_gemv(q, s, [w_qkv, w_z], [proj, z])
                C.gdn_core(proj, z, xn, wa, wb, conv_w, st["conv"], st["pb"], st["qb"], ctl, dt_bias, g_decay, st["rec"],
                           st["gates"], st["sums"], nw[:DH], 1e-6, DH ** -0.5, HK, core=core, raw=True)
            outs[name] = (proj, z, core)
        torch.cuda.synchronize()
        for i, what in enumerate(("proj", "z", "core")):
            assert torch.equal(outs["fold"][i], outs["split"][i]), f"{what} step {step}"
        for k in ("conv", "pb", "qb", "rec", "gates"):
            assert torch.equal(A[k], B[k]), f"{k} step {step}"
        # the gate factors: bf16(z / (1 + e^-z)) of the z outputs, within an ulp of torch's (the library's
        # own expf), and exactly what the gated RMSNorm takes (test_gnorm_linear_matches_prep_then_gemv)
        zf = outs["split"][1].float()
        assert (zg.float() - (zf * torch.sigmoid(zf)).bfloat16().float()).abs().max() <= 2 ** -7 * zf.abs().max() + 1e-6
        if step < 3:
            assert not A["gates"][p, R:].any(), "gates of rows past R"
        # accept a path of the tree for the next step: the chain, cut at a depth that varies by step
        chain = [0]
        while len(chain) < R:
            kids = [r for r in range(R) if parents[r] == chain[-1]]
            if not kids:
                break
            chain.append(kids[0])
        pending = 1 + (step * 3) % len(chain)
        accepted = chain[:pending] + [0] * (slots - pending)


def _projected_z(C, dev, gen, rows):
    """z outputs of a projection launch (mdx_gdn_proj) over random weights and their gate factors."""
    from mdx import _lib, hybrid
    slots = 8 if rows <= 8 else 16
    w_qkv, w_z = hybrid._gptq(NCH, H, gen, dev), hybrid._gptq(HV * DH, H, gen, dev)
    bf = lambda *s: torch.randn(*s, generator=gen, device=dev).bfloat16()
    st = _state(gen, dev, slots)
    x = bf(rows, H)
    xn = torch.empty_like(x)
    q, s = C.rms_rot_quant(x, torch.ones(H, dtype=torch.bfloat16, device=dev), 1e-6, _lib.ROT_NONE, None, xn_out=xn)
    ctl = torch.tensor([0, 0] + [0] * slots + [r - 1 for r in range(rows)] + [-1] * (slots - rows) + [r | 32 for r in range(rows)]
                       + [0] * (slots - rows), dtype=torch.int32, device=dev)
    proj = torch.empty(rows, NCH, dtype=torch.bfloat16, device=dev)
    z, zg = torch.empty(rows, HV * DH, dtype=torch.bfloat16, device=dev), torch.empty(rows, HV * DH, dtype=torch.bfloat16, device=dev)
    C.gdn_proj(q, s, w_qkv, w_z, proj, z, xn, bf(HV, H) * 0.02, bf(HV, H) * 0.02, bf(NCH, 4), st["conv"], st["pb"], st["qb"],
               ctl, torch.zeros(HV, device=dev), -torch.ones(HV, device=dev), st["gates"], HK, z_gate=zg)
    return z, zg


def test_fold_rejects_bad_shapes(C, dev):
    from mdx import hybrid
    gen = torch.Generator(device=dev).manual_seed(3)
    w_qkv = hybrid._gptq(NCH, H, gen, dev)
    w_z = hybrid._gptq(HV * DH + 16, H, gen, dev)  # z must be HV x 128 wide
    st = _state(gen, dev, 8)
    q = torch.zeros(1, H, dtype=torch.int8, device=dev)
    s = torch.ones(1, device=dev)
    bf = lambda *sh: torch.zeros(*sh, dtype=torch.bfloat16, device=dev)
    ctl = torch.tensor([0, 0] + [0] * 8 + [-1] * 8 + [32] + [0] * 7, dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError):
        C.gdn_proj(q, s, w_qkv, w_z, bf(1, NCH), bf(1, HV * DH + 16), bf(1, H), bf(HV, H), bf(HV, H), bf(NCH, 4),
                   st["conv"], st["pb"], st["qb"], ctl, torch.zeros(HV, device=dev), torch.zeros(HV, device=dev),
                   st["gates"], HK)


@pytest.mark.parametrize("rows,integral,gated", [(1, False, True), (2, False, False), (1, True, False), (2, True, True),
                                                 (3, False, True), (8, True, False)])
def test_gnorm_linear_matches_prep_then_gemv(C, dev, rows, integral, gated):
    """mdx_gnorm_linear (the gated RMSNorm + quantisation in the out_proj's prologue at one or two rows;
    two launches above) against mdx_gnorm_rot_quant then mdx_stream_gemv, bit for bit: the output with its
    residual, the normalised rows; the trace names the gated-norm source where it applies. gated: z given
    as the gate factors mdx_gdn_proj stores (z_gate of a projection launch whose z is z)."""
    from mdx import _lib, hybrid
    print(f"case gnorm_linear rows={rows} integral={integral}", flush=True)
    gen = torch.Generator(device=dev).manual_seed(11 + rows)
    w = hybrid._gptq(H, HV * DH, gen, dev, integral)
    bf = lambda *s: torch.randn(*s, generator=gen, device=dev).bfloat16()
    y, z, res = bf(rows, HV * DH), bf(rows, HV * DH), bf(rows, H)
    zin = z
    if gated:  # z and its gate factors from one projection launch
        z, zin = _projected_z(C, dev, gen, rows)
    y[0, :DH] = 0  # a head of zeros (rsq of eps alone)
    gnw = (1 + 0.1 * torch.randn(DH, generator=gen, device=dev)).bfloat16()
    q = torch.empty(rows, HV * DH, dtype=torch.int8, device=dev)
    s = torch.empty(rows, device=dev)
    yn, out = torch.empty_like(y), torch.empty(rows, H, dtype=torch.bfloat16, device=dev)
    _lib.gemv_trace()
    C.gnorm_linear(y, zin, gnw, 1e-6, w, out, residual=res, y_out=yn, q=q, scale=s, z_gated=gated)
    tr = _lib.gemv_trace()
    assert len(tr) == 1 and (tr[0]["src"] == _lib.SRC_GN) == (rows <= 2), tr
    yw = torch.empty_like(y)
    q2, s2 = torch.empty_like(q), torch.empty_like(s)
    _lib.call("mdx_gnorm_rot_quant", _lib.ptr(y), _lib.ptr(z), _lib.ptr(gnw), 1e-6, _lib.ptr(yw), None, _lib.ROT_NONE,
              _lib.ptr(q2), _lib.ptr(s2), rows, HV * DH, _lib.stream_of(y))
    want = torch.empty_like(out)
    C.stream_gemv(q2, s2, [w], [want], residuals=[res])
    torch.cuda.synchronize()
    assert torch.equal(yn, yw), "normalised rows"
    assert torch.equal(out, want), "out_proj output"
