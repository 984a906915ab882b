"""Gated-DeltaNet core on the GPU against the float64 oracle over two deferred steps (verify a tree,
accept a path, replay it next step): the core rows and the committed recurrent state within the
bound of the reference's attention / GDN tests (max <= 1.5 x e_ref.max + 1e-3, mean <= 1.5 x
e_ref.mean + 1e-5, e_ref = the float32 chain's error), the control path exact (conv history, the
projection buffer of the next step, which rows are produced)."""
import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits
from oracle import ref

pytestmark = pytest.mark.gpu

HK, HV, DH = 16, 32, 128
NCH = 2 * HK * DH + HV * DH


def _bf(a):
    return ref.bf16_to_f32(ref.f32_to_bf16(np.asarray(a, np.float32)))


def _tensor(a, dev, dt=torch.bfloat16):
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    return t.to(dt).to(dev)


def _bound(got, want, chain, what):
    e_ref = np.abs(chain - want)
    err = np.abs(got - want)
    assert err.max() <= 1.5 * e_ref.max() + 1e-3, (what, err.max(), e_ref.max())
    assert err.mean() <= 1.5 * e_ref.mean() + 1e-5, (what, err.mean(), e_ref.mean())


@pytest.mark.parametrize("slots,widths", [(8, (4, 3)), (8, (1,) * 7), (16, (4, 3, 2, 2, 2)), (8, (1,)), (8, ())])
def test_gdn_two_steps_match_f64(C, dev, slots, widths):
    rng = np.random.default_rng(40 + slots + len(widths))
    conv_w = _bf(rng.standard_normal((NCH, 4)) * 0.5)
    dt_bias = rng.uniform(-1, 1, HV).astype(np.float32)
    g_decay = (-np.exp(rng.uniform(-1, 0.5, HV))).astype(np.float32)
    gnw = _bf(1 + rng.standard_normal(DH) * 0.1)
    wa = _bf(rng.standard_normal((HV, 4096)) * 0.02)
    wb = _bf(rng.standard_normal((HV, 4096)) * 0.02)
    eps, qscale = 1e-6, DH ** -0.5
    st64 = dict(conv_state=_bf(rng.standard_normal((NCH, 3))), pb=np.zeros((2, slots, NCH), np.float32),
                qb=np.zeros((2, slots, NCH), np.float32),
                rec=(rng.standard_normal((HV, DH, DH)) * 0.1).astype(np.float32),
                gates=np.zeros((2, slots, HV, 2), np.float32), sums=np.zeros((2, slots, HK, 2), np.float32))
    st32 = {k: v.copy() for k, v in st64.items()}
    d = {k: _tensor(v, dev, torch.bfloat16 if k in ("conv_state", "pb", "qb") else torch.float32)
         for k, v in st64.items()}
    tree = ref.tree_from_spec(ref.spec_of_widths(widths), slots)
    R = 1 + sum(widths)
    parents = tree[0][:R] + [-1] * (slots - R)
    prog = ref.verify_program(tree[0][:R], R) + [0] * (slots - R)
    accepted = [0] * slots
    pending = 0
    for step in range(2):
        p = step % 2
        print(f"case gdn slots={slots} widths={widths} R={R} step={step}", flush=True)
        ctl = [pending, p] + accepted + parents + prog
        proj = _bf(rng.standard_normal((R, NCH)))
        z = _bf(rng.standard_normal((R, HV * DH)))
        xn = _bf(rng.standard_normal((R, 4096)))
        xb, wab, wbb = ref.f32_to_bf16(xn), ref.f32_to_bf16(wa), ref.f32_to_bf16(wb)
        args = (conv_w, dt_bias, g_decay, gnw, eps, qscale, np.array(ctl), R, HK, slots)
        a64, b64 = ref.gdn_ab(xb, wab, wbb)
        a32, b32 = ref.gdn_ab(xb, wab, wbb, np.float32)
        c64 = ref.gdn_step(st64, proj, z, a64, b64, *args[:6], args[6], R, HK, slots)
        c32 = ref.gdn_step(st32, proj, z, a32, b32, *args[:6], args[6], R, HK, slots, dtype=np.float32)
        core = C.gdn_core(_tensor(proj, dev), _tensor(z, dev), _tensor(xn, dev), _tensor(wa, dev), _tensor(wb, dev),
                          _tensor(conv_w, dev),
                           d["conv_state"], d["pb"], d["qb"], torch.tensor(ctl, dtype=torch.int32, device=dev),
                           _tensor(dt_bias, dev, torch.float32), _tensor(g_decay, dev, torch.float32), d["rec"],
                           d["gates"], d["sums"], _tensor(gnw, dev), eps, qscale, HK)
        got = core.float().cpu().numpy()
        _bound(got, c64, c32, f"core step {step}")
        # exact control: the conv history and the projection buffer of the next step
        assert_bits_equal(bits(d["conv_state"]), ref.f32_to_bf16(st64["conv_state"]), f"conv state {step}")
        assert_bits_equal(bits(d["pb"])[p], ref.f32_to_bf16(st64["pb"][p]), f"proj buffer {step}")
        _bound(d["rec"].cpu().numpy(), st64["rec"], st32["rec"], f"state step {step}")
        # accept a path of the tree for the next step: the chain, cut at a random depth
        chain = [0]
        while len(chain) < R:
            kids = [r for r in range(R) if parents[r] == chain[-1]]
            if not kids:
                break
            chain.append(kids[0])
        n = int(rng.integers(1, len(chain) + 1))
        pending = n
        accepted = chain[:n] + [0] * (slots - n)


def test_gdn_first_step_without_history_rows(C, dev):
    """pending = 0 leaves the recurrent state untouched (nothing replayed)."""
    rng = np.random.default_rng(1)
    slots, R = 8, 3
    rec = torch.randn(HV, DH, DH, device=dev) * 0.1
    before = rec.clone()
    ctl = torch.tensor([0, 0] + [0] * 8 + [-1, 0, 1] + [-1] * 5 + [32, 33, 2] + [0] * 5, dtype=torch.int32, device=dev)
    bf = lambda *s: torch.randn(*s, device=dev).bfloat16()
    C.gdn_core(bf(R, NCH), bf(R, HV * DH), bf(R, 4096), bf(HV, 4096), bf(HV, 4096), bf(NCH, 4), bf(NCH, 3), torch.zeros(2, slots, NCH, dtype=torch.bfloat16,
                device=dev), torch.zeros(2, slots, NCH, dtype=torch.bfloat16, device=dev), ctl,
                torch.zeros(HV, device=dev), -torch.ones(HV, device=dev), rec, torch.zeros(2, slots, HV, 2, device=dev),
                torch.zeros(2, slots, HK, 2, device=dev), torch.ones(DH, device=dev).bfloat16(), 1e-6, DH ** -0.5, HK)
    assert torch.equal(rec, before)


@pytest.mark.parametrize("bad", [-1, 8])
def test_gdn_invalid_accepted_slot_replays_nothing(C, dev, bad):
    """A pending list with an out-of-range slot: nothing is replayed or verified (the state and the
    outputs stay as they are, csrc/mono_gdn.sycl:398-407,568); the conv history reads the slot clamped
    into range, as the oracle does."""
    print(f"case gdn invalid slot {bad}", flush=True)
    rng = np.random.default_rng(60 + bad)
    slots = 8
    tree = ref.tree_from_spec(ref.spec_of_widths((4, 3)), slots)
    R = 8
    parents = tree[0][:R]
    ctl = [3, 0] + [0, bad, 2] + [0] * (slots - 3) + parents + ref.verify_program(parents, R)
    conv_w = _bf(rng.standard_normal((NCH, 4)) * 0.5)
    st = dict(conv_state=_bf(rng.standard_normal((NCH, 3))), pb=_bf(rng.standard_normal((2, slots, NCH))),
              qb=_bf(rng.standard_normal((2, slots, NCH))), rec=(rng.standard_normal((HV, DH, DH)) * 0.1).astype(np.float32),
              gates=rng.uniform(0.1, 0.9, (2, slots, HV, 2)).astype(np.float32),
              sums=rng.uniform(0.5, 2, (2, slots, HK, 2)).astype(np.float32))
    d = {k: _tensor(v, dev, torch.bfloat16 if k in ("conv_state", "pb", "qb") else torch.float32) for k, v in st.items()}
    rec0 = d["rec"].clone()
    proj, z, xn = (_bf(rng.standard_normal(s_)) for s_ in ((R, NCH), (R, HV * DH), (R, 4096)))
    wa, wb = (_bf(rng.standard_normal((HV, 4096)) * 0.02) for _ in range(2))
    dt_bias = rng.uniform(-1, 1, HV).astype(np.float32)
    g_decay = (-np.exp(rng.uniform(-1, 0.5, HV))).astype(np.float32)
    gnw = _bf(1 + rng.standard_normal(DH) * 0.1)
    core = C.gdn_core(_tensor(proj, dev), _tensor(z, dev), _tensor(xn, dev), _tensor(wa, dev), _tensor(wb, dev),
                      _tensor(conv_w, dev), d["conv_state"], d["pb"], d["qb"], torch.tensor(ctl, dtype=torch.int32, device=dev),
                      _tensor(dt_bias, dev, torch.float32), _tensor(g_decay, dev, torch.float32), d["rec"], d["gates"],
                      d["sums"], _tensor(gnw, dev), 1e-6, DH ** -0.5, HK)
    assert torch.equal(d["rec"], rec0)
    assert not core.float().abs().sum().item()
    want = ref.gdn_step(st, proj, z, *ref.gdn_ab(ref.f32_to_bf16(xn), ref.f32_to_bf16(wa), ref.f32_to_bf16(wb)), conv_w,
                        dt_bias, g_decay, gnw, 1e-6, DH ** -0.5, np.array(ctl), R, HK, slots)
    assert not want.any()
    assert_bits_equal(bits(d["conv_state"]), ref.f32_to_bf16(st["conv_state"]), "conv history")
