"""rope_kv / qk_norm_rope_kv and the MTP loop bookkeeping on the GPU against the CPU oracle, bit for
bit. Reference tests mirrored: tests/test_rope_kv.py, tests/test_mtp_accept.py."""
import random

import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits
from oracle import ref

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=torch.bfloat16):
    if dtype == torch.bfloat16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("D,rd,Hq,Hk", [(256, 64, 16, 4), (128, 128, 32, 8), (128, 32, 32, 8), (64, 64, 4, 2)])
def test_rope_kv_matches_oracle(C, dev, D, rd, Hq, Hk):
    g = torch.Generator().manual_seed(D + rd)
    cap = 64
    for t in range(12):
        S = (1, 3, 8, 16)[t % 4]
        qn = (torch.randn(S, Hq, D, generator=g) * torch.exp(torch.randn(S, Hq, D, generator=g) * 2)).bfloat16()
        kn = (torch.randn(S, Hk, D, generator=g) * 30).bfloat16()
        vn = torch.randn(S, Hk, D, generator=g).bfloat16()
        f = torch.randn(S, rd // 2, 2, 2, generator=g)
        pos = torch.randperm(cap, generator=g)[:S]
        key = torch.randn(1, Hk, cap, D, generator=g).bfloat16()
        val = torch.randn(1, Hk, cap, D, generator=g).bfloat16()
        wq, wk, ek, ev = ref.rope_kv(bits(qn), bits(kn), bits(vn), f.numpy(), bits(key)[0], bits(val)[0],
                                     pos.numpy(), rd)
        kd, vd = key.to(dev), val.to(dev)
        q, k = C.rope_kv(qn.to(dev), kn.to(dev), vn.to(dev), f.to(dev), kd, vd, pos.to(dev), rd)
        assert q.shape == (1, Hq, S, D) and k.shape == (1, Hk, S, D)
        assert_bits_equal(bits(q)[0], wq, f"q S={S}")
        assert_bits_equal(bits(k)[0], wk, f"k S={S}")
        assert_bits_equal(bits(kd)[0], ek, "key cache")
        assert_bits_equal(bits(vd)[0], ev, "value cache")


@pytest.mark.parametrize("D", [128, 256])
def test_qk_norm_rope_kv_matches_oracle(C, dev, D):
    g = torch.Generator().manual_seed(211 + D)
    for i in range(36):
        S = (1, 3, 8, 16)[i % 4]
        Hq, Hk = ((16, 4), (4, 2), (32, 8))[(i // 4) % 3]
        rd = (64, D)[(i // 12) % 2]
        kind = i % 3 if i < 24 else 3
        qg = torch.randn(1, S, Hq, 2 * D, generator=g)
        k = torch.randn(1, S, Hk, D, generator=g)
        if kind == 1:
            qg *= torch.exp(torch.randn(qg.shape, generator=g) * 2)
            k *= 30
        elif kind == 2:
            qg *= 1e-4
            k *= 1e-4
        elif kind == 3:
            qg.zero_()
            qg[..., ::2] = -0.0
            k.zero_()
            k[..., ::2] = -0.0
        qg, k = qg.bfloat16(), k.bfloat16()
        gated = i % 2 == 0
        q = qg[..., :D] if gated else qg[..., :D].contiguous()
        v = torch.randn(k.shape, generator=g).bfloat16()
        wq = (1 + torch.randn(D, generator=g) * .3).bfloat16()
        wk = (1 + torch.randn(D, generator=g) * .3).bfloat16()
        f = torch.randn(S, rd // 2, 2, 2, generator=g)
        pos = torch.randperm(64, generator=g)[:S]
        key = torch.randn(1, Hk, 64, D, generator=g).bfloat16()
        val = torch.randn(1, Hk, 64, D, generator=g).bfloat16()
        wantq, wantk, ek, ev = ref.rope_kv(bits(q)[0], bits(k)[0], bits(v)[0], f.numpy(), bits(key)[0],
                                           bits(val)[0], pos.numpy(), rd, bits(wq), bits(wk), 1e-6, 2e-5)
        qd = qg.to(dev)[..., :D] if gated else q.to(dev)
        kd, vd = key.to(dev), val.to(dev)
        oq, ok = C.qk_norm_rope_kv(qd, k.to(dev), v.to(dev), wq.to(dev), wk.to(dev), f.to(dev), kd, vd,
                                   pos.to(dev), 1e-6, 2e-5, rd)
        assert_bits_equal(bits(oq)[0], wantq, f"q case {i}")
        assert_bits_equal(bits(ok)[0], wantk, f"k case {i}")
        assert_bits_equal(bits(kd)[0], ek, f"key case {i}")
        assert_bits_equal(bits(vd)[0], ev, f"value case {i}")


def test_rope_contract_rejects(C, dev):
    S, H, D = 2, 2, 128
    x = torch.zeros(S, H, D, dtype=torch.bfloat16, device=dev)
    key = torch.zeros(1, H, 8, D, dtype=torch.bfloat16, device=dev)
    pos = torch.arange(S, device=dev)
    with pytest.raises(RuntimeError):
        C.rope_kv(x, x, x, torch.zeros(S, 16, 2, 2, device=dev), key, key.clone(), pos, 33)  # odd rd
    with pytest.raises(RuntimeError):
        y = torch.zeros(S, H, 96, dtype=torch.bfloat16, device=dev)  # head_dim 96
        C.rope_kv(y, y, y, torch.zeros(S, 16, 2, 2, device=dev), torch.zeros(1, H, 8, 96, dtype=torch.bfloat16,
                  device=dev), torch.zeros(1, H, 8, 96, dtype=torch.bfloat16, device=dev), pos, 32)


SPECS8 = [ref.spec_of_widths(w) for w in ((4, 3), (7,), (1, 1, 1, 1, 1, 1, 1), (2, 2, 3), (3, 1, 1, 2))] + \
         [[[[[[]], []], []], []], [[[[[]]]]]]
SPECS16 = [ref.spec_of_widths(w) for w in ((4, 3, 2, 2, 2), (8, 4), (2,) * 7, (1,) * 15, (5, 5, 3))]


def _children_table(children, slots):
    ch = np.full((slots, slots), -1, np.int32)
    for r, cs in enumerate(children[:slots]):
        for j, c in enumerate(cs):
            ch[r, j] = c
    return ch.reshape(-1)


@pytest.mark.parametrize("slots,spec_index", [(8, i) for i in range(len(SPECS8))] +
                         [(16, i) for i in range(len(SPECS16))])
def test_mtp_accept_matches_oracle(C, dev, slots, spec_index):
    spec = (SPECS8 if slots == 8 else SPECS16)[spec_index]
    rng = random.Random(1000 + 31 * slots + spec_index)
    parent, children, depth_of, chain = ref.tree_from_spec(spec, slots)
    rows = slots
    Hd, HK, CAP, D = 64, 4, 96, 128
    ch = torch.from_numpy(_children_table(children, slots)).to(dev)
    for trial in range(20):
        toks = [rng.randrange(50) for _ in range(rows)]
        dr = [rng.randrange(50) for _ in range(rows)]
        for r in range(rows):
            if children[r] and rng.random() < 0.8:
                dr[rng.choice(children[r])] = toks[r]
        nc = 7 * max(chain, 7)
        cand = [rng.randrange(50) for _ in range(nc)]
        for node in range(chain):
            if rng.random() < 0.7:
                cand[7 * node + rng.randrange(7)] = toks[node]
        use_cand = trial % 4 != 3
        pos, mtp_pos = rng.randrange(0, 90), rng.randrange(0, 30)
        path, commit, ranks, row, on_chain, kept = ref.accept_walk(children, toks, dr, chain,
                                                                   cand if use_cand else None)
        st = torch.tensor([pos, mtp_pos, 0, 0], dtype=torch.long, device=dev)
        x = torch.randn(1, rows, Hd).bfloat16().to(dev)
        nt = torch.empty(1, 1, dtype=torch.long, device=dev)
        hb = torch.empty(1, 1, Hd, dtype=torch.bfloat16, device=dev)
        ctl = torch.zeros(2 + 3 * slots, dtype=torch.int32, device=dev)
        keys = [torch.randn(1, HK, CAP, D).bfloat16().to(dev) for _ in range(4)]
        before = [bits(k)[0] for k in keys]
        ptrs = torch.tensor([p - (1 << 64) if p >= (1 << 63) else p for p in (k.data_ptr() for k in keys)],
                            dtype=torch.long, device=dev)
        result = torch.zeros(slots + 24, dtype=torch.long, device=dev)
        t_cand = torch.tensor(cand, dtype=torch.long, device=dev).view(-1, 7) if use_cand else \
            torch.empty(0, dtype=torch.long, device=dev)
        C.mtp_accept(st, torch.tensor([toks], dtype=torch.long, device=dev),
                     torch.tensor([dr], dtype=torch.long, device=dev), t_cand, ch, rows, chain, x, nt, hb, ctl,
                     ptrs, HK, CAP, D, result)
        want = ref.accept_record(slots, path, commit, ranks, row, on_chain, kept, pos)
        got = result.tolist()
        assert got[:len(want)] == want, (trial, got, want)
        assert st.tolist() == [pos + len(path), mtp_pos + kept, 0, 0]
        c = ctl.tolist()
        assert c[0] == len(path) and c[2:2 + slots] == path + list(range(len(path), slots))
        assert nt.item() == toks[row] and torch.equal(hb.view(-1), x[0, row])
        for k_before, k_after in zip(before, keys):
            assert_bits_equal(bits(k_after)[0], ref.commit_path(k_before, path, on_chain, pos), f"kv trial {trial}")


@pytest.mark.parametrize("slots", [8, 16])
def test_mtp_prep_matches_host_prepare(C, dev, slots):
    st = torch.tensor([37, 11, 0, 0], dtype=torch.long, device=dev)
    ftab = torch.randn(1, 1, 64, 32, 2, 2, device=dev)
    freqs = torch.empty(1, 1, 1, 32, 2, 2, device=dev)
    mpos, mseq = torch.empty(slots, dtype=torch.long, device=dev), torch.empty(1, dtype=torch.int32, device=dev)
    C.mtp_prep_draft(st, 2, ftab, freqs, mpos, mseq)
    assert torch.equal(freqs, ftab[:, :, 39:40]) and mpos.tolist() == list(range(13, 13 + slots))
    assert mseq.item() == 14
    # past the table's end the last row is used
    C.mtp_prep_draft(st, 40, ftab, freqs, mpos, mseq)
    assert torch.equal(freqs, ftab[:, :, 63:64])
    apos, aseq = torch.empty(slots, dtype=torch.long, device=dev), torch.empty(1, dtype=torch.int32, device=dev)
    tpos = torch.tensor(([0, 1, 2, 3, 4, 1, 2, 1] * 2)[:slots], dtype=torch.long, device=dev)
    vpos = torch.empty(1, slots, dtype=torch.long, device=dev)
    ctl = torch.zeros(2 + 3 * slots, dtype=torch.int32, device=dev)
    tctl = torch.arange(100, 100 + 2 * slots, dtype=torch.int32, device=dev)
    C.mtp_prep_verify(st, apos, aseq, vpos, tpos, ctl, tctl, 1, 5)
    assert apos.tolist() == list(range(37, 37 + slots)) and aseq.item() == 37
    assert vpos.view(-1).tolist() == [37 + 5 + d for d in tpos.tolist()]
    assert ctl.tolist()[1] == 1 and ctl.tolist()[2 + slots:] == list(range(100, 100 + 2 * slots))
    assert ctl.tolist()[0] == 0 and ctl.tolist()[2:2 + slots] == [0] * slots


@pytest.mark.parametrize("slots,rows", [(8, 8), (16, 16), (8, 3)])
def test_mtp_prep_verify_rows_matches_ops(C, dev, slots, rows):
    """mtp_prep_verify_rows (one launch) against mtp_prep_verify, the root token's copy and the two
    index_select gathers of the verify rows, bit for bit; a position past the RoPE table reads its last
    row."""
    print(f"case prep_verify_rows slots={slots} rows={rows}", flush=True)
    g = torch.Generator(device=dev).manual_seed(slots + rows)
    V, Hd, P = 5000, 4096, 96
    embed = torch.randn(V, Hd, generator=g, device=dev).bfloat16()
    ftab = torch.randn(P, 32, 2, 2, generator=g, device=dev)
    st = torch.tensor([60, 3, 0, 0], dtype=torch.long, device=dev)
    tpos = torch.tensor(([0, 1, 2, 3, 4, 1, 2, 1] * 2)[:rows], dtype=torch.long, device=dev)
    tctl = torch.arange(100, 100 + 2 * slots, dtype=torch.int32, device=dev)
    nt = torch.tensor([4321], dtype=torch.long, device=dev)
    outs = []
    for fused in (True, False):
        apos, aseq = torch.empty(slots, dtype=torch.long, device=dev), torch.empty(1, dtype=torch.int32, device=dev)
        vpos = torch.empty(1, rows, dtype=torch.long, device=dev)
        ctl = torch.zeros(2 + 3 * slots, dtype=torch.int32, device=dev)
        vtok = torch.randint(0, V, (1, rows), generator=torch.Generator(device=dev).manual_seed(1), device=dev)
        x = torch.empty(rows, Hd, dtype=torch.bfloat16, device=dev)
        vf = torch.empty(rows, 32, 2, 2, device=dev)
        if fused:
            C.mtp_prep_verify_rows(st, apos, aseq, vpos, tpos, ctl, tctl, 1, 34, nt, vtok, embed, ftab, x, vf)
        else:
            vtok[0, 0:1].copy_(nt)
            C.mtp_prep_verify(st, apos, aseq, vpos, tpos, ctl, tctl, 1, 34)
            torch.index_select(ftab, 0, vpos.view(-1).clamp(max=P - 1), out=vf)
            torch.index_select(embed, 0, vtok.view(-1), out=x)
        outs.append((apos, aseq, vpos, ctl, vtok, x, vf))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert outs[0][2].view(-1).max().item() >= P  # some positions ran past the table (clamped to its last row)
