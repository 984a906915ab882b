"""The draft pick (second stage of the two-stage draft lm_head) on the GPU.

int8 head (the reference's contract, csrc/draft_lmhead.sycl:82-291): against the oracle's exact int8
logits and torch XPU topk / argmax order, with approximate scores that are exact, noisy or tie-heavy --
the cases of the reference's own test (tests/test_draft_lmhead.py:11-61: N 60000, K 1024, the strongest
rows duplicated across the vocabulary for exact ties, noise 1-2% of the largest logit), plus the real
vocabulary size at K 4096 and the exact-scores mode (no weight).

bf16 head (this library's own form): the two-stage result -- int4 scoring copy through the W4A8 GEMV,
then the pick -- equals the one-stage head (bf16_linear + fast_topk) bit for bit, indices and values."""
import numpy as np
import pytest
import torch

from conftest import bits
from oracle import ref

pytestmark = pytest.mark.gpu


def _case(N, K, seed, ties):
    g = torch.Generator().manual_seed(seed)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = torch.rand(N, generator=g) * 1e-3 + 1e-4
    qx = torch.randint(-127, 128, (K,), generator=g, dtype=torch.int8)
    if ties:  # the strongest rows duplicated across the vocabulary: exact ties at the top
        acc0 = (w.long() * qx.long()).sum(-1)
        for j, r in enumerate(acc0.topk(4).indices.tolist()):
            for d in range(1, 4):
                dst = (r + d * 12347 + j * 999) % N
                w[dst], sw[dst] = w[r], sw[r]
    sx = torch.rand(1, generator=g) * 0.05 + 0.01
    exact = ref.int8_head_logits(qx.numpy(), sx.numpy(), w.numpy(), sw.numpy())
    return w, sw, qx, sx, exact


@pytest.mark.parametrize("N,K,seed,ties,noise", [(60000, 1024, 1, False, 0.0), (60000, 1024, 2, False, 0.02),
                                                 (60000, 1024, 3, True, 0.0), (60000, 1024, 4, True, 0.01),
                                                 (151936, 4096, 5, False, 0.01)])
def test_draft_pick_int8_matches_oracle(C, dev, N, K, seed, ties, noise):
    print(f"case pick int8 N={N} K={K} seed={seed} ties={ties} noise={noise}", flush=True)
    w, sw, qx, sx, exact = _case(N, K, seed, ties)
    ef = ref.bf16_to_f32(exact)
    g = torch.Generator().manual_seed(seed + 100)
    approx = torch.from_numpy(ef + noise * np.abs(ef).max() * torch.randn(N, generator=g).numpy()).bfloat16()
    wd, swd, qxd, sxd, ad = w.to(dev), sw.to(dev), qx.to(dev), sx.to(dev), approx.to(dev)
    calls = torch.zeros(1, dtype=torch.long, device=dev)
    rows = 8
    for nout, amf, children in ((7, False, [1, 2, 5]), (3, True, [3, 4, 6]), (1, True, [2]), (8, False, list(range(8)))):
        top = torch.full((8,), -1, dtype=torch.long, device=dev)
        ranks = torch.full((8,), -1, dtype=torch.long, device=dev)
        token = torch.full((1,), -1, dtype=torch.long, device=dev)
        vtok = torch.full((rows,), -1, dtype=torch.long, device=dev)
        C.draft_pick(ad, qxd, sxd, wd, swd, nout, amf, top, ranks, token, vtok, children, calls)
        wtop, wtok, wvtok = ref.draft_pick(exact, nout, amf, children, rows)
        assert top.tolist()[:nout] == wtop.tolist() and ranks.tolist()[:nout] == wtop.tolist(), (nout, amf)
        assert top.tolist()[nout:] == [-1] * (8 - nout)
        assert token.item() == wtok
        assert vtok.tolist() == wvtok.tolist()
    assert calls.item() == 4
    if noise == 0.0:
        # the scores are the logits (no weight): a top-n pick with the outputs, no recompute
        e8 = torch.empty(0, dtype=torch.int8, device=dev)
        ef32 = torch.empty(0, dtype=torch.float32, device=dev)
        exd = torch.from_numpy(exact.view(np.int16)).view(torch.bfloat16).to(dev)
        top = torch.full((7,), -1, dtype=torch.long, device=dev)
        token = torch.full((1,), -1, dtype=torch.long, device=dev)
        vtok = torch.full((8,), -1, dtype=torch.long, device=dev)
        C.draft_pick(exd, e8, ef32, e8, ef32, 7, False, top, top[:0], token, vtok, [1, 2], None)
        wtop, wtok, _ = ref.draft_pick(exact, 7, False, [1, 2], 8)
        assert top.tolist() == wtop.tolist() and token.item() == wtok


@pytest.mark.parametrize("N,tiled", [(151936, True), (32768, False)])
def test_draft_pick_bf16_equals_one_stage_head(C, dev, N, tiled):
    """Two-stage (int4 scores + pick) against bf16_linear + fast_topk on the same head and rows."""
    from mdx import layout
    K = 4096
    g = torch.Generator(device=dev).manual_seed(N)
    w = (torch.randn(N, K, generator=g, device=dev) * 0.02).bfloat16()
    wt = layout.tile_major_bf16(w) if tiled else w
    lm4 = layout.int4_scoring_copy(w)
    for trial in range(6):
        print(f"case pick bf16 N={N} tiled={tiled} trial={trial}", flush=True)
        x = torch.randn(1, K, generator=g, device=dev).bfloat16()
        if trial == 5:  # a row that makes many logits tie (coarse values)
            x = (torch.round(x.float() * 4) / 4).bfloat16()
        q, s = C.quant_rows(x)
        approx = torch.empty(1, N, dtype=torch.bfloat16, device=dev)
        C.stream_gemv(q, s.view(-1), [lm4], [approx])
        logits = C.bf16_linear(x, wt, tiled=tiled)
        for nout, amf in ((4, False), (3, False), (8, True)):
            wv, wi = C.fast_topk(logits, nout, False)
            top = torch.full((nout,), -1, dtype=torch.long, device=dev)
            vals = torch.zeros(nout, dtype=torch.bfloat16, device=dev)
            token = torch.full((1,), -1, dtype=torch.long, device=dev)
            vtok = torch.full((8,), -1, dtype=torch.long, device=dev)
            children = list(range(1, nout + 1)) if nout < 8 else list(range(8))
            C.draft_pick_bf16(approx.view(-1), x.view(-1), wt, nout, amf, top, vals, token, vtok, children, tiled=tiled)
            assert top.tolist() == wi.view(-1).tolist(), (trial, nout)
            assert torch.equal(vals.view(torch.int16), wv.view(-1).view(torch.int16)), (trial, nout)
            want_tok = C.fast_topk(logits, 1, True)[1].item() if amf else wi.view(-1)[0].item()
            assert token.item() == want_tok
            assert vtok[children[0]].item() == want_tok
            for j, c in enumerate(children[1:], 1):
                assert vtok[c].item() == wi.view(-1)[j].item()


@pytest.mark.parametrize("tiled", [False, True])
def test_draft_pick_bf16_odd_k(C, dev, tiled):
    """K = 1056 (33 chunks of 32, split into 3 K slices at N = 32768; rows gathered in the MFMA operand
    layout): the pick against bf16_linear + fast_topk, with the scores the logits themselves and the
    logits plus a small perturbation."""
    from mdx import layout
    N, K = 32768, 1056
    g = torch.Generator(device=dev).manual_seed(K)
    w = (torch.randn(N, K, generator=g, device=dev) * 0.03).bfloat16()
    wt = layout.tile_major_bf16(w) if tiled else w
    for trial in range(3):
        print(f"case pick bf16 odd K={K} tiled={tiled} trial={trial}", flush=True)
        x = torch.randn(1, K, generator=g, device=dev).bfloat16()
        logits = C.bf16_linear(x, wt, tiled=tiled)
        approx = logits.view(-1).clone() if trial == 0 else (
            logits.view(-1).float() + 0.002 * torch.randn(N, generator=g, device=dev)).bfloat16()
        for nout, amf in ((4, False), (8, True)):
            wv, wi = C.fast_topk(logits, nout, False)
            top = torch.full((nout,), -1, dtype=torch.long, device=dev)
            vals = torch.zeros(nout, dtype=torch.bfloat16, device=dev)
            token = torch.full((1,), -1, dtype=torch.long, device=dev)
            vtok = torch.full((8,), -1, dtype=torch.long, device=dev)
            children = list(range(1, nout + 1)) if nout < 8 else list(range(8))
            C.draft_pick_bf16(approx, x.view(-1), wt, nout, amf, top, vals, token, vtok, children, tiled=tiled)
            assert top.tolist() == wi.view(-1).tolist(), (trial, nout)
            assert torch.equal(vals.view(torch.int16), wv.view(-1).view(torch.int16)), (trial, nout)
            want_tok = C.fast_topk(logits, 1, True)[1].item() if amf else wi.view(-1)[0].item()
            assert token.item() == want_tok
