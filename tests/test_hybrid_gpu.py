"""The synthetic hybrid stack's device loop on the GPU (a small shape: 4 layers, MLP 4096, vocab
32768): prefill, eager steps and graph-replayed steps. Checks the orchestration: the committed
length advances by each step's accepted count, every accepted token is a tree token, eager and
replayed steps agree (greedy), the KV rows of accepted positions are the verify's rows."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _model(dev, seed=5, greedy=True):
    from mdx import hybrid
    cfg = hybrid.HybridConfig(layers=4, inter=4096, vocab=32768, cap=256, greedy=greedy)
    m = hybrid.HybridModel(cfg, dev, seed=seed)
    g = torch.Generator().manual_seed(1)
    m.prefill(torch.randint(0, cfg.vocab, (37,), generator=g))
    return m


def test_prefill_commits_the_prompt(dev):
    m = _model(dev)
    assert m.st[0].item() == 36 and m.st[1].item() == 36
    # GDN replay state: the last chunk is pending
    assert m.ctl[0].item() == 36 - 32


def test_eager_steps_advance_counters(dev):
    m = _model(dev)
    for step in range(4):
        st0 = m.st[0].item()
        m.step(m.parity)
        m.parity ^= 1
        torch.cuda.synchronize()
        n = m.result[0].item()
        assert 1 <= n <= m.R
        assert m.st[0].item() == st0 + n
        assert m.result[1 + n - 1].item() == m.nt.item()  # the last committed token is the next root
        assert m.ctl[0].item() == n


def test_graph_replay_matches_eager(dev):
    a, b = _model(dev), _model(dev)
    for _ in range(3):
        a.step(a.parity)
        a.parity ^= 1
    b.capture()  # captures after two eager warm-up steps (one per parity)
    b.replay(1)
    torch.cuda.synchronize()
    assert torch.equal(a.st, b.st) and torch.equal(a.nt, b.nt) and torch.equal(a.result, b.result)
    assert torch.equal(a.hbuf, b.hbuf)


@pytest.mark.parametrize("head", ["bf16", "int8"])
def test_two_stage_drafts_equal_one_stage(dev, head):
    """The two-stage draft head (int4 scores + the draft pick) gives the same decode as the full lm_head (bf16,
    or the int8 ConvRot head): counters, accept records, next tokens and hidden rows after eager steps and
    a graph replay."""
    from mdx import hybrid
    ms = []
    for two in (False, True):
        cfg = hybrid.HybridConfig(layers=4, inter=4096, vocab=32768, cap=256, greedy=True, two_stage=two, head=head)
        m = hybrid.HybridModel(cfg, dev, seed=7)
        m.prefill(torch.randint(0, cfg.vocab, (37,), generator=torch.Generator().manual_seed(2)))
        ms.append(m)
    for step in range(3):
        print(f"case two-stage eager step {step}", flush=True)
        for m in ms:
            m.step(m.parity)
            m.parity ^= 1
        torch.cuda.synchronize()
        a, b = ms
        assert torch.equal(a.vtok, b.vtok) and torch.equal(a.result, b.result) and torch.equal(a.nt, b.nt)
    for m in ms:
        m.capture()
        m.replay(2)
    torch.cuda.synchronize()
    a, b = ms
    assert torch.equal(a.st, b.st) and torch.equal(a.result, b.result) and torch.equal(a.hbuf, b.hbuf)


def test_full_stack_steps(dev):
    """The full decode stack (32 layers: 24 GDN + 8 attention, hidden 4096, MLP 12288, vocab 151936, tree
    (4, 3)): eager steps give finite logits, advance the counters by the accepted count and commit only
    tree tokens; a captured graph replayed from the same state reproduces the eager steps."""
    from mdx import hybrid
    ms = []
    for _ in range(2):
        cfg = hybrid.HybridConfig(cap=256, greedy=True)
        m = hybrid.HybridModel(cfg, dev, seed=9)
        m.prefill(torch.randint(0, cfg.vocab, (41,), generator=torch.Generator().manual_seed(4)))
        ms.append(m)
    a, b = ms
    for step in range(3):
        print(f"case full stack eager step {step}", flush=True)
        st0 = a.st[0].item()
        a.step(a.parity)
        a.parity ^= 1
        torch.cuda.synchronize()
        assert torch.isfinite(a.logits.float()).all()
        n = a.result[0].item()
        assert 1 <= n <= a.R and a.st[0].item() == st0 + n
        committed = a.result[1:1 + n].tolist()
        assert all(t in a.vtok[0].tolist() or t == a.nt.item() for t in committed)
    print("case full stack graph replay", flush=True)
    b.capture()  # two eager warm-up steps, one per parity
    b.replay(1)
    torch.cuda.synchronize()
    assert torch.equal(a.st, b.st) and torch.equal(a.nt, b.nt) and torch.equal(a.result, b.result)
    assert torch.equal(a.hbuf, b.hbuf) and torch.equal(a.logits, b.logits)


def test_auto_tree_records_ranks_and_adapts(dev):
    """auto: the drafts keep 7 candidates and the accept records the verify token's rank among them, the
    decode itself unchanged; decode_auto folds ranks and device times and, with random weights (no draft is
    ever accepted), shrinks the tree to one draft."""
    from mdx import hybrid
    ms = []
    for auto in (False, True):
        cfg = hybrid.HybridConfig(layers=4, inter=4096, vocab=32768, cap=1024, greedy=True, auto=auto)
        m = hybrid.HybridModel(cfg, dev, seed=5)
        m.prefill(torch.randint(0, cfg.vocab, (37,), generator=torch.Generator().manual_seed(1)))
        ms.append(m)
    a, b = ms
    S = a.cfg.slots
    for step in range(3):
        print(f"case auto eager step {step}", flush=True)
        for m in ms:
            m.step(m.parity)
            m.parity ^= 1
        torch.cuda.synchronize()
        ra, rb = a.result.tolist(), b.result.tolist()
        assert ra[:S + 3] == rb[:S + 3] and ra[S + 11:S + 13] == rb[S + 11:S + 13]
        nranks = rb[S + 3]
        assert ra[S + 3] == 0 and 1 <= nranks <= 2
        cand = b.cand.view(7, 7)[0].tolist()
        tok0 = b.toks[0, 0].item()
        assert rb[S + 4] == (cand.index(tok0) if tok0 in cand else 7)
    print("case auto decode", flush=True)
    st0 = b.st[0].item()
    out = b.decode_auto(72, fold_every=16)
    torch.cuda.synchronize()
    assert out["steps"] == 72 and len(out["widths"]) == 72 and out["tokens"] == b.st[0].item() - st0
    assert out["widths"][0] == (4, 3) and out["widths"][-1] == (1,)
    assert out["draft_ms"] > 0 and out["verify_ms"] > 0


@pytest.mark.parametrize("greedy", [True, False])
def test_predictable_weights_commit_every_draft(dev, greedy):
    """Synthetic weights whose next token is predictable (t -> t + 1 mod vocab, HybridConfig.predictable):
    the drafts follow the chain, the verify (sampled or greedy) accepts them, and every step commits
    len(widths) + 1 consecutive tokens, eagerly and from a replayed graph."""
    from mdx import hybrid
    cfg = hybrid.HybridConfig(layers=4, inter=4096, vocab=32768, cap=512, greedy=greedy, predictable=True)
    m = hybrid.HybridModel(cfg, dev, seed=3)
    m.prefill(torch.randint(0, cfg.vocab, (37,), generator=torch.Generator().manual_seed(6)))
    torch.cuda.synchronize()
    want_n = len(cfg.widths) + 1
    root = m.nt.item()

    def check(step):
        nonlocal root
        n = m.result[0].item()
        got = m.result[1:1 + n].tolist()
        assert n == want_n, (step, n, got, root)
        assert got == [(root + 1 + i) % cfg.vocab for i in range(n)], (step, got, root)
        assert m.nt.item() == got[-1]
        root = got[-1]

    for step in range(3):
        print(f"case predictable greedy={greedy} eager step {step}", flush=True)
        st0 = m.st[0].item()
        m.step(m.parity)
        m.parity ^= 1
        torch.cuda.synchronize()
        check(step)
        assert m.st[0].item() == st0 + want_n
    print(f"case predictable greedy={greedy} replay", flush=True)
    m.capture()  # two more eager warm-up steps
    torch.cuda.synchronize()
    root = m.nt.item()
    for step in range(3):
        m.replay(1)
        torch.cuda.synchronize()
        check(3 + step)


def test_tree_switch_and_back_replays_the_first_trees_graphs(dev):
    """A -> B -> A: a model whose graphs were captured for tree A, then for tree B, replays A's graphs again
    after switching back. Those graphs hold the addresses of A's tree tensors (masks, children, positions,
    the verify program), so the tensors must still be A's: the replayed steps equal the same steps run
    eagerly on a second model, with freed-memory reuse provoked in between."""
    a, b = _model(dev), _model(dev)
    A, B = (4, 3), (2, 2, 1)

    def eager(m, n):
        for _ in range(n):
            m.step(m.parity)
            m.parity ^= 1

    print("case tree A capture + replay", flush=True)
    b.capture()  # two eager warm-up steps, one per parity
    b.replay(1)
    eager(a, 3)
    print("case tree B capture + replay", flush=True)
    for m in (a, b):
        m._set_tree(B)
    # small allocations of every size the tree tensors have, filled with junk: a freed A tensor would be
    # handed out again here and overwritten
    junk = [torch.full((n,), -7, dtype=dt, device=dev) for n in (8, 16, 64, 256) for dt in (torch.int32, torch.int64)]
    b.capture()
    b.replay(1)
    eager(a, 3)
    print("case tree A again: replay of the first graphs", flush=True)
    for m in (a, b):
        m._set_tree(A)
    b.replay(2)
    eager(a, 2)
    torch.cuda.synchronize()
    del junk
    assert torch.equal(a.st, b.st) and torch.equal(a.nt, b.nt) and torch.equal(a.result, b.result)
    assert torch.equal(a.hbuf, b.hbuf) and torch.equal(a.ctl, b.ctl)
