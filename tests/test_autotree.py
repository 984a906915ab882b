"""The adaptive tree's statistics and choice (mdx/autotree.py) on the CPU: the rank histogram's decay and
counts (comfy_mono_decode_xpu/mtp_loop.py:414-423), the timing average's warm-up skip and 1/8 smoothing
(autotree.py:62-76 there), the expected-token closed form on hand-worked trees, the candidate set, and
best_widths against an exhaustive search (with its 2% hysteresis), at the two ends: drafts that never
hit shrink the tree to one draft, drafts whose chain always hits grow it to the deepest chain."""
import pytest

from mdx import autotree as at


def test_hits_decay_and_fill_forward():
    h = at.Hits()
    assert h.probs() is None
    h.add([0, 2])
    h.add([7])
    assert h.h[0][0] == pytest.approx(at.DECAY) and h.h[1][2] == pytest.approx(at.DECAY) and h.h[0][7] == 1
    p = h.probs()
    s0 = at.DECAY + 1
    assert p[0][0] == pytest.approx(at.DECAY / s0) and p[0][7] == pytest.approx(1 / s0)
    assert p[1] == [0, 0, 1, 0, 0, 0, 0, 0]
    assert all(p[k] == p[1] for k in range(2, 7))  # deeper levels without data take the deepest seen


def test_clock_skips_warm_up_then_smooths():
    c = at.Clock()
    for _ in range(8):
        c.add(100.0, 100.0)
    assert not c.ready and c.draft_ms == 0
    c.add(1.0, 2.0)
    assert c.ready and (c.draft_ms, c.verify_ms) == (1.0, 2.0)
    c.add(9.0, 10.0)
    assert c.draft_ms == pytest.approx(1.0 + (9.0 - 1.0) / 8) and c.verify_ms == pytest.approx(2.0 + 1.0)


def test_expected_tokens_closed_form():
    p0 = [0.5, 0.25, 0, 0, 0, 0, 0, 0.25]
    p1 = [0.4, 0.1, 0.1, 0, 0, 0, 0, 0.4]
    probs = [p0, p1] + [p1] * 5
    assert at.expected_tokens((1,), probs) == pytest.approx(1.5)
    assert at.expected_tokens((2,), probs) == pytest.approx(1.75)
    assert at.expected_tokens((2, 1), probs) == pytest.approx(1 + 0.75 + 0.5 * 0.4)
    assert at.expected_tokens((2, 3), probs) == pytest.approx(1 + 0.75 + 0.5 * 0.6)
    assert at.expected_tokens((1, 1, 1), probs) == pytest.approx(1 + 0.5 + 0.5 * 0.4 + 0.5 * 0.4 * 0.4)


def test_candidates_fit_the_slots():
    cs = at.candidates(16)
    assert (4, 3) in cs and (1,) in cs and (7,) in cs and (1,) * 7 in cs
    assert all(1 + sum(c) <= 16 and 1 <= len(c) <= 7 and list(c) == sorted(c, reverse=True) for c in cs)
    assert len(cs) == len(set(cs))


def _probs(chain_hit, sibling_hit=0.0):
    p = [chain_hit, sibling_hit] + [0] * 5 + [1 - chain_hit - sibling_hit]
    return [p] * 7


@pytest.mark.parametrize("chain_hit,sibling,draft_ms,verify_ms", [(0.0, 0.0, 0.1, 3.0), (1.0, 0.0, 0.05, 3.0),
                                                                    (0.6, 0.2, 0.1, 3.0), (0.3, 0.3, 0.5, 1.0)])
def test_best_widths_is_the_exhaustive_maximum(chain_hit, sibling, draft_ms, verify_ms):
    probs = _probs(chain_hit, sibling)
    best = at.best_widths((4, 3), probs, draft_ms, verify_ms)
    scores = {c: at.score(c, probs, draft_ms, verify_ms) for c in at.candidates(16)}
    top = max(scores.values())
    cur = at.score((4, 3), probs, draft_ms, verify_ms)
    if top > cur * at.HYSTERESIS:
        assert scores[best] == pytest.approx(top)
    else:
        assert best == (4, 3)
    if chain_hit == 0.0:
        assert best == (1,)      # nothing is accepted: one draft, the cheapest step
    if chain_hit == 1.0:
        assert best == (1,) * 7  # every chain draft is accepted: the deepest chain


def test_no_statistics_keeps_the_tree():
    assert at.best_widths((4, 3), at.Hits(), 0.1, 3.0) == (4, 3)
    assert at.best_widths((4, 3), _probs(0.0), 0.0, 3.0) == (4, 3)
