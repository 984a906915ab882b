"""Adaptive MTP tree ("auto"): choose the draft tree's widths from measured acceptance and device time
(comfy_mono_decode_xpu/autotree.py:1-194 feeds ComfyUI's qwen35.best_widths with device timings; the
device loop gathers the per-depth acceptance ranks, comfy_mono_decode_xpu/mtp_loop.py:264,414-441).

Statistics, restated from the reference's loop:
  hits[level][rank]: for every decode step, each chain depth the accept walk reached records the rank (0..6)
  of the verify's token among that draft's 7 candidates, or 7 for none (mtp_accept's record); before a
  step is added every count decays by 63/64.
  draft_ms / verify_ms: device time of one draft and of the verify part (verify, lm_head, top-k, sampling,
  accept) per step from HIP events; the first 8 steps are not learned (graph capture and warm-up), step 9
  sets the averages, later steps move them by 1/8.

The choice (best_widths) is this library's own: ComfyUI's scoring is third-party and not part of the
reference, so its rule is restated here from what it optimises, accepted tokens per millisecond. For a chain
of widths (w_1 .. w_D) -- depth d drafts w_d candidates, the first continues the chain -- with acceptance
distribution p_d over ranks (hits normalised per level; a level without data takes the deepest level
that has data):
  E = 1 + sum_d reach_d * sum_{r < w_d} p_d[r],   reach_1 = 1, reach_{d+1} = reach_d * p_d[0]
  T = D * draft_ms + verify_ms
and the widths with the largest E / T among the trees that fit the slots (1 + sum w_d <= slots, D <= 7,
w_d <= 7, non-increasing) win, unless they beat the current widths' score by less than 2% (no flapping
between near-equal trees, each change costs a graph capture). Parity unpinned against ComfyUI's own
best_widths (not available); the rule is pinned by its closed form in the tests.
"""
from __future__ import annotations

import itertools

DECAY = 0.984375
LEVELS, RANKS = 7, 8
HYSTERESIS = 1.02


class Hits:
    def __init__(self):
        self.h = [[0.0] * RANKS for _ in range(LEVELS)]

    def add(self, ranks):
        """One step's ranks (level order): decay, then count."""
        for row in self.h:
            for i in range(RANKS):
                row[i] *= DECAY
        for level, rank in enumerate(ranks[:LEVELS]):
            self.h[level][min(max(int(rank), 0), RANKS - 1)] += 1

    def probs(self):
        """Per-level rank distributions, or None when nothing was recorded."""
        out, last = [], None
        for row in self.h:
            s = sum(row)
            if s > 0:
                last = [v / s for v in row]
            out.append(last)
        if last is None:
            return None
        # levels before the first recorded one cannot exist (level 0 is always reached): fill forward only
        first = next(p for p in out if p is not None)
        return [p if p is not None else first for p in out]


class Clock:
    """The reference's smoothing of per-step device times."""

    def __init__(self):
        self.steps = 0
        self.draft_ms = 0.0
        self.verify_ms = 0.0

    def add(self, draft_ms_per_draft, verify_ms):
        self.steps += 1
        if self.steps <= 8:
            return
        mix = 1.0 if self.steps == 9 else 0.125
        self.draft_ms += mix * (draft_ms_per_draft - self.draft_ms)
        self.verify_ms += mix * (verify_ms - self.verify_ms)

    @property
    def ready(self):
        return self.steps > 8


def expected_tokens(widths, probs):
    e, reach = 1.0, 1.0
    for d, w in enumerate(widths):
        p = probs[min(d, len(probs) - 1)]
        e += reach * sum(p[:w])
        reach *= p[0]
    return e


def candidates(slots=16, max_depth=7, max_width=7):
    """Every non-increasing width chain that fits the slots, fewest tree rows first (then fewest drafts):
    best_widths keeps the first of equal scores, so ties go to the smaller verify."""
    out = []
    for depth in range(1, max_depth + 1):
        for ws in itertools.combinations_with_replacement(range(max_width, 0, -1), depth):
            if 1 + sum(ws) <= slots:
                out.append(tuple(ws))
    return sorted(out, key=lambda ws: (sum(ws), len(ws), [-w for w in ws]))


def score(widths, probs, draft_ms, verify_ms):
    return expected_tokens(widths, probs) / (len(widths) * draft_ms + verify_ms)


def best_widths(widths, hits, draft_ms, verify_ms, slots=16):
    """The widths to use next (the current ones when there is nothing to decide on)."""
    probs = hits.probs() if isinstance(hits, Hits) else hits
    widths = tuple(widths)
    if probs is None or draft_ms <= 0 or verify_ms <= 0:
        return widths
    cur = score(widths, probs, draft_ms, verify_ms)
    best, best_s = widths, cur
    for ws in candidates(slots):
        s = score(ws, probs, draft_ms, verify_ms)
        if s > best_s:
            best, best_s = ws, s
    return best if best_s > cur * HYSTERESIS else widths
