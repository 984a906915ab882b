"""Pins of the oracle's draft pick (oracle/ref.py: int8_head_logits, draft_pick) on the CPU: the exact
int8 logits against torch (int64 dot, fp32 products, bf16), the outputs against a brute-force sort on
distinct logits and hand-worked placements of the token and the children's verify tokens."""
import numpy as np
import torch

from oracle import ref


def test_int8_head_logits_against_torch():
    g = torch.Generator().manual_seed(3)
    w = torch.randint(-127, 128, (300, 512), generator=g, dtype=torch.int8)
    qx = torch.randint(-127, 128, (512,), generator=g, dtype=torch.int8)
    sx = torch.rand(1, generator=g) * 0.05 + 0.01
    sw = torch.rand(300, generator=g) * 1e-3 + 1e-4
    acc = (w.long() * qx.long()).sum(-1)
    want = ((acc.float() * sx) * sw).bfloat16().view(torch.int16).numpy().view(np.uint16)
    got = ref.int8_head_logits(qx.numpy(), sx.numpy(), w.numpy(), sw.numpy())
    assert np.array_equal(got, want)


def test_draft_pick_outputs_on_distinct_logits():
    rng = np.random.default_rng(5)
    lb = rng.permutation(np.arange(0x3F80, 0x3F80 + 8192, dtype=np.uint16))  # distinct positive bf16 values
    vals = ref.bf16_to_f32(lb)
    order = np.argsort(-vals, kind="stable")
    top, tok, vtok = ref.draft_pick(lb, 5, False, [1, 3, 4], 8)
    assert top.tolist() == order[:5].tolist()
    assert tok == order[0]
    assert vtok.tolist() == [-1, order[0], -1, order[1], order[2], -1, -1, -1]
    # argmax_first: the token is the argmax, the children after the first take top[1:]
    top, tok, vtok = ref.draft_pick(lb, 3, True, [6, 2], 8)
    assert tok == order[0] and vtok[6] == order[0] and vtok[2] == order[1]


def test_draft_pick_argmax_rules():
    """A NaN is the argmax (torch's rule) while topk places it first too; -0 and +0 tie by index."""
    lb = ref.f32_to_bf16(np.array([1.0, 3.0, -0.0, 0.0, 2.0] * 2000, dtype=np.float32))
    lb[7] = 0x7FC0
    _, tok, _ = ref.draft_pick(lb, 2, True, [0], 4)
    assert tok == 7
