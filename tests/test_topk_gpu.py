"""fast_topk / fast_pick / topk_rows on the GPU against the CPU oracle's rank order: values and indices
bit for bit, including tie-heavy, +-0, all-equal and NaN rows. Reference tests mirrored:
tests/test_fast_topk.py, tests/test_topk_rows.py (whose torch-XPU outputs are the contract the
oracle restates; torch-CPU's topk tie order differs and is not used)."""
import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits
from oracle import ref

pytestmark = pytest.mark.gpu


def _rows(V, n):
    g = torch.Generator().manual_seed(0)
    for trial in range(n):
        x = (torch.randn(1, V, generator=g) * 3).to(torch.bfloat16)
        if trial % 2:
            x = (torch.round(x.float() * 2) / 2).to(torch.bfloat16)  # many ties
        if trial % 3 == 0:
            x[0, torch.randint(0, V, (6,), generator=g)] = x.max()
        if trial % 7 == 0:
            x[0, torch.randint(0, V, (3,), generator=g)] = 0.0
            x[0, 5] = -0.0
        if trial % 11 == 0:
            x = torch.zeros(1, V, dtype=torch.bfloat16)
        if trial % 13 == 5:
            x[0, torch.randint(0, V, (4,), generator=g)] = float("nan")
        yield trial, x


@pytest.mark.parametrize("V", [151936, 248320, 32768])
def test_fast_topk_and_pick_match_oracle(C, dev, V):
    for trial, x in _rows(V, 16 if V != 32768 else 8):
        xb = bits(x)[0]
        wv, wi = ref.fast_topk(xb, 8)
        am = ref.argmax_bf16(xb)
        xd = x.to(dev)
        for k in (1, 2, 3, 7, 8):
            v, i = C.fast_topk(xd, k, False)
            assert v.shape == (1, k) and i.shape == (1, k)
            assert i.cpu().numpy()[0].tolist() == wi[:k].tolist(), (trial, k)
            assert_bits_equal(bits(v)[0], wv[:k], f"values trial {trial} k {k}")
        _, ai = C.fast_topk(xd, 1, True)
        assert ai.item() == am, trial
        v8, i8, a8 = C.fast_pick(xd, 8)
        assert i8.cpu().numpy()[0].tolist() == wi.tolist() and a8.item() == am, trial
        assert_bits_equal(bits(v8)[0], wv, f"pick values trial {trial}")


def _topk_rows_input(kind, R, N, g):
    if kind == "bf16":
        return torch.randn(R, N, generator=g).bfloat16().float()
    if kind == "ties":
        return torch.randint(0, 6, (R, N), generator=g).float()
    if kind == "few":
        return (torch.randn(R, N, generator=g) * 3).round() / 0.7
    if kind == "zeros":
        x = torch.randint(-3, 3, (R, N), generator=g).float()
        x[x == 0] = -0.0
        x[:, ::97] = 0.0
        return x
    if kind == "equal":
        return torch.ones(R, N)
    x = torch.randn(R, N, generator=g).bfloat16().float()
    x[:, torch.randint(0, N, (50,), generator=g)] = float("nan")
    return x


@pytest.mark.parametrize("kind", ["bf16", "ties", "few", "zeros", "equal", "nan"])
@pytest.mark.parametrize("R,k,N", [(8, 20, 151936), (8, 64, 248320), (3, 7, 151936), (1, 1, 4096),
                                   (16, 64, 151936), (16, 20, 5000)])
def test_topk_rows_matches_oracle(C, dev, kind, R, k, N):
    g = torch.Generator().manual_seed(hash((kind, R, k, N)) % (1 << 31))
    x = _topk_rows_input(kind, R, N, g)
    wv, wi = ref.topk_rows(x.numpy(), k)
    v, i = C.topk_rows(x.to(dev), k)
    assert np.array_equal(i.cpu().numpy(), wi), kind
    assert_bits_equal(bits(v), wv.view(np.uint32), f"values {kind}")
    if kind not in ("few", "nan"):  # bf16-valued rows: the bf16 input gives the top-k of its fp32 values
        xb = x.bfloat16()
        wv, wi = ref.topk_rows(bits(xb), k)
        v, i = C.topk_rows(xb.to(dev), k)
        assert np.array_equal(i.cpu().numpy(), wi), kind
        assert_bits_equal(bits(v), wv.view(np.uint32), f"bf16 values {kind}")


def test_topk_rejects_unsupported(C, dev):
    with pytest.raises(RuntimeError):
        C.fast_topk(torch.zeros(1, 1024, dtype=torch.bfloat16, device=dev), 4, False)  # row too short
    with pytest.raises(RuntimeError):
        C.fast_topk(torch.zeros(1, 151936, dtype=torch.bfloat16, device=dev), 9, False)  # k > 8
    with pytest.raises(RuntimeError):
        C.topk_rows(torch.zeros(17, 8192, device=dev), 4)  # rows > 16
    with pytest.raises(RuntimeError):
        C.topk_rows(torch.zeros(2, 8192, device=dev), 65)  # k > 64


def test_topk_repeated_launches_reuse_workspace(C, dev):
    """Counters return to zero: many launches in a row (and inside one graph) stay correct."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(8, 151936, generator=g).bfloat16()
    wv, wi = ref.topk_rows(bits(x), 20)
    xd = x.to(dev)
    for _ in range(50):
        v, i = C.topk_rows(xd, 20)
    torch.cuda.synchronize()
    assert np.array_equal(i.cpu().numpy(), wi)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        C.topk_rows(xd, 20)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gv, gi = C.topk_rows(xd, 20)
    for rep in range(3):
        gi.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(gi.cpu().numpy(), wi), rep


@pytest.mark.parametrize("temperature", [1.0, 0.7])
def test_topk_sample_matches_torch_expression(C, dev, temperature):
    """The fused Gumbel-max pick equals the decode loop's torch expression on the same uniforms
    (fp32 roundings of the same operations; ties to the first position, as torch.argmax), with the
    clamp's edges among the uniforms."""
    g = torch.Generator(device=dev).manual_seed(int(temperature * 100))
    for R, k in ((8, 20), (1, 1), (16, 64), (3, 7)):
        print(f"case topk_sample R={R} k={k} T={temperature}", flush=True)
        vals = (torch.randn(R, k, generator=g, device=dev) * 3).sort(dim=1, descending=True).values
        vals[:, k // 2:] = vals[:, k // 2:].round()  # ties among the scores' first terms
        idx = torch.randint(0, 151936, (R, k), generator=g, device=dev)
        u = torch.rand(R, k, generator=g, device=dev)
        u[0, 0] = 0.0
        if k > 2:
            u[0, 1], u[0, 2] = 1e-30, 0.99999994
        got = C.topk_sample(vals, idx, u, temperature)
        gum = -torch.log(-torch.log(u.clone().clamp_(1e-20, 1.0)))
        pick = torch.argmax(vals / temperature + gum, dim=1, keepdim=True)
        want = torch.gather(idx, 1, pick).view(R)
        assert torch.equal(got, want), (got, want)


def test_topk_sample_seeded_matches_oracle_uniforms(C, dev):
    """topk_sample_seeded draws its uniforms on the device from (seed, counter[0], row, slot): the picks
    equal topk_sample's on the oracle's restatement of those uniforms, for two counters (a captured
    graph's successive replays), and differ between counters."""
    from oracle import ref
    g = torch.Generator(device=dev).manual_seed(9)
    R, k, seed = 8, 20, 0x5EED5EED
    vals = torch.randn(R, k, generator=g, device=dev).sort(dim=1, descending=True).values * 0.3
    idx = torch.randint(0, 151936, (R, k), generator=g, device=dev)
    picks = []
    for cnt in (1061, 1062):
        print(f"case topk_sample_seeded counter={cnt}", flush=True)
        counter = torch.tensor([cnt, 0, 0, 0], dtype=torch.int64, device=dev)
        u = torch.tensor([[float(ref.seeded_uniform(seed, cnt, r, j)) for j in range(k)] for r in range(R)],
                         dtype=torch.float32, device=dev)
        got = C.topk_sample_seeded(vals, idx, seed, counter, 1.0)
        want = C.topk_sample(vals, idx, u, 1.0)
        assert torch.equal(got, want), (got, want)
        picks.append(got)
    assert not torch.equal(picks[0], picks[1])
