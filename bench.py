"""Benchmark of the W4A8 decode path on one MI355X.

Default workload: the fused W4A8 SwiGLU MLP block (hidden 4096, intermediate 12288, RMSNorm eps 1e-6
in front, GPTQ int4 weights in groups of 128 with fp16 scales ~U(0.005, 0.02), per-token int8
activations), one decode row. A "step" is one MLP call. Weights live in a ring of distinct copies
(> 2x the 256 MB Infinity Cache) so each call streams its weights from HBM; the ring is captured
in one HIP graph and replayed. The default run then also decodes the full synthetic 32-layer hybrid
stack (the metric's second half: tok/s, ms per step) and reports it under "decode".

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--rows M]
                    [--workload mlp|linear|lmhead|attn|stack|copy] [--ctx L] [--prompt P]

Prints one JSON line: value = whole-job achieved HBM GB/s (algorithmic bytes / wall time), plus
`roofline` for the dominant kernel (the gate/up GEMV launch, timed on its own graph of launches;
`traffic` from the committed rocprofv3 PMC summary) and `cpu_baseline` (the CPU oracle of the same
operator chain on a bounded sample).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "comfy-mono-decode-xpu_amd"))

PEAK_HBM_GBS = 8000.0
METRIC = "W4A8 GEMV achieved HBM GB/s (% of peak); decode tok/s at 9B hybrid, 8-draft tree"


def pmc_traffic(key):
    """HBM bytes per launch of a workload's dominant kernel, from the committed rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE scaled by the counters' readings for a 256 MiB copy), or None."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            return json.load(f)[key]["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def gptq_weight(N, K, gen, dev, tiled=True):
    import torch
    from mdx import _lib, layout
    q = torch.randint(-8, 8, (N, K), generator=gen, device=dev, dtype=torch.int8)
    s = (torch.rand(N, K // 128, generator=gen, device=dev) * 0.015 + 0.005).half()
    packed, s_rel, sch, _ = layout.gptq_pack(q, s, 128, integral=True)
    w = layout.W4(packed, s_rel, sch, None, decode=_lib.DECODE_INTEGRAL)  # integral scales by construction
    return w.tiled() if tiled else w


def mlp_bytes(rows, H=4096, I=12288):
    codes = 3 * H * I // 2
    scales = 3 * H * I // 128 * 2
    sch = (2 * I + H) * 4
    io = rows * H * 2 * 2 + H * 2  # x in, out, norm weight
    return codes + scales + sch + io


def gateup_bytes(rows, H=4096, I=12288):
    return 2 * (I * H // 2 + I * H // 128 * 2 + I * 4) + rows * (H + 4) + rows * I * 2


def linear_bytes(rows, N=4096, K=4096):
    return N * K // 2 + N * K // 128 * 2 + N * 4 + rows * (K + 4) + rows * N * 2


def graph_time(fn, replays, warmup):
    """Capture fn() once in a HIP graph; seconds per replay over `replays` timed replays."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # eager warm-up (workspace, LDS attributes)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(max(warmup, 1)):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / replays


def cpu_threads():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline_mlp(ring0, rows, xb, nwb, lutb, budget_s=20.0):
    """The oracle's operator chain (RMSNorm, quantise, decode + int dot, SiLU, quantise, decode +
    int dot) on the host, on one set of the same weights; median over a bounded number of calls."""
    import numpy as np
    sys.path.insert(0, ROOT)
    from oracle import ref
    d = []
    for w in ring0:
        from mdx import layout
        q = layout.row_major_codes(w.q).cpu().numpy()
        s = w.s.float().cpu().numpy()
        d.append(dict(packed=q, s=s, sch=w.sc.cpu().numpy(), cb=None, G=128))
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 and (not times or time.perf_counter() + times[-1] < t_end):
        for dd in d:
            dd.pop("w8", None)  # the decode is part of every call of the chain
        t0 = time.perf_counter()
        xn = ref.rmsnorm(xb, nwb, 1e-6)
        ref.mono_mlp(xn, "none", None, lutb, *d)
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def bench_mlp(args, dev):
    import torch
    from mdx import _C, _lib, layout
    gen = torch.Generator(device=dev).manual_seed(2)
    H, I, M = 4096, 12288, args.rows
    per = mlp_bytes(M)
    ring_n = max(2, -(-2 * 256 * 2 ** 20 // (3 * H * I // 2)) + 1)  # > 2x the 256 MB Infinity Cache
    ring = [(gptq_weight(I, H, gen, dev), gptq_weight(I, H, gen, dev), gptq_weight(H, I, gen, dev))
            for _ in range(ring_n)]
    x = torch.randn(M, H, generator=gen, device=dev).to(torch.bfloat16)
    nw = (1 + 0.02 * torch.randn(H, generator=gen, device=dev)).to(torch.bfloat16)
    lut = layout.silu_lut(dev)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
    ws = torch.zeros(_lib.lib().mdx_mono_mlp_workspace(M, H, I), dtype=torch.uint8, device=dev)

    def all_ring():
        for g_, u_, d_ in ring:
            _C.mono_mlp_w4(x, _lib.ROT_NONE, None, lut, g_, u_, d_, norm_w=nw, eps=1e-6, out=out, ws=ws)

    reps = max(1, args.steps // ring_n)
    t_call = graph_time(all_ring, reps, args.warmup) / ring_n
    # the dominant kernel alone: the gate/up GEMV launch over the same ring
    q1, s1 = _C.rms_rot_quant(x, nw, 1e-6)
    hbuf = torch.empty(M, I, dtype=torch.bfloat16, device=dev)

    def all_gateup():
        for g_, u_, _ in ring:
            _C.stream_gemv(q1, s1, [g_, u_], [hbuf], gate_up=True, silu_lut=lut)

    t_gu = graph_time(all_gateup, reps, args.warmup) / ring_n
    gu_b = gateup_bytes(M)
    res = {
        "metric": METRIC,
        "value": round(per / t_call / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": reps * ring_n,
        "warmup": args.warmup,
        "ms_per_step": round(t_call * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xint4->int32, bf16 out",
        "data": "synthetic (seeded GPTQ int4 weights, fp16 G128 scales, N(0,1) activations)",
        "config": {"workload": f"fused W4A8 SwiGLU MLP 4096->2x12288->4096, RMSNorm 1e-6, rows={M}, "
                               f"tile-major weights, {ring_n}-copy weight ring",
                   "rows": M, "hidden": H, "intermediate": I, "group_size": 128,
                   "algorithmic_bytes_per_step": per, "frac_of_peak": round(per / t_call / 1e9 / PEAK_HBM_GBS, 4)},
        "roofline": {"bound": "hbm", "kernel": "gemv_kernel (gate/up pair, SiLU epilogue)",
                     "achieved": round(gu_b / t_gu / 1e9, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gu_b / t_gu / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": pmc_traffic("mlp_gateup_rows1") if M == 1 else None,
                     "algorithmic_bytes_per_launch": gu_b, "avg_launch_us": round(t_gu * 1e6, 3)},
    }
    if not args.no_cpu:
        from oracle import ref as _ref  # noqa: F401
        xb = x.view(torch.int16).cpu().numpy().view("uint16")
        nwb = nw.view(torch.int16).cpu().numpy().view("uint16")
        lutb = lut.view(torch.int16).cpu().numpy().view("uint16")
        t_cpu, n = cpu_baseline_mlp(ring[0], M, xb, nwb, lutb)
        res["cpu_baseline"] = {"value": round(per / t_cpu / 1e9, 4), "unit": "GB/s", "cores": cpu_threads(),
                               "kind": "port", "ms_per_step": round(t_cpu * 1e3, 1),
                               "sample": f"{n} MLP calls of the numpy oracle chain (decode + float64 int dot), "
                                         f"same weights and rows"}
    return res


def bench_linear(args, dev):
    import torch
    from mdx import _C
    gen = torch.Generator(device=dev).manual_seed(1)
    N = K = 4096
    M = args.rows
    per = linear_bytes(M)
    ring_n = -(-2 * 256 * 2 ** 20 // (N * K // 2)) + 1
    ring = [gptq_weight(N, K, gen, dev) for _ in range(ring_n)]
    x = torch.randn(M, K, generator=gen, device=dev).to(torch.bfloat16)
    q, s = _C.quant_rows(x)
    s = s.view(-1)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)

    def all_ring():
        for w in ring:
            _C.stream_gemv(q, s, [w], [out])

    reps = max(1, args.steps // ring_n)
    t = graph_time(all_ring, reps, args.warmup) / ring_n
    return {
        "metric": METRIC, "value": round(per / t / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": reps * ring_n,
        "warmup": args.warmup, "ms_per_step": round(t * 1e3, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8xint4->int32, bf16 out",
        "data": "synthetic (seeded GPTQ int4 weights, fp16 G128 scales)",
        "config": {"workload": f"single W4A8 linear M={M} K=N=4096 G128, {ring_n}-copy weight ring", "rows": M,
                   "algorithmic_bytes_per_step": per},
        "roofline": {"bound": "hbm", "kernel": "gemv_kernel", "achieved": round(per / t / 1e9, 2),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(per / t / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": pmc_traffic("linear_rows1") if M == 1 else None, "avg_launch_us": round(t * 1e6, 3)},
    }


def _ring_count(per_call_bytes):
    """Copies cycled per replay so the working set exceeds 2x the 256 MB Infinity Cache."""
    return max(1, -(-2 * 256 * 2 ** 20 // per_call_bytes) + 1) if per_call_bytes < 2 * 256 * 2 ** 20 else 1


def _line(args, value, unit, t, steps, dtype, data, config, roofline=None):
    res = {"metric": METRIC, "value": value, "unit": unit, "n_gpus": 1, "steps": steps, "warmup": args.warmup,
           "ms_per_step": round(t * 1e3, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": dtype, "data": data, "config": config}
    if roofline:
        res["roofline"] = roofline
    return res


def bench_lmhead(args, dev):
    """bf16 lm_head of the hybrid stack: vocab 151936 x hidden 4096, `rows` decode rows."""
    import torch
    from mdx import _C, layout
    gen = torch.Generator(device=dev).manual_seed(5)
    V, H, M = 151936, 4096, args.rows
    per = V * H * 2 + M * H * 2 + M * V * 2
    w = layout.tile_major_bf16((torch.randn(V, H, generator=gen, device=dev) * 0.02).bfloat16())
    x = torch.randn(M, H, generator=gen, device=dev).bfloat16()
    out = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
    reps = max(1, args.steps // 10)
    t = graph_time(lambda: _C.bf16_linear(x, w, tiled=True, out=out), reps, args.warmup)
    gbs = per / t / 1e9
    return _line(args, round(gbs, 2), "GB/s", t, reps, "bf16 x bf16 -> fp32 acc, bf16 out",
                 "synthetic (seeded N(0, 0.02) weights, N(0,1) rows)",
                 {"workload": f"bf16 lm_head 151936x4096, rows={M}, tile-major", "rows": M,
                  "algorithmic_bytes_per_step": per},
                 {"bound": "hbm", "kernel": "bf16_linear_kernel", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS,
                  "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
                  "avg_launch_us": round(t * 1e6, 3)})


def bench_attn(args, dev):
    """Tree-verify decode attention of the hybrid stack's attention layer: 32 q / 8 kv heads, head_dim
    128, 16 tree rows, context `--ctx` tokens; KV caches cycled in a ring."""
    import torch
    from mdx import _C
    sys.path.insert(0, ROOT)
    gen = torch.Generator(device=dev).manual_seed(3)
    H, Hk, D, S, L = 32, 8, 128, 16, args.ctx
    cap = L + 64
    per = 2 * Hk * L * D * 2 + H * S * D * 2 * 2 + 2 * Hk * S * D * 2
    ring_n = _ring_count(per)
    caches = [((torch.randn(1, Hk, cap, D, generator=gen, device=dev)).bfloat16(),
               (torch.randn(1, Hk, cap, D, generator=gen, device=dev)).bfloat16()) for _ in range(ring_n)]
    q = torch.randn(1, H, S, D, generator=gen, device=dev).bfloat16()
    xk = torch.randn(1, Hk, S, D, generator=gen, device=dev).bfloat16()
    xv = torch.randn(1, Hk, S, D, generator=gen, device=dev).bfloat16()
    parents = [-1, 0, 1, 2, 3, 4, 5, 6, 0, 8, 1, 10, 2, 12, 3, 14]
    m = []
    for r, p in enumerate(parents):
        m.append((m[p] if p >= 0 else 0) | (1 << r))
    mask = torch.tensor(m, dtype=torch.int32, device=dev)
    sl = torch.tensor([L], dtype=torch.int32, device=dev)

    def all_ring():
        for k, v in caches:
            _C.attn_dpas(q, k, v, sl, xk, xv, mask, 0)

    reps = max(1, args.steps // ring_n)
    t = graph_time(all_ring, reps, args.warmup) / ring_n
    gbs = per / t / 1e9
    return _line(args, round(gbs, 2), "GB/s", t, reps * ring_n, "bf16 x bf16 -> fp32 (MFMA), bf16 out",
                 "synthetic (seeded N(0,1) KV cache and rows)",
                 {"workload": f"tree-verify decode attention, 32q/8kv heads, head_dim 128, 16 rows, ctx={L}, "
                              f"{ring_n}-copy KV ring", "ctx": L, "rows": S, "algorithmic_bytes_per_step": per},
                 {"bound": "hbm", "kernel": "attn_kernel", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS,
                  "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
                  "avg_launch_us": round(t * 1e6, 3)})


def bench_stack(args, dev):
    """The full synthetic 32-layer hybrid stack (3 GDN : 1 attention, hidden 4096, MLP 12288, W4A8
    GPTQ G128), 1-layer bf16 MTP draft block, bf16 lm_head over 151936, tree_spec (4, 3) (8 rows, 2
    drafts per step), top-k 20 sampling; a seeded random prompt is prefilled (not timed), then each
    decode step is one replayed HIP graph. value = accepted tokens per second."""
    import torch
    from mdx import hybrid
    steps, warm = args.steps, max(args.warmup, 2)
    cap = args.prompt + 8 * (steps + warm + 4) + 64
    cfg = hybrid.HybridConfig(cap=cap)
    t0 = time.perf_counter()
    m = hybrid.HybridModel(cfg, dev, seed=5)
    prompt = torch.randint(0, cfg.vocab, (args.prompt,), generator=torch.Generator().manual_seed(5))
    m.prefill(prompt)
    m.capture()
    m.replay(warm)
    torch.cuda.synchronize()
    setup = time.perf_counter() - t0
    st0 = int(m.st[0].item())
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    m.replay(steps)
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) / 1e3
    tokens = int(m.st[0].item()) - st0
    per_step = t / steps
    return _line(args, round(tokens / t, 2), "tok/s", per_step, steps, "W4A8 int8 x int4 -> int32; bf16 draft, lm_head",
                 "synthetic (random-init weights, seeded random prompt)",
                 {"workload": f"32-layer W4A8 hybrid (24 GDN + 8 attention), hidden 4096, MLP 12288, vocab 151936, "
                              f"MTP draft, tree (4, 3), top-k 20, prompt {args.prompt}, {steps} decode steps",
                  "prompt": args.prompt, "steps": steps, "tokens": tokens,
                  "accepted_per_step": round(tokens / steps, 3), "ms_per_step": round(per_step * 1e3, 4),
                  "setup_s": round(setup, 1)})


def bench_copy(args, dev):
    """Calibration workload: a plain device copy of 256 MiB (read 256 MiB, write 256 MiB). Its
    FETCH_SIZE / WRITE_SIZE counters give the scale factor of the traffic figures."""
    import torch
    n = 256 * 2 ** 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    reps = max(1, args.steps // 100)
    t = graph_time(lambda: dst.copy_(src), reps, args.warmup)
    return {"metric": "device copy GB/s (read + write)", "value": round(2 * n / t / 1e9, 2), "unit": "GB/s",
            "n_gpus": 1, "steps": reps, "warmup": args.warmup, "ms_per_step": round(t * 1e3, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8", "data": "synthetic",
            "config": {"workload": "copy of 256 MiB (traffic calibration)", "bytes_read": n, "bytes_written": n}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--rows", type=int, default=1)
    ap.add_argument("--workload", choices=["mlp", "linear", "copy", "lmhead", "attn", "stack"], default="mlp")
    ap.add_argument("--prompt", type=int, default=1024, help="stack: prompt tokens (prefilled, not timed)")
    ap.add_argument("--ctx", type=int, default=8192, help="attention context length")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-decode", action="store_true", help="mlp: skip the full-stack decode leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU only: the 9B stack scales as one "
                                   "data-parallel replica per GPU (about 5 GB each); tensor-parallel "
                                   "sharding of the GEMVs, heads and lm_head is not implemented or "
                                   "measured here", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm device"}))
        sys.exit(1)
    dev = torch.device("cuda", 0)
    res = {"mlp": bench_mlp, "linear": bench_linear, "copy": bench_copy, "lmhead": bench_lmhead,
           "attn": bench_attn, "stack": bench_stack}[args.workload](args, dev)
    if args.workload == "mlp" and not args.no_decode:
        # the second half of the metric: decode tok/s of the full synthetic hybrid stack (1024-token
        # prompt, 64 graph-replayed steps)
        sub = argparse.Namespace(**vars(args))
        sub.steps, sub.warmup, sub.prompt = 64, 4, 1024
        d = bench_stack(sub, dev)
        res["decode"] = {"metric": "decode tok/s at 9B hybrid, 8-draft tree", "value": d["value"], "unit": "tok/s",
                         "ms_per_step": d["config"]["ms_per_step"],
                         "accepted_per_step": d["config"]["accepted_per_step"], "workload": d["config"]["workload"]}
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
