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
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "comfy-mono-decode-xpu_amd"))

PEAK_HBM_GBS = 8000.0
PEAK_I8_OPS = 5.0e15      # dense int8 MFMA, MI355X
PEAK_BF16_FLOPS = 2.5e15  # dense bf16 MFMA, MI355X
METRIC = "W4A8 GEMV achieved HBM GB/s (% of peak); decode tok/s at 9B hybrid, 8-draft tree"


def pmc_traffic(key):
    """HBM bytes per launch of a workload's dominant kernel, from the committed rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE scaled by the counters' readings for a 256 MiB copy), or None."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            return json.load(f)[key]["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def read_roof(key):
    """The single-launch streaming-read roof (GB/s) at a launch size, from the committed summary of
    `bench.py --workload read` (the best over the work-group counts tried), or None."""
    try:
        with open(os.path.join(ROOT, "profiles", "read_roof.json")) as f:
            return json.load(f)["roof_gbs"][key]
    except (OSError, KeyError, ValueError):
        return None


def gptq_weight(N, K, gen, dev, tiled=True, integral=False):
    """A random GPTQ int4 matrix (q ~ U{-8..7}, fp16 G128 scales ~ U(0.005, 0.02)) in the packed-W4
    contract. integral=False (default): the fp16 group scales relative to the channel scale, decoded
    per weight by rint (the reference contract); True: the group scales become 4-bit integer multiples
    of a channel scale (the integral decode; up to smax / (30 s_g) relative scale error per group)."""
    import torch
    from mdx import _lib, layout
    q = torch.randint(-8, 8, (N, K), generator=gen, device=dev, dtype=torch.int8)
    s = (torch.rand(N, K // 128, generator=gen, device=dev) * 0.015 + 0.005).half()
    packed, s_rel, sch, _ = layout.gptq_pack(q, s, 128, integral=integral)
    w = layout.W4(packed, s_rel, sch, None, decode=_lib.DECODE_INTEGRAL if integral else _lib.DECODE_AUTO)
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


def ring_time(call, ring_n, steps, warmup):
    """Seconds per call of exactly `steps` calls call(0), call(1), ... cycling through a ring of
    `ring_n` weight copies: one captured graph of a whole ring replayed steps // ring_n times, then a
    graph of the remaining steps % ring_n calls (HIP events on the capturing stream's order)."""
    import torch
    full, rem = divmod(steps, ring_n)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(ring_n):
            call(i)  # eager warm-up (workspaces, LDS attributes)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graphs = []
    for n in (ring_n if full else 0, rem):
        if n:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(n):
                    call(i)
            graphs.append((g, full if n == ring_n and full else 1))
    for _ in range(max(1, -(-warmup // ring_n))):
        graphs[0][0].replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for g, reps in graphs:
        for _ in range(reps):
            g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / steps


def fresh_pool():
    """Hand the caching allocator's unused segments back to the runtime, so the next leg's model is
    allocated as a fresh serving process would allocate it, not carved out of the segments the previous
    legs' weight rings left behind."""
    import gc
    import torch
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def cpu_info():
    """(model name, threads used by the CPU baseline): numpy's BLAS pool is pinned to the process's
    affinity count for the timed leg."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model, cpu_threads()


def cpu_threads():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline_mlp(ring0, rows, xb, nwb, lutb, budget_s=25.0):
    """The oracle's operator chain (RMSNorm, quantise, decode + int dot, SiLU, quantise, decode +
    int dot) on the host, on one set of the same weights: 3 warm-up calls, then the median of the
    timed calls (>= 10; up to 100 within the budget). The oracle's C restatement (oracle/cpu_mlp.c, one
    thread per share of the output channels on every core of the process's affinity; bit-identical to
    the numpy chain) where it loads, else the numpy chain with its BLAS threads pinned to that count.
    Returns (median s, calls, CPU model, threads, form)."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    sys.path.insert(0, ROOT)
    from oracle import ref
    from mdx import layout
    d = []
    for w in ring0:
        q = layout.row_major_codes(w.q).cpu().numpy()
        d.append(dict(packed=q, s=w.s.float().cpu().numpy(), sch=w.sc.cpu().numpy(), cb=None, G=128))
    model, threads = cpu_info()
    try:
        from oracle import cpu_port
        cpu_port.load(build=False)
        form = "c"
    except OSError:
        form = "numpy"
    times = []
    t_end = time.perf_counter() + budget_s
    with threadpool_limits(limits=threads):
        for i in range(103 if form == "c" else 13):
            for dd in d:
                dd.pop("w8", None)  # the decode is part of every call of the chain
            t0 = time.perf_counter()
            if form == "c":
                cpu_port.mlp(xb, nwb, 1e-6, lutb, *d, threads=threads)
            else:
                xn = ref.rmsnorm(xb, nwb, 1e-6)
                ref.mono_mlp(xn, "none", None, lutb, *d)
            dt = time.perf_counter() - t0
            if i >= 3:
                times.append(dt)
            if time.perf_counter() + dt > t_end and len(times) >= 10:
                break
    return float(np.median(times)), len(times), model, threads, form


def cpu_decode_estimate(mlp_s, mlp_algo_bytes, budget_s=20.0):
    """Config-5 CPU tok/s, composed from timed pieces of the oracle on the host (a whole 32-layer step
    on the CPU takes tens of seconds): every W4A8 GEMV of a step at the MLP chain's measured rate per
    weight byte (the CPU baseline's chain: the same decode + int dot), the bf16 lm_head (verify + 2 drafts) and the MTP
    block's bf16 GEMMs at the rate of a timed 8-row slice of the float64 bf16 linear, 24 timed GDN
    steps (8 tree rows) and 8 timed attention calls (8 rows over a 1024-token context); norms,
    RoPE, top-k and the accept walk are left out. One accepted token per step, as in the GPU line."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    sys.path.insert(0, ROOT)
    from oracle import ref
    rng = np.random.default_rng(5)
    H, I, V = 4096, 12288, 151936
    bf = lambda *shape: ref.f32_to_bf16(rng.standard_normal(shape).astype(np.float32) * 0.05)

    def med(fn, n=3):
        ts = []
        t_end = time.perf_counter() + budget_s / 4
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
            if time.perf_counter() > t_end:
                break
        return float(np.median(ts))

    w4_layer = {"mlp": 3 * H * I, "gdn": (2 * 16 * 128 + 32 * 128 + 32 * 128) * H + H * 32 * 128,
                "attn": (2 * 32 * 128 + 2 * 8 * 128) * H + H * 32 * 128}
    w4_bytes = (32 * w4_layer["mlp"] + 24 * w4_layer["gdn"] + 8 * w4_layer["attn"]) * (0.5 + 2 / 128)
    w4_s = mlp_s * w4_bytes / mlp_algo_bytes
    _, threads = cpu_info()
    with threadpool_limits(limits=threads):
        xs, ws = bf(8, H), bf(16384, H)
        bf_rate = 16384 * H * 2 / med(lambda: ref.bf16_linear_f64(xs, ws))
        mtp_bytes = 486.5e6
        bf_s = (3 * V * H * 2 + 2 * mtp_bytes) / bf_rate
        HK, HV, R, slots = 16, 32, 8, 8
        C = 2 * HK * 128 + HV * 128
        tree = ref.tree_from_spec(ref.spec_of_widths((4, 3)), slots)
        parents = tree[0][:R]
        ctl = np.array([0, 0] + [0] * slots + parents + ref.verify_program(parents, R))
        st = dict(conv_state=ref.bf16_to_f32(bf(C, 3)), pb=np.zeros((2, slots, C), np.float32),
                  qb=np.zeros((2, slots, C), np.float32), rec=(rng.standard_normal((HV, 128, 128)) * 0.1).astype(np.float32),
                  gates=np.zeros((2, slots, HV, 2), np.float32), sums=np.zeros((2, slots, HK, 2), np.float32))
        a, b = ref.gdn_ab(bf(R, H), bf(HV, H), bf(HV, H))
        args_g = (ref.bf16_to_f32(bf(R, C)), ref.bf16_to_f32(bf(R, HV * 128)), a, b, ref.bf16_to_f32(bf(C, 4)),
                  rng.uniform(-1, 1, HV).astype(np.float32), -np.exp(rng.uniform(-1, 0.5, HV)).astype(np.float32),
                  ref.bf16_to_f32(bf(128)), 1e-6, 128 ** -0.5, ctl, R, HK, slots)
        gdn_s = med(lambda: ref.gdn_step({k: v.copy() for k, v in st.items()}, *args_g))
        L = 1024
        q, k, v = (rng.standard_normal(sh).astype(np.float32) for sh in ((32, R, 128), (8, L + 64, 128), (8, L + 64, 128)))
        xk, xv = (rng.standard_normal((8, R, 128)).astype(np.float32) for _ in range(2))
        attn_s = med(lambda: ref.attention_f64(q, k, v, L, xk, xv, ref.tree_mask(tree[0][:R])))
    step_s = w4_s + bf_s + 24 * gdn_s + 8 * attn_s
    return {"value": round(1.0 / step_s, 5), "unit": "tok/s", "cores": threads, "kind": "port",
            "ms_per_step": round(step_s * 1e3, 1),
            "components_ms": {"w4a8_gemvs": round(w4_s * 1e3, 1), "bf16_gemms": round(bf_s * 1e3, 1),
                              "gdn_steps": round(24 * gdn_s * 1e3, 1), "attention": round(8 * attn_s * 1e3, 1)},
            "sample": "composed from timed oracle pieces: W4A8 GEMVs at the MLP chain's rate (per weight byte, the "
                      "CPU baseline's MLP chain), one 8-row 16384-row "
                      "slice of the bf16 linear, one GDN step and one attention call (medians of up to 3), "
                      "scaled to a 32-layer step; norms, RoPE and top-k left out"}


SCALES_DATA = {
    "faithful": "fp16 G128 group scales ~U(0.005, 0.02) kept as fp16 ratios to a per-channel scale (the "
                "reference's W4 contract, the form checkpoint ingestion produces), decoded per weight by rint",
    "integral": "fp16 G128 group scales ~U(0.005, 0.02) re-quantised to 4-bit integer multiples of a channel "
                "scale (up to smax / (30 s_g) relative scale error per group), integral decode",
}

# the gate/up kernel each scale form runs at 1 row (template arguments: MFMA, R, scale dtype, ring, source)
GATEUP_KERNEL = {
    "faithful": "gemv_kernel<true, 4, 1, 4, 8> (gate/up pair, int8 activation staged by DMA, per-weight decode through "
                "16-byte LDS tables, products on v_mfma_i32_16x16x32_i8)",
    "integral": "gemv_kernel<false, 1, 1, 4, 4> (gate/up pair, int8 activation staged by DMA, integral decode only, "
                "v_dot4_i32_i8)",
}
LINEAR_KERNEL = {
    "faithful": "gemv_kernel<true, 4, 1, 4, 8> (per-weight decode through 16-byte LDS tables, MFMA products)",
    "integral": "gemv_kernel<false, 1, 1, 4, 4> (integral decode only, v_dot4_i32_i8)",
}


def bench_mlp(args, dev):
    """Config 2: the fused MLP block over a weight ring, in the scale form args.scales (faithful by
    default); the other form is timed beside it as a labelled extra unless --no-extra."""
    import torch
    from mdx import _C, _lib, layout
    gen = torch.Generator(device=dev).manual_seed(2)
    H, I, M = 4096, 12288, args.rows
    per = mlp_bytes(M)
    ring_n = max(2, -(-2 * 256 * 2 ** 20 // (3 * H * I // 2)) + 1)  # > 2x the 256 MB Infinity Cache
    primary = args.scales
    other = "integral" if primary == "faithful" else "faithful"

    def make_ring(form):
        integral = form == "integral"
        return [(gptq_weight(I, H, gen, dev, integral=integral), gptq_weight(I, H, gen, dev, integral=integral),
                 gptq_weight(H, I, gen, dev, integral=integral)) for _ in range(ring_n)]

    ring = make_ring(primary)
    x = torch.randn(M, H, generator=gen, device=dev).to(torch.bfloat16)
    nw = (1 + 0.02 * torch.randn(H, generator=gen, device=dev)).to(torch.bfloat16)
    lut = layout.silu_lut(dev)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
    ws = torch.zeros(_lib.lib().mdx_mono_mlp_workspace(M, H, I), dtype=torch.uint8, device=dev)

    def mlp(r):
        def call(i):
            g_, u_, d_ = r[i]
            _C.mono_mlp_w4(x, _lib.ROT_NONE, None, lut, g_, u_, d_, norm_w=nw, eps=1e-6, out=out, ws=ws)
        return call

    # the dominant kernel alone: the gate/up GEMV launch over the same ring
    q1, s1 = _C.rms_rot_quant(x, nw, 1e-6)
    hbuf = torch.empty(M, I, dtype=torch.bfloat16, device=dev)

    def gateup(r):
        def call(i):
            g_, u_, _ = r[i]
            _C.stream_gemv(q1, s1, [g_, u_], [hbuf], gate_up=True, silu_lut=lut)
        return call

    t_call = ring_time(mlp(ring), ring_n, args.steps, args.warmup)
    t_gu = ring_time(gateup(ring), ring_n, args.steps, args.warmup)
    gu_b = gateup_bytes(M)
    res = {
        "metric": METRIC,
        "value": round(per / t_call / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_call * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xint4->int32, bf16 out",
        "data": f"synthetic (seeded GPTQ int4 weights; {SCALES_DATA[primary]}; N(0,1) activations)",
        "config": {"workload": f"fused W4A8 SwiGLU MLP 4096->2x12288->4096, RMSNorm 1e-6, rows={M}, "
                               f"tile-major weights, {ring_n}-copy weight ring",
                   "rows": M, "hidden": H, "intermediate": I, "group_size": 128, "scales": primary,
                   "algorithmic_bytes_per_step": per, "frac_of_peak": round(per / t_call / 1e9 / PEAK_HBM_GBS, 4)},
        "roofline": {"bound": "hbm", "kernel": GATEUP_KERNEL[primary] if M == 1 else "gemv_kernel (gate/up pair)",
                     "achieved": round(gu_b / t_gu / 1e9, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gu_b / t_gu / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": pmc_traffic(f"mlp_gateup_rows1_{primary}") if M == 1 else None,
                     "algorithmic_bytes_per_launch": gu_b, "avg_launch_us": round(t_gu * 1e6, 3),
                     "single_launch_read_roof_gbs": read_roof("52MB")},
    }
    if M >= 2:
        # the MFMA path (v_mfma_i32_16x16x32_i8 on rows padded to 16): issued int8 operations of the gate/up
        # launch per second against the dense int8 peak (counters: profiles/mfma_mlp8_attn16.md)
        ops = 2 * 16 * -(-M // 16) * 2 * I * H
        res["roofline"]["mfma_util"] = round(ops / t_gu / PEAK_I8_OPS, 4)
        res["roofline"]["mfma_useful_util"] = round(2 * M * 2 * I * H / t_gu / PEAK_I8_OPS, 4)
    cpu_ring = ring[0]
    if not args.no_extra:
        # the same block and gate/up launch in the other scale form (a labelled extra, not the headline)
        del ring
        torch.cuda.empty_cache()
        ring_o = make_ring(other)
        t_o = ring_time(mlp(ring_o), ring_n, args.steps, args.warmup)
        t_ogu = ring_time(gateup(ring_o), ring_n, args.steps, args.warmup)
        res[f"{other}_scales"] = {
            "value": round(per / t_o / 1e9, 2), "unit": "GB/s", "ms_per_step": round(t_o * 1e3, 5),
            "gateup_us": round(t_ogu * 1e6, 3), "gateup_gbs": round(gu_b / t_ogu / 1e9, 2),
            "gateup_kernel": GATEUP_KERNEL[other] if M == 1 else "gemv_kernel (gate/up pair)",
            "data": SCALES_DATA[other]}
        if primary == "integral":
            cpu_ring = ring_o[0]
    if not args.no_cpu:
        xb = x.view(torch.int16).cpu().numpy().view("uint16")
        nwb = nw.view(torch.int16).cpu().numpy().view("uint16")
        lutb = lut.view(torch.int16).cpu().numpy().view("uint16")
        t_cpu, n, model, threads, form = cpu_baseline_mlp(cpu_ring, M, xb, nwb, lutb)
        res["_cpu_mlp_s"] = t_cpu
        what = (f"the oracle's C restatement (oracle/cpu_mlp.c: per-group decode tables, int32 dots, {threads} "
                f"threads over the output channels; bit-identical to the numpy oracle)" if form == "c" else
                f"the numpy oracle chain (decode + float64 int dot; BLAS threads pinned to {threads})")
        res["cpu_baseline"] = {"value": round(per / t_cpu / 1e9, 4), "unit": "GB/s", "cores": threads,
                               "kind": "port", "ms_per_step": round(t_cpu * 1e3, 2), "cpu_model": model,
                               "sample": f"median of {n} MLP calls (after 3 warm-up calls) of {what} on one weight "
                                         f"set of the fp16-faithful form, same rows"}
    return res


def bench_linear(args, dev):
    import torch
    from mdx import _C
    gen = torch.Generator(device=dev).manual_seed(1)
    N = K = 4096
    M = args.rows
    per = linear_bytes(M)
    ring_n = -(-2 * 256 * 2 ** 20 // (N * K // 2)) + 1
    ring = [gptq_weight(N, K, gen, dev, integral=args.scales == "integral") for _ in range(ring_n)]
    x = torch.randn(M, K, generator=gen, device=dev).to(torch.bfloat16)
    q, s = _C.quant_rows(x)
    s = s.view(-1)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)

    t = ring_time(lambda i: _C.stream_gemv(q, s, [ring[i]], [out]), ring_n, args.steps, args.warmup)
    return {
        "metric": METRIC, "value": round(per / t / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(t * 1e3, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8xint4->int32, bf16 out",
        "data": f"synthetic (seeded GPTQ int4 weights; {SCALES_DATA[args.scales]})",
        "config": {"workload": f"single W4A8 linear M={M} K=N=4096 G128, {ring_n}-copy weight ring", "rows": M,
                   "scales": args.scales, "algorithmic_bytes_per_step": per},
        "roofline": {"bound": "hbm", "kernel": LINEAR_KERNEL[args.scales] if M == 1 else "gemv_kernel",
                     "achieved": round(per / t / 1e9, 2),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(per / t / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": pmc_traffic(f"linear_rows1_{args.scales}") if M == 1 else None, "avg_launch_us": round(t * 1e6, 3),
                     "single_launch_read_roof_gbs": read_roof("8.7MB")},
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
    """bf16 lm_head of the hybrid stack: vocab 151936 x hidden 4096, `rows` decode rows (--head int8: the
    int8 ConvRot head through the W8A8 linear)."""
    import torch
    from mdx import _C, layout
    gen = torch.Generator(device=dev).manual_seed(5)
    V, H, M = 151936, 4096, args.rows
    if args.head == "int8":
        per = V * H + V * 4 + M * (H + 4) + M * V * 2
        w8 = layout.tile_major_i8(torch.randint(-127, 128, (V, H), generator=gen, device=dev, dtype=torch.int8))
        s8 = torch.rand(V, generator=gen, device=dev) * 1e-3 + 1e-4
        x8 = torch.randint(-128, 128, (M, H), generator=gen, device=dev, dtype=torch.int8)
        xs = torch.rand(M, generator=gen, device=dev) * 0.05 + 0.01
        out = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
        steps = max(1, args.steps // 5)
        t = ring_time(lambda i: _C.int8_linear_prequantized(x8, xs, w8, s8, tiled=True, out=out), 1, steps, args.warmup)
        gbs = per / t / 1e9
        return _line(args, round(gbs, 2), "GB/s", t, steps, "int8 x int8 -> int32 (MFMA), bf16 out",
                     "synthetic (seeded int8 weights and rows, per-row scales)",
                     {"workload": f"int8 ConvRot lm_head 151936x4096, rows={M}, tile-major", "rows": M,
                      "algorithmic_bytes_per_step": per},
                     {"bound": "hbm", "kernel": "int8_linear_kernel", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS,
                      "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
                      "avg_launch_us": round(t * 1e6, 3)})
    per = V * H * 2 + M * H * 2 + M * V * 2
    w = layout.tile_major_bf16((torch.randn(V, H, generator=gen, device=dev) * 0.02).bfloat16())
    x = torch.randn(M, H, generator=gen, device=dev).bfloat16()
    out = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
    steps = max(1, args.steps // 10)  # (about 0.2 ms per call)
    t = ring_time(lambda i: _C.bf16_linear(x, w, tiled=True, out=out), 1, steps, args.warmup)
    gbs = per / t / 1e9
    return _line(args, round(gbs, 2), "GB/s", t, steps, "bf16 x bf16 -> fp32 acc, bf16 out",
                 "synthetic (seeded N(0, 0.02) weights, N(0,1) rows)",
                 {"workload": f"bf16 lm_head 151936x4096, rows={M}, tile-major", "rows": M,
                  "algorithmic_bytes_per_step": per},
                 {"bound": "hbm", "kernel": "bf16_stream_kernel", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS,
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

    t = ring_time(lambda i: _C.attn_dpas(q, caches[i][0], caches[i][1], sl, xk, xv, mask, 0), ring_n, args.steps,
                  args.warmup)
    gbs = per / t / 1e9
    return _line(args, round(gbs, 2), "GB/s", t, args.steps, "bf16 x bf16 -> fp32 (MFMA), bf16 out",
                 "synthetic (seeded N(0,1) KV cache and rows)",
                 {"workload": f"tree-verify decode attention, 32q/8kv heads, head_dim 128, 16 rows, ctx={L}, "
                              f"{ring_n}-copy KV ring", "ctx": L, "rows": S, "algorithmic_bytes_per_step": per},
                 {"bound": "hbm", "kernel": "attn2_kernel + attn_merge_kernel", "achieved": round(gbs, 2),
                  "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                  # fetched and written bytes of both launches per call (the partials included)
                  "traffic": pmc_traffic(f"attn_tree16_ctx{L}"),
                  "avg_launch_us": round(t * 1e6, 3),
                  # S^T = K Q^T and O^T = V^T P^T on bf16 MFMA: 4 H S L D flops per call against the dense peak
                  "mfma_util": round(4 * H * S * L * D / t / PEAK_BF16_FLOPS, 4)})


def bench_stack(args, dev, tokens=0, two_stage=False, head="bf16"):
    """The full synthetic 32-layer hybrid stack (3 GDN : 1 attention, hidden 4096, MLP 12288, W4A8
    GPTQ G128), 1-layer bf16 MTP draft block, bf16 lm_head over 151936, tree_spec (4, 3) (8 rows, 2
    drafts per step), top-k 20 sampling; a seeded random prompt is prefilled (not timed), then each
    decode step is one replayed HIP graph. value = accepted tokens per second. tokens > 0: decode
    until that many tokens are committed (chunks of 64 steps, each timed by events, the committed
    count read between chunks); else exactly `steps` steps. head "int8": the int8 ConvRot lm_head (W8A8) for
    the verify and the drafts instead of the bf16 one."""
    import torch
    from mdx import hybrid
    fresh_pool()
    steps, warm = args.steps, max(args.warmup, 2)
    per = 3  # at most len(widths) + 1 tokens committed per step
    budget = tokens + 64 if tokens else steps
    cap = args.prompt + per * (budget + warm + 4) + 64
    cfg = hybrid.HybridConfig(cap=cap, two_stage=two_stage, head=head, predictable=getattr(args, "predictable", False),
                              scales=args.scales, gdn_fold=not getattr(args, "gdn_split", False))
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
    t, done, got = 0.0, 0, 0
    while True:
        n = min(64, steps - done) if not tokens else 64
        if n <= 0 or (tokens and got >= tokens):
            break
        torch.cuda.synchronize()
        e0.record()
        m.replay(n)
        e1.record()
        torch.cuda.synchronize()
        t += e0.elapsed_time(e1) / 1e3
        done += n
        got = int(m.st[0].item()) - st0
    per_step = t / done
    what = f"{got} tokens decoded" if tokens else f"{done} decode steps"
    hd = "int8 ConvRot lm_head (W8A8)" if head == "int8" else "bf16 lm_head"
    return _line(args, round(got / t, 2), "tok/s", per_step, done, f"W4A8 int8 x int4 -> int32; bf16 draft block, {hd}",
                 f"synthetic (random-init weights, GPTQ int4 with {SCALES_DATA[args.scales]}; seeded random prompt)",
                 {"workload": f"32-layer W4A8 hybrid (24 GDN + 8 attention), hidden 4096, MLP 12288, vocab 151936 "
                              f"({hd}), MTP draft{' (two-stage head)' if two_stage else ''}, tree (4, 3), top-k 20, "
                              f"prompt {args.prompt}, {what}",
                  "prompt": args.prompt, "steps": done, "tokens": got, "scales": args.scales,
                  "accepted_per_step": round(got / done, 3), "ms_per_step": round(per_step * 1e3, 4),
                  "setup_s": round(setup, 1)})


def bench_stack_auto(args, dev, tokens=512):
    """The full stack with the adaptive tree (auto): decode until `tokens` are committed; each step replays the
    current tree's draft and verify graphs with events between them, every 32 steps the acceptance ranks and
    device times choose the tree. value = committed tokens per second of wall time (the adaptive
    bookkeeping, its host reads and any new tree's capture included)."""
    import torch
    from mdx import hybrid
    fresh_pool()
    cap = args.prompt + 8 * (tokens + 64) + 64
    cfg = hybrid.HybridConfig(cap=cap, auto=True, two_stage=args.two_stage, head=args.head,
                              predictable=getattr(args, "predictable", False), scales=args.scales,
                              gdn_fold=not getattr(args, "gdn_split", False))
    t0 = time.perf_counter()
    m = hybrid.HybridModel(cfg, dev, seed=5)
    m.prefill(torch.randint(0, cfg.vocab, (args.prompt,), generator=torch.Generator().manual_seed(5)))
    m.decode_auto(64)  # warm: the first trees captured, the clock past its warm-up
    torch.cuda.synchronize()
    setup = time.perf_counter() - t0
    got = steps = 0
    widths = []
    t1 = time.perf_counter()
    while got < tokens:
        out = m.decode_auto(64)
        got += out["tokens"]
        steps += out["steps"]
        widths += out["widths"]
    torch.cuda.synchronize()
    t = time.perf_counter() - t1
    final = widths[-1]
    return _line(args, round(got / t, 2), "tok/s", t / steps, steps, "W4A8 int8 x int4 -> int32; bf16 draft block",
                 "synthetic (" + ("predictable" if cfg.predictable else "random-init") + " weights, seeded random prompt)",
                 {"workload": f"32-layer W4A8 hybrid, vocab 151936, MTP draft, adaptive tree (auto), top-k 20, prompt "
                              f"{args.prompt}, {got} tokens decoded", "prompt": args.prompt, "steps": steps,
                  "tokens": got, "accepted_per_step": round(got / steps, 3), "final_widths": list(final),
                  "trees_used": sorted({str(list(w)) for w in widths}), "ms_per_step": round(t / steps * 1e3, 4),
                  "draft_ms": round(out["draft_ms"], 4), "verify_ms": round(out["verify_ms"], 4),
                  "setup_s": round(setup, 1)})


def w4_bytes(w):
    return w.q.numel() + w.s.numel() * w.s.element_size() + w.sc.numel() * 4


def bench_attn_layer(args, dev):
    """One full-attention decoder layer's mixer for 16 tree-verify rows: RMSNorm + int8 quantisation,
    W4A8 q/k/v (one launch), Q/K RMSNorm + RoPE (theta 1e7, 64 rotary dims) + the KV cache write and the GQA
    tree-verify attention over `--ctx` cached tokens (32 q / 8 kv heads, head_dim 128) in one launch as the
    decode step runs them (two under MDX_ROPE_ATTN=0), quantisation of its output, W4A8 o_proj with the
    residual. Weights and KV caches cycle through a ring > 2x the Infinity Cache."""
    import torch
    from mdx import _C, _lib, hybrid
    gen = torch.Generator(device=dev).manual_seed(3)
    integ = args.scales == "integral"
    H, Hk, D, S, L, Hd = 32, 8, 128, 16, args.ctx, 4096
    cap = L + S
    cfg = hybrid.HybridConfig(cap=cap + 8)
    ftab = hybrid.rope_table(cfg, dev)
    parents = [-1, 0, 1, 2, 3, 4, 5, 6, 0, 8, 1, 10, 2, 12, 3, 14]
    depth, m = [], []
    for r, p_ in enumerate(parents):
        depth.append(depth[p_] + 1 if p_ >= 0 else 0)
        m.append((m[p_] if p_ >= 0 else 0) | (1 << r))
    mask = torch.tensor(m, dtype=torch.int32, device=dev)
    pos = torch.arange(L, L + S, dtype=torch.int64, device=dev)
    freqs = torch.index_select(ftab, 0, torch.tensor(depth, device=dev) + L).contiguous()
    seq = torch.tensor([L], dtype=torch.int32, device=dev)
    def layer_w():
        return dict(q=gptq_weight(H * D, Hd, gen, dev, integral=integ), k=gptq_weight(Hk * D, Hd, gen, dev, integral=integ),
                    v=gptq_weight(Hk * D, Hd, gen, dev, integral=integ), o=gptq_weight(Hd, H * D, gen, dev, integral=integ),
                    key=torch.randn(1, Hk, cap, D, generator=gen, device=dev).bfloat16(),
                    value=torch.randn(1, Hk, cap, D, generator=gen, device=dev).bfloat16())
    first = layer_w()
    per_w = sum(w4_bytes(first[k]) for k in "qkvo")
    per = per_w + 2 * Hk * L * D * 2 + 2 * Hk * S * D * 2 + 2 * S * Hd * 2 + Hd * 2
    ring_n = _ring_count(per_w + 2 * Hk * cap * D * 2)
    ring = [first] + [layer_w() for _ in range(ring_n - 1)]
    x = torch.randn(S, Hd, generator=gen, device=dev).bfloat16()
    nw = (1 + 0.02 * torch.randn(Hd, generator=gen, device=dev)).bfloat16()
    qn = (1 + 0.1 * torch.randn(D, generator=gen, device=dev)).bfloat16()
    kn = (1 + 0.1 * torch.randn(D, generator=gen, device=dev)).bfloat16()
    xo = torch.empty_like(x)
    xn = torch.empty_like(x)
    qkv = [torch.empty(S, n, dtype=torch.bfloat16, device=dev) for n in (H * D, Hk * D, Hk * D)]
    qh = torch.empty(1, H, S, D, dtype=torch.bfloat16, device=dev)
    kh = torch.empty(1, Hk, S, D, dtype=torch.bfloat16, device=dev)
    y = torch.empty(1, S, H * D, dtype=torch.bfloat16, device=dev)
    q2 = torch.empty(S, H * D, dtype=torch.int8, device=dev)
    s2 = torch.empty(S, dtype=torch.float32, device=dev)

    fused = _C.rope_attn_fits(H, Hk, S, D, 64)

    def call(i):
        w = ring[i]
        q1, s1 = _C.rms_rot_quant(x, nw, 1e-6, _lib.ROT_NONE, None, xn_out=xn)
        _C.stream_gemv(q1, s1, [w["q"], w["k"], w["v"]], qkv)
        vv = qkv[2].view(1, S, Hk, D)
        if fused:  # the decode step's form: the Q/K norm, RoPE and KV write inside the attention launch
            _C.qk_norm_rope_attn(qkv[0].view(1, S, H, D), qkv[1].view(1, S, Hk, D), vv, qn, kn, freqs, w["key"],
                                 w["value"], pos, 1e-6, 1e-6, 64, seq, mask, kh, out=y)
        else:
            _C.qk_norm_rope_kv(qkv[0].view(1, S, H, D), qkv[1].view(1, S, Hk, D), vv, qn, kn, freqs, w["key"],
                               w["value"], pos, 1e-6, 1e-6, 64, outs=(qh, kh))
            _C.attn_dpas(qh, w["key"], w["value"], seq, kh, vv.transpose(1, 2), mask, 0, out=y)
        _lib.call("mdx_rot_quant", _lib.ptr(y), None, _lib.ROT_NONE, _lib.ptr(q2), _lib.ptr(s2), S, H * D,
                  _lib.stream_of(y))
        _C.stream_gemv(q2, s2, [w["o"]], [xo], residuals=[x])

    t = ring_time(call, ring_n, args.steps, args.warmup)
    gbs = per / t / 1e9
    return _line(args, round(gbs, 2), "GB/s", t, args.steps, "W4A8 int8 x int4 -> int32; bf16 attention (MFMA)",
                 f"synthetic (seeded GPTQ int4 weights; {SCALES_DATA[args.scales]}; N(0,1) KV cache and rows)",
                 {"workload": f"full-attention layer mixer, 16 tree rows, 32q/8kv heads, head_dim 128, ctx={L}, "
                              f"{ring_n}-copy weight + KV ring", "ctx": L, "rows": S,
                  "algorithmic_bytes_per_step": per, "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4),
                  "launches_per_step": 6 if fused else 7,
                  "rope": "in the attention launch" if fused else "its own launch"})


def bench_gdn_layer(args, dev):
    """One Gated-DeltaNet layer's mixer for `--rows` chain rows (1 or 8): RMSNorm + int8 quantisation,
    W4A8 qkv | z (one launch), the causal conv (kernel 4) + gates + L2 norms and the delta-rule update of
    the fp32 128x128 state of each of 32 value heads (every row committed; one launch), the gated RMSNorm +
    quantisation, W4A8 out_proj with the residual. Weights and states cycle through a ring > 2x the
    Infinity Cache."""
    import torch
    from mdx import _C, _lib
    gen = torch.Generator(device=dev).manual_seed(4)
    integ = args.scales == "integral"
    M, Hd, HK, HV, DH, S = args.rows, 4096, 16, 32, 128, 8
    if not 1 <= M <= S:
        raise SystemExit("gdn_layer: --rows must be 1..8")
    C = 2 * HK * DH + HV * DH
    bf = dict(dtype=torch.bfloat16, device=dev)

    def layer_w():
        return dict(qkv=gptq_weight(C, Hd, gen, dev, integral=integ), z=gptq_weight(HV * DH, Hd, gen, dev, integral=integ), o=gptq_weight(Hd, HV * DH, gen, dev, integral=integ),
                    wa=(torch.randn(HV, Hd, generator=gen, device=dev) * 0.02).bfloat16(),
                    wb=(torch.randn(HV, Hd, generator=gen, device=dev) * 0.02).bfloat16(),
                    conv_w=(torch.randn(C, 4, generator=gen, device=dev) * 0.5).bfloat16(),
                    conv=torch.randn(C, 3, generator=gen, device=dev).bfloat16(),
                    pb=torch.zeros(2, S, C, **bf), qb=torch.zeros(2, S, C, **bf),
                    rec=torch.randn(HV, DH, DH, generator=gen, device=dev) * 0.1,
                    gates=torch.zeros(2, S, HV, 2, device=dev), sums=torch.zeros(2, S, HK, 2, device=dev))
    first = layer_w()
    per_w = sum(w4_bytes(first[k]) for k in ("qkv", "z", "o"))
    per = (per_w + 2 * HV * Hd * 2 + C * 4 * 2 + 2 * C * 3 * 2 + 2 * HV * DH * DH * 4 + 2 * M * Hd * 2 + Hd * 2 + DH * 2)
    ring_n = _ring_count(per)
    ring = [first] + [layer_w() for _ in range(ring_n - 1)]
    dt_bias = torch.rand(HV, generator=gen, device=dev) * 2 - 1
    g_decay = -torch.exp(torch.rand(HV, generator=gen, device=dev) * 1.5 - 1)
    gnw = (1 + 0.1 * torch.randn(DH, generator=gen, device=dev)).bfloat16()
    nw = (1 + 0.02 * torch.randn(Hd, generator=gen, device=dev)).bfloat16()
    x = torch.randn(M, Hd, generator=gen, device=dev).bfloat16()
    xo, xn = torch.empty_like(x), torch.empty_like(x)
    proj = torch.empty(M, C, **bf)
    z = torch.empty(M, HV * DH, **bf)
    zg = torch.empty(M, HV * DH, **bf)
    core = torch.empty(M, HV * DH, **bf)
    q2 = torch.empty(M, HV * DH, dtype=torch.int8, device=dev)
    s2 = torch.empty(M, dtype=torch.float32, device=dev)
    # nothing pending; a chain of M verify rows, each committed (program bit 5)
    ctl = torch.tensor([0, 0] + [0] * S + [r - 1 for r in range(M)] + [-1] * (S - M) + [r | 32 for r in range(M)]
                       + [0] * (S - M), dtype=torch.int32, device=dev)

    fold = not args.gdn_split

    def call(i):
        w = ring[i]
        q1 = s1 = None
        if not (fold and M == 1):  # (one row folded: the row prep runs in the projection launch)
            q1, s1 = _C.rms_rot_quant(x, nw, 1e-6, _lib.ROT_NONE, None, xn_out=xn)
        if fold:
            _C.gdn_proj(q1, s1, w["qkv"], w["z"], proj, z, None if M == 1 else xn, w["wa"], w["wb"], w["conv_w"],
                        w["conv"], w["pb"], w["qb"], ctl, dt_bias, g_decay, w["gates"], HK, z_gate=zg,
                        x_row=x if M == 1 else None, norm_w=nw, eps=1e-6)
            _C.gdn_delta(w["qb"], ctl, w["rec"], w["gates"], DH ** -0.5, HK, core)
        else:
            _C.stream_gemv(q1, s1, [w["qkv"], w["z"]], [proj, z])
            _C.gdn_core(proj, z, xn, w["wa"], w["wb"], w["conv_w"], w["conv"], w["pb"], w["qb"], ctl, dt_bias, g_decay,
                        w["rec"], w["gates"], w["sums"], gnw, 1e-6, DH ** -0.5, HK, core=core, raw=True)
        if fold:  # the gated RMSNorm + quantisation in the out_proj's launch at one or two rows
            _C.gnorm_linear(core, zg, gnw, 1e-6, w["o"], xo, residual=x, q=q2, scale=s2, z_gated=True)
        else:
            _lib.call("mdx_gnorm_rot_quant", _lib.ptr(core), _lib.ptr(z), _lib.ptr(gnw), 1e-6, _lib.ptr(core), None,
                      _lib.ROT_NONE, _lib.ptr(q2), _lib.ptr(s2), M, HV * DH, _lib.stream_of(core))
            _C.stream_gemv(q2, s2, [w["o"]], [xo], residuals=[x])

    t = ring_time(call, ring_n, args.steps, args.warmup)
    gbs = per / t / 1e9
    return _line(args, round(gbs, 2), "GB/s", t, args.steps, "W4A8 int8 x int4 -> int32; fp32 recurrent state",
                 f"synthetic (seeded GPTQ int4 weights; {SCALES_DATA[args.scales]}; state N(0, 0.1))",
                 {"workload": f"Gated-DeltaNet layer mixer, {M} chain rows, 16 key / 32 value heads of 128, conv 4, "
                              f"{ring_n}-copy weight + state ring", "rows": M,
                  "algorithmic_bytes_per_step": per, "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4),
                  "launches_per_step": (3 if M == 1 else 4 if M <= 2 else 5) if fold else 6,
                  "gdn_path": (("row prep, " if M == 1 else "") + "conv + gates in the projection launch" +
                               ("; gated RMSNorm + quantisation in the out_proj launch" if M <= 2 else ""))
                              if fold else "six launches"})


def bench_read(args, dev):
    """Single-launch read roofs: one streaming read (the GEMV's load pattern, libmdx's calibration
    kernel) per launch at the decode path's matrix sizes, over a ring of buffers > 2x the Infinity
    Cache, for several work-group counts. The best per size is the roof a one-launch GEMV of that size
    can reach."""
    import torch
    from mdx import _lib
    sizes = {"8.7MB": 8679424, "26MB": 25990144, "52MB": 52031488, "78MB": 77996032}
    buf_bytes = max(sizes.values())
    ring_n = -(-2 * 256 * 2 ** 20 // min(sizes.values())) + 1
    bufs = [torch.ones(buf_bytes // 4, dtype=torch.int32, device=dev) for _ in range(min(ring_n, 16))]
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    out = {}
    for key, nbytes in sizes.items():
        nbytes = nbytes // 1024 * 1024
        # distinct regions (buffer, offset) of this size, enough to exceed 2x the cache
        regions = [b.data_ptr() + off for off in range(0, buf_bytes - nbytes + 1, nbytes) for b in bufs]
        rn = min(len(regions), max(2, -(-2 * 256 * 2 ** 20 // nbytes) + 1))
        best = None
        for wgs in (256, 512, 768, 1024, 2048):
            t = ring_time(lambda i: _lib.call("mdx_stream_read", ctypes.c_void_p(regions[i]), nbytes, wgs,
                                              _lib.ptr(sink), _lib.stream_of(sink)), rn, args.steps, args.warmup)
            gbs = nbytes / t / 1e9
            out[f"{key}_wg{wgs}"] = {"us": round(t * 1e6, 3), "gbs": round(gbs, 1)}
            best = gbs if best is None else max(best, gbs)
        out[key] = round(best, 1)
    roof = {k: v for k, v in out.items() if "_wg" not in k}
    return {"metric": "single-launch streaming read GB/s", "value": roof["52MB"], "unit": "GB/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "u8", "data": "synthetic",
            "config": {"workload": "read roof per launch size (calibration)", "roof_gbs": roof},
            "detail": {k: v for k, v in out.items() if "_wg" in k}}


def bench_copy(args, dev):
    """Calibration workload: a plain device copy of 256 MiB (read 256 MiB, write 256 MiB). Its
    FETCH_SIZE / WRITE_SIZE counters give the scale factor of the traffic figures."""
    import torch
    n = 256 * 2 ** 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    steps = max(1, args.steps // 100)
    t = ring_time(lambda i: dst.copy_(src), 1, steps, args.warmup)
    return {"metric": "device copy GB/s (read + write)", "value": round(2 * n / t / 1e9, 2), "unit": "GB/s",
            "n_gpus": 1, "steps": steps, "warmup": args.warmup, "ms_per_step": round(t * 1e3, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8", "data": "synthetic",
            "config": {"workload": "copy of 256 MiB (traffic calibration)", "bytes_read": n, "bytes_written": n}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--rows", type=int, default=1)
    ap.add_argument("--workload", choices=["mlp", "linear", "copy", "lmhead", "attn", "stack", "read", "attn_layer",
                                           "gdn_layer"], default="mlp")
    ap.add_argument("--tokens", type=int, default=0, help="stack: decode until this many tokens are committed")
    ap.add_argument("--predictable", action="store_true", help="stack: synthetic weights whose next token is "
                    "predictable (t -> t + 1), so the drafts are accepted (HybridConfig.predictable)")
    ap.add_argument("--two-stage", action="store_true", help="stack: drafts score the vocabulary with an int4 copy "
                                                               "of the lm_head and recompute their candidates exactly")
    ap.add_argument("--auto", action="store_true", help="stack: the adaptive tree (decode_auto)")
    ap.add_argument("--head", choices=["bf16", "int8"], default="bf16",
                    help="stack / lmhead: the bf16 lm_head or the int8 ConvRot one (W8A8)")
    ap.add_argument("--prompt", type=int, default=1024, help="stack: prompt tokens (prefilled, not timed)")
    ap.add_argument("--ctx", type=int, default=8192, help="attention context length")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-decode", action="store_true", help="mlp: skip the full-stack decode leg")
    ap.add_argument("--no-extra", action="store_true", help="mlp: skip the other scale form's leg")
    ap.add_argument("--gdn-split", action="store_true",
                    help="gdn_layer / stack: the conv + gates as their own launch instead of in the projection launch")
    ap.add_argument("--scales", choices=["faithful", "integral"], default="faithful",
                    help="W4 group scales: fp16 ratios decoded per weight (the reference contract, default) or "
                         "the lossy 4-bit integral re-quantisation")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU only: the 9B stack scales as one "
                                   "data-parallel replica per GPU (about 5 GB each); tensor-parallel "
                                   "sharding of the GEMVs, heads and lm_head is not implemented or "
                                   "measured here", "n_gpus": args.gpus}))
        sys.exit(2)
    # kernel arguments read from host memory rather than a device-memory copy (a HIP runtime setting,
    # read when the runtime starts): the graph-replayed decode step measured 2.80 against 2.87 ms per
    # step with it, the MLP lines unchanged. A value the caller set is kept.
    os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "0")
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm device"}))
        sys.exit(1)
    dev = torch.device("cuda", 0)
    if args.workload == "stack":
        if args.auto:
            res = bench_stack_auto(args, dev, tokens=args.tokens or 512)
        else:
            res = bench_stack(args, dev, tokens=args.tokens, two_stage=args.two_stage, head=args.head)
    else:
        res = {"mlp": bench_mlp, "linear": bench_linear, "copy": bench_copy, "lmhead": bench_lmhead,
               "attn": bench_attn, "read": bench_read, "attn_layer": bench_attn_layer,
               "gdn_layer": bench_gdn_layer}[args.workload](args, dev)
    if args.workload == "mlp" and not args.no_decode:
        # the second half of the metric: decode tok/s of the full synthetic hybrid stack (1024-token
        # prompt, 512 tokens decoded by graph-replayed steps)
        sub = argparse.Namespace(**vars(args))
        sub.steps, sub.warmup, sub.prompt = 0, 4, 1024
        # drafts score the vocabulary with an int4 copy of the bf16 head and recompute their candidates'
        # logits exactly (the verify pass keeps the full bf16 lm_head and its exact top-20): a draft only
        # proposes tokens, the verify decides what is committed
        d = bench_stack(sub, dev, tokens=512, two_stage=True)
        res["decode"] = {"metric": "decode tok/s at 9B hybrid, 8-draft tree", "value": d["value"], "unit": "tok/s",
                         "ms_per_step": d["config"]["ms_per_step"], "scales": args.scales,
                         "accepted_per_step": d["config"]["accepted_per_step"], "workload": d["config"]["workload"]}
        # the same decode on the other scale form's weights (a labelled extra)
        osub = argparse.Namespace(**vars(sub))
        osub.scales = "integral" if args.scales == "faithful" else "faithful"
        do = bench_stack(osub, dev, tokens=512, two_stage=True)
        res[f"decode_{osub.scales}_scales"] = {"value": do["value"], "unit": "tok/s",
                                                "ms_per_step": do["config"]["ms_per_step"],
                                                "accepted_per_step": do["config"]["accepted_per_step"],
                                                "data": SCALES_DATA[osub.scales]}
        # the same decode with the drafts' full bf16 lm_head (one stage)
        d2 = bench_stack(sub, dev, tokens=512)
        res["decode_one_stage_drafts"] = {"value": d2["value"], "unit": "tok/s", "ms_per_step": d2["config"]["ms_per_step"],
                                          "accepted_per_step": d2["config"]["accepted_per_step"],
                                          "workload": d2["config"]["workload"]}
        # the same decode with the reference's own head format: an int8 ConvRot lm_head (W8A8) for the verify
        # and the drafts' exact pick
        d4 = bench_stack(sub, dev, tokens=512, two_stage=True, head="int8")
        res["decode_int8_convrot_head"] = {"value": d4["value"], "unit": "tok/s", "ms_per_step": d4["config"]["ms_per_step"],
                                           "accepted_per_step": d4["config"]["accepted_per_step"],
                                           "workload": d4["config"]["workload"]}
        # the same decode on weights whose next token is predictable: the drafts are accepted, every step
        # commits len(widths) + 1 tokens (the same kernels on the same shapes)
        sub.predictable = True
        d3 = bench_stack(sub, dev, tokens=512, two_stage=True)
        res["decode_predictable_weights"] = {"value": d3["value"], "unit": "tok/s", "ms_per_step": d3["config"]["ms_per_step"],
                                             "accepted_per_step": d3["config"]["accepted_per_step"],
                                             "workload": d3["config"]["workload"] + ", predictable synthetic weights"}
        if "_cpu_mlp_s" in res:
            res["decode"]["cpu_baseline"] = cpu_decode_estimate(res["_cpu_mlp_s"], mlp_bytes(1))
        # the other configurations' units, each timed by its own workload (weights and caches in rings
        # larger than twice the Infinity Cache): the 16-row full-attention layer at two context lengths,
        # the GDN layer step at 1 and 8 rows
        layers = {}
        for key, fn, kw in (("attention_layer_16rows_ctx2048", bench_attn_layer, {"ctx": 2048}),
                            ("attention_layer_16rows_ctx8192", bench_attn_layer, {"ctx": 8192}),
                            ("gdn_layer_1row", bench_gdn_layer, {"rows": 1}),
                            ("gdn_layer_8rows", bench_gdn_layer, {"rows": 8})):
            lsub = argparse.Namespace(**vars(args))
            lsub.steps, lsub.warmup = 200, 10
            for k, v in kw.items():
                setattr(lsub, k, v)
            fresh_pool()
            r = fn(lsub, dev)
            layers[key] = {"value": r["value"], "unit": r["unit"], "us_per_step": round(r["ms_per_step"] * 1e3, 2),
                           "frac_of_peak": round(r["value"] / PEAK_HBM_GBS, 4), "workload": r["config"]["workload"]}
        res["layers"] = layers
    res.pop("_cpu_mlp_s", None)
    res["runtime"] = {"HIP_FORCE_DEV_KERNARG": os.environ["HIP_FORCE_DEV_KERNARG"]}
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
