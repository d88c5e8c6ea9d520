#!/usr/bin/env python3
"""Benchmark: µs per INT4 FFN decode call (M=1) on one MI355X, plus achieved HBM GB/s.

Workload (default): the Qwen3-4B-shaped dense FFN, hidden 2560,
intermediate 9728, INT4 group-128 weights with BF16 scales, BF16 activation, one decode token.
Weights are synthetic (BF16 ~N(0, 0.02), quantized on the device by the library's quantizer,
re-laid into tile order), activations BF16 ~N(0, 1). 16 distinct weight sets (616 MB) rotate
so the 256 MB Infinity Cache cannot serve the stream; one "step" is one FFN call (fused
gate/up/SiLU kernel + down kernel) on the next set, inputs already resident in HBM.

``--config 2`` runs the 27B FFN (hidden 5120, intermediate 17408) over 64 distinct layers
(8.8 GB); ``--config 4`` its tp=2 rank-0 slice; ``--config 0`` the single K=2560, N=9728
linear; ``--config 3`` config 1 at M = --m; ``--config 5`` the single linear at the shape the
reference publishes its per-call INT4 figures for (N=4096, K=5120: 52.1 us at M=1 on an A40,
reference docs/plan-numeric-contract.md:1753, and its --time sweep at M = 2 / 16 / 64 / 128,
:1775-1778), at M = --m or over --m-sweep, quoted beside this run's.

Timing: the calls of one pass over the rotating sets are captured in a HIP graph (the first
pass's graph also holds the steps % sets extra calls); exactly --steps calls are replayed in
the timed region, with a HIP event on the replay stream before it and after every pass, so ``value`` is device
time per call over all --steps calls (gaps between kernels included, not Python's launch rate)
and ``config.pass_us_per_call`` gives the median, min and max over the passes.

Prints ONE JSON line.
* ``roofline`` is the dominant kernel's (the fused gate/up/SiLU GEMV, or the linear):
  algorithmic bytes per launch (packed nibbles + BF16 scales of its weight) over its average
  duration. ``frac`` uses the rocprofv3 kernel-trace average of the same workload's committed
  profile (profiles/kernel_avg_<config>.json, over the dispatches of the live-timing sections),
  ``frac_live`` the live measurement: --steps eager calls, the kernel's dispatch in each timed
  by the start/end events of w4a16_time_next_launch (hipExtLaunchKernel), whose window also
  holds the dispatch's setup (about 1 us more than the trace's duration).
* ``floor_us`` / ``floor`` (FFN configs): a pure streaming read of the call's bytes in one
  launch, as two dependent launches, and an empty launch pair, on the same rotation
  (libw4a16_floor.so).
* ``secondary`` (config 1): config 3's verify rows M = 2, 4, 8, 16 on the same weight sets.
* ``cpu_baseline`` times the CPU dequant+matmul path (numpy, BLAS) over a bounded sample.
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "haskell-infer-demo_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
CACHE_ROTATE_BYTES = 512 << 20   # rotate at least this many weight bytes (MALL is 256 MB)
KERNEL_TIMING_CHUNK = 32         # eager calls enqueued behind one spin kernel (kernel_us)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=1, choices=(0, 1, 2, 3, 4, 5))
    ap.add_argument("--m", type=int, default=None,
                    help="activation rows: --config 3 (default 4) and --config 5 (default 1)")
    ap.add_argument("--m-sweep", default=None,
                    help="--config 5 only: comma-separated row counts (e.g. 1,2,4,8,16,32,64,128), "
                         "each timed like the main line and reported in `sweep`")
    ap.add_argument("--no-secondary", action="store_true",
                    help="config 1: skip the C3 verify-row timings reported in `secondary`")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--pmc-pass", action="store_true",
                    help="for rocprofv3 --pmc: eager (no graph) calls of the two FFN kernels plus "
                         "a plain 256 MiB device copy whose byte counts calibrate the counters")
    return ap.parse_args()


def shapes(cfg, m):
    """(hidden, intermediate, M, layers-or-sets, name)."""
    if cfg == 0:
        return 2560, 9728, 1, "config0: single W4A16 linear M=1 K=2560 N=9728"
    if cfg == 1:
        return 2560, 9728, 1, "config1: Qwen3-4B dense FFN decode M=1 H=2560 I=9728"
    if cfg == 2:
        return 5120, 17408, 1, "config2: 27B dense FFN decode M=1 H=5120 I=17408, 64 layers"
    if cfg == 3:
        return 2560, 9728, m, f"config3: Qwen3-4B dense FFN verify rows M={m}"
    if cfg == 5:
        return 5120, 4096, m, (f"config5: the reference's published shape, W4A16 linear M={m} "
                               f"K=5120 N=4096")
    return 5120, 8704, 1, "config4: tp=2 rank-0 slice of config2 (I/2=8704), FP32 partial"


def make_sets(torch, w4a16, hidden, inter, count, linear_only, seed=1234):
    """Device-generated weight sets in tile order (gate/up pair + down), or single linears."""
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    sets = []
    for _ in range(count):
        def quantized(n, k):
            w = (torch.randn(n, k, generator=gen, device=dev) * 0.02).to(torch.bfloat16).float()
            p, s = w4a16.quantize_device(w)
            del w
            return p, s

        if linear_only:
            p, s = quantized(inter, hidden)
            sets.append((w4a16.TiledWeight.from_device_artifact(p, s, inter, hidden), None, (p, s)))
            continue
        gp, gs = quantized(2 * inter, hidden)   # gate rows then up rows, as the F1 pair
        dp, ds = quantized(hidden, inter)
        gu = w4a16.TiledWeight.from_device_artifact(gp, gs, 2 * inter, hidden, pair=True)
        dn = w4a16.TiledWeight.from_device_artifact(dp, ds, hidden, inter)
        keep = (gp, gs, dp, ds) if not sets else None   # artifact of set 0 for the CPU leg
        sets.append((gu, dn, keep))
    torch.cuda.synchronize()
    return sets


def _median_us(run, seconds, cap=50):
    run()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        run()
        times.append((time.perf_counter() - t0) * 1e6)
        if len(times) >= cap:
            break
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baseline(sets, hidden, inter, m, linear_only, seconds):
    """The reference's CPU path on the GPU box's host: (i) dequantize per call + FP32 BLAS matmul
    (reported as value), (ii) the matmul alone on weights dequantized once (matmul_only)."""
    import numpy as np

    from oracle import oracle

    try:
        from threadpoolctl import threadpool_info

        cores = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:  # pragma: no cover
        cores = os.cpu_count() or 1
    keep = sets[0][2]
    x = oracle.synth_activation(m, hidden, 7)
    if linear_only:
        p, s = (t.cpu().numpy() for t in keep)
        s = s.view(np.uint16)
        xf = oracle.bf16_to_f32(x).reshape(m, hidden)

        def run():
            w = oracle.dequantize_numpy(p, s, inter, hidden)
            return oracle.bf16_bits(xf @ w.T)

        w_once = oracle.dequantize_numpy(p, s, inter, hidden)

        def run_ii():
            return oracle.bf16_bits(xf @ w_once.T)
    else:
        gp, gs, dp, ds = (t.cpu().numpy() for t in keep)
        gs, ds = gs.view(np.uint16), ds.view(np.uint16)

        def run():
            return oracle.ffn_cpu_baseline(x, gp, gs, dp, ds, hidden, inter)

        wgu = oracle.dequantize_numpy(gp, gs, 2 * inter, hidden)
        wdn = oracle.dequantize_numpy(dp, ds, hidden, inter)

        def run_ii():
            return oracle.ffn_cpu_matmul_only(x, wgu, wdn, hidden, inter)
    v_i, n_i = _median_us(run, seconds)
    v_ii, n_ii = _median_us(run_ii, max(2.0, seconds / 3))
    return {"value": round(v_i, 1), "unit": "us per call", "cores": cores, "kind": "port",
            "sample": f"{n_i} calls of numpy dequantize-per-call + FP32 BLAS matmul (BF16 "
                      f"rounding at the reference's points) on one weight set, median",
            "matmul_only": {"value": round(v_ii, 1), "unit": "us per call",
                            "sample": f"{n_ii} calls of the FP32 BLAS matmuls on weights "
                                      f"dequantized once, median"}}


class HipEvents:
    """hipEvent_t handles from the HIP runtime the process already loaded (torch's and the
    library's are one: same soname), for w4a16_time_next_launch."""

    def __init__(self):
        import ctypes

        self.ct = ctypes
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]

    def create(self, n):
        out = []
        for _ in range(n):
            h = self.ct.c_void_p()
            if self.hip.hipEventCreate(self.ct.byref(h)) != 0:
                raise RuntimeError("hipEventCreate failed")
            out.append(h.value)
        return out

    def elapsed_us(self, a, b):
        self.hip.hipEventSynchronize(b)
        ms = self.ct.c_float()
        if self.hip.hipEventElapsedTime(self.ct.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value * 1e3

    def destroy(self, handles):
        for h in handles:
            self.hip.hipEventDestroy(h)


def profile_json(kind, tag):
    """The committed rocprofv3 figures of one workload (profiles/<kind>_<tag>.json), or {}."""
    path = os.path.join(ROOT, "profiles", f"{kind}_{tag}.json")
    if not os.path.exists(path):
        return {}, None
    with open(path) as handle:
        return json.load(handle), os.path.relpath(path, ROOT)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the tensor-parallel slice is benchmarked on one GPU as --config 4)",
              file=sys.stderr)
        sys.exit(2)
    if args.m is None:
        args.m = 4 if args.config == 3 else 1
    if args.m != 1 and args.config not in (3, 5):
        sys.exit("bench.py: --m applies to --config 3 and --config 5")
    if args.m_sweep and args.config != 5:
        sys.exit("bench.py: --m-sweep applies to --config 5")
    import torch

    import w4a16

    hidden, inter, m, name = shapes(args.config, args.m)
    linear_only = args.config in (0, 5)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if linear_only:
        per_set = inter * hidden // 2 + inter * hidden // 128 * 2
    else:
        per_set = 3 * (inter * hidden // 2 + inter * hidden // 128 * 2)
    count = 64 if args.config == 2 else max(16, -(-CACHE_ROTATE_BYTES // per_set))
    print(f"bench: {name}; generating {count} weight sets ({count * per_set / 2**20:.0f} MiB)",
          file=sys.stderr, flush=True)
    sets = make_sets(torch, w4a16, hidden, inter, count, linear_only)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    partial = args.config == 4
    events = HipEvents()

    def buffers(rows):
        x = torch.randn(rows, hidden, generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
        act = torch.empty(rows, inter, dtype=torch.int16, device=dev)
        out = torch.empty(rows, inter if linear_only else hidden,
                          dtype=torch.float32 if partial else torch.int16, device=dev)
        return x, act, out

    x, act, out = buffers(m)

    def make_calls(x, act, out):
        def ffn_call(i):
            gu, dn, _ = sets[i % count]
            if linear_only:
                w4a16.gemm_int4_bf16(x, gu, out)
            else:
                w4a16.mlp_int4(x, gu, dn, out=out, act_ws=act, partial_f32=partial)

        def first_kernel(i):
            gu = sets[i % count][0]
            if linear_only:
                w4a16.gemm_int4_bf16(x, gu, out)
            else:
                w4a16.gate_up_silu(x, gu, act)

        return ffn_call, first_kernel

    ffn_call, first_kernel = make_calls(x, act, out)

    # Launches are captured into HIP graphs (one graph = one pass over all rotating weight sets;
    # the first pass's graph also holds the steps % count extra calls) so the timed region
    # measures the device, not Python's launch rate.
    def capture(fn, n=None):
        n = count if n is None else n
        for i in range(n):              # eager warm-up of exactly the captured work
            fn(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(n):
                fn(i)
        torch.cuda.synchronize()
        return graph

    def timed(fn, steps, warmup):
        """Exactly `steps` calls of fn, replayed from graphs, after at least `warmup` untimed
        calls; returns (device us per call over all steps, wall us per call, per-pass us per
        call list)."""
        # one graph per pass over the rotating sets; the steps % count extra calls ride in the
        # first pass's graph (a separate short graph would add a whole graph launch to few calls)
        rest = steps % count
        if steps < count:
            first = capture(fn, steps)
            passes = [(first, steps)]
            full = first
        else:
            full = capture(fn)
            first = capture(fn, count + rest) if rest else full
            passes = [(first, count + rest)] + [(full, count)] * (steps // count - 1)
        for _ in range(max(1, -(-warmup // count))):
            full.replay()
        if first is not full:   # its first replay uploads the graph: keep that out of the timing
            first.replay()
            full.replay()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(len(passes) + 1)]
        t0 = time.perf_counter()
        evs[0].record(stream)
        for i, (graph, _) in enumerate(passes):
            graph.replay()
            evs[i + 1].record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        per_pass = [evs[i].elapsed_time(evs[i + 1]) * 1e3 / n for i, (_, n) in enumerate(passes)]
        total_us = evs[0].elapsed_time(evs[-1]) * 1e3
        return total_us / steps, wall * 1e6 / steps, per_pass

    spin_cycles_per_us = []

    def busy_stream(us):
        """Hold the current stream for about `us` microseconds (torch's spin kernel)."""
        if not spin_cycles_per_us:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(1000)
            a.record()
            torch.cuda._sleep(1 << 20)
            b.record()
            torch.cuda.synchronize()
            spin_cycles_per_us.append((1 << 20) / max(a.elapsed_time(b) * 1e3, 1.0))
        torch.cuda._sleep(int(spin_cycles_per_us[0] * us))

    def kernel_us(fn, steps, warmup, skip=0):
        """Average duration of the kernel fn launches after `skip` others, over `steps` eager
        calls (after `warmup`), each timed by the events of w4a16_time_next_launch on the stream
        it runs on: the dispatch's own start and end, as a kernel trace reports them."""
        for i in range(max(warmup, 1)):
            fn(i)
        torch.cuda.synchronize()
        handles = events.create(2 * steps)
        for i in range(steps):
            if i % KERNEL_TIMING_CHUNK == 0:
                # A host-side launch takes longer than the call runs, so the stream would drain
                # between eager calls and each kernel would start on an idle GPU. A spin kernel
                # ahead of every chunk holds the stream while the chunk's calls are enqueued;
                # they then run back to back, as in the graph-replayed call.
                busy_stream(KERNEL_TIMING_CHUNK * 60.0)
            w4a16.lib.w4a16_time_next_launch(skip, handles[2 * i], handles[2 * i + 1])
            fn(i)
        torch.cuda.synchronize()
        total = sum(events.elapsed_us(handles[2 * i], handles[2 * i + 1]) for i in range(steps))
        events.destroy(handles)
        return total / steps

    if args.pmc_pass:
        for i in range(args.steps):
            ffn_call(i)
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_pass": name, "calls": args.steps, "copy_bytes": 256 << 20}))
        return

    if args.steps < 1:
        sys.exit("bench.py: --steps must be at least 1")
    us_per_call, wall_us, per_pass = timed(ffn_call, args.steps, args.warmup)
    ms_total = us_per_call * args.steps / 1e3
    k1_graph, _, _ = timed(first_kernel, args.steps, args.warmup)
    k1_live = kernel_us(ffn_call, args.steps, args.warmup)              # the call's first kernel
    k2_live = 0.0
    if not linear_only:
        k2_live = kernel_us(ffn_call, args.steps, args.warmup, skip=1)   # the call's down kernel
    norm_us = f2_us = None
    if not linear_only:
        # forward_mlp: the same call with the post-attention RMSNorm folded in (plain style)
        norm_w = (1.0 + 0.1 * torch.randn(hidden, generator=gen, device=dev)).to(
            torch.bfloat16).view(torch.int16)
        ws = torch.empty(m, hidden + inter, dtype=torch.int16, device=dev)

        def norm_call(i):
            gu, dn, _ = sets[i % count]
            w4a16.mlp_int4_norm(x, norm_w, 1, 1e-6, gu, dn, out=out, ws=ws, partial_f32=partial)

        norm_us, _, _ = timed(norm_call, args.steps, args.warmup)
        if not partial:
            # plan F2: residual update + norm + FFN + residual add (the residual drifts over the
            # replays, which changes no timing: the call's work does not depend on the values)
            residual = x.clone()
            sub = torch.randn(m, hidden, generator=gen, device=dev).to(torch.bfloat16).view(
                torch.int16)

            def f2_call(i):
                gu, dn, _ = sets[i % count]
                w4a16.mlp_int4_residual_norm(residual, sub, norm_w, 1, 1e-6, gu, dn, out=out,
                                             ws=ws)

            f2_us, _, _ = timed(f2_call, args.steps, args.warmup)
    # the dominant launch: the fused gate/up + SiLU kernel, or the linear of configs 0 and 5
    if linear_only:
        dom_bytes = per_set
        dom_role = "gemm_int4_bf16"
    else:
        dom_bytes = 2 * inter * hidden // 2 + 2 * inter * hidden // 128 * 2
        dom_role = "fused gate/up + SiLU x up"
    down_bytes = inter * hidden // 2 + inter * hidden // 128 * 2
    achieved = dom_bytes / (k1_live * 1e-6) / 1e9
    tag = f"config{args.config}" + (f"_m{m}" if args.config == 3 or (args.config == 5 and m != 1)
                                    else "")
    # The committed rocprofv3 summaries of the same configuration (profiles/): the kernel the
    # dominant launch runs and its kernel-trace average (the figure `frac` uses; the live event
    # window above runs about 1 us longer), and its HBM bytes per launch from FETCH_SIZE /
    # WRITE_SIZE scaled by a plain copy.
    kdoc, rocprof_src = profile_json("kernel_avg", tag)
    dom_kernel = kdoc.get("dominant", {}).get("kernel")
    # the trace average over the dispatches of the live-timing sections (the context the live
    # figure measures), and over every dispatch of the kernel in the traced run
    rocprof_avg = kdoc.get("dominant", {}).get("avg_us_live_sections")
    rocprof_all = kdoc.get("dominant", {}).get("avg_us")
    if rocprof_avg is None:
        rocprof_avg = rocprof_all
    tdoc, traffic_src = profile_json("traffic", tag)
    traffic = tdoc.get("dominant", {}).get("traffic_bytes")
    if not traffic:
        traffic_src = None
    dom_name = f"{dom_kernel or 'gemv'} ({dom_role})"
    achieved_rp = dom_bytes / (rocprof_avg * 1e-6) / 1e9 if rocprof_avg else None
    ffn_gbs = per_set / (us_per_call * 1e-6) / 1e9
    srt = sorted(per_pass)
    pass_stats = {"passes": len(per_pass), "median": round(srt[len(srt) // 2], 3),
                  "min": round(srt[0], 3), "max": round(srt[-1], 3)}

    result = {
        "metric": "µs per INT4 FFN decode call (M=1) + achieved HBM GB/s vs peak, 1 MI355X",
        "value": round(us_per_call, 3),
        "unit": "us per FFN call" if not linear_only else "us per linear call",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_total / args.steps, 6),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "int4 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic (device-generated BF16 ~N(0,0.02) weights quantized by the library, "
                "BF16 ~N(0,1) activations)",
        "config": {"workload": name, "hidden": hidden, "intermediate": inter, "M": m,
                   "weight_sets_rotated": count, "bytes_per_call": per_set,
                   "ffn_achieved_GBps": round(ffn_gbs, 1),
                   "ffn_frac_of_peak": round(ffn_gbs / HBM_PEAK_GBS, 4),
                   "wall_us_per_call": round(wall_us, 3),
                   "pass_us_per_call": pass_stats,
                   "kernel_avg_us": {"dominant": round(k1_live, 3), "second": round(k2_live, 3),
                                     "source": "live: per-launch dispatch events "
                                               "(w4a16_time_next_launch), eager launches"},
                   "with_rmsnorm_us_per_call": None if norm_us is None else round(norm_us, 3),
                   "with_residual_rmsnorm_us_per_call": None if f2_us is None else round(f2_us, 3)},
        "roofline": {"bound": "hbm", "kernel": dom_name,
                     # achieved / frac from the kernel-trace average of this workload's committed
                     # profile (its live-timing sections); the live event window beside it
                     "achieved": round(achieved_rp if rocprof_avg else achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round((achieved_rp if rocprof_avg else achieved) / HBM_PEAK_GBS, 4),
                     "frac_source": "rocprof_avg_us" if rocprof_avg else "avg_launch_us_live",
                     "traffic": traffic, "traffic_source": traffic_src,
                     "bytes_per_launch": dom_bytes,
                     "rocprof_avg_us": rocprof_avg, "rocprof_avg_us_all_dispatches": rocprof_all,
                     "rocprof_source": rocprof_src,
                     "avg_launch_us_live": round(k1_live, 3),
                     "frac_live": round(achieved / HBM_PEAK_GBS, 4),
                     "live_source": "dispatch start/end events of each launch "
                                    "(w4a16_time_next_launch), eager calls enqueued back to back "
                                    "behind a spin kernel; the event window also holds the "
                                    "dispatch's setup",
                     "graph_us_per_launch": round(k1_graph, 3)},
    }
    if not linear_only:
        floor = floor_us(torch, dev, count, dom_bytes, down_bytes, events, timed_fn=timed,
                         steps=args.steps, warmup=args.warmup)
        result["floor_us"] = floor["one_launch_read_us"]
        result["floor"] = floor
    if args.config == 5:
        # the reference's own per-call figures at this shape, on its hardware (A40, ~696 GB/s)
        pub = {1: 52.1, 2: 924.1, 16: 996.7, 64: 2247.7, 128: 3316.1}
        result["config"]["reference_published"] = {
            "us_per_call": pub.get(m), "GBps": 207.6 if m == 1 else None,
            "hardware": "NVIDIA A40", "frac_of_its_peak": round(207.6 / 696.0, 3) if m == 1 else None,
            "source": "reference docs/plan-numeric-contract.md:1753 (M=1), :1775-1778 (M=2, 16, "
                      "64, 128), docs/worklog.md:514"}
        if args.m_sweep:
            result["sweep"] = m_sweep(torch, w4a16, sets, count, hidden, inter, gen, dev,
                                      [int(v) for v in args.m_sweep.split(",")], capture,
                                      kernel_us, args, pub)
    if args.config == 1 and not args.no_secondary:
        result["secondary"] = secondary_rows(torch, w4a16, sets, count, hidden, inter, gen, dev,
                                             timed, kernel_us, args, dom_bytes)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(sets, hidden, inter, m, linear_only,
                                              args.cpu_seconds)
    print(json.dumps(result), flush=True)


def floor_us(torch, dev, count, gu_bytes, dn_bytes, events, timed_fn, steps, warmup):
    """What any implementation of the call can reach here, on buffers of the call's byte counts
    rotated like the weight sets (libw4a16_floor.so): one launch reading both operands, the two
    operands as two dependent launches, and a pair of empty dependent launches (graph-replayed,
    as the call is). Each as us per call."""
    import ctypes

    floor = ctypes.CDLL(os.path.join(PKG, "libw4a16_floor.so"))
    floor.w4a16_floor_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                       ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    floor.w4a16_floor_empty.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    gu_b, dn_b = -(-gu_bytes // 16) * 16, -(-dn_bytes // 16) * 16
    bufs = [(torch.full((gu_b,), 17, dtype=torch.uint8, device=dev),
             torch.full((dn_b,), 23, dtype=torch.uint8, device=dev)) for _ in range(count)]
    sink = torch.zeros(4, dtype=torch.int32, device=dev)

    def stream():
        return torch.cuda.current_stream().cuda_stream

    def one(i):
        a, b = bufs[i % count]
        floor.w4a16_floor_read(a.data_ptr(), gu_b, b.data_ptr(), dn_b, sink.data_ptr(), stream())

    def two(i):
        a, b = bufs[i % count]
        floor.w4a16_floor_read(a.data_ptr(), gu_b, None, 0, sink.data_ptr(), stream())
        floor.w4a16_floor_read(b.data_ptr(), dn_b, None, 0, sink.data_ptr(), stream())

    def empty(i):
        floor.w4a16_floor_empty(2, 256, 256, stream())

    res = {}
    for key, fn in (("one_launch_read_us", one), ("two_launch_read_us", two),
                    ("empty_launch_pair_us", empty)):
        res[key] = round(timed_fn(fn, steps, warmup)[0], 3)
    res["bytes"] = [gu_bytes, dn_bytes]
    res["note"] = ("pure streaming reads of the call's weight bytes (non-temporal 16-byte loads, "
                   "all of a lane's loads issued first), rotated over the same number of sets, "
                   "graph-replayed like the call; libw4a16_floor.so")
    del bufs
    return res


def secondary_rows(torch, w4a16, sets, count, hidden, inter, gen, dev, timed, kernel_us, args,
                   dom_bytes):
    """Config 3 on config 1's weight sets: the FFN call at M = 2, 4, 8, 16 verify rows, us per
    call (graph-replayed, --steps calls), the live average of its gate/up kernel and that
    kernel's fraction of peak, beside the committed rocprofv3 figure of the same workload."""
    rows = {}
    for mm in (2, 4, 8, 16):
        x = torch.randn(mm, hidden, generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
        act = torch.empty(mm, inter, dtype=torch.int16, device=dev)
        out = torch.empty(mm, hidden, dtype=torch.int16, device=dev)

        def call(i, x=x, act=act, out=out):
            gu, dn, _ = sets[i % count]
            w4a16.mlp_int4(x, gu, dn, out=out, act_ws=act)

        us, _, _ = timed(call, args.steps, args.warmup)
        k1 = kernel_us(call, args.steps, args.warmup)      # the call's gate/up kernel
        kdoc, src = profile_json("kernel_avg", f"config3_m{mm}")
        rp = kdoc.get("dominant", {}).get("avg_us_live_sections") or kdoc.get("dominant", {}).get("avg_us")
        rows[f"M={mm}"] = {
            "us_per_call": round(us, 3),
            "GBps_whole_call": round(3 * dom_bytes / 2 / (us * 1e-6) / 1e9, 1),
            "gate_up_us_live": round(k1, 3),
            "gate_up_frac_live": round(dom_bytes / (k1 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "gate_up_kernel": kdoc.get("dominant", {}).get("kernel"),
            "gate_up_rocprof_avg_us": rp, "rocprof_source": src,
            "gate_up_frac_from_rocprof": None if not rp else
            round(dom_bytes / (rp * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    return {"workload": "config3: config 1's weight sets with M verify rows", "rows": rows}


def m_sweep(torch, w4a16, sets, count, hidden, inter, gen, dev, ms, capture, kernel_us, args, pub):
    """The reference's --time sweep shape (N=4096, K=5120) at each M: us per linear call
    (graph-replayed over the rotating sets, --steps calls) and live kernel average."""
    rows = {}
    per_set = inter * hidden // 2 + inter * hidden // 128 * 2
    for mm in ms:
        x = torch.randn(mm, hidden, generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
        out = torch.empty(mm, inter, dtype=torch.int16, device=dev)

        def call(i, x=x, out=out):
            w4a16.gemm_int4_bf16(x, sets[i % count][0], out)

        graph = capture(call)
        for _ in range(2):
            graph.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = max(1, args.steps // count)
        a.record()
        for _ in range(reps):
            graph.replay()
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / (reps * count)
        k = kernel_us(call, args.steps, args.warmup)
        rows[f"M={mm}"] = {"us_per_call": round(us, 3), "kernel_us_live": round(k, 3),
                           "GBps": round(per_set / (us * 1e-6) / 1e9, 1),
                           "frac_of_peak": round(per_set / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                           "reference_A40_us": pub.get(mm)}
    return rows


if __name__ == "__main__":
    main()
