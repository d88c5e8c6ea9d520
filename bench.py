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
reference publishes its one per-call INT4 figure for (N=4096, K=5120, M=1: 52.1 us, 207.6 GB/s
on an A40, reference docs/plan-numeric-contract.md:1753), quoted beside this run's.

Timing: the calls of one pass over the rotating sets are captured in a HIP graph (and the first
steps % sets calls in a second graph); exactly --steps calls are replayed in the timed region,
with a HIP event on the replay stream before it and after every pass, so ``value`` is device
time per call over all --steps calls (gaps between kernels included, not Python's launch rate)
and ``config.pass_us_per_call`` gives the median, min and max over the passes.

Prints ONE JSON line. ``roofline`` is the dominant kernel's (the fused gate/up/SiLU GEMV):
algorithmic bytes per launch (packed nibbles + BF16 scales of its weight) over its average
launch duration, from a graph holding only that kernel's launches, timed the same way.
``cpu_baseline`` times the CPU dequant+matmul path (numpy, BLAS) over a bounded sample.
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


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=1, choices=(0, 1, 2, 3, 4, 5))
    ap.add_argument("--m", type=int, default=4, help="rows for --config 3")
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
        return 5120, 4096, 1, "config5: the reference's published shape, W4A16 linear M=1 K=5120 N=4096"
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


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the tensor-parallel slice is benchmarked on one GPU as --config 4)",
              file=sys.stderr)
        sys.exit(2)
    import numpy as np
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
    x = torch.randn(m, hidden, generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
    act = torch.empty(m, inter, dtype=torch.int16, device=dev)
    partial = args.config == 4
    out = torch.empty(m, inter if linear_only else hidden,
                      dtype=torch.float32 if partial else torch.int16, device=dev)
    down_out = torch.empty(m, hidden, dtype=torch.int16, device=dev)

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

    def second_kernel(i):
        if not linear_only:
            w4a16.gemm_int4_bf16(act, sets[i % count][1], down_out)

    # Launches are captured into HIP graphs (one graph = one pass over all rotating weight sets,
    # plus one holding the first steps % count calls) so the timed region measures the device,
    # not Python's launch rate.
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
        full = capture(fn)
        rest = steps % count
        tail = capture(fn, rest) if rest else None
        for _ in range(max(1, -(-warmup // count))):
            full.replay()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        passes = [(full, count)] * (steps // count) + ([(tail, rest)] if tail else [])
        events = [torch.cuda.Event(enable_timing=True) for _ in range(len(passes) + 1)]
        t0 = time.perf_counter()
        events[0].record(stream)
        for i, (graph, _) in enumerate(passes):
            graph.replay()
            events[i + 1].record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        per_pass = [events[i].elapsed_time(events[i + 1]) * 1e3 / n
                    for i, (_, n) in enumerate(passes)]
        total_us = events[0].elapsed_time(events[-1]) * 1e3
        return total_us / steps, wall * 1e6 / steps, per_pass

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
    k1_avg, _, _ = timed(first_kernel, args.steps, args.warmup)
    k2_avg = 0.0
    if not linear_only:
        k2_avg, _, _ = timed(second_kernel, args.steps, args.warmup)
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
    achieved = dom_bytes / (k1_avg * 1e-6) / 1e9
    tag = f"config{args.config}" + (f"_m{m}" if args.config == 3 else "")
    # The committed rocprofv3 summaries of the same configuration (profiles/): the kernel the
    # dominant launch runs and its kernel-trace average (a cross-check of the live event timing
    # above), and its HBM bytes per launch from FETCH_SIZE / WRITE_SIZE scaled by a plain copy.
    dom_kernel, rocprof_avg, rocprof_src, traffic, traffic_src = None, None, None, None, None
    kpath = os.path.join(ROOT, "profiles", f"kernel_avg_{tag}.json")
    if os.path.exists(kpath):
        with open(kpath) as handle:
            dom = json.load(handle).get("dominant", {})
        dom_kernel, rocprof_avg = dom.get("kernel"), dom.get("avg_us")
        rocprof_src = os.path.relpath(kpath, ROOT)
    tpath = os.path.join(ROOT, "profiles", f"traffic_{tag}.json")
    if os.path.exists(tpath):
        with open(tpath) as handle:
            dom = json.load(handle).get("dominant", {})
        traffic = dom.get("traffic_bytes")
        traffic_src = os.path.relpath(tpath, ROOT) if traffic else None
    dom_name = f"{dom_kernel or 'gemv'} ({dom_role})"
    ffn_gbs = per_set / (us_per_call * 1e-6) / 1e9
    srt = sorted(per_pass)
    pass_stats = {"passes": len(per_pass), "median": round(srt[len(srt) // 2], 3),
                  "min": round(srt[0], 3), "max": round(srt[-1], 3)}

    result = {
        "metric": "\u00b5s per INT4 FFN decode call (M=1) + achieved HBM GB/s vs peak, 1 MI355X",
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
                   "kernel_avg_us": {"dominant": round(k1_avg, 3), "second": round(k2_avg, 3)},
                   # the down projection is timed through gemm_int4_bf16 on row-major rows;
                   # from M = 4 the FFN call runs it on its chunk-major intermediate instead
                   **({"second_as_timed": "gemm_int4_bf16 (row-major rows), not the FFN's "
                       "chunk-major down kernel"} if 4 <= m <= 16 and not linear_only else {}),
                   "with_rmsnorm_us_per_call": None if norm_us is None else round(norm_us, 3),
                   "with_residual_rmsnorm_us_per_call": None if f2_us is None else round(f2_us, 3)},
        "roofline": {"bound": "hbm", "kernel": dom_name, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src, "bytes_per_launch": dom_bytes,
                     "avg_launch_us": round(k1_avg, 3), "rocprof_avg_us": rocprof_avg,
                     "rocprof_source": rocprof_src,
                     "frac_from_rocprof": None if not rocprof_avg else
                     round(dom_bytes / (rocprof_avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
    }
    if args.config == 5:
        # the reference's own per-call figure at this shape, on its hardware (A40, ~696 GB/s)
        result["config"]["reference_published"] = {
            "us_per_call": 52.1, "GBps": 207.6, "hardware": "NVIDIA A40",
            "frac_of_its_peak": round(207.6 / 696.0, 3),
            "source": "reference docs/plan-numeric-contract.md:1753, docs/worklog.md:514"}
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(sets, hidden, inter, m, linear_only,
                                              args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
