"""fp8lin benchmark: block-FP8 decode GEMV (HBM roofline) and prefill GEMM
(MFMA roofline) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick]

A step is one decode pass of the one-rank layer chain at M=1 (benchmark
config 2): gate/up 17408x5120, down 5120x8704 and QKV-gate 7168x5120, E4M3FN
weights with 128x128 block scales (seed 0, N(0, 0.02)), BF16 activations
N(0,1).  Weight sets are rotated so the working set exceeds twice the 256 MB
Infinity Cache, so the GB/s figures are HBM, not cache.  `value` is the
algorithmic bytes of the timed steps divided by their wall time on the GPU
(HIP events bracketing the timed region).  One JSON line is printed last.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "a100-vision-infer_amd"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
METRIC = "FP8 GEMV HBM GB/s (% peak) at M=1; prefill GEMM TFLOP/s (% MFMA peak)"
# HBM bytes per launch of the roofline kernel (gate/up GEMV, M=1), from two
# rocprofv3 --pmc passes: 2.000 x FETCH_SIZE (44 962.1 KiB) + 1.000 x WRITE_SIZE
# (68.0 KiB); the factors are what the counters read for a 256 MiB device copy
# (`bench.py --calibrate`).  Re-measure when the kernel changes.
GATE_UP_TRAFFIC_BYTES = 92_152_013
# One M=4096 gate/up+SwiGLU prefill call (gemm_fp8_kernel<8, true> and its
# tail_reduce_kernel), copy-calibrated FETCH_SIZE x2 + WRITE_SIZE, rotated.
PREFILL_TRAFFIC_BYTES = 1_119_594_086
# MFMA busy fraction of the prefill kernel over its whole dispatch (M=4096
# gate/up+SwiGLU), one --pmc pass: SQ_VALU_MFMA_BUSY_CYCLES summed over the
# 1024 SIMDs, per SIMD, over the dispatch's cycles.  GRBM_GUI_ACTIVE comes back
# summed over the 8 XCDs (8 x the dispatch's cycles at the shader clock), so
# rocprofv3's own MfmaUtil formula reads 8x low on this part.  Re-measure when
# the kernel changes.
PREFILL_MFMA_BUSY = 0.730
PREFILL_MFMA_BUSY_SOURCE = ("rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE: 715.7e6 busy cycles "
                            "/ 1024 SIMDs over GRBM_GUI_ACTIVE / 8 XCDs = 0.957e6 cycles (1.60 GHz)")
SHAPES = [("gate_up", 17408, 5120), ("down", 5120, 8704), ("qkv_gate", 7168, 5120)]


# Least bytes of weight copies each rotation holds: more than twice the
# 256 MB Infinity Cache, so a weight is evicted before it comes round again.
ROTATION_BYTES = 600_000_000


def weight_bytes(n, k):
    """Codes and row-expanded block scales of one N x K weight."""
    return n * k + 4 * n * ((k + 127) // 128)


def rotations(fp8lin, dev, copies):
    """Per decode shape, at least ROTATION_BYTES of seeded weight copies (and
    at least `copies`): copy c of shape i has Philox tag 1 + 16 c + i for the
    first `copies`, 500 + 32 i + c after."""
    rot = {}
    for i, (name, n, k) in enumerate(SHAPES):
        count = max(copies, -(-ROTATION_BYTES // weight_bytes(n, k)))
        rot[name] = [fp8lin.gen_weights(n, k, seed=0, tag=(1 + 16 * c + i) if c < copies else (500 + 32 * i + c),
                                        device=dev) for c in range(count)]
    return rot


def algo_bytes(m, n, k, n_out=None):
    """N*K codes + 4*N*ceil(K/128) scales + 2*M*K activations + 2*M*N_out output."""
    n_out = n if n_out is None else n_out
    return n * k + 4 * n * ((k + 127) // 128) + 2 * m * k + 2 * m * n_out


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1000)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--copies", type=int, default=4, help="rotated weight sets (>= 512 MB total)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--quick", action="store_true", help="skip the secondary measurements")
    p.add_argument("--sections", default="gemv,small,prefill,refbench,chain,inproj,head,stream,ceiling",
                   help="secondary measurements to run (comma list of gemv, small, prefill, refbench, "
                        "chain, inproj, head, stream, ceiling)")
    p.add_argument("--prefill-m", default="128,512,1024,4096",
                   help="prefill row counts of the prefill section (comma list)")
    p.add_argument("--calibrate", action="store_true",
                   help="also run a 256 MiB device copy (known HBM bytes) for counter scaling")
    return p.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "tensor-parallel sharding is designed but not run on more than one GPU", file=sys.stderr)
        sys.exit(2)
    import torch
    import fp8lin

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    assert fp8lin.lib().fp8lin_init() == 0, fp8lin.lib().fp8lin_last_error()

    # ---- inputs: seed 0, generated on the device ---------------------------------
    # Each shape's weights rotate over copies of at least ROTATION_BYTES
    # (more than twice the 256 MB Infinity Cache), so every figure that
    # rotates through them streams from HBM; the decode step takes the first
    # `copies` of each.
    rot = rotations(fp8lin, dev, args.copies)
    sets = [{name: rot[name][c] for name, _, _ in SHAPES} for c in range(args.copies)]
    xs = {k: fp8lin.gen_activations(1, k, seed=0, tag=2, device=dev) for k in {5120, 8704}}
    ys = {name: torch.empty((1, n), dtype=torch.bfloat16, device=dev) for name, n, _ in SHAPES}
    torch.cuda.synchronize()
    step_bytes = sum(algo_bytes(1, n, k) for _, n, k in SHAPES)
    working_set = args.copies * sum(weight_bytes(n, k) for _, n, k in SHAPES)
    log(f"working set {working_set / 1e6:.1f} MB over {args.copies} weight copies; per-shape rotations " +
        ", ".join(f"{name} {len(rot[name])} x {weight_bytes(n, k) / 1e6:.1f} MB" for name, n, k in SHAPES))

    L = fp8lin.lib()
    import ctypes
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)

    def gemv(name, ws, y):
        n, k = {s[0]: (s[1], s[2]) for s in SHAPES}[name]
        codes, scales = ws[name]
        rc = L.fp8lin_linear(ctypes.c_void_p(xs[k].data_ptr()), ctypes.c_void_p(codes.data_ptr()),
                             ctypes.c_void_p(scales.data_ptr()), (k + 127) // 128,
                             ctypes.c_void_p(y.data_ptr()), 1, n, k, 1, sp)
        if rc:
            raise RuntimeError(L.fp8lin_last_error())

    def step(i):
        ws = sets[i % len(sets)]
        gemv("gate_up", ws, ys["gate_up"])
        gemv("down", ws, ys["down"])
        gemv("qkv_gate", ws, ys["qkv_gate"])

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # The decode step also runs as a captured HIP graph (the reference's decode
    # loop is CUDA-graph captured): one graph holds one step per weight copy.
    copies = len(sets)
    cap = torch.cuda.Stream(dev)
    graph = torch.cuda.CUDAGraph()
    cap.wait_stream(stream)
    with torch.cuda.stream(cap):
        sp_cap = ctypes.c_void_p(cap.cuda_stream)
        sp_saved, sp.value = sp.value, sp_cap.value
        with torch.cuda.graph(graph, stream=cap):
            for c in range(copies):
                step(c)
        sp.value = sp_saved
    stream.wait_stream(cap)
    replays = max(1, (args.steps + copies - 1) // copies)
    steps = args.steps
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()

    # ---- timed region: K steps of eager back-to-back launches ----------------------
    # (On this ROCm stack graph replay of the 3-kernel step is slower than eager
    # launches; the graph figure is reported in `extra`.)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for i in range(steps):
        step(i)
    t1.record()
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    ms_per_step = total_ms / steps
    value = step_bytes * steps / (total_ms * 1e-3) / 1e9

    r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    r0.record()
    for _ in range(replays):
        graph.replay()
    r1.record()
    torch.cuda.synchronize()
    graph_ms = r0.elapsed_time(r1) / (replays * copies)

    # Dominant kernel: gate/up GEMV, back-to-back launches over its rotation
    # (at least ROTATION_BYTES) in a graph, timed with HIP events around the
    # replays.
    gu_graph = torch.cuda.CUDAGraph()
    gu_rot = rot["gate_up"]
    reps_in_graph = 4 * len(gu_rot)
    with torch.cuda.stream(cap):
        sp_saved, sp.value = sp.value, cap.cuda_stream
        with torch.cuda.graph(gu_graph, stream=cap):
            for i in range(reps_in_graph):
                gemv("gate_up", {"gate_up": gu_rot[i % len(gu_rot)]}, ys["gate_up"])
        sp.value = sp_saved
    gu_graph.replay()
    torch.cuda.synchronize()
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g0.record()
    for _ in range(10):
        gu_graph.replay()
    g1.record()
    torch.cuda.synchronize()
    gu_avg_ms = g0.elapsed_time(g1) / (10 * reps_in_graph)
    gu_bytes = algo_bytes(1, 17408, 5120)
    gu_gbs = gu_bytes / (gu_avg_ms * 1e-3) / 1e9
    log(f"decode chain: {ms_per_step * 1e3:.2f} us/step, {value:.1f} GB/s; gate/up GEMV "
        f"avg {gu_avg_ms * 1e3:.2f} us ({gu_gbs:.1f} GB/s)")
    log(f"decode chain (graph replay): {graph_ms * 1e3:.2f} us/step, "
        f"{step_bytes / (graph_ms * 1e-3) / 1e9:.1f} GB/s")

    extra = {"graph_us_per_step": round(graph_ms * 1e3, 3),
             "graph_GBs": round(step_bytes / (graph_ms * 1e-3) / 1e9, 1)}
    if not args.quick:
        extra.update(secondary(torch, fp8lin, dev, rot, log, set(args.sections.split(",")),
                               [int(v) for v in args.prefill_m.split(",") if v]))
    if args.calibrate:
        extra.update(calibrate(torch, dev, log))

    cpu = None
    if not args.no_cpu:
        cpu, cpu_extra = cpu_baseline(sets[0], xs, args.cpu_seconds, log)
        extra.update(cpu_extra)

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seed-0 Philox N(0,0.02) weights quantized to E4M3FN per 128x128 block; "
                "BF16 N(0,1) activations)",
        "config": {
            "workload": "decode GEMV, M=1, one TP-rank layer chain: gate/up 17408x5120 + "
                        "down 5120x8704 + QKV-gate 7168x5120 (config 2)",
            "batch_rows": 1,
            "weight_format": "E4M3FN codes + FP32 128x128 block scales (row-expanded)",
            "accumulate": "fp32",
            "bytes_per_step": step_bytes,
            "working_set_bytes": working_set,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "gemv_ring_kernel<1,2,5,fp8,x in LDS> (gate/up 17408x5120, M=1)",
            "achieved": round(gu_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
            "traffic": GATE_UP_TRAFFIC_BYTES,
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE x2.000 + WRITE_SIZE x1.000 (copy-calibrated)",
            "avg_launch_us": round(gu_avg_ms * 1e3, 3),
            "algorithmic_bytes_per_launch": gu_bytes,
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    if "prefill_swiglu_m4096_TFLOPs" in extra:
        tf = extra["prefill_swiglu_m4096_TFLOPs"]
        out["roofline_prefill"] = {
            "bound": "mfma",
            "kernel": "gemm_fp8_kernel<8, true> + tail_reduce_kernel<8, true> (gate/up+SwiGLU 17408x5120, M=4096)",
            "achieved": tf,
            "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tf / BF16_PEAK_TFLOPS, 4),
            "avg_call_us": extra["prefill_swiglu_m4096_us"],
            "algorithmic_flop_per_call": 2 * 4096 * 17408 * 5120,
            "mfma_busy": PREFILL_MFMA_BUSY,
            "mfma_busy_source": PREFILL_MFMA_BUSY_SOURCE,
            "traffic": PREFILL_TRAFFIC_BYTES,
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE x2.000 + WRITE_SIZE x1.000 (copy-calibrated), "
                              "GEMM + tail reduce of one call",
            "algorithmic_bytes_per_call": 4096 * 5120 * 2 + 17408 * 5120 + 17408 * 40 * 4 + 4096 * 8704 * 2,
        }
    print(json.dumps(out), flush=True)


def timed(torch, fn, iters, warm=3):
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters


def graph_timed(torch, fn, sp, reps=20, replays=20):
    """Per-call time of `fn` with the host out of the loop: `reps` calls
    captured in one HIP graph (fn launches on sp, a ctypes stream handle that
    is pointed at the capture stream meanwhile), replayed `replays` times."""
    cap = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.stream(cap):
        saved, sp.value = sp.value, cap.cuda_stream
        try:
            fn()
            cap.synchronize()
            with torch.cuda.graph(graph, stream=cap):
                for _ in range(reps):
                    fn()
        finally:
            sp.value = saved
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (replays * reps)


def secondary(torch, fp8lin, dev, rot, log, sections, prefill_m=(128, 512, 1024, 4096)):
    """Per-shape and per-path figures through the C ABI with preallocated
    outputs, each call on the next of its shape's rotated weight copies
    (`rot`, at least ROTATION_BYTES per shape); decode figures are graph
    replays of back-to-back launches (the host's launch rate stays out of
    them), prefill figures eager back-to-back calls."""
    import ctypes
    L = fp8lin.lib()
    P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    extra = {}

    def ok(rc):
        if rc:
            raise RuntimeError(L.fp8lin_last_error())

    # per-shape decode GEMV (rotating copies), plus config 1 (N = K = 4096)
    # over 32 copies (554 MB) so it too streams from HBM
    cfg1 = [fp8lin.gen_weights(4096, 4096, seed=0, tag=100 + c, device=dev)
            for c in range(32)] if "gemv" in sections else []
    gemv_cases = [(name, n, k, rot[name]) for name, n, k in SHAPES]
    gemv_cases.append(("cfg1_4096", 4096, 4096, cfg1))
    for name, n, k, copies in (gemv_cases if "gemv" in sections else []):
        x = fp8lin.gen_activations(1, k, seed=0, tag=2, device=dev)
        y = torch.empty((1, n), dtype=torch.bfloat16, device=dev)
        i = [0]

        def run():
            c, s = copies[i[0] % len(copies)]
            i[0] += 1
            ok(L.fp8lin_linear(P(x), P(c), P(s), s.size(1), P(y), 1, n, k, 1, sp))
        ms = graph_timed(torch, run, sp, reps=4 * len(copies), replays=10)
        gbs = algo_bytes(1, n, k) / (ms * 1e-3) / 1e9
        extra[f"gemv_m1_{name}_GBs"] = round(gbs, 1)
        extra[f"gemv_m1_{name}_us"] = round(ms * 1e3, 2)
        log(f"gemv M=1 {name}: {ms * 1e3:.2f} us {gbs:.1f} GB/s")
    del cfg1
    # small M (config 3): GEMV and matrix-core paths on the three shapes and
    # the reference benchmark's 8240 x 5120 (in_proj_all, all FP8; 13 copies)
    small_copies = dict(rot)
    if "small" in sections:
        small_copies["in_proj_all"] = [fp8lin.gen_weights(8240, 5120, seed=0, tag=400 + c, device=dev)
                                       for c in range(13)]
    for name, n, k in (SHAPES + [("in_proj_all", 8240, 5120)] if "small" in sections else []):
        # M = 16 and 32: fp8lin_linear only (fp8_tensor_small takes 2..8 rows)
        for m in (2, 4, 8, 16, 32):
            x = fp8lin.gen_activations(m, k, seed=0, tag=2, device=dev)
            y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
            ws = torch.empty(4 * 4 * m * n, dtype=torch.uint8, device=dev)
            paths = {
                "gemv": lambda c, s: ok(L.fp8lin_linear(P(x), P(c), P(s), s.size(1), P(y), m, n, k, 1, sp)),
                "tensor_s1": lambda c, s: ok(L.fp8lin_tensor_small(P(x), P(c), P(s), P(y), m, n, k, 1,
                                                                  None, 0, sp)),
                "tensor_s4": lambda c, s: ok(L.fp8lin_tensor_small(P(x), P(c), P(s), P(y), m, n, k, 4,
                                                                  P(ws), ws.numel(), sp)),
            }
            if m > 8:
                paths = {"gemv": paths["gemv"]}
            for label, fn in paths.items():
                i = [0]

                def run():
                    c, s = small_copies[name][i[0] % len(small_copies[name])]
                    i[0] += 1
                    fn(c, s)
                ms = graph_timed(torch, run, sp, reps=2 * len(small_copies[name]), replays=10)
                gbs = algo_bytes(m, n, k) / (ms * 1e-3) / 1e9
                extra[f"m{m}_{name}_{label}_GBs"] = round(gbs, 1)
                log(f"M={m} {name} {label}: {ms * 1e3:.2f} us {gbs:.1f} GB/s")
    del small_copies
    # prefill GEMM with fused SwiGLU (config 4), each call on the next gate/up
    # copy of the rotation
    n, k = 17408, 5120
    gu = rot["gate_up"]
    for m in (prefill_m if "prefill" in sections else ()):
        x = fp8lin.gen_activations(m, k, seed=0, tag=2, device=dev)
        y = torch.empty((m, n // 2), dtype=torch.bfloat16, device=dev)
        need = L.fp8lin_linear_swiglu_workspace_bytes(m, n, k)
        pws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
        i = [0]

        def call():
            c, s = gu[i[0] % len(gu)]
            i[0] += 1
            ok(L.fp8lin_linear_swiglu_ws(P(x), P(c), P(s), s.size(1), P(y), m, n, k, P(pws), need, sp))
        ms = timed(torch, call, 2 * len(gu) if m == 4096 else 4 * len(gu), warm=len(gu))
        tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        extra[f"prefill_swiglu_m{m}_TFLOPs"] = round(tflops, 1)
        extra[f"prefill_swiglu_m{m}_us"] = round(ms * 1e3, 2)
        extra[f"prefill_swiglu_m{m}_frac"] = round(tflops / BF16_PEAK_TFLOPS, 4)
        log(f"prefill M={m} gate/up+SwiGLU: {ms:.3f} ms {tflops:.1f} TFLOP/s "
            f"({100 * tflops / BF16_PEAK_TFLOPS:.1f}% of BF16 peak)")
    # Practical-ceiling reference, not part of the library: the platform's
    # BF16 GEMM (torch.mm -> hipBLASLt) on the same M=4096 shape with plain
    # BF16 weights (no dequantization, no SwiGLU epilogue).
    if "prefill" in sections and 4096 in prefill_m:
        m = 4096
        xa = fp8lin.gen_activations(m, k, seed=0, tag=2, device=dev)
        wb = torch.randn(k, n, device=dev, dtype=torch.bfloat16)
        ms = timed(torch, lambda: torch.mm(xa, wb), 10)
        tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        extra["reference_hipblaslt_bf16_m4096_TFLOPs"] = round(tflops, 1)
        log(f"reference: torch.mm BF16 (hipBLASLt) M={m} N={n} K={k}: {ms:.3f} ms {tflops:.1f} TFLOP/s")
        del xa, wb
    # The drop-in operator (fp8_linear through fp8lin_linear_ws, as the ATen
    # shim calls it) on the prefill projections whose tiles leave CUs idle,
    # against the same call without a workspace (M = 64 and 128: the small-M
    # kernels; M = 512: every tile whole); graph replays over the rotation, as
    # the chain section times the engine branch.
    for name, n, k in (SHAPES[1:] if "prefill" in sections else ()):
        for m in (64, 128, 512):
            x = fp8lin.gen_activations(m, k, seed=0, tag=2, device=dev)
            y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
            need = L.fp8lin_linear_workspace_bytes(m, n, k)
            lws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
            copies = rot[name]
            for label, split in (("linear_ws", True), ("linear", False)):
                i = [0]

                def call():
                    c, s = copies[i[0] % len(copies)]
                    i[0] += 1
                    if split:
                        ok(L.fp8lin_linear_ws(P(x), P(c), P(s), s.size(1), P(y), m, n, k, 1, P(lws), need, sp))
                    else:
                        ok(L.fp8lin_linear(P(x), P(c), P(s), s.size(1), P(y), m, n, k, 1, sp))
                ms = graph_timed(torch, call, sp, reps=2 * len(copies), replays=10)
                tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
                extra[f"dropin_m{m}_{name}_{label}_us"] = round(ms * 1e3, 2)
                log(f"fp8_linear M={m} {name} ({label}): {ms * 1e3:.2f} us {tf:.1f} TFLOP/s")
    if "refbench" in sections:
        extra.update(reference_benchmark_shapes(torch, fp8lin, dev, log))
    if "chain" in sections:
        extra.update(layer_chain(torch, fp8lin, dev, rot, log))
    if "inproj" in sections:
        extra.update(in_proj_all(torch, fp8lin, dev, log))
    if "head" in sections:
        extra.update(head_and_epilogue(torch, fp8lin, dev, log))
    # streaming-read ceiling: 1 GiB and each decode weight size.  Each launch
    # reads the next region of a 1 GiB buffer (as the GEMV benchmarks rotate
    # weight copies), so the reads come from HBM, not the 256 MB Infinity Cache.
    if "stream" in sections:
        buf = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        sink = torch.zeros(4096, dtype=torch.float32, device=dev)
        for label, nbytes in (("1GiB", 1 << 30), ("gate_up", 17408 * 5120), ("down", 5120 * 8704),
                              ("qkv_gate", 7168 * 5120), ("cfg1", 4096 * 4096)):
            regions = max(1, (1 << 30) // ((nbytes + 4095) // 4096 * 4096))
            step = (1 << 30) // regions // 4096 * 4096
            i = [0]

            def read():
                src = ctypes.c_void_p(buf.data_ptr() + (i[0] % regions) * step)
                i[0] += 1
                ok(L.fp8lin_stream_read(src, nbytes, P(sink), sp))
            ms = graph_timed(torch, read, sp, reps=max(4, 2 * regions), replays=5)
            extra[f"stream_read_{label}_GBs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
            log(f"stream read {label}: {extra[f'stream_read_{label}_GBs']} GB/s")
    # MFMA ceiling: register-only BF16 MFMA on every CU for about a second
    # (the clock settles), then the last launch's rate and shader clock.
    if "ceiling" in sections:
        sink = torch.zeros(1, dtype=torch.float32, device=dev)
        clocks = torch.zeros(2, dtype=torch.int64, device=dev)
        iters = 20000
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        flop = cus * 4 * iters * 16 * 32768
        t_end = time.time() + 1.0
        while True:
            ms = timed(torch, lambda: ok(L.fp8lin_mfma_ceiling(iters, P(sink), P(clocks), sp)), 1, warm=0)
            if time.time() > t_end:
                break
        c = clocks.cpu().tolist()
        tflops = flop / (ms * 1e-3) / 1e12
        extra["mfma_ceiling_TFLOPs"] = round(tflops, 1)
        extra["mfma_ceiling_clock_MHz"] = round(c[0] / c[1] * 100.0, 0)
        log(f"MFMA ceiling (register-only BF16 MFMA, {cus} CUs): {tflops:.1f} TFLOP/s "
            f"({100 * tflops / BF16_PEAK_TFLOPS:.1f}% of nominal peak) at {c[0] / c[1] * 100.0:.0f} MHz")
    return extra


def head_and_epilogue(torch, fp8lin, dev, log):
    """The output head and the decode epilogue (src/speculative.cpp:25-27,
    src/dual_path.cu): the vocab-sharded head 75968 x 5120 alone and followed
    by its vocabulary candidates, at M = 1 and 4; residual add + RMSNorm at
    hidden 5120.  Timed as graph replays: these calls are short enough that
    eager timing through the C ABI measures the host's launch rate."""
    import ctypes
    L = fp8lin.lib()
    P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    extra = {}

    def ok(rc):
        if rc:
            raise RuntimeError(L.fp8lin_last_error())

    n, k = 75968, 5120
    c, s = fp8lin.gen_weights(n, k, seed=0, tag=90, device=dev)
    for m in (1, 4):
        x = fp8lin.gen_activations(m, k, seed=0, tag=2, device=dev)
        logits = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        out = torch.empty((m, 2), dtype=torch.float64, device=dev)
        vws = torch.empty(L.fp8lin_vocab_candidates_workspace_bytes(m, n), dtype=torch.uint8, device=dev)
        hws = torch.empty(L.fp8lin_linear_candidates_workspace_bytes(m, n, k), dtype=torch.uint8, device=dev)

        def head():
            ok(L.fp8lin_linear(P(x), P(c), P(s), s.size(1), P(logits), m, n, k, 1, sp))

        def head_candidates():
            ok(L.fp8lin_linear_candidates(P(x), P(c), P(s), s.size(1), m, n, k, 0, P(out), P(hws),
                                          hws.numel(), sp))

        def candidates():
            ok(L.fp8lin_vocab_candidates(P(logits), m, n, 0, P(out), P(vws), vws.numel(), sp))
        # Engine::local_candidates with the small-M matrix-core option
        # (src/engine.cpp:206-213): the head at rows 2..8 on that path
        topt = fp8lin.LinearOptions(fp8_tensor_small=True)
        rec = fp8lin.Weight()
        rec.data, rec.scales, rec.scale_cols, rec.cached_bf16, rec.N, rec.K = c.data_ptr(), s.data_ptr(), s.size(1), None, n, k
        ews_n = L.fp8lin_engine_linear_candidates_workspace_bytes(ctypes.byref(topt), ctypes.byref(rec), m)
        ews = torch.empty(max(ews_n, 16), dtype=torch.uint8, device=dev)

        def engine_candidates():
            ok(L.fp8lin_engine_linear_candidates(ctypes.byref(topt), ctypes.byref(rec), P(x), m, 0, P(out), P(ews),
                                                 ews_n, None, sp))
        nbytes = algo_bytes(m, n, k)
        paths = [("linear", head), ("linear_candidates", head_candidates), ("candidates_only", candidates)]
        if m > 1:
            paths.append(("tensor_small_candidates", engine_candidates))
        for label, fn in paths:
            ms = graph_timed(torch, fn, sp)
            extra[f"head_m{m}_{label}_us"] = round(ms * 1e3, 2)
            if label != "candidates_only":
                extra[f"head_m{m}_{label}_GBs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
            log(f"head M={m} {label}: {ms * 1e3:.2f} us (graph replay)")
    del c, s
    d = 5120
    w = fp8lin.gen_activations(1, d, seed=1, tag=3, device=dev)
    for m in (1, 512, 4096):
        x = fp8lin.gen_activations(m, d, seed=0, tag=2, device=dev)
        u = fp8lin.gen_activations(m, d, seed=0, tag=4, device=dev)
        res, y = torch.empty_like(x), torch.empty_like(x)
        ms = graph_timed(torch, lambda: ok(L.fp8lin_residual_rms(P(x), P(u), P(w), P(res), P(y), m, d, 1e-6, 1,
                                                                 sp)), sp)
        nbytes = (4 * m * d + d) * 2
        extra[f"residual_rms_m{m}_us"] = round(ms * 1e3, 2)
        extra[f"residual_rms_m{m}_GBs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        log(f"residual_rms M={m} D={d}: {ms * 1e3:.2f} us {nbytes / (ms * 1e-3) / 1e9:.1f} GB/s")
        # the TP=2 row-parallel reduce folded in: two gathered partials
        parts = torch.stack([u, fp8lin.gen_activations(m, d, seed=1, tag=5, device=dev)]).contiguous()
        ms = graph_timed(torch, lambda: ok(L.fp8lin_reduce_residual_rms(P(x), P(parts), 2, P(w), P(res), P(y), m, d,
                                                                        1e-6, 1, sp)), sp)
        nbytes = (5 * m * d + d) * 2
        extra[f"reduce2_residual_rms_m{m}_us"] = round(ms * 1e3, 2)
        extra[f"reduce2_residual_rms_m{m}_GBs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        log(f"reduce(2 ranks)+residual_rms M={m} D={d}: {ms * 1e3:.2f} us {nbytes / (ms * 1e-3) / 1e9:.1f} GB/s")
    # Q/K epilogue of a full-attention layer (TP=2 rank: 12 query, 2 key heads
    # of 256, rotary 64): fused, and the unfused sequence it replaces
    # (fused_rms of the query and key heads, then fused_rope of each).
    H, HK, D, R = 12, 2, 256, 64
    qw = fp8lin.gen_activations(1, D, seed=2, tag=3, device=dev)
    for t in (1, 4096):
        proj = fp8lin.gen_activations(t, 2 * (H + HK) * D, seed=0, tag=6, device=dev)
        pos = torch.randint(0, 8192, (3, t), dtype=torch.int64, device=dev)
        q = torch.empty((t, H, D), dtype=torch.bfloat16, device=dev)
        k = torch.empty((t, HK, D), dtype=torch.bfloat16, device=dev)
        args = (t, H, HK, D, R, 1e7, 11, 10, 1e-6, sp)
        ms = graph_timed(torch, lambda: ok(L.fp8lin_qk_norm_rope(P(proj), proj.size(1), P(qw), P(qw), P(pos), P(q),
                                                                 P(k), *args)), sp)
        nbytes = 2 * t * (H + HK) * D * 2 + 2 * D * 2 + 3 * t * 8
        qv, _, kv, _ = fp8lin.LinearEngine.qkv_gate_views(proj, H, HK, D)
        qc, kc = qv.contiguous(), kv.contiguous()
        qn, kn = torch.empty_like(qc), torch.empty_like(kc)

        def unfused():
            ok(L.fp8lin_rms(P(qc), P(qw), P(qn), t * H, D, 1e-6, 1, sp))
            ok(L.fp8lin_rms(P(kc), P(qw), P(kn), t * HK, D, 1e-6, 1, sp))
            ok(L.fp8lin_rope(P(qn), P(pos), P(q), t, H, D, R, 1e7, 11, 10, sp))
            ok(L.fp8lin_rope(P(kn), P(pos), P(k), t, HK, D, R, 1e7, 11, 10, sp))
        ms_u = graph_timed(torch, unfused, sp)
        extra[f"qk_norm_rope_t{t}_us"] = round(ms * 1e3, 2)
        extra[f"qk_norm_rope_t{t}_GBs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        extra[f"qk_norm_rope_t{t}_unfused_us"] = round(ms_u * 1e3, 2)
        log(f"qk_norm_rope T={t} (H={H}, HK={HK}, D={D}): {ms * 1e3:.2f} us {nbytes / (ms * 1e-3) / 1e9:.1f} GB/s; "
            f"unfused rms+rope {ms_u * 1e3:.2f} us (graph replay)")
    return extra


def layer_chain(torch, fp8lin, dev, rot, log):
    """Config 5: QKV-gate -> gate/up+SwiGLU -> down -> vocab-sharded head
    (75968 x 5120) at M = 512 and M = 1, each link fed by the previous one's
    output where the shapes chain (QKV-gate and gate/up both read the layer
    input; attention between them is out of scope).  Every link rotates over
    at least ROTATION_BYTES of its own weight copies (the layer links over
    their `rot` lists, the head over two 389 MB copies), so every figure
    streams from HBM, for the whole chain and for each link alone.  M = 1 is
    timed as graph replays of back-to-back calls (the host's launch rate
    stays out), M = 512 eagerly."""
    import ctypes
    L = fp8lin.lib()
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    heads = [fp8lin.gen_weights(75968, 5120, seed=0, tag=90 + c, device=dev) for c in range(2)]
    shapes = {"qkv_gate": (7168, 5120, False), "gate_up_swiglu": (17408, 5120, True),
              "down": (5120, 8704, False), "head": (75968, 5120, False)}
    weights = {"qkv_gate": rot["qkv_gate"], "gate_up_swiglu": rot["gate_up"], "down": rot["down"], "head": heads}
    copies = max(len(v) for v in weights.values())
    extra = {}

    def ok(rc):
        if rc:
            raise RuntimeError(L.fp8lin_last_error())

    def record(w, n, k):
        c, s = w
        r = fp8lin.Weight()
        r.data, r.scales, r.scale_cols, r.cached_bf16, r.N, r.K = c.data_ptr(), s.data_ptr(), s.size(1), None, n, k
        return r

    for m in (1, 512):
        x = fp8lin.gen_activations(m, 5120, seed=0, tag=2, device=dev)
        outs = {name: torch.empty((m, n // 2 if sw else n), dtype=torch.bfloat16, device=dev)
                for name, (n, _, sw) in shapes.items()}
        feeds = {"qkv_gate": x, "gate_up_swiglu": x, "down": outs["gate_up_swiglu"], "head": outs["down"]}

        # Non-SwiGLU links go through Engine::linear's dispatch (split-K for
        # the few-tile prefill projections); gate/up through the fused kernel,
        # with its workspace.
        opt = fp8lin.LinearOptions()
        recs = {name: [record(w, n, k) for w in weights[name]] for name, (n, k, _) in shapes.items()}
        wss = {}
        for name, (n, k, sw) in shapes.items():
            need = (L.fp8lin_linear_swiglu_workspace_bytes(m, n, k) if sw else
                    L.fp8lin_engine_linear_workspace_bytes(ctypes.byref(opt), ctypes.byref(recs[name][0]), m))
            wss[name] = (torch.empty(need, dtype=torch.uint8, device=dev) if need else None, need)

        def call(name, i):
            n, k, sw = shapes[name]
            ws, need = wss[name]
            wp = P(ws) if ws is not None else None
            if sw:
                c, s = weights[name][i % len(weights[name])]
                ok(L.fp8lin_linear_swiglu_ws(P(feeds[name]), P(c), P(s), s.size(1), P(outs[name]), m, n, k, wp,
                                             need, sp))
            else:
                rec = recs[name][i % len(recs[name])]
                ok(L.fp8lin_engine_linear(ctypes.byref(opt), ctypes.byref(rec), P(feeds[name]), m,
                                          P(outs[name]), n, wp, need, None, sp))

        def rotating(fn):
            i = [0]

            def run():
                fn(i[0])
                i[0] += 1
            return run

        def chain(i):
            for name in shapes:
                call(name, i)

        def time_it(fn):
            if m == 1:
                return graph_timed(torch, rotating(fn), sp, reps=2 * copies, replays=10)
            return timed(torch, rotating(fn), copies, warm=copies)
        total_ms = time_it(chain)
        tot_bytes = tot_flops = 0
        for name, (n, k, sw) in shapes.items():
            ms = time_it(lambda i: call(name, i))
            nbytes = algo_bytes(m, n, k, n // 2 if sw else n)
            flops = 2.0 * m * n * k
            tot_bytes += nbytes
            tot_flops += flops
            key = f"chain_m{m}_{name}"
            extra[key + "_us"] = round(ms * 1e3, 2)
            if m == 1:
                extra[key + "_GBs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
            else:
                extra[key + "_TFLOPs"] = round(flops / (ms * 1e-3) / 1e12, 1)
        extra[f"chain_m{m}_total_us"] = round(total_ms * 1e3, 2)
        if m == 1:
            gbs = tot_bytes / (total_ms * 1e-3) / 1e9
            extra["chain_m1_GBs"] = round(gbs, 1)
            log(f"chain M=1: {total_ms * 1e3:.2f} us, {gbs:.1f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% HBM)")
            # The same four links as one launch (fp8lin_decode_chain) on the
            # same rotation: each link waiting for the previous one (the
            # layer's order), and with no waits (the links read inputs
            # already in HBM), each on a workspace of its own.
            order = list(shapes)

            def chain_recs(i, strict):
                recs = (fp8lin._lib.ChainLink * 4)()
                for j, name in enumerate(order):
                    n, k, sw = shapes[name]
                    c, s = weights[name][i % len(weights[name])]
                    r = recs[j]
                    r.codes, r.scales, r.scale_cols, r.N, r.K = c.data_ptr(), s.data_ptr(), s.size(1), n, k
                    r.x, r.y = feeds[name].data_ptr(), outs[name].data_ptr()
                    r.swiglu, r.after = int(sw), j - 1 if strict else -1
                return recs
            for strict, label in ((True, "one_launch"), (False, "one_launch_independent")):
                cws = torch.zeros(L.fp8lin_decode_chain_workspace_bytes(4), dtype=torch.uint8, device=dev)
                chain_sets = [chain_recs(i, strict) for i in range(copies)]
                pms = time_it(lambda i: ok(L.fp8lin_decode_chain(chain_sets[i % copies], 4, P(cws), cws.numel(),
                                                                 sp)))
                sync = cws.view(torch.int64).cpu()
                if sync[0] != 0:
                    raise RuntimeError(f"decode chain: {int(sync[0])} waits gave up")
                pgbs = tot_bytes / (pms * 1e-3) / 1e9
                extra[f"chain_m1_{label}_us"] = round(pms * 1e3, 2)
                extra[f"chain_m1_{label}_GBs"] = round(pgbs, 1)
                log(f"chain M=1, one launch (fp8lin_decode_chain), {'each link after the previous' if strict else 'no waits'}: "
                    f"{pms * 1e3:.2f} us, {pgbs:.1f} GB/s ({100 * pgbs / HBM_PEAK_GBS:.1f}% HBM)")
        else:
            tf = tot_flops / (total_ms * 1e-3) / 1e12
            extra[f"chain_m{m}_TFLOPs"] = round(tf, 1)
            log(f"chain M={m}: {total_ms:.3f} ms, {tf:.1f} TFLOP/s ({100 * tf / BF16_PEAK_TFLOPS:.1f}% MFMA)")
        log("  " + ", ".join(f"{name} {extra[f'chain_m{m}_{name}_us']} us" for name in shapes))
    return extra


def reference_benchmark_shapes(torch, fp8lin, dev, log):
    """The reference benchmark's remaining shapes (tests/linear_benchmark.cpp:
    22-23): 5120 x 5120 and the 124160 x 5120 head at M = 2, 4, 8, through
    fp8_linear and fp8_tensor_small with split 1 and 4, as graph replays.
    5120 x 5120 rotates over 23 copies (613 MB); the 655 MB head is one
    matrix, larger than twice the Infinity Cache."""
    import ctypes
    L = fp8lin.lib()
    P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    extra = {}

    def ok(rc):
        if rc:
            raise RuntimeError(L.fp8lin_last_error())
    for name, n, k, count in (("5120x5120", 5120, 5120, 23), ("head124160", 124160, 5120, 1)):
        copies = [fp8lin.gen_weights(n, k, seed=0, tag=700 + c, device=dev) for c in range(count)]
        for m in (2, 4, 8):
            x = fp8lin.gen_activations(m, k, seed=0, tag=2, device=dev)
            y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
            paths = {
                "linear": lambda c, s: ok(L.fp8lin_linear(P(x), P(c), P(s), s.size(1), P(y), m, n, k, 1, sp)),
                "tensor_s1": lambda c, s: ok(L.fp8lin_tensor_small(P(x), P(c), P(s), P(y), m, n, k, 1, None, 0,
                                                                  sp)),
                "tensor_s4": lambda c, s: ok(L.fp8lin_tensor_small(P(x), P(c), P(s), P(y), m, n, k, 4, None, 0,
                                                                  sp)),
            }
            for label, fn in paths.items():
                i = [0]

                def run():
                    c, s = copies[i[0] % len(copies)]
                    i[0] += 1
                    fn(c, s)
                ms = graph_timed(torch, run, sp, reps=max(4, 2 * len(copies)), replays=10)
                gbs = algo_bytes(m, n, k) / (ms * 1e-3) / 1e9
                extra[f"refbench_m{m}_{name}_{label}_us"] = round(ms * 1e3, 2)
                extra[f"refbench_m{m}_{name}_{label}_GBs"] = round(gbs, 1)
                log(f"reference shape {name} M={m} {label}: {ms * 1e3:.2f} us {gbs:.1f} GB/s")
        del copies
    return extra


def in_proj_all(torch, fp8lin, dev, log):
    """The GDN in_proj_all group at one rank's size (src/engine.cpp:198-199,
    tests/linear_benchmark.cpp:22): qkv + z fused into 8192 FP8 rows, then the
    BF16 b and a projections (24 + 24 rows), K = 5120, through
    fp8lin_engine_linear_groups into one [M, 8240] output.  M = 1 and 4 are
    decode (M = 4 with the small-M matrix-core option, as the reference's
    benchmark runs its tensor-small variants), M = 512 a prefill chunk.  The
    FP8 group rotates over 13 copies (545 MB), so the decode figures are HBM
    figures."""
    import ctypes
    L = fp8lin.lib()
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    k, nf, nb = 5120, 8192, 48
    fp8 = [fp8lin.gen_weights(nf, k, seed=0, tag=300 + c, device=dev) for c in range(13)]
    bf16 = (fp8lin.gen_activations(nb, k, seed=1, tag=20, device=dev).float() * 0.02).to(torch.bfloat16)
    extra = {}

    def ok(rc):
        if rc:
            raise RuntimeError(L.fp8lin_last_error())

    def groups(c, s):
        g = (fp8lin.Weight * 2)()
        g[0].data, g[0].scales, g[0].scale_cols, g[0].cached_bf16, g[0].N, g[0].K = (
            c.data_ptr(), s.data_ptr(), s.size(1), None, nf, k)
        g[1].data, g[1].scales, g[1].scale_cols, g[1].cached_bf16, g[1].N, g[1].K = (
            bf16.data_ptr(), None, 0, None, nb, k)
        return g
    recs = [groups(c, s) for c, s in fp8]
    for m in (1, 4, 512):
        opt = fp8lin.LinearOptions(fp8_tensor_small=(m == 4))
        x = fp8lin.gen_activations(m, k, seed=0, tag=7, device=dev)
        y = torch.empty((m, nf + nb), dtype=torch.bfloat16, device=dev)
        need = max(L.fp8lin_engine_linear_workspace_bytes(ctypes.byref(opt), ctypes.byref(recs[0][j]), m)
                   for j in range(2))
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
        i = [0]

        def run():
            g = recs[i[0] % len(recs)]
            i[0] += 1
            ok(L.fp8lin_engine_linear_groups(ctypes.byref(opt), g, 2, P(x), m, P(y), nf + nb, P(ws), need, sp))
        ms = (graph_timed(torch, run, sp, reps=2 * len(recs), replays=10) if m <= 8 else
              timed(torch, run, 2 * len(recs)))
        nbytes = algo_bytes(m, nf, k) + nb * k * 2 + 2 * m * nb
        key = f"in_proj_all_m{m}"
        extra[key + "_us"] = round(ms * 1e3, 2)
        if m <= 8:
            extra[key + "_GBs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
            log(f"in_proj_all M={m} (8192 FP8 + 48 BF16 rows, K=5120): {ms * 1e3:.2f} us "
                f"{nbytes / (ms * 1e-3) / 1e9:.1f} GB/s")
        else:
            tf = 2.0 * m * (nf + nb) * k / (ms * 1e-3) / 1e12
            extra[key + "_TFLOPs"] = round(tf, 1)
            log(f"in_proj_all M={m}: {ms:.3f} ms {tf:.1f} TFLOP/s")
    return extra


def calibrate(torch, dev, log):
    """A 256 MiB device-to-device copy (256 MiB read + 256 MiB written): the
    known-size kernel that scales the FETCH_SIZE / WRITE_SIZE counters."""
    src = torch.empty(1 << 28, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    ms = timed(torch, lambda: dst.copy_(src), 5)
    gbs = 2 * (1 << 28) / (ms * 1e-3) / 1e9
    log(f"calibration copy 256 MiB: {ms * 1e3:.1f} us ({gbs:.1f} GB/s read+write)")
    return {"calibration_copy_256MiB_us": round(ms * 1e3, 1)}


def cpu_model():
    """The host CPU's model name and logical CPU count (what lscpu prints as
    "Model name" and "CPU(s)"), from /proc/cpuinfo."""
    try:
        with open("/proc/cpuinfo") as f:
            names = [line.split(":", 1)[1].strip() for line in f if line.startswith("model name")]
    except OSError:
        return None
    if not names:
        return None
    return f"{names[0]} ({len(names)} logical CPUs; {os.cpu_count()} visible)"


def cpu_baseline(ws, xs, seconds, log):
    """The CPU oracle (C restatement of tests/fp8_tensor_test.cpp:11-22,
    OpenMP over output rows) on the same step, repeated for ~`seconds`."""
    import numpy as np
    from oracle import oracle as O  # test infrastructure: the checker, timed as a baseline
    host = {name: (c.cpu().numpy(), s.cpu().numpy()) for name, (c, s) in ws.items()}
    xh = {k: x.view(dtype=__import__("torch").int16).cpu().numpy().view(np.uint16) for k, x in xs.items()}
    threads = O.max_threads()

    def one():
        for name, n, k in SHAPES:
            c, s = host[name]
            O.linear(xh[k], c, s, threads=threads)
    one()
    reps, t0 = 0, time.perf_counter()
    while True:
        one()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 1000:
            break
    per = el / reps
    step_bytes = sum(algo_bytes(1, n, k) for _, n, k in SHAPES)
    gbs = step_bytes / per / 1e9
    log(f"cpu oracle: {per * 1e3:.1f} ms/step on {threads} threads ({gbs:.2f} GB/s)")

    # one thread, one step
    t0 = time.perf_counter()
    for name, n, k in SHAPES:
        c, s = host[name]
        O.linear(xh[k], c, s, threads=1)
    per1 = time.perf_counter() - t0
    log(f"cpu oracle: {per1 * 1e3:.1f} ms/step on 1 thread ({step_bytes / per1 / 1e9:.2f} GB/s)")

    # prefill M=4096 gate/up: 64 of the 17408 weight rows, scaled linearly
    xp = O.gen_activations(0, 2, 4096, 5120)
    c, s = host["gate_up"]
    t0 = time.perf_counter()
    O.linear(xp, c, s, rows=(0, 64), threads=threads)
    part = time.perf_counter() - t0
    est = part * 17408 / 64
    log(f"cpu oracle prefill M=4096 gate/up: {est:.1f} s extrapolated from 64 rows ({part:.2f} s)")
    cpu = {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port", "cpu_model": cpu_model(),
           "sample": f"{reps} full decode steps (3 GEMVs, M=1) in {el:.1f} s; "
                     f"{per * 1e3:.1f} ms per step; FP64 oracle, OpenMP over output rows"}
    extra = {"cpu_1thread_ms_per_step": round(per1 * 1e3, 1),
             "cpu_1thread_GBs": round(step_bytes / per1 / 1e9, 3),
             "cpu_prefill_m4096_gate_up_s_extrapolated": round(est, 1),
             "cpu_prefill_m4096_TFLOPs_extrapolated": round(2.0 * 4096 * 17408 * 5120 / est / 1e12, 5)}
    return cpu, extra


if __name__ == "__main__":
    main()
