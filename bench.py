"""Benchmark of the MXFP8 FMHA forward (hd128) on one MI355X: the reference's headline metric.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload cfg2|cfg3|cfg4|cfg5|cfg1|quant|t128] [--no-cpu]

One step = one call of fmha_fwd_hd128_mxfp8_auto (dispatch + validate + launch, plus the combine on the KV-split
path) on inputs already resident in HBM. Prints ONE JSON line. TFLOP/s = 4 B H S SK 128 / t (algorithmic,
non-causal count, tests/gpu/ref_host.cpp:403); the causal workload counts only the visible
(query, key) pairs, key <= query + SK - S (bottom-right mask).

Timing. Before anything is timed the GPU runs the step for at least CLOCK_WARMUP_MS of wall time (the clock ramps for
tens of milliseconds under this load, whatever --warmup says), then the --warmup untimed steps, then exactly --steps
steps bracketed by synchronisations and HIP events on the launch stream: ms_per_step is their event time / steps
(the wall time is reported beside it). The reference's own method (docs/perf-matrix.md:11: 100 launches, median of 5
repetitions) is reported as `ref_method`.

roofline: the dominant kernel's algorithmic FLOP per launch / its duration, against the dense MXFP8 MFMA peak. The
kernel is launched alone through the C-ABI launcher, timed with HIP events on its stream, median of 5 repetitions of
100 launches, interleaved with repetitions of the whole step so that both see the same clock. cpu_baseline: the oracle's fp32 attention on the dequantised
inputs, all host cores, on a bounded sample of the same workload (rank 0, N = 1).
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_MXFP8_TFLOPS = 5000.0      # MI355X dense MXFP8 MFMA peak, published figure (5.0 PFLOP/s)
PEAK_HBM_GBS = 8000.0           # MI355X HBM3E
REF_PUBLISHED_TFLOPS = 1811.8   # reference, B4H8S2048 vs128 (docs/perf-matrix.md:41)
CLOCK_WARMUP_MS = 400.0         # wall time of untimed steps before any timing (the clock's ramp)
REF_LAUNCHES, REF_REPS = 100, 5 # the reference's timing method (docs/perf-matrix.md:11)

WORKLOADS = {
    # name: (B, H, HK, S, SK, causal, path, splits, description)
    "cfg2": (4, 8, 8, 2048, 2048, False, "auto", None, "B4H8S2048 non-causal (BASELINE configs[1], vs128)"),
    "cfg3": (1, 8, 8, 8192, 8192, False, "auto", None, "B1H8S8192 non-causal (configs[2], vs128)"),
    "cfg4": (2, 8, 8, 2048, 2048, True, "auto", None, "B2H8S2048 causal bottom-right (configs[3])"),
    "cfg5": (1, 8, 8, 128, 16384, False, "kvsplit", 8, "B1H8 Sq128 SK16384 split 8 (configs[4])"),
    "cfg1": (1, 1, 1, 256, 256, False, "auto", None, "B1H1S256 (configs[0], t128)"),
    # the on-GPU quantisers producing cfg2's inputs from bf16 (not the headline metric; an HBM-bound side path)
    "quant": (4, 8, 8, 2048, 2048, False, None, None, "MXFP8 quantisation of B4H8S2048 bf16 Q, K, V"),
    # the reference-named _t128 kernel under its own contract (256 threads, grid (ceil(S/128), H, B)) on every shape the
    # reference publishes for the t128 path; not the headline metric
    "t128": (None, 8, 8, None, None, False, "t128", None, "fmha_fwd_hd128_mxfp8_v3_t128, 256 threads, the 8 published t128 shapes"),
}
# docs/perf-matrix.md: (B, S, SK) -> the reference's TF/s on the t128 path
T128_PUBLISHED = [((1, 512, 512), 104.8), ((1, 1024, 1024), 283.8), ((2, 512, 512), 204.8), ((2, 1024, 1024), 538.5),
                  ((4, 512, 512), 390.2), ((1, 1000, 1000), 256.7), ((1, 2048, 1337), 554.1), ((1, 1000, 1337), 283.4)]


def flops_of(B, H, S, SK, causal):
    if not causal:
        return 4.0 * B * H * S * SK * 128
    vis = sum(max(0, min(SK, i + SK - S + 1)) for i in range(S))
    return 4.0 * B * H * vis * 128


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo) and the core count the OS reports."""
    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    name = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return f"{name} ({os.cpu_count()} logical CPUs on the host)"


def cpu_baseline(B, H, HK, S, SK, causal, budget_s=12.0):
    """fp32 attention on the dequantised inputs (oracle), all host cores, bounded sample: whole (b, h) slices of the
    workload's shape with the first `rows` query rows, rows chosen so the run takes about `budget_s`."""
    import oracle
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    inp = oracle.Inputs(B, H, S, SK, HK=HK, causal=causal)
    rows = min(S, 64)
    secs, _ = oracle.attention_fp32(inp, rows=rows, threads=threads, want_out=False)
    # scale the sample up to the time budget (never beyond the whole workload)
    if secs > 0:
        rows = int(min(S, max(rows, rows * budget_s / max(secs, 1e-3) * 0.5)))
        secs, _ = oracle.attention_fp32(inp, rows=rows, threads=threads, want_out=False)
    if causal:
        vis = sum(max(0, min(SK, i + SK - S + 1)) for i in range(rows))
        fl = 4.0 * B * H * vis * 128
    else:
        fl = 4.0 * B * H * rows * SK * 128
    return {"value": round(fl / secs / 1e12, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"fp32 attention on dequantised MXFP8 inputs, B{B} H{H} SK{SK}, first {rows} of {S} query rows of every "
                      f"(b,h) ({fl / 1e9:.1f} GFLOP in {secs:.2f} s, {threads} threads, oracle/mxfp8_oracle.c)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="cfg2", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--copy-calibration", type=int, metavar="MIB", default=0,
                    help="only run a plain device copy of MIB MiB (steps times): the known-size kernel that scales the "
                         "FETCH_SIZE / WRITE_SIZE counters into bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (the path has no cross-GPU component; --gpus {args.gpus} is not "
              "supported). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "launches": args.steps}), flush=True)
        return
    from amdgpu_rustdsl_amd import lib, ops

    if args.workload == "quant":
        return main_quant(args, torch, lib, ops)
    if args.workload == "t128":
        return main_t128(args, torch, lib, ops)
    B, H, HK, S, SK, causal, path, splits, desc = WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    q, k, v, qs, ks, vs = ops.random_inputs(B, H, S, SK, HK=HK, device=dev, seed=1234)
    out = torch.empty(B, S, H, 128, dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream(dev)

    # the first call goes through the torch-facing op (shape checks, workspace); the timed steps call the C-ABI entry
    # fmha_fwd_hd128_mxfp8_auto directly with the same prepared parameters (dispatch + validate + launch per step)
    used = ops.fmha_fwd_mxfp8(q, k, v, qs, ks, vs, out, path=path, splits=splits, causal=causal)
    p = lib.Params()
    p.o, p.q, p.k, p.v = out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr()
    p.q_descale, p.k_descale, p.v_descale, p.lse = qs.data_ptr(), ks.data_ptr(), vs.data_ptr(), None
    p.bytes_q, p.bytes_k, p.bytes_v, p.bytes_o = ops._cap(q), ops._cap(k), ops._cap(v), ops._cap(out)
    p.bytes_q_descale, p.bytes_k_descale, p.bytes_v_descale = ops._cap(qs), ops._cap(ks), ops._cap(vs)
    p.B, p.H, p.HK, p.S, p.SK = B, H, HK, S, SK
    p.path = -1 if path == "auto" else lib.PATH_IDS[path]
    p.splits, p.causal = splits or 0, int(causal)
    # the KV split's workspace as the op sizes it: the entry's workspace slots of the partials that ran
    ws_bytes = lib.WORKSPACE_SLOTS * ((lib.workspace_bytes(B, H, S, used.partials) + 255) // 256 * 256) if used[0] == "kvsplit" else 0
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    turn = ctypes.c_uint32(0)   # the caller-owned turn word of the workspace slots
    p.ws_turn = ctypes.pointer(turn)
    st = stream.cuda_stream

    # one step = one call of the C entry; its arguments are built once (ctypes objects cost microseconds per call,
    # which a short timed window would otherwise see as GPU idle time before the first launch)
    entry = lib.raw.fmha_fwd_hd128_mxfp8_auto
    po, so, errbuf = ctypes.c_int(-1), ctypes.c_int(0), ctypes.create_string_buffer(512)
    call_args = (ctypes.byref(p), ws.data_ptr(), ws_bytes, st, ctypes.byref(po), ctypes.byref(so), errbuf, 512)

    def step():
        if entry(*call_args) != 0:
            raise RuntimeError(f"fmha_fwd_hd128_mxfp8_auto: {errbuf.value.decode()}")

    assert lib.run_auto(p, ws.data_ptr(), ws_bytes, st) == used
    torch.cuda.synchronize()
    # the configs[1] line is quoted with the LSE saved: the natural-log LSE output (vs128 / t128) is on for the timed
    # steps of the full-sequence paths
    lse = None
    if used[0] in ("vs128", "t128"):
        lse = torch.empty(B, H, S, dtype=torch.float32, device=dev)
        p.lse = lse.data_ptr()
        assert lib.run_auto(p, ws.data_ptr(), ws_bytes, st) == used

    def timed(fn, n):
        """Event time (ms) of n calls of fn on the stream, bracketed by synchronisations; the wall time beside it."""
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1), (time.perf_counter() - t0) * 1e3

    # clock warm-up by wall time, then the --warmup steps, then exactly --steps timed steps
    t_end = time.perf_counter() + CLOCK_WARMUP_MS / 1e3
    clock_steps = 0
    while time.perf_counter() < t_end:
        for _ in range(50):
            step()
        clock_steps += 50
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    ev_ms, wall_ms = timed(step, args.steps)
    ms = ev_ms / args.steps
    ms_wall = wall_ms / args.steps
    fl = flops_of(B, H, S, SK, causal)
    tflops = fl / (ms * 1e-3) / 1e12

    # the dominant kernel alone through its C-ABI launcher, and the reference's timing method (median of 5 repetitions
    # of 100 launches) for the step and the kernel, repetitions interleaved
    launch, kern_name = kernel_launcher(lib, q, k, v, qs, ks, vs, out, lse, used, B, H, HK, S, SK, causal, stream)
    rcs = []
    kern = lambda: rcs.append(launch())
    step_reps, kern_reps = [], []
    for _ in range(REF_REPS):
        step_reps.append(timed(step, REF_LAUNCHES)[0] / REF_LAUNCHES)
        kern_reps.append(timed(kern, REF_LAUNCHES)[0] / REF_LAUNCHES)
    assert all(rc == 0 for rc in rcs), f"kernel launches failed: {sorted(set(rcs))}"
    med = lambda xs: sorted(xs)[len(xs) // 2]
    ref_ms, kern_ms = med(step_reps), med(kern_reps)
    kern_tflops = fl / (kern_ms * 1e-3) / 1e12
    print(f"bench: clock warm-up {clock_steps} steps; {args.steps} steps: events {ms * 1e3:.2f} us/step, wall {ms_wall * 1e3:.2f} "
          f"us/step; reference method: step {ref_ms * 1e3:.2f} us, kernel {kern_name} {kern_ms * 1e3:.2f} us "
          f"(reps step {[round(x * 1e3, 2) for x in step_reps]}, kernel {[round(x * 1e3, 2) for x in kern_reps]})", file=sys.stderr)
    # on the single-kernel paths the step is one launch of the same kernel, so the two agree within the clock noise
    # (about 0.3 %); more than 1 % above both step timings means the kernel leg measured something else
    if kern_ms > 1.01 * max(ms, ref_ms):
        print(f"bench: WARNING kernel_ms {kern_ms:.5f} > ms_per_step {ms:.5f}", file=sys.stderr)
    traffic = None
    tfile = os.path.join(ROOT, "profiles", f"traffic_{args.workload}.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    line = {
        "metric": "FMHA fwd TFLOP/s + % MXFP8 MFMA peak, hd128 B4H8S2048, 1 MI355X",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_warmup": {"ms": CLOCK_WARMUP_MS, "steps": clock_steps},
        "ms_per_step": round(ms, 5),
        "ms_per_step_wall": round(ms_wall, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(tflops / REF_PUBLISHED_TFLOPS, 4) if args.workload == "cfg2" else None,
        "ref_method": {"launches": REF_LAUNCHES, "reps": REF_REPS, "ms_per_step": round(ref_ms, 5),
                       "value": round(fl / (ref_ms * 1e-3) / 1e12, 2),
                       "vs_baseline": round(fl / (ref_ms * 1e-3) / 1e12 / REF_PUBLISHED_TFLOPS, 4) if args.workload == "cfg2" else None},
        "dtype": "e4m3 (MXFP8, E8M0/32 scales, fp32 accumulate)",
        "data": "synthetic: N(0,1) Q/K/V quantised to MXFP8 like the reference's REF_DATA=normal generator, drawn on the GPU",
        "config": {"workload": f"fmha_fwd_hd128_mxfp8_auto {desc}", "B": B, "H": H, "HK": HK, "S": S, "SK": SK,
                   "causal": causal, "path": used[0], "splits": used[1], "kv_partials": used.partials if used[0] == "kvsplit" else None, "lse": lse is not None,
                   "pct_mxfp8_peak": round(100 * tflops / PEAK_MXFP8_TFLOPS, 2)},
        "roofline": {"bound": "mfma", "achieved": round(kern_tflops, 2), "peak": PEAK_MXFP8_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(kern_tflops / PEAK_MXFP8_TFLOPS, 4), "traffic": traffic,
                     "kernel": kern_name, "kernel_ms": round(kern_ms, 5)},
    }
    if used[0] == "kvsplit":
        # the KV split is HBM-bound (about 226 FLOP per byte at config 5, below the ridge of 5.0e15 / 8e12): its
        # split kernel reads Q, K, V and their scales once and writes the fp16 partial rows and LSE words
        rows = B * S * H
        split_bytes = rows * (128 + 4) + 2 * B * SK * HK * 128 + B * SK * HK * 4 + used.partials * rows * (256 + 4)
        gbs = split_bytes / (kern_ms * 1e-3) / 1e9
        line["roofline"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                            "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic, "algorithmic_bytes": split_bytes,
                            "kernel": kern_name, "kernel_ms": round(kern_ms, 5),
                            "mfma_tflops": round(kern_tflops, 2), "mfma_frac": round(kern_tflops / PEAK_MXFP8_TFLOPS, 4)}
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(B, H, HK, S, SK, causal)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


def main_t128(args, torch, lib, ops):
    """The reference-named fmha_fwd_hd128_mxfp8_v3_t128 launched as a reference launcher would (fmha_mxfp8_launch_t128:
    block 256, grid (ceil(S/128), H, B)) on each published t128 shape, timed by the reference's method (100 launches,
    median of 5), after the clock warm-up. value = the smallest ratio to the reference's published TF/s; the per-shape
    figures are in config.shapes."""
    import ctypes
    _, H, HK, _, _, _, _, _, desc = WORKLOADS["t128"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    st = stream.cuda_stream
    shapes, keep = [], []
    for (B, S, SK), ref in T128_PUBLISHED:
        q, k, v, qs, ks, vs = ops.random_inputs(B, H, S, SK, HK=HK, device=dev, seed=1234)
        out = torch.empty(B, S, H, 128, dtype=torch.bfloat16, device=dev)
        a = lib.fill_args(out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), qs.data_ptr(), ks.data_ptr(), vs.data_ptr(),
                          B, H, HK, S, SK)
        grid = (math.ceil(S / 128), H, B)
        sz = lib.BufferSizes(ops._cap(q), ops._cap(k), ops._cap(v), ops._cap(out), ops._cap(qs), ops._cap(ks), ops._cap(vs), 0, 0)
        rc, msg = lib.validate("t128", a, sz, grid, HK=HK)
        assert rc == 0, msg
        keep.append((q, k, v, qs, ks, vs, out, a))
        shapes.append(((B, S, SK), ref, a, grid))
    rcs = []
    def launcher(a, grid):
        return lambda: rcs.append(lib.raw.fmha_mxfp8_launch_t128(ctypes.byref(a), *grid, st))
    # clock warm-up on the first shape
    f0 = launcher(shapes[0][2], shapes[0][3])
    t_end = time.perf_counter() + CLOCK_WARMUP_MS / 1e3
    while time.perf_counter() < t_end:
        for _ in range(50):
            f0()
        torch.cuda.synchronize()
    res = []
    for (B, S, SK), ref, a, grid in shapes:
        f = launcher(a, grid)
        for _ in range(max(args.warmup, 20)):
            f()
        reps = []
        for _ in range(REF_REPS):
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(REF_LAUNCHES):
                f()
            e1.record(stream)
            torch.cuda.synchronize()
            reps.append(e0.elapsed_time(e1) / REF_LAUNCHES)
        ms = sorted(reps)[len(reps) // 2]
        tf = flops_of(B, H, S, SK, False) / (ms * 1e-3) / 1e12
        res.append({"B": B, "S": S, "SK": SK, "us": round(ms * 1e3, 2), "tflops": round(tf, 1), "reference": ref,
                    "ratio": round(tf / ref, 3)})
        print(f"bench t128: B{B}H{H}S{S}SK{SK} {ms * 1e3:.2f} us {tf:.1f} TF/s ({tf / ref:.3f}x the reference)", file=sys.stderr)
    assert all(rc == 0 for rc in rcs), f"kernel launches failed: {sorted(set(rcs))}"
    worst = min(r["ratio"] for r in res)
    line = {
        "metric": "fmha_fwd_hd128_mxfp8_v3_t128 under its 256-thread contract / the reference's published t128 TF/s (worst shape)",
        "value": worst, "unit": "ratio", "n_gpus": 1, "steps": REF_LAUNCHES * REF_REPS, "warmup": max(args.warmup, 20),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": worst, "dtype": "e4m3 (MXFP8, E8M0/32 scales, fp32 accumulate)",
        "data": "synthetic: N(0,1) Q/K/V quantised to MXFP8 like the reference's REF_DATA=normal generator, drawn on the GPU",
        "config": {"workload": desc, "H": H, "shapes": res},
    }
    print(json.dumps(line), flush=True)


def main_quant(args, torch, lib, ops):
    """One step = quantise the bf16 Q, K (rows, E8M0 per 32) and V (one f32 descale) of B4H8S2048 on the GPU.
    value = algorithmic bytes (bf16 read once, e4m3 + scales written once) / step time, in GB/s; roofline = the rows
    kernel on Q alone against HBM bandwidth."""
    B, H, HK, S, SK, _, _, _, desc = WORKLOADS["quant"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    xq = torch.randn(B, S, H, 128, generator=g, device=dev, dtype=torch.bfloat16)
    xk = torch.randn(B, SK, HK, 128, generator=g, device=dev, dtype=torch.bfloat16)
    xv = torch.randn(B, SK, HK, 128, generator=g, device=dev, dtype=torch.bfloat16)
    qs, ks = ops.alloc_scales(B, S, H, dev), ops.alloc_scales(B, SK, HK, dev)
    q8, k8, v8 = (torch.empty(x.shape, dtype=torch.uint8, device=dev) for x in (xq, xk, xv))
    vs = torch.zeros(1024, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    st = stream.cuda_stream
    cap = ops._cap
    mul = ops.LOG2E_OVER_SQRT_D
    nq, nk = xq.numel(), xk.numel()

    def rows_q():
        lib.quantize_rows(xq.data_ptr(), q8.data_ptr(), qs.data_ptr(), nq // 128, mul, cap(xq), cap(q8), cap(qs), st)

    def step():
        rows_q()
        lib.quantize_rows(xk.data_ptr(), k8.data_ptr(), ks.data_ptr(), nk // 128, 1.0, cap(xk), cap(k8), cap(ks), st)
        lib.quantize_tensor(xv.data_ptr(), v8.data_ptr(), vs.data_ptr(), nk, cap(xv), cap(v8), cap(vs), st)

    def timed(fn, n):
        for _ in range(max(args.warmup // 10, 20)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return max(e0.elapsed_time(e1) / n, (time.perf_counter() - t0) * 1e3 / n)

    steps = max(args.steps // 10, 10)
    ms = timed(step, steps)
    bytes_step = (nq * 3 + nq // 8) + (nk * 3 + nk // 8) + nk * 3 + 4
    rows_ms = timed(rows_q, steps)
    rows_bytes = nq * 3 + nq // 8
    gbs = bytes_step / (ms * 1e-3) / 1e9
    rows_gbs = rows_bytes / (rows_ms * 1e-3) / 1e9
    print(f"bench quant: {steps} steps, {ms * 1e3:.2f} us/step; rows kernel {rows_ms * 1e3:.2f} us", file=sys.stderr)
    line = {
        "metric": "MXFP8 input quantisation GB/s (bf16 Q, K, V of B4H8S2048), 1 MI355X",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": max(args.warmup // 10, 20),
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 -> e4m3 + E8M0", "data": "synthetic N(0,1) bf16 drawn on the GPU",
        "config": {"workload": desc, "B": B, "H": H, "HK": HK, "S": S, "SK": SK, "bytes_per_step": bytes_step},
        "roofline": {"bound": "hbm", "achieved": round(rows_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(rows_gbs / PEAK_HBM_GBS, 4), "traffic": None, "kernel": "fmha_mxfp8_quant_rows",
                     "kernel_ms": round(rows_ms, 5)},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def kernel_launcher(lib, q, k, v, qs, ks, vs, out, lse, used, B, H, HK, S, SK, causal, stream):
    """A launch of the main kernel alone (no combine) through its C-ABI launcher, validated once, and its name."""
    import ctypes
    import torch
    from amdgpu_rustdsl_amd.ops import _cap
    a = lib.fill_args(out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), qs.data_ptr(), ks.data_ptr(), vs.data_ptr(),
                      B, H, HK, S, SK)
    a.flags = 1 if causal else 0
    a.ptr_lse = lse.data_ptr() if lse is not None else None
    sz = lib.BufferSizes(_cap(q), _cap(k), _cap(v), _cap(out), _cap(qs), _cap(ks), _cap(vs), 0, 0)
    st = stream.cuda_stream
    path = used[0]
    kernel = "fmha_fwd_hd128_mxfp8_v3_" + path
    if path in ("vs128", "t128"):
        split_tiles = lib.uses_split_tiles(path, B, H, S, SK, causal)
        # the kernel the one-call entry runs: the split-tile kernel (t128's grid, 512 threads), the 256-thread t128
        # kernel (128-row grids below the split-tile threshold) or the path's own; vs128 takes the 128-row grid when
        # its 256-row grid is at most half the chip, and under the causal mask from 4 key tiles on
        row128 = math.ceil(S / 256) * H * B <= 128 or (causal and math.ceil(SK / 128) >= 4)
        on_t128 = path == "t128" or split_tiles or row128
        grid = (math.ceil(S / (128 if on_t128 else 256)), H, B)
        rc, msg = lib.validate("t128" if on_t128 else "vs128", a, sz, grid, HK=HK)
        assert rc == 0, msg
        if split_tiles:
            launch = lambda: lib.raw.fmha_mxfp8_launch_t128_split_tiles(ctypes.byref(a), *grid, st)
        elif on_t128:
            launch = lambda: lib.raw.fmha_mxfp8_launch_t128(ctypes.byref(a), *grid, st)
        else:
            launch = lambda: lib.raw.fmha_mxfp8_launch_vs128(ctypes.byref(a), *grid, st)
        if split_tiles:
            kernel = "fmha_fwd_hd128_mxfp8_v3_t128_split_tiles"
    else:
        # the split kernel as the entry runs it: the partials that ran (the KV fill's), over the entry's workspace slots
        # in turn (one slot would have each launch write over the lines the previous one wrote)
        nsplit = used.partials
        rows_total = B * S * H
        need = lib.workspace_bytes(B, H, S, nsplit)
        stride = (need + 255) // 256 * 256
        ws = torch.empty(lib.WORKSPACE_SLOTS * stride, dtype=torch.uint8, device=q.device)
        kas = []
        for slot in range(lib.WORKSPACE_SLOTS):
            ka = lib.KvsplitArgs()
            ctypes.memmove(ctypes.addressof(ka), ctypes.addressof(a), 0x270)
            ka.ptr_ohat = ws.data_ptr() + slot * stride
            ka.ptr_lse = ka.ptr_ohat + nsplit * rows_total * 512
            ka.kvs_splits, ka.kvs_rows_total = nsplit, rows_total
            kas.append(ka)
        grid = (math.ceil(S / 256), H, B * nsplit)
        sz.ptr_ohat, sz.ptr_lse = nsplit * rows_total * 512, nsplit * rows_total * 4
        rc, msg = lib.validate("kvsplit", kas[0], sz, grid, B=B, HK=HK, KL=0)
        assert rc == 0, msg
        turn = [0]

        def launch(ws=ws):   # (the default argument keeps the workspace tensor alive with the launcher)
            turn[0] += 1
            return lib.raw.fmha_mxfp8_launch_kvsplit(ctypes.byref(kas[turn[0] % len(kas)]), *grid, st)
    for _ in range(20):
        assert launch() == 0
    torch.cuda.synchronize()
    return launch, kernel


if __name__ == "__main__":
    main()
