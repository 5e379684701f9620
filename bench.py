"""Headline benchmark: effective FP64 TFLOPS of emulated mm_nt at n=8192 with
the default plan, on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--n 8192] [--no-accuracy]
                [--no-cpu] [--no-configs] [--no-traffic] [--configs [--config NAME]]
                [--accuracy-grid] [--bmm-sweep] [--square-sweep] [--card-grid]
                [--small-n] [--first-call] [--ceilings] [--calibrate-copy]

One step = one emulated mm_nt of resident 8192x8192 float64 operands (iid
N(0,1) from CPU seeds 2000/2001, configs[1]) through the C ABI
(fp64emu_mm_nt_events, workspace allocated once).  W untimed warm-up calls,
then exactly K calls between two device synchronisations; value = 2 n^3 /
(mean ms per call; the median call's time beside it).  Prints one JSON line.
Before the timing, two rocprofv3 --pmc child runs of this script count the
GEMM launch's L2-boundary traffic (roofline.traffic).  Besides the contract
fields it reports: the per-phase ms (events recorded by each timed call at its
phase boundaries), the ceilings this part attains in the same run (the GEMM's
MFMA loop with operands in registers, read from LDS, and fed by its copies;
HBM streams), the same step through the torch op fp64_emu.mm_nt, native rocBLAS
DGEMM (torch.matmul float64 on the device) throughput, correct bits of both
against a device double-double GEMM, the plan-adjusted INT8 roofline
fraction, the `roofline` object for the dominant kernel (the modular GEMM,
its duration from the events bracketing its launch in every timed call), the CPU
baseline (the oracle port on a bounded sample of the same workload), torch
float64 matmul on the host's cores, and under "configs" every other benchmark
config (c1, c3a, c3b, c4, c5, c5 reduced) plus c2 with the fp64 combine (c2i)
and at the reduced plan (c2r), each with its ms, TFLOP/s, plan fraction,
phases, native comparator and correct bits.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "fp64-emu_amd"))

# The native comparator is rocBLAS DGEMM: torch's float64 matmul with the
# hipBLASLt preference off, set before torch initialises its BLAS handles.
os.environ.setdefault("TORCH_BLAS_PREFER_HIPBLASLT", "0")

INT8_PEAK_TOPS = 5000.0    # MI355X dense INT8 MFMA, 5.0 POP/s
HBM_PEAK_GBS = 8000.0
METRIC = "effective FP64 TFLOPS, mm_nt n=8192 default plan; correct bits vs double-double"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--n", type=int, default=8192)
    ap.add_argument("--no-accuracy", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="leave out the per-config records (c1, c2 inexact and reduced, c3a, "
                         "c3b, c4, c5, c5 reduced) that the headline line carries under "
                         "\"configs\"")
    ap.add_argument("--configs", action="store_true",
                    help="instead of the headline line, one JSON line per benchmark config "
                         "(c1, c2, c3a, c3b, c4, c5 default and reduced)")
    ap.add_argument("--config", choices=CONFIG_NAMES, default=None,
                    help="with --configs: only this config (for a profiler run)")
    ap.add_argument("--accuracy-grid", action="store_true",
                    help="only the correct-bits table of the reference's accuracy study "
                         "(six distributions x K 512/4096 at M = N = 128: native, default, "
                         "reduced) and of its default-call depths, as JSON lines")
    ap.add_argument("--bmm-sweep", action="store_true",
                    help="only the reference's batched grid (bench/bmmbench.py: batch x n = "
                         "64x256 .. 4x4096): native torch.bmm, emulated bmm and a loop of "
                         "emulated mm over the members, as JSON lines")
    ap.add_argument("--square-sweep", action="store_true",
                    help="only square mm_nt products n = 1000 .. 10000 (not multiples of the "
                         "tile size): native float64 matmul against the emulation, as JSON lines")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a float64 streaming kernel over 1 GiB (read 1 GiB, write "
                         "1 GiB) three times: the scale of the FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--ceilings", action="store_true",
                    help="only the ceiling probes: the modular GEMM's inner loop with its "
                         "operands in registers, read from LDS, and fed by its global->LDS "
                         "copies from L2 (TOP/s and shader clock), and HBM read / write / copy "
                         "streams (GB/s), as one JSON line")
    ap.add_argument("--card-grid", action="store_true",
                    help="only the reference's card protocol (bench/card_bench.py): n = 256 .. "
                         "16384, native, default plan and reduced plan, median of timed calls, "
                         "as JSON lines")
    ap.add_argument("--small-n", action="store_true",
                    help="only the reference's small-n table (bench/smalln.py): n = 64 .. 512, "
                         "eager mm against HIP-graph replay of the same call against native, "
                         "as JSON lines")
    ap.add_argument("--first-call", action="store_true",
                    help="only the first-call cost at n = 2048 (the process's first call, the "
                         "first call of a new shape, steady state), as one JSON line; run it "
                         "in a fresh process")
    ap.add_argument("--no-traffic", action="store_true",
                    help="leave roofline.traffic null instead of measuring it with two "
                         "rocprofv3 --pmc child runs (FETCH_SIZE, WRITE_SIZE) before the timing")
    ap.add_argument("--traffic-child", action="store_true", help=argparse.SUPPRESS)
    return ap.parse_args()


CONFIG_NAMES = ("c1", "c2", "c2i", "c2r", "c3a", "c3b", "c4", "c5", "c5r")


def calibrate_copy():
    import torch
    n = (1 << 30) // 8
    src = torch.ones(n, dtype=torch.float64, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy": "torch.neg float64", "bytes_read": n * 8,
                      "bytes_written": n * 8, "launches": 3}), flush=True)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _event_ms(fn, torch):
    """One call of fn bracketed by events on the current stream, in ms."""
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def measure_ceilings(dev, seconds=0.25):
    """The rates this part attains, measured by the library's probes
    (fp64emu_probe_mfma, fp64emu_probe_stream):

    - mfma_registers: the modular GEMM's MFMA loop (one group of 4 waves
      per CU, 8 x 8 accumulator quads per wave, 64 v_mfma_i32_16x16x64_i8
      per step in its order) on random balanced residues held in registers:
      the INT8 rate this part sustains under its power limit;
    - mfma_lds_reads: the same with the GEMM's fragment reads from its LDS
      ring and its per-step wait and barrier;
    - mfma_lds_copies: that plus its global->LDS copies from an L2-resident
      source: the GEMM's inner loop without HBM traffic, prologue, epilogue
      or tail.
    Each is the median of 3 launches of about `seconds`; the shader clock is
    the median over groups of s_memtime against the 100 MHz s_memrealtime.
    Then HBM streams over 1 GiB buffers (median of 5): read, write, and
    read-plus-write (the byte phases' shape)."""
    import statistics
    import numpy as np
    import torch
    from fp64_emu import capi
    groups = torch.cuda.get_device_properties(dev).multi_processor_count
    src = torch.from_numpy(capi.probe_source(11)).to(dev)
    ops_per_step = groups * 4 * 64 * 16 * 16 * 64 * 2
    out = {"groups": groups}
    for mode, name in ((0, "mfma_registers"), (1, "mfma_lds_reads"), (2, "mfma_lds_copies")):
        steps = 2001
        capi.probe_mfma(src, groups, steps, mode)          # warm-up
        t = _event_ms(lambda: capi.probe_mfma(src, groups, steps, mode), torch)
        steps = max(2001, int(steps * seconds * 1e3 / t)) | 1
        ts, ghz = [], []
        for _ in range(3):
            res = {}

            def run():
                res["clk"] = capi.probe_mfma(src, groups, steps, mode)[1]
            ts.append(_event_ms(run, torch))
            c = res["clk"].cpu().numpy().astype(np.float64)
            ghz.append(float(np.median((c[:, 1] - c[:, 0]) / (c[:, 3] - c[:, 2]) * 0.1)))
        t = statistics.median(ts)
        out[name] = {"tops": round(ops_per_step * steps / (t * 1e-3) / 1e12, 1),
                     "clock_ghz": round(statistics.median(ghz), 3), "steps": steps,
                     "ms": round(t, 3)}
    n = (1 << 30) // 8
    a = torch.ones(n, dtype=torch.float64, device=dev)
    b = torch.empty_like(a)
    for mode, name, nbytes in ((0, "hbm_read", 8 * n), (1, "hbm_write", 8 * n),
                               (2, "hbm_copy", 16 * n)):
        for _ in range(2):
            capi.probe_stream(b, a, mode)
        t = statistics.median(_event_ms(lambda: capi.probe_stream(b, a, mode), torch)
                              for _ in range(5))
        out[name] = {"gbs": round(nbytes / (t * 1e-3) / 1e9, 1), "ms": round(t, 4),
                     "bytes": nbytes}
    del a, b
    torch.cuda.empty_cache()
    return out


def traffic_child(n):
    """Run under rocprofv3 --pmc by measure_traffic: the copy probe over
    1 GiB (known bytes, the counters' scale), then two c2 calls."""
    import torch
    import fp64_emu
    from fp64_emu import capi
    dev = torch.device("cuda:0")
    m = (1 << 30) // 8
    a = torch.ones(m, dtype=torch.float64, device=dev)
    b = torch.empty_like(a)
    capi.probe_stream(b, a, 2)
    torch.cuda.synchronize()
    del a, b
    g = torch.Generator().manual_seed(2000)
    A = torch.randn(n, n, dtype=torch.float64, generator=g).to(dev)
    g = torch.Generator().manual_seed(2001)
    Bt = torch.randn(n, n, dtype=torch.float64, generator=g).to(dev)
    for _ in range(2):
        fp64_emu.mm_nt(A, Bt)
    torch.cuda.synchronize()
    print("traffic child done", flush=True)


def measure_traffic(n, timeout=240):
    """The modular GEMM's traffic across the L2 boundary per launch (reads
    from MALL or HBM plus writes), from two rocprofv3 --pmc child runs of
    traffic_child: FETCH_SIZE, then WRITE_SIZE (KiB per dispatch), each
    scaled by what the same counter reads for the copy probe's 1 GiB read
    and 1 GiB write in that run.  None (with the reason logged) when
    rocprofv3 is missing or a run fails."""
    import csv
    import shutil
    import subprocess
    import tempfile
    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(prof):
        log("traffic: rocprofv3 not found")
        return None
    # Under a profiler the children would inherit its preloaded tool library,
    # which opens the GPU in every process of the child's launch chain
    # before that chain execs the next program: skip the measurement.
    if "rocprofiler" in os.environ.get("LD_PRELOAD", "") or "ROCP_TOOL_LIBRARIES" in os.environ:
        log("traffic: skipped (this run is itself under rocprofv3)")
        return None
    res = {}
    env = dict(os.environ, TMPDIR="/tmp")
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="fp64emu_pmc_", dir="/tmp")
        cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "t", "--",
               sys.executable, os.path.abspath(__file__), "--traffic-child", "--n", str(n)]
        log(f"traffic: {counter} child run")
        try:
            r = subprocess.run(cmd, cwd="/tmp", env=env, timeout=timeout, capture_output=True,
                               text=True)
        except subprocess.TimeoutExpired:
            log(f"traffic: {counter} run timed out")
            return None
        files = [os.path.join(dp, f) for dp, _, fs in os.walk(d) for f in fs
                 if f.endswith("counter_collection.csv")]
        if r.returncode != 0 or "traffic child done" not in r.stdout or not files:
            log(f"traffic: {counter} run failed (rc {r.returncode}): {r.stderr[-300:]}")
            return None
        gemm, copy = [], []
        with open(files[0]) as f:
            for row in csv.DictReader(f):
                if row["Counter_Name"] != counter:
                    continue
                if "modgemm_kernel" in row["Kernel_Name"]:
                    gemm.append(float(row["Counter_Value"]))
                elif "stream_probe_kernel<2>" in row["Kernel_Name"]:
                    copy.append(float(row["Counter_Value"]))
        shutil.rmtree(d, ignore_errors=True)
        if not gemm or len(copy) != 1:
            log(f"traffic: {counter}: no dispatches found")
            return None
        scale = copy[0] * 1024 / float(1 << 30)     # counter KiB per true byte / 1024
        res[counter] = {"kib_per_dispatch": round(sum(gemm) / len(gemm), 1),
                        "dispatches": len(gemm), "copy_probe_kib": round(copy[0], 1),
                        "scale": round(scale, 5),
                        "bytes": int(sum(gemm) / len(gemm) * 1024 / scale)}
    total = res["FETCH_SIZE"]["bytes"] + res["WRITE_SIZE"]["bytes"]
    log(f"traffic: {res['FETCH_SIZE']['bytes'] / 1e9:.2f} GB fetched + "
        f"{res['WRITE_SIZE']['bytes'] / 1e9:.2f} GB written per GEMM launch")
    return {"bytes_per_launch": total, "counters": res,
            "method": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE child runs of this script "
                      "(--traffic-child: the copy probe over 1 GiB for the scale, then two c2 "
                      "calls), averaged over the modgemm dispatches"}


def card_grid():
    """The reference's card protocol (bench/card_bench.py:14-44, README.md:
    125-138): n = 256 .. 16384, randn operands (CPU seeds 8000 + n), native
    float64 matmul (rocBLAS) and the emulated mm at the default plan
    (plan_config(n)) and the reduced plan (one modulus fewer, no
    correction), each the median of timed calls (host clock, a
    synchronisation per call, after 3 warm-ups; 30 calls up to n = 1024, 3
    at 16384, else 8; native half as many, at least 3)."""
    import statistics
    import torch
    import fp64_emu
    dev = torch.device("cuda:0")
    pin_rocblas()

    def timed(fn, iters, warmup=3):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(iters):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    for n in (256, 1024, 2048, 4096, 8192, 16384):
        flop = 2.0 * n ** 3
        it = 3 if n >= 16384 else (30 if n <= 1024 else 8)
        g = torch.Generator().manual_seed(8000 + n)
        A = torch.randn(n, n, dtype=torch.float64, generator=g).to(dev)
        Bt = torch.randn(n, n, dtype=torch.float64, generator=g).to(dev)
        B = Bt.t().contiguous()
        tn = timed(lambda: A @ Bt, max(3, it // 2))
        P, corr = fp64_emu.plan_config(n)
        rec = {"table": "card_grid", "n": n, "native": {"ms": round(tn * 1e3, 4),
                                                       "tflops": round(flop / tn / 1e12, 2)}}
        for cfg, pp, cc in (("default", P, corr), ("reduced", P - 1, False)):
            t = timed(lambda: fp64_emu.mm(A, B, nprimes=pp, corr=cc), it)
            rec[cfg] = {"plan": [pp, cc], "ms": round(t * 1e3, 4),
                        "tflops": round(flop / t / 1e12, 2), "x_native": round(tn / t, 2)}
        print(json.dumps(rec), flush=True)
        del A, Bt, B
        torch.cuda.empty_cache()


def small_n():
    """The reference's small-n table (bench/smalln.py:29-50, paper.tex:
    650-652): n = 64 .. 512, randn A and B (CPU seeds), the emulated mm
    eager against a HIP-graph replay of the same call against native
    float64 matmul, each the median of 200 host-timed calls (a
    synchronisation per call) after 20 warm-ups; the replay's output is
    checked against an eager call."""
    import statistics
    import torch
    import fp64_emu
    dev = torch.device("cuda:0")
    pin_rocblas()

    def timed(fn, iters=200, warm=20):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(iters):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    for n in (64, 128, 256, 512):
        g = torch.Generator().manual_seed(8500 + n)
        A = torch.randn(n, n, dtype=torch.float64, generator=g).to(dev)
        B = torch.randn(n, n, dtype=torch.float64, generator=g).to(dev)
        te = timed(lambda: fp64_emu.mm(A, B))
        tn = timed(lambda: A @ B.t())
        for _ in range(3):
            fp64_emu.mm(A, B)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            C = fp64_emu.mm(A, B)
        graph.replay()
        torch.cuda.synchronize()
        ok = bool(torch.equal(C, fp64_emu.mm(A, B)))
        tg = timed(graph.replay)
        print(json.dumps({"table": "small_n", "n": n, "eager_us": round(te * 1e6, 1),
                          "graph_us": round(tg * 1e6, 1), "native_us": round(tn * 1e6, 1),
                          "eager_over_graph": round(te / tg, 2),
                          "graph_vs_native": round(tn / tg, 2), "graph_equals_eager": ok}),
              flush=True)
        del graph, C, A, B
        torch.cuda.empty_cache()


def first_call():
    """First-call cost (paper.tex:674-677 reports the reference's first call
    at a new shape, which runs its dispatch probe: 16.6 ms against 1.41 ms
    steady at n = 2048).  This build keeps no per-shape state, so a first
    call costs the workspace allocation plus, once per process, the loading
    of the library's code objects.  In this process, with resident randn
    operands: (1) the process's first emulated mm call (n = 1024), (2) the
    1024 steady state, (3) after torch's cached blocks are released, the
    first call at the new shape n = 2048, (4) the 2048 steady state, the
    median of 20 calls; host clock, a synchronisation per call.  Run it as
    its own process."""
    import statistics
    import torch
    import fp64_emu
    dev = torch.device("cuda:0")

    def once(fn):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3

    g = torch.Generator().manual_seed(8900)
    A = torch.randn(2048, 2048, dtype=torch.float64, generator=g).to(dev)
    B = torch.randn(2048, 2048, dtype=torch.float64, generator=g).to(dev)
    a, b = A[:1024, :1024].contiguous(), B[:1024, :1024].contiguous()
    torch.cuda.synchronize()
    first = once(lambda: fp64_emu.mm(a, b))
    steady_1024 = statistics.median(once(lambda: fp64_emu.mm(a, b)) for _ in range(20))
    torch.cuda.empty_cache()
    new_shape = once(lambda: fp64_emu.mm(A, B))
    steady = statistics.median(once(lambda: fp64_emu.mm(A, B)) for _ in range(20))
    print(json.dumps({"table": "first_call", "process_first_ms_n1024": round(first, 3),
                      "steady_ms_n1024": round(steady_1024, 3),
                      "new_shape_first_ms_n2048": round(new_shape, 3),
                      "steady_ms_n2048": round(steady, 3),
                      "process_first_over_steady": round(first / steady_1024, 2),
                      "new_shape_over_steady": round(new_shape / steady, 2)}), flush=True)


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build runs on one GPU only (the emulated GEMM has no "
              "multi-GPU path); use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.traffic_child:
        traffic_child(args.n)
        return
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.ceilings:
        import torch
        print(json.dumps({"table": "ceilings", **measure_ceilings(torch.device("cuda:0"))}),
              flush=True)
        return
    if args.card_grid:
        card_grid()
        return
    if args.small_n:
        small_n()
        return
    if args.first_call:
        first_call()
        return
    if args.accuracy_grid:
        accuracy_grid()
        return
    if args.bmm_sweep:
        bmm_sweep()
        return
    if args.square_sweep:
        square_sweep()
        return
    if args.configs:
        run_configs(max(args.steps, 3), max(args.warmup, 1),
                    [args.config] if args.config else CONFIG_NAMES)
        return

    # The modular GEMM's L2-boundary traffic per launch, counted in two
    # rocprofv3 child runs before this process touches the GPU.
    traffic = None
    if not args.no_traffic:
        traffic = measure_traffic(args.n)

    import torch
    import fp64_emu
    from fp64_emu import capi

    dev = torch.device("cuda:0")
    pin_rocblas()
    n = args.n
    M = N = K = n
    P, corr = fp64_emu.plan_config(K)
    G = P + (2 if corr else 0)
    flop = 2.0 * M * N * K

    g = torch.Generator().manual_seed(2000)
    A = torch.randn(M, K, dtype=torch.float64, generator=g).to(dev)
    g = torch.Generator().manual_seed(2001)
    Bt = torch.randn(K, N, dtype=torch.float64, generator=g).to(dev)
    torch.cuda.synchronize()
    log(f"inputs resident: {n}^3, plan P={P} corr={corr} G={G}")

    # Timed region: K calls through the C ABI's instrumented mm_nt on a
    # workspace and output allocated once; every call records its phase
    # boundaries on the stream the kernels run on (no synchronisation).
    primes = fp64_emu._PRIMES[:P]
    lay = capi.layout(1, M, N, K, P, corr)
    ws = torch.empty(int(lay.total), dtype=torch.uint8, device=dev)
    C = torch.empty(M, N, dtype=torch.float64, device=dev)
    evs = [capi.PhaseEvents() for _ in range(max(args.steps, 1))]
    for i in range(args.warmup):
        capi.mm_nt_events(A, Bt, primes, C, ws, evs[i % len(evs)], use_corr=corr)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        capi.mm_nt_events(A, Bt, primes, C, ws, evs[i], use_corr=corr)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed * 1e3 / max(args.steps, 1)
    value = flop / (ms * 1e-3) / 1e12
    log(f"timed {args.steps} steps: {ms:.3f} ms/step, {value:.1f} TFLOP/s")
    phases = [e.phases_ms() for e in evs[:max(args.steps, 1)]]
    avg = [sum(p[i] for p in phases) / len(phases) for i in range(4)]
    gemm_ms = avg[1]    # events 1 -> 2 bracket exactly the one modgemm launch
    gemm_tops = 2.0 * M * N * K * G / (gemm_ms * 1e-3) / 1e12
    # Per call, events 0 -> 4 bracket the whole call on the device: the
    # median call (BASELINE's protocol) beside the mean of the wall clock.
    calls = sorted(sum(p) for p in phases)
    med_ms = calls[len(calls) // 2] if len(calls) % 2 else 0.5 * (
        calls[len(calls) // 2 - 1] + calls[len(calls) // 2])
    gemms = sorted(p[1] for p in phases)
    med_gemm_ms = gemms[len(gemms) // 2]
    log(f"phases ms (avg of {len(phases)}): {['%.3f' % x for x in avg]}; median call "
        f"{med_ms:.3f} ms")
    del ws, evs

    # The same step through the drop-in torch op (workspace from torch's
    # caching allocator), for comparison.
    for _ in range(2):
        C2 = fp64_emu.mm_nt(A, Bt)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    op_steps = max(3, min(args.steps, 10))
    for _ in range(op_steps):
        C2 = fp64_emu.mm_nt(A, Bt)
    torch.cuda.synchronize()
    op_ms = (time.perf_counter() - t0) * 1e3 / op_steps
    assert torch.equal(C, C2), "torch op and C ABI results differ"
    del C2
    log(f"torch op mm_nt: {op_ms:.3f} ms/step")

    # Native DGEMM comparator (rocBLAS through torch.matmul float64).
    for _ in range(2):
        Cn = A @ Bt
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    nat_steps = max(3, min(args.steps, 10))
    for _ in range(nat_steps):
        Cn = A @ Bt
    torch.cuda.synchronize()
    nat_ms = (time.perf_counter() - t0) * 1e3 / nat_steps
    nat_tf = flop / (nat_ms * 1e-3) / 1e12
    log(f"native DGEMM: {nat_ms:.3f} ms, {nat_tf:.1f} TFLOP/s")

    acc = {}
    if not args.no_accuracy:
        hi, lo = capi.ddgemm_nt(A, Bt.t().contiguous())
        torch.cuda.synchronize()
        scale = hi.abs().max().item()

        def bits(X):
            err = ((X - hi) - lo).abs().max().item()
            return 53.0 if err == 0 else -math.log2(err / scale)

        acc = {"correct_bits_emu": round(bits(C), 2), "correct_bits_native": round(bits(Cn), 2)}
        del hi, lo
        log(f"correct bits: emu {acc['correct_bits_emu']}, native {acc['correct_bits_native']}")
    del Cn

    # The attainable rates of this part, measured in the same run after the
    # timed calls (the probes run the chip at its power limit).
    ceil = measure_ceilings(dev)
    mfma_ceiling = ceil["mfma_registers"]["tops"]
    log(f"ceilings: MFMA in registers {mfma_ceiling:.0f} TOP/s at "
        f"{ceil['mfma_registers']['clock_ghz']:.2f} GHz, with LDS reads "
        f"{ceil['mfma_lds_reads']['tops']:.0f}, with copies {ceil['mfma_lds_copies']['tops']:.0f}; "
        f"HBM copy {ceil['hbm_copy']['gbs']:.0f} GB/s")

    cpu = None
    cpu_torch = None
    if not args.no_cpu:
        cpu = cpu_baseline(A, Bt, P, corr)
        cpu_torch = cpu_torch_baseline(A, Bt)

    configs = None
    if not args.no_configs and n == 8192:
        # Every other benchmark config (and c2's other operating points) in
        # the same run, timed through the torch op like the reference's
        # benchmarks; the headline c2 line above is this table's c2 row.
        del A, Bt, C
        torch.cuda.empty_cache()
        configs = run_configs(3, 1, [c for c in CONFIG_NAMES if c != "c2"], emit=False)
        for r in configs:
            log(f"config {r['config']}: {r['ms']:.3f} ms, {r['tflops']:.2f} TFLOP/s, "
                f"{r['tflops'] / r['native_tflops']:.2f}x native, bits {r['correct_bits_emu']} / "
                f"{r['correct_bits_native']}")

    rec = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic",
        "config": {"workload": f"mm_nt M=N=K={n}, A/Bt iid N(0,1) (CPU seeds 2000/2001), "
                               f"default plan_config({K}) = ({P}, corr={corr})",
                   "M": M, "N": N, "K": K, "nprimes": P, "corr": corr, "gemms": G,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": "modgemm_kernel",
                     "achieved": round(gemm_tops, 1), "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(gemm_tops / INT8_PEAK_TOPS, 4),
                     "traffic": traffic["bytes_per_launch"] if traffic else None,
                     "work": "2*M*N*K*G INT8 ops per launch",
                     "measured_peak": round(mfma_ceiling, 1),
                     "frac_of_measured": round(gemm_tops / mfma_ceiling, 4),
                     "measured_loop": round(ceil["mfma_lds_copies"]["tops"], 1),
                     "frac_of_measured_loop": round(gemm_tops / ceil["mfma_lds_copies"]["tops"], 4)},
        "plan_roofline_frac": round(value / (INT8_PEAK_TOPS / G), 4),
        "median_call_ms": round(med_ms, 4),
        "value_at_median_call": round(flop / (med_ms * 1e-3) / 1e12, 3),
        "median_gemm_ms": round(med_gemm_ms, 4),
        "phases_ms": [round(x, 4) for x in avg],
        "torch_op_ms_per_step": round(op_ms, 4),
        "native_dgemm_tflops": round(nat_tf, 2),
        "native_dgemm_ms": round(nat_ms, 3),
        "speedup_vs_native": round(value / nat_tf, 3),
        **acc,
        "cpu_baseline": cpu,
        "cpu_torch_f64": cpu_torch,
        "ceilings": ceil,
        "traffic": traffic,
        "native_blas": native_blas(),
        "configs": configs,
    }
    print(json.dumps(rec), flush=True)


def accuracy_grid():
    """Correct bits against the device double-double GEMM on the input
    distributions of the reference's accuracy study (bench/accuracy.py:85-118,
    README.md:200-213) and its default-call depths (bench/defaultcheck.py),
    with inputs from the CPU seeds the GPU parity tests use."""
    import torch
    import fp64_emu
    from fp64_emu import capi
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from distributions import DISTS, make, seed_of
    dev = torch.device("cuda:0")

    def bits(X, hi, lo):
        err = ((X - hi) - lo).abs().max().item()
        return 53.0 if err == 0 else round(-math.log2(err / hi.abs().max().item()), 2)

    for dist in DISTS:
        for K in (512, 4096):
            A, Bt = make(dist, 128, K, 128, seed_of(dist, K))
            A, Bt = A.to(dev), Bt.to(dev)
            hi, lo = capi.ddgemm_nt(A, Bt.t().contiguous())
            rec = {"table": "grid", "dist": dist, "K": K, "native": bits(A @ Bt, hi, lo),
                   "default": bits(fp64_emu.mm_nt(A, Bt), hi, lo),
                   "reduced": bits(fp64_emu.mm_nt(A, Bt, nprimes=13, corr=False), hi, lo)}
            print(json.dumps(rec), flush=True)
    for K in (64, 256, 1024, 4096):
        for dist in ("randn", "wide16", "illcond40", "spike"):
            A, Bt = make(dist, 128, K, 128, seed_of(dist, K) + 1)
            A, Bt = A.to(dev), Bt.to(dev)
            hi, lo = capi.ddgemm_nt(A, Bt.t().contiguous())
            P, corr = fp64_emu.plan_config(K)
            rec = {"table": "default_call", "dist": dist, "K": K, "plan": [P, corr],
                   "native": bits(A @ Bt, hi, lo),
                   "default": bits(fp64_emu.mm(A, Bt.t().contiguous()), hi, lo)}
            print(json.dumps(rec), flush=True)


def _median_event_time(fn, torch, reps=8):
    """Median of `reps` event-timed calls of fn after 3 warm-ups, in seconds."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e-3)
    return sorted(ts)[len(ts) // 2]


def square_sweep():
    """Square mm_nt products of sizes that are not multiples of the GEMM tile
    (randn A and Bt, CPU seeds 9500 + n): native float64 matmul (rocBLAS)
    against the emulation at the default plan, each the median of 8
    event-timed calls after 3 warm-ups."""
    import torch
    import fp64_emu
    dev = torch.device("cuda:0")
    pin_rocblas()
    for n in (1000, 1500, 2000, 3000, 5000, 6000, 10000):
        g = torch.Generator().manual_seed(9500 + n)
        A = torch.randn((n, n), dtype=torch.float64, generator=g).to(dev)
        Bt = torch.randn((n, n), dtype=torch.float64, generator=g).to(dev)
        flop = 2.0 * n ** 3
        tn = _median_event_time(lambda: A @ Bt, torch)
        te = _median_event_time(lambda: fp64_emu.mm_nt(A, Bt), torch)
        print(json.dumps({"table": "square_sweep", "n": n,
                          "native_tflops": round(flop / tn / 1e12, 2),
                          "emu_tflops": round(flop / te / 1e12, 2),
                          "emu_vs_native": round(tn / te, 2),
                          "ms": {"native": round(tn * 1e3, 4), "emu": round(te * 1e3, 4)}}),
              flush=True)
        del A, Bt
        torch.cuda.empty_cache()


def bmm_sweep():
    """The reference's batched grid (bench/bmmbench.py:29-43, README.md:156-172):
    for batch x n in 64x256 .. 4x4096, randn A and B (CPU seeds), effective
    FP64 TFLOP/s of native torch.bmm (rocBLAS), of the emulated bmm (one launch
    chain for the batch), and of a loop of emulated mm over the members; each
    the median of 8 event-timed calls after 3 warm-ups."""
    import torch
    import fp64_emu
    dev = torch.device("cuda:0")
    pin_rocblas()

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(8):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e-3)
        return sorted(ts)[len(ts) // 2]

    for b, n in ((64, 256), (32, 512), (16, 1024), (8, 2048), (4, 4096)):
        g = torch.Generator().manual_seed(7000 + n)
        A = torch.randn(b, n, n, dtype=torch.float64, generator=g).to(dev)
        Bt = torch.randn(b, n, n, dtype=torch.float64, generator=g).to(dev)
        Bm = Bt.transpose(1, 2).contiguous()
        flop = 2.0 * b * n ** 3
        tn = timed(lambda: torch.bmm(A, Bt))
        tb = timed(lambda: fp64_emu.bmm(A, Bm))
        tl = timed(lambda: torch.stack([fp64_emu.mm(A[i], Bm[i]) for i in range(b)]))
        print(json.dumps({"table": "bmm_sweep", "batch": b, "n": n,
                          "native_tflops": round(flop / tn / 1e12, 2),
                          "emu_bmm_tflops": round(flop / tb / 1e12, 2),
                          "emu_vs_native": round(tn / tb, 2),
                          "looped_mm_tflops": round(flop / tl / 1e12, 2),
                          "bmm_vs_looped": round(tl / tb, 2),
                          "ms": {"native": round(tn * 1e3, 4), "emu_bmm": round(tb * 1e3, 4),
                                 "looped_mm": round(tl * 1e3, 4)}}), flush=True)
        del A, Bt, Bm
        torch.cuda.empty_cache()


def _config_inputs(name, torch):
    """Inputs of the benchmark configs c1 .. c5, generated on the CPU (seeds 1000 cfg,
    1000 cfg + 1)."""
    g = lambda seed: torch.Generator().manual_seed(seed)  # noqa: E731
    if name == "c1":
        return "mm_nt", torch.randn(128, 4096, dtype=torch.float64, generator=g(1000)), \
            torch.randn(4096, 128, dtype=torch.float64, generator=g(1001)), None
    if name in ("c2", "c2i", "c2r"):
        # c2i: the fp64 combine (exact=False, README.md:117-121); c2r: the
        # reduced operating point, 13 moduli and no correction (README.md:137).
        plan = {"c2": None, "c2i": (14, True, False), "c2r": (13, False)}[name]
        return "mm_nt", torch.randn(8192, 8192, dtype=torch.float64, generator=g(2000)), \
            torch.randn(8192, 8192, dtype=torch.float64, generator=g(2001)), plan
    if name == "c3a":
        def wide(seed):
            gg = g(seed)
            sgn = torch.randint(0, 2, (4096, 4096), generator=gg) * 2 - 1
            m = 1 + torch.rand(4096, 4096, generator=gg, dtype=torch.float64)
            e = torch.randint(-20, 21, (4096, 4096), generator=gg)
            return sgn * torch.ldexp(m, e)
        return "mm_nt", wide(3000), wide(3001), None
    if name == "c3b":
        r = lambda seed: torch.randint(-2 ** 20, 2 ** 20 + 1, (4096, 4096), generator=g(seed)).double()  # noqa: E731
        return "mm_nt", r(3100), r(3101), None
    if name == "c4":
        return "bmm_nt", torch.randn(64, 512, 512, dtype=torch.float64, generator=g(4000)), \
            torch.randn(64, 512, 512, dtype=torch.float64, generator=g(4001)), None
    u = lambda shape, seed: torch.rand(shape, dtype=torch.float64, generator=g(seed)) * 2 - 1  # noqa: E731
    A, B = u((1023, 32769), 5000), u((32769, 2049), 5001)
    return "mm_nt", A, B, ((13, False) if name == "c5r" else None)


def run_configs(steps, warmup, names, emit=True):
    """One record per benchmark config: effective FP64 TFLOPS, the
    plan-adjusted INT8 roofline fraction, per-phase ms (mm_nt forms), the
    native float64 comparator and correct bits against the device
    double-double GEMM.  Printed as JSON lines when `emit`; returned."""
    import torch
    import fp64_emu
    from fp64_emu import capi
    dev = torch.device("cuda:0")
    pin_rocblas()
    records = []
    for name in names:
        kind, A, B, plan = _config_inputs(name, torch)
        A, B = A.to(dev), B.to(dev)
        batched = kind == "bmm_nt"
        K = A.shape[-1]
        P, corr = plan[:2] if plan else fp64_emu.plan_config(K)
        exact = plan[2] if plan and len(plan) > 2 else True
        G = P + (2 if corr else 0)
        M, N = A.shape[-2], B.shape[-1]
        batch = A.shape[0] if batched else 1
        flop = 2.0 * batch * M * N * K
        emu = (lambda: fp64_emu.bmm_nt(A, B, nprimes=P, corr=corr, exact=exact)) if batched else \
            (lambda: fp64_emu.mm_nt(A, B, nprimes=P, corr=corr, exact=exact))
        nat = (lambda: torch.bmm(A, B)) if batched else (lambda: A @ B)

        def timed(fn):
            # At least `steps` calls and about 50 ms of them (small configs
            # take tens of microseconds, where a handful of calls would time
            # mostly the host's synchronisation), after at least `warmup`
            # calls and about 100 ms of them: each config follows seconds of
            # host-side input generation with the GPU idle, and a shorter
            # warm-up timed the clock's ramp (c3a: 1.142 ms per call against
            # 1.051 ms summed over its phases in the same run).
            t0 = time.perf_counter()
            i = 0
            while i < warmup or time.perf_counter() - t0 < 0.1:
                fn()
                i += 1
                if i % 8 == 0:
                    torch.cuda.synchronize()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            one = time.perf_counter() - t0
            n = max(steps, min(500, int(0.05 / max(one, 1e-6))))
            t0 = time.perf_counter()
            for _ in range(n):
                fn()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e3 / n

        ms = timed(emu)
        nat_ms = timed(nat)
        # Per-phase times: events at the phase boundaries of each call
        # (fp64emu_mm_nt_events / fp64emu_bmm_nt_events), averaged.
        primes = fp64_emu._PRIMES[:P]
        lay = capi.layout(batch, M, N, K, P, corr)
        ws = torch.empty(int(lay.total), dtype=torch.uint8, device=dev)
        C = torch.empty((batch, M, N) if batched else (M, N), dtype=torch.float64, device=dev)
        evs = [capi.PhaseEvents() for _ in range(steps)]
        for i in range(steps):
            if batched:
                capi.bmm_nt_events(A, B, primes, C, ws, evs[i], use_corr=corr, exact=exact)
            else:
                capi.mm_nt_events(A, B, primes, C, ws, evs[i], use_corr=corr, exact=exact)
        torch.cuda.synchronize()
        ph = [e.phases_ms() for e in evs]
        phases = [round(sum(p[i] for p in ph) / len(ph), 4) for i in range(4)]
        del ws, C, evs
        Ce, Cn = emu(), nat()
        bits = {}
        for tag, X in (("emu", Ce), ("native", Cn)):
            errs, scale = 0.0, 0.0
            for b in range(batch):
                Ab = A[b] if batched else A
                Bb = B[b] if batched else B
                hi, lo = capi.ddgemm_nt(Ab, Bb.t().contiguous())
                Xb = X[b] if batched else X
                errs = max(errs, ((Xb - hi) - lo).abs().max().item())
                scale = max(scale, hi.abs().max().item())
                if batched and b >= 7:
                    break            # 8 members suffice for the correct-bit estimate
            bits[tag] = 53.0 if errs == 0 else round(-math.log2(errs / scale), 2)
        value = flop / (ms * 1e-3) / 1e12
        rec = {"config": name, "kind": kind, "batch": batch, "M": M, "N": N, "K": K,
               "nprimes": P, "corr": corr, "exact": exact, "gemms": G, "ms": round(ms, 4),
               "tflops": round(value, 2),
               "plan_roofline_frac": round(value / (INT8_PEAK_TOPS / G), 4),
               "phases_ms": phases, "native_ms": round(nat_ms, 4),
               "native_tflops": round(flop / (nat_ms * 1e-3) / 1e12, 2),
               "correct_bits_emu": bits["emu"], "correct_bits_native": bits["native"]}
        if emit:
            print(json.dumps(rec), flush=True)
        records.append(rec)
        del A, B, Ce, Cn
        torch.cuda.empty_cache()
    return records


def _host_cores():
    """The cores this process may use: its CPU affinity, capped at the 16
    cores a one-GPU box of this pool allots to a GPU (OMP_NUM_THREADS there)."""
    try:
        cores = len(os.sched_getaffinity(0))
    except Exception:
        cores = os.cpu_count() or 1
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return max(1, min(cores, cap) if cap > 0 else cores)


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def pin_rocblas():
    """Route torch's device GEMMs through rocBLAS (torch's "cublas" backend on
    ROCm) rather than hipBLASLt, for the native comparator."""
    import torch
    try:
        torch.backends.cuda.preferred_blas_library("cublas")
    except Exception as e:   # older torch: the environment variable set above
        log(f"preferred_blas_library unavailable: {e}")


def native_blas():
    """Which library serves the native float64 comparator on the device."""
    import torch
    try:
        pref = str(torch.backends.cuda.preferred_blas_library())
    except Exception:
        pref = "unknown"
    return {"library": "rocBLAS (torch.matmul float64)", "torch_preferred_blas": pref,
            "TORCH_BLAS_PREFER_HIPBLASLT": os.environ.get("TORCH_BLAS_PREFER_HIPBLASLT")}


def cpu_torch_baseline(A, Bt):
    """torch float64 matmul of the same workload on the host's cores (the
    comparison the reference's benchmarks quote beside native DGEMM): one
    warm-up, then the median of three full products."""
    import re
    import statistics
    import torch
    cores = _host_cores()
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    a, bt = A.cpu(), Bt.cpu()
    torch.matmul(a, bt)                               # warm-up
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        torch.matmul(a, bt)
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    used = torch.get_num_threads()
    torch.set_num_threads(prev)
    cfg = torch.__config__.show()
    blas = re.search(r"BLAS_INFO=([^,\n]+)", cfg)
    n = a.shape[0]
    val = 2.0 * n * bt.shape[1] * a.shape[1] / t / 1e12
    log(f"cpu torch float64 matmul ({used} threads, {_cpu_model()}): median {t:.2f} s, "
        f"{val:.4f} TFLOP/s")
    return {"value": round(val, 5), "unit": "TFLOP/s", "cores": used, "seconds": round(t, 3),
            "runs_s": [round(x, 3) for x in ts], "cpu_model": _cpu_model(),
            "affinity_cores": len(os.sched_getaffinity(0)),
            "blas": blas.group(1).strip() if blas else "unknown",
            "sample": "the full workload, torch.matmul float64 on host tensors; median of 3 "
                      "after 1 warm-up"}


def cpu_baseline(A, Bt, P, corr):
    """The oracle port (the reference pipeline restated in C) on the host's
    cores, on a bounded sample of the workload: the first 4096 rows of A and
    columns of Bt at the full depth K, same plan (about 10 s on 16 cores).
    Effective FP64 TFLOPS of that sample (2 * 4096 * 4096 * K / t)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    cores = _host_cores()
    m = 4096
    a = A[:m].cpu().numpy()
    bt = Bt[:, :m].contiguous().cpu().numpy()
    K = a.shape[1]
    t0 = time.perf_counter()
    O.mm(a, bt, 1, O.PRIMES[:P], use_corr=corr, nthreads=cores)
    t = time.perf_counter() - t0
    val = 2.0 * m * m * K / t / 1e12
    log(f"cpu baseline (oracle port, {cores} threads): {t:.2f} s, {val:.4f} TFLOP/s")
    return {"value": round(val, 5), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"mm_nt {m}x{m}x{K} (rows/cols 0..{m - 1} of the workload, full depth), "
                      f"same plan, oracle/fp64emu_oracle.c with OpenMP",
            "seconds": round(t, 3)}


if __name__ == "__main__":
    main()
