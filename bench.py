#!/usr/bin/env python3
"""Benchmark of the KERNIX forward hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--no-cpu] [--no-forward] [--no-small]

Headline (`value`): int8 GEMM Y = relu(((float)(A·Wᵀ)·sa[m])·sw[n] + bias[n]) at M = K = N = 4096 with int32
accumulation, inputs resident in HBM, through the C ABI (knx_hip_i8gemm), in TOPS (1 MAC = 2 ops), sustained: W
untimed warm-up launches and at least 200 ms more of back-to-back launches (past the first milliseconds, in which
the clocks are still above their loaded level), then exactly K launches back to back, bracketed by device
synchronizations and timed by HIP events on the launch stream.  Windows of 50 launches after them give the median
and spread, and the burst figure (K launches right after the W warm-up launches, no further warm-up) is reported
beside it.  `roofline` relates the
sustained figure to the int8 MFMA peak and carries the HBM traffic per launch measured with rocprofv3 counters
(read from profiles/i8gemm_4096_traffic.json).
Also reported: the GEMM at M ∈ {1, 16, 256} (HBM-bound), with the same operands every launch (the last-level cache
then holds the weights) and rotating over enough operand copies (> 256 MB) that every launch reads them from HBM; the
bandwidth-bound row kernels the same two ways; the convolution layers and the attention core; the .knx forward
samples/sec of the int8 MLP, fp32 MLP, CNN and int8-weight Transformer workloads (device-resident and end to end
through kernix_capi_forward), each beside the reference's CPU path (oracle/cpu_forward.py: the plain-C kernels of
the oracle) timed on this machine's host cores on a sample of the same batch; and the CPU oracle's int8 GEMM.
Each of these lines is timed after 100 ms of untimed launches of its own (the clock ramps up over the first tens of
milliseconds of work after an idle spell; --warm-ms sets it, and profiling runs with --no-sustained skip it unless
--warm-ms is given).  A forward line's `forwards` counts the device and host-buffer forwards the run made.
One JSON line is printed on stdout.
"""
import argparse
import ctypes
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_I8_TOPS = 5000.0      # MI355X dense int8 MFMA
PEAK_F32_TFLOPS = 157.3    # MI355X fp32 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
WARM_MS = 100.0            # untimed launches before each line beside the headline (clock ramp)
METRIC = "int8 GEMM TOPS + .knx forward samples/sec on 1 MI355X, % of roofline"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_launches(fn, steps, warmup, warm_ms=0.0):
    """(ms per launch, wall ms per launch): `steps` launches back to back between two HIP events on torch's current
    stream, which is the stream the launches go to.  An event pair around every single launch would add a
    system-scope cache flush per launch (≈10 µs for a 64 MB output) that a kernel-trace profile does not see.
    warm_ms > 0: after the `warmup` launches, more untimed launches until that much time has passed (the GPU's clock
    ramps up over the first tens of milliseconds of work after an idle spell: the CNN forward's convolutions ran 12%
    slower in its first 45 forwards than in the next)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < warm_ms:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return start.elapsed_time(end) / steps, wall


def time_sustained(fn, steps, warm_ms=200.0, windows=20, per_window=50):
    """After at least warm_ms of back-to-back launches (untimed, past the clock ramp of the first milliseconds):
    exactly `steps` launches timed between two HIP events on torch's current stream with a device synchronization
    on both sides (ms per launch), then `windows` windows of `per_window` back-to-back launches each bracketed by
    events (median, p10, p90 ms per launch)."""
    import statistics

    import torch

    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < warm_ms:
        for _ in range(per_window):
            fn()
        torch.cuda.synchronize()
    ms, _ = time_launches(fn, steps, 0)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(windows + 1)]
    ev[0].record()
    for w in range(windows):
        for _ in range(per_window):
            fn()
        ev[w + 1].record()
    torch.cuda.synchronize()
    per = sorted(ev[w].elapsed_time(ev[w + 1]) / per_window for w in range(windows))
    return ms, statistics.median(per), per[len(per) // 10], per[(9 * len(per)) // 10]


def i8gemm_bench(M, steps, warmup, N=4096, K=4096, sustained=True, rotate_bytes=0, warm_ms=0.0):
    """The int8 GEMM at M×N×K.  rotate_bytes > 0: launches cycle over copies of A and W (and of the output) that
    together exceed rotate_bytes, so no launch finds its operands in the 256 MB last-level cache."""
    import numpy as np
    import torch

    from kernix_amd import configs, hipabi

    L = hipabi.lib()
    hipabi.check(L.knx_hip_init())
    A, W, sa, sw, bias = configs.i8gemm_inputs(M, N, K)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    dsa, dsw, db = dev(sa), dev(sw), dev(bias)
    P = hipabi.ptr
    per_copy = M * K + N * K + 4 * M * N
    copies = max(1, -(-rotate_bytes // per_copy)) if rotate_bytes else 1
    dA, dW = dev(A), dev(W)
    sets = [(dA, dW, torch.empty((M, N), dtype=torch.float32, device="cuda"))]
    for _ in range(copies - 1):
        sets.append((dA.clone(), dW.clone(), torch.empty((M, N), dtype=torch.float32, device="cuda")))
    args = [(M, N, K, P(a), K, P(dsa), P(w), K, P(dsw), P(db), 0, 0.0, 0, P(y), N, None, 0, hipabi.stream())
            for a, w, y in sets]
    turn = [0]

    def run():
        hipabi.check(L.knx_hip_i8gemm(*args[turn[0]]))
        turn[0] = (turn[0] + 1) % len(args)

    ms, wall = time_launches(run, steps, warmup, warm_ms)
    sus = time_sustained(run, steps) if sustained else (ms, ms, ms, ms)
    ops, algo_bytes = configs.i8gemm_work(M, N, K)
    return dict(M=M, N=N, K=K, ms=sus[0], ms_median=sus[1], ms_p10=sus[2], ms_p90=sus[3], burst_ms=ms, wall_ms=wall,
                tops=ops / (sus[0] * 1e-3) / 1e12, burst_tops=ops / (ms * 1e-3) / 1e12,
                gbs=algo_bytes / (sus[0] * 1e-3) / 1e9, algo_bytes=algo_bytes, ops=ops, copies=copies,
                A=A, W=W, sa=sa, sw=sw, bias=bias, Y=sets[0][2])


def cpu_baseline(g, threads, target_s=10.0):
    """Oracle int8 GEMM (plain C, the reference's scalar int8 arithmetic) on rows of the same workload."""
    import numpy as np

    from oracle import knx_ref

    A, W, sa, sw, bias = g["A"], g["W"], g["sa"], g["sw"], g["bias"]
    N, K = W.shape
    rows = min(64, A.shape[0])
    t0 = time.perf_counter()
    knx_ref.i8gemm(A[:rows], W, sa[:rows], sw, bias, act_id=0, threads=threads)
    dt = time.perf_counter() - t0
    rate = rows / max(dt, 1e-6)                      # rows per second
    rows = int(min(A.shape[0], max(rows, rate * target_s)))
    reps, total, y = 0, 0.0, None
    while reps == 0 or (total < target_s * 0.5 and reps < 5):
        t0 = time.perf_counter()
        y, _ = knx_ref.i8gemm(A[:rows], W, sa[:rows], sw, bias, act_id=0, threads=threads)
        total += time.perf_counter() - t0
        reps += 1
    sec = total / reps
    ops = 2.0 * rows * N * K
    got = g["Y"][:rows].cpu().numpy()
    return dict(tops=ops / sec / 1e12, seconds=sec, rows=rows, reps=reps, bit_exact=bool(np.array_equal(got, y)))


ROTATE_BYTES = 320 << 20  # more than the 256 MB last-level cache: a rotating working set comes from HBM


def rows_bench(steps, warmup, warm_ms=0.0):
    """The bandwidth-bound kernels at the Transformer / CNN workload shapes: algorithmic bytes (every fp32 input read
    once, every output written once) per launch ÷ time, against HBM peak.  Two figures each: `cached`, the same
    buffers every launch (16-134 MB working sets stay in the 256 MB last-level cache, so this can exceed what HBM
    delivers; it is what a forward sees when a step's input was just written), and `hbm`, launches rotating over
    copies whose total exceeds the cache, so every byte comes from HBM."""
    import torch

    from kernix_amd import hipabi

    L = hipabi.lib()
    hipabi.check(L.knx_hip_init())
    P, S = hipabi.ptr, hipabi.stream()
    rnd = lambda *shape: torch.randn(*shape, device="cuda", dtype=torch.float32)  # noqa: E731
    out = {}

    def run(name, make, call, nbytes):
        """make(): one set of buffers; call(set): the launch on it"""
        copies = max(2, -(-ROTATE_BYTES // nbytes))
        sets = [make() for _ in range(copies)]
        res = {"bytes": int(nbytes)}
        for mode in ("cached", "hbm"):
            turn = [0]

            def one():
                hipabi.check(call(sets[turn[0]]))
                if mode == "hbm":
                    turn[0] = (turn[0] + 1) % copies

            ms, _ = time_launches(one, steps, warmup, warm_ms)
            gbs = nbytes / (ms * 1e-3) / 1e9
            res[mode] = dict(us=round(ms * 1e3, 2), gbs=round(gbs, 1), hbm_frac=round(gbs / PEAK_HBM_GBS, 4))
        res["rotating_copies"] = copies
        out[name] = res
        log(f"{name}: cached {res['cached']['us']} us {res['cached']['gbs']:.0f} GB/s, "
            f"from HBM {res['hbm']['us']} us {res['hbm']['gbs']:.0f} GB/s")
        del sets
        torch.cuda.empty_cache()

    g, b = rnd(512), rnd(512)
    run("layernorm_8192x512", lambda: (rnd(8192, 512), torch.empty(8192, 512, device="cuda")),
        lambda t: L.knx_hip_layernorm(P(t[0]), P(t[1]), 8192, 512, P(g), P(b), 1e-5, S), 2 * 8192 * 512 * 4 + 2 * 512 * 4)
    run("softmax_65536x128_inplace", lambda: (rnd(65536, 128),),
        lambda t: L.knx_hip_softmax(P(t[0]), P(t[0]), 65536, 128, S), 2 * 65536 * 128 * 4)
    hb = rnd(2048)
    run("bias_gelu_8192x2048_inplace", lambda: (rnd(8192, 2048),),
        lambda t: L.knx_hip_bias_act(P(t[0]), P(t[0]), 8192, 2048, P(hb), 1, 0.0, S), 2 * 8192 * 2048 * 4 + 2048 * 4)
    run("binary_add_8192x512", lambda: (rnd(8192, 512), rnd(8192, 512), torch.empty(8192, 512, device="cuda")),
        lambda t: L.knx_hip_binary(0, P(t[0]), 512, 512, P(t[1]), 512, 512, P(t[2]), 16, 512, 512, S),
        3 * 8192 * 512 * 4)
    run("global_avg_pool_256x64x256", lambda: (rnd(256 * 64, 256), torch.empty(256, 256, device="cuda")),
        lambda t: L.knx_hip_global_pool(1, P(t[0]), 256, 64, 256, P(t[1]), S), 256 * 64 * 256 * 4 + 256 * 256 * 4)
    run("quantize_rows_8192x2048",
        lambda: (rnd(8192, 2048), torch.empty(8192, 2048, dtype=torch.int8, device="cuda"), torch.empty(8192, device="cuda")),
        lambda t: L.knx_hip_quantize_rows(P(t[0]), 2048, 8192, 2048, 2048, P(t[1]), 2048, P(t[2]), S),
        8192 * 2048 * 5 + 8192 * 4)
    return out


def conv_bench(steps, warmup, warm_ms=0.0):
    """The four convolutions of the CNN configuration (batch 256, NHWC, 3×3, pad 1, bias + ReLU fused) through
    knx_hip_conv_t: algorithmic flops 2·B·Ho·Wo·Co·9·Cin per launch against the fp32 MFMA peak, and the minimum HBM
    bytes (input + weights + output once)."""
    import torch

    from kernix_amd import hipabi

    L = hipabi.lib()
    hipabi.check(L.knx_hip_init())
    P, S = hipabi.ptr, hipabi.stream()
    out = {}
    for name, (h, cin, cout, st) in {"c1_3to64_s1": (32, 3, 64, 1), "c2_64to64_s1": (32, 64, 64, 1),
                                     "c3_64to128_s2": (32, 64, 128, 2), "c4_128to256_s2": (16, 128, 256, 2)}.items():
        ho = (h + 2 - 3) // st + 1
        g = hipabi.ConvGeom(256, h, h, cin, ho, ho, cout, 3, 3, st, st, 1, 1, 1, 1, 1)
        x = torch.randn(256, h, h, cin, device="cuda")
        wt = torch.randn(cout, 9 * cin, device="cuda") * (2.0 / (9 * cin)) ** 0.5  # Co × K, the model's device layout
        b = torch.randn(cout, device="cuda") * 0.01
        y = torch.empty(256, ho, ho, cout, device="cuda")
        ms, _ = time_launches(lambda: hipabi.check(L.knx_hip_conv_t(ctypes.byref(g), P(x), P(wt), P(b), 0, 0.0, P(y), S)),
                              steps, warmup, warm_ms)
        flops = 2.0 * 256 * ho * ho * cout * 9 * cin
        nbytes = 4 * (x.numel() + wt.numel() + cout + y.numel())
        tf = flops / (ms * 1e-3) / 1e12
        out[name] = dict(us=round(ms * 1e3, 2), tflops=round(tf, 2), mfma_frac=round(tf / PEAK_F32_TFLOPS, 4),
                         gbs=round(nbytes / (ms * 1e-3) / 1e9, 1))
        log(f"conv {name}: {ms * 1e3:.1f} us  {tf:.1f} TFLOP/s  {nbytes / (ms * 1e-3) / 1e9:.0f} GB/s")
    return out


def attention_bench(steps, warmup, warm_ms=0.0):
    """The attention core of the Transformer configuration (batch 64, 8 heads, 128 queries and keys, dk = dv = 64):
    algorithmic flops 2·B·H·Rq·S·(dk + dv) per launch against the fp32 MFMA peak, and the minimum HBM bytes (Q, K,
    V read once, the context written once), for the fused kernel and for the three-launch path it replaces."""
    import torch

    from kernix_amd import hipabi

    L = hipabi.lib()
    hipabi.check(L.knx_hip_init())
    P, S = hipabi.ptr, hipabi.stream()
    B, H, T, d = 64, 8, 128, 64
    q, k, v = (torch.randn(B * T, H * d, device="cuda") for _ in range(3))
    ctx = torch.empty(B * T, H * d, device="cuda")
    sc = torch.empty(B * H * T, T, device="cuda")
    vt = torch.empty(H * d, B * T, device="cuda")
    flops = 2.0 * B * H * T * T * (2 * d)
    nbytes = 4 * 4 * B * T * H * d
    out = {}
    for name, env in (("fused", None), ("unfused", "unfused")):
        if env:
            os.environ["KNX_ATTN_KERNEL"] = env
        try:
            ms, _ = time_launches(lambda: hipabi.check(L.knx_hip_attention_core_ex(
                P(q), H * d, P(k), H * d, P(v), H * d, P(vt), P(ctx), P(sc), B, H, T, T, d, d, 0.125, 0, S)), steps,
                warmup, warm_ms)
        finally:
            os.environ.pop("KNX_ATTN_KERNEL", None)
        tf = flops / (ms * 1e-3) / 1e12
        out[name] = dict(us=round(ms * 1e3, 2), tflops=round(tf, 2), mfma_frac=round(tf / PEAK_F32_TFLOPS, 4),
                         gbs=round(nbytes / (ms * 1e-3) / 1e9, 1))
        log(f"attention b64 h8 s128 d64 {name}: {ms * 1e3:.1f} us  {tf:.1f} TFLOP/s")
    return out


def measured_traffic():
    """HBM bytes per launch of the M=N=K=4096 GEMM from the committed rocprofv3 counter summary (FETCH_SIZE and
    WRITE_SIZE per dispatch, each scaled by the same counter on a kernel of known traffic), or None without it."""
    path = os.path.join(ROOT, "profiles", "i8gemm_4096_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)["traffic_bytes"]
    except (OSError, ValueError, KeyError):
        return None


def cpu_model_name():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_forward_baseline(path, xr, seq_len, threads, target_s):
    """The reference's CPU forward path (oracle/cpu_forward.py, plain C) on `threads` host threads, on the first
    samples of the same batch: samples/s, timed over about target_s seconds (at least one sample, whole forwards)."""
    from oracle import knx_ref
    from oracle.cpu_forward import CpuModel

    cm = CpuModel(knx_ref.parse(path))
    B = xr.shape[0] // seq_len
    n = 1
    t0 = time.perf_counter()
    cm.forward(xr[: n * seq_len], threads)
    per = max(time.perf_counter() - t0, 1e-6)
    n = int(min(B, max(1, target_s / per)))
    if n > 1:  # the batch the reference would run at once, within the time budget
        t0 = time.perf_counter()
        cm.forward(xr[: n * seq_len], threads)
        per = (time.perf_counter() - t0) / n
    reps = int(min(2000, target_s / 2 / max(per * n, 1e-6)))
    if n == B and reps > 1:  # a whole small batch: forwards repeated for a stable figure
        t0 = time.perf_counter()
        for _ in range(reps):
            cm.forward(xr[: n * seq_len], threads)
        per = (time.perf_counter() - t0) / (reps * n)
        return dict(value=round(1.0 / per, 1), unit="samples/s", cores=threads, kind="port",
                    sample=f"the {B} samples, mean of {reps} forwards")
    return dict(value=round(1.0 / per, 1), unit="samples/s", cores=threads, kind="port",
                sample=f"first {n} of the {B} samples, one forward")


def forward_bench(name, make, flops, steps, warmup, mode="ref", i8_ops=0.0, cpu=None, warm_ms=0.0):
    """`flops` of one forward, `i8_ops` of them on the int8 MFMA (`i8` mode): the roofline time is the fp32 part at
    the fp32 MFMA peak plus the int8 part at the int8 peak, and roofline_frac that time over the measured one.
    cpu: None, or (list of thread counts, seconds per measurement) for the CPU baseline of the same workload."""
    import numpy as np
    import torch

    from kernix_amd.kernix import INT8_I8, Model

    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, name + ".knx")
        x = make(path)
        m = Model(path, workspace_mb=0)
        if mode == "i8":
            m.set_int8_mode(INT8_I8)
        xr = x
        if m.channels_first and x.ndim >= 3:
            xr = np.moveaxis(x, 1, -1)
        xr = np.ascontiguousarray(xr, np.float32).reshape(-1, m.in_dim)
        B = xr.shape[0] // m.seq_len
        dx = torch.from_numpy(xr).cuda()
        dy = torch.empty((B, m.out_dim), dtype=torch.float32, device="cuda")
        # a dedicated stream: the library runs the forward on the handle it is given (NULL would mean the model's
        # own stream), and the timing events are recorded on the same one
        stream = torch.cuda.Stream()
        st = stream.cuda_stream

        # end to end through kernix_capi_forward (host buffers, PCIe included), before the device forwards (so that
        # the timed device forwards end the run of identical launch sequences in a kernel trace): untimed calls for
        # 50 ms (at least one), then calls back to back for at least 0.2 s (at least 2) — a handful of calls after an
        # idle spell times the clock ramp, not the path
        n_host = 0
        t0 = time.perf_counter()
        while n_host < 1 or time.perf_counter() - t0 < 0.05:
            m(x)
            n_host += 1
        n_e2e = 0
        t0 = time.perf_counter()
        while n_e2e < 2 or time.perf_counter() - t0 < 0.2:
            m(x)
            n_e2e += 1
        e2e = (time.perf_counter() - t0) * 1e3 / n_e2e
        n_host += n_e2e

        n_dev = [0]

        def run():
            m.forward_device(dx.data_ptr(), xr.shape[0], dy.data_ptr(), st)
            n_dev[0] += 1

        with torch.cuda.stream(stream):
            ms, _ = time_launches(run, steps, warmup, warm_ms)
        seq = m.seq_len
        m.close()
        base = {}
        if cpu is not None:
            threads, secs = cpu
            for t in threads:
                base[str(t)] = cpu_forward_baseline(path, xr, seq, t, secs)
    tf = flops / (ms * 1e-3) / 1e12
    ideal_ms = ((flops - i8_ops) / (PEAK_F32_TFLOPS * 1e12) + i8_ops / (PEAK_I8_TOPS * 1e12)) * 1e3
    res = dict(batch=B, ms=round(ms, 4), samples_per_s=round(B / (ms * 1e-3), 1),
               e2e_ms=round(e2e, 3), e2e_samples_per_s=round(B / (e2e * 1e-3), 1),
               tflops=round(tf, 2), roofline_frac=round(ideal_ms / ms, 4), mode=mode,
               forwards={"device": n_dev[0], "host": n_host})
    if base:
        res["cpu_baseline"] = base
    return res


def run_parts(args, out, want, configs):
    """the lines beside the headline: small-M GEMMs, row kernels, convolutions, attention, .knx forwards"""
    ncpu = len(os.sched_getaffinity(0))
    threads = [8] + ([ncpu] if ncpu != 8 else [])
    # profiling runs (--no-sustained) take the launch counts as given; otherwise enough launches for stable figures
    few = args.no_sustained
    n_small = (args.steps, args.warmup) if few else (max(args.steps, 50), max(args.warmup, 20))
    n_layer = (args.steps, args.warmup) if few else (max(args.steps, 20), max(args.warmup, 3))
    warm_ms = args.warm_ms if args.warm_ms is not None else 0.0 if few else WARM_MS
    small = {}
    for M in (() if args.no_small or not want("gemm_small") else (1, 16, 256)):
        entry = {}
        for mode, rot in (("cached", 0), ("hbm", ROTATE_BYTES)):
            r = i8gemm_bench(M, n_small[0], n_small[1], sustained=False, rotate_bytes=rot,
                             warm_ms=warm_ms)
            entry[mode] = dict(us=round(r["burst_ms"] * 1e3, 2), tops=round(r["burst_tops"], 2),
                               gbs=round(r["algo_bytes"] / (r["burst_ms"] * 1e-3) / 1e9, 1),
                               hbm_frac=round(r["algo_bytes"] / (r["burst_ms"] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4))
            log(f"i8gemm M={M} {mode}: {r['burst_ms'] * 1e3:.2f} us  {entry[mode]['gbs']:.0f} GB/s algorithmic")
            if mode == "cached" and not args.no_cpu:  # the oracle's int8 GEMM on the same M rows
                entry["cpu_baseline"] = {}
                for t in threads:
                    c = cpu_baseline(r, t, target_s=1.0)
                    entry["cpu_baseline"][str(t)] = dict(us=round(c["seconds"] * 1e6, 1), tops=round(c["tops"], 4),
                                                         cores=t, kind="port", rows=c["rows"],
                                                         gpu_rows_bit_exact=c["bit_exact"])
                log(f"i8gemm M={M} cpu: " + ", ".join(f"{v['us']:.0f} us on {t}" for t, v in entry["cpu_baseline"].items()))
        entry["bytes"] = int(configs.i8gemm_work(M)[1])
        small[str(M)] = entry

    if small:
        out["i8gemm_small_m"] = small
    if not args.no_small and want("rows"):
        out["row_kernels"] = rows_bench(*n_small, warm_ms)
    if not args.no_small and want("conv"):
        out["conv_layers"] = conv_bench(*n_layer, warm_ms)
    if not args.no_small and want("attention"):
        out["attention_core"] = attention_bench(*n_layer, warm_ms)
    if not args.no_forward and want("forward"):
        fw = {}
        st = max(10, args.steps)
        fwarm = max(3, args.warmup)
        cpu = None if args.no_cpu else (threads, 2.0)
        mlp = (784, 512, 256, 10)
        kw = dict(cpu=cpu, warm_ms=warm_ms)
        lines = {
            "int8_mlp_784_512_256_10_b64": lambda: forward_bench(
                "mlp", lambda p: configs.int8_mlp(p, batch=64), configs.mlp_flops(64, mlp), st, fwarm, **kw),
            # batch 1: the reference's int8 latency path (int8 arithmetic at ≤ 2 rows), quantize fused into the GEMM
            "int8_mlp_784_512_256_10_b1": lambda: forward_bench(
                "mlp", lambda p: configs.int8_mlp(p, batch=1), configs.mlp_flops(1, mlp), st, fwarm,
                i8_ops=configs.mlp_flops(1, mlp), **kw),
            "int8_mlp_784_512_256_10_b64_i8": lambda: forward_bench(
                "mlp", lambda p: configs.int8_mlp(p, batch=64), configs.mlp_flops(64, mlp), st, fwarm, mode="i8",
                i8_ops=configs.mlp_flops(64, mlp), **kw),
            "fp32_mlp_4096_4096_4096_1000_b8192": lambda: forward_bench(
                "f32", lambda p: configs.fp32_mlp(p), configs.mlp_flops(8192, (4096, 4096, 4096, 1000)), st, fwarm,
                **kw),
            "cnn_b256": lambda: forward_bench("cnn", lambda p: configs.cnn(p), configs.cnn_flops(), st, fwarm, **kw),
            "transformer_4l_d512_b64": lambda: forward_bench(
                "tr", lambda p: configs.transformer(p), configs.transformer_flops(), st, fwarm, **kw),
            "transformer_4l_d512_b64_i8": lambda: forward_bench(
                "tr", lambda p: configs.transformer(p), configs.transformer_flops(), st, fwarm, mode="i8",
                i8_ops=configs.transformer_ffn_flops(), **kw),
        }
        # recurrent models (reference kernix_rnn_dir): LSTM over T = 32 steps of 128 features, 128 units, then a
        # dense 10; each timestep's h·U + cell in one launch of the whole sequence, and the same forward with one
        # launch per timestep for the product and another for the cell (KNX_RNN_PERSISTENT=0) beside it
        for bsz in (1, 64):
            for q8, mode in ((False, "ref"), (True, "ref" if bsz <= 2 else "i8")):
                key = f"lstm{'_int8' if q8 else ''}_t32_f128_u128_b{bsz}{'_i8' if mode == 'i8' else ''}"
                fl = configs.lstm_flops(batch=bsz)
                rec_i8 = configs.lstm_flops(batch=bsz, fin=0, classes=0) if q8 and (mode == "i8" or bsz <= 2) else 0.0

                def line(bsz=bsz, q8=q8, mode=mode, fl=fl, rec_i8=rec_i8):
                    mk = lambda p: configs.lstm(p, batch=bsz, int8=q8)  # noqa: E731
                    r = forward_bench("lstm", mk, fl, st, fwarm, mode=mode, i8_ops=rec_i8, **kw)
                    os.environ["KNX_RNN_PERSISTENT"] = "0"
                    try:
                        r0 = forward_bench("lstm", mk, fl, st, fwarm, mode=mode, i8_ops=rec_i8, warm_ms=warm_ms)
                    finally:
                        del os.environ["KNX_RNN_PERSISTENT"]
                    r["per_timestep_launches"] = dict(ms=r0["ms"], samples_per_s=r0["samples_per_s"])
                    return r

                lines[key] = line
        only = {k for k in args.forward_only.split(",") if k}
        for k, run in lines.items():
            if not only or k in only:
                fw[k] = run()
        for k, v in fw.items():
            cpu_txt = ""
            if "cpu_baseline" in v:
                cpu_txt = "  cpu " + ", ".join(f"{c['value']:.0f}/s on {t}" for t, c in v["cpu_baseline"].items())
            log(f"forward {k}: {v['ms']:.3f} ms  {v['samples_per_s']:.0f} samples/s  {v['tflops']:.1f} TFLOP/s{cpu_txt}")
        out["forward"] = fw
        if not args.no_cpu:
            out["forward_cpu"] = {"cpu": cpu_model_name(), "threads": threads,
                                  "path": "oracle/cpu_forward.py: fp32 native GEMM, im2col convolution, row ops, "
                                          "int8 kernel at <= 2 rows (the reference's CPU dispatch), plain C; the i8 "
                                          "lines' baseline is that dispatch for the same model (the reference has no "
                                          "int8-at-every-row mode)"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-forward", action="store_true")
    ap.add_argument("--no-small", action="store_true", help="skip the small-M GEMM, row, convolution, attention lines")
    ap.add_argument("--only", default="",
                    help="comma-separated subset for profiling runs: gemm4096, gemm_small, rows, conv, attention, "
                         "forward (the JSON line then lacks the parts not run)")
    ap.add_argument("--forward-only", default="",
                    help="comma-separated subset of the .knx forward lines (their keys, e.g. cnn_b256), for profiling runs")
    ap.add_argument("--no-sustained", action="store_true",
                    help="time the headline GEMM only in the burst form (profiling runs with few launches)")
    ap.add_argument("--warm-ms", type=float, default=None,
                    help="untimed launches (ms) before each line beside the headline; default 100, 0 with "
                         "--no-sustained")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run a 256 MiB read (sum) and a 256 MiB copy: reference kernels of known HBM traffic for "
                         "scaling the FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: multi-GPU runs are not part of this build "
              "(the forward shards by rows with no exchange; see the design notes)", file=sys.stderr)
        sys.exit(2)

    import torch

    from kernix_amd import configs

    assert torch.cuda.is_available(), "bench.py needs the MI355X"
    log(f"device: {torch.cuda.get_device_name(0)}")
    only = set(filter(None, args.only.split(",")))
    want = lambda part: not only or part in only  # noqa: E731
    if only and "gemm4096" not in only:
        args.no_cpu = True
    if args.calibrate:  # kernels of known traffic, in the same process as the kernels profiled
        n = 256 << 20
        src = torch.ones(n // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            src.sum()
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration: {n} byte read (sum) and {n} byte copy issued 3 times")
    g = i8gemm_bench(4096, args.steps, args.warmup, sustained=not args.no_sustained) if want("gemm4096") else None
    if g is None:
        out = {"metric": METRIC, "only": sorted(only)}
        run_parts(args, out, want, configs)
        print(json.dumps(out), flush=True)
        return
    log(f"i8gemm M=4096: sustained {g['ms'] * 1e3:.1f} us ({g['tops']:.1f} TOPS; windows median "
        f"{g['ms_median'] * 1e3:.1f}, p10-p90 {g['ms_p10'] * 1e3:.1f}-{g['ms_p90'] * 1e3:.1f} us), burst "
        f"{g['burst_ms'] * 1e3:.1f} us "
        f"({g['burst_tops']:.1f} TOPS)")
    out = {
        "metric": METRIC,
        "value": round(g["tops"], 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "int8 GEMM relu(((float)(A_i8·W_i8^T)·sa[m])·sw[n] + bias[n]), int32 accumulate",
                   "M": 4096, "N": 4096, "K": 4096},
        "roofline": {"bound": "mfma", "achieved": round(g["tops"], 2), "peak": PEAK_I8_TOPS, "unit": "TOP/s",
                     "frac": round(g["tops"] / PEAK_I8_TOPS, 4), "traffic": measured_traffic(),
                     "kernel_us": round(g["ms"] * 1e3, 2),
                     "timing": "sustained: the K timed launches follow at least 200 ms of back-to-back launches",
                     "windows_us": {"median": round(g["ms_median"] * 1e3, 2), "p10": round(g["ms_p10"] * 1e3, 2),
                                    "p90": round(g["ms_p90"] * 1e3, 2), "windows": 20, "launches_per_window": 50}},
        "burst": {"steps": args.steps, "warmup": args.warmup, "kernel_us": round(g["burst_ms"] * 1e3, 2),
                  "tops": round(g["burst_tops"], 2), "frac": round(g["burst_tops"] / PEAK_I8_TOPS, 4)},
    }
    ncpu = len(os.sched_getaffinity(0))
    threads = [8] + ([ncpu] if ncpu != 8 else [])
    if not args.no_cpu:
        c8 = cpu_baseline(g, 8)
        out["cpu_baseline"] = {"value": round(c8["tops"], 4), "unit": "TOPS", "cores": 8, "kind": "port",
                               "sample": f"oracle int8 GEMM (plain C, -O3), rows 0..{c8['rows'] - 1} of the "
                                         f"M=4096 workload ({c8['rows']}x4096x4096), mean of {c8['reps']}",
                               "gpu_rows_bit_exact": c8["bit_exact"], "cpu": cpu_model_name()}
        log(f"cpu 8 threads: {c8['tops'] * 1e3:.1f} GOPS, GPU rows bit-exact: {c8['bit_exact']}")
        if ncpu != 8:
            cn = cpu_baseline(g, ncpu, target_s=5.0)
            out["cpu_baseline_all_cores"] = {"value": round(cn["tops"], 4), "unit": "TOPS", "cores": ncpu}
    run_parts(args, out, want, configs)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
