"""Benchmark of the int8 quantised-matmul hot path on one MI355X.

Metric: int8 GEMM TOPS + GEMV HBM GB/s (% of MI355X roofline), 1 GPU.

One step = one pass of the reference operator try_int8_gemm (per-row int8
quantisation of the f16 activations + W8A8 int8-MFMA GEMM with the fused
epilogue, f32 out) over the north_star GEMM "4096x3072x12288" in both
orientations: M=4096,K=3072,N=12288 and M=4096,K=12288,N=3072. ``value`` is
int8 TOPS = 2*M*N*K / time over the timed steps, inputs resident in HBM.

The weight-only GEMV (M=1, K=4096, N=14336, fp16 scales) is reported beside
it under "gemv", in HBM GB/s, over a rotation of weight copies larger than the
256 MB Infinity Cache so that no launch re-reads its weights from that cache.

Launches are captured into HIP graphs and replayed, bracketed by HIP events
on the stream the kernels run on, so host launch overhead is not timed.
"roofline" describes the dominant kernel (the W8A8 GEMM), timed alone; "cpu_baseline" times the CPU
oracle (a C restatement of the reference's int8_host::gemm, single thread)
on a bounded sample of the same workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "omni-rs_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

PEAK_INT8_TOPS = 5000.0     # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E, 8 TB/s
PEAK_F16_TFLOPS = 2500.0    # MI355X dense fp16 MFMA, 2.5 PFLOP/s
GEMM_SHAPES = [(4096, 3072, 12288), (4096, 12288, 3072)]  # (M, K, N)
GEMV_SHAPE = (1, 4096, 14336)
GEMV_ROTATION_BYTES = 1 << 30


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="bounded CPU-baseline sample length")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a 256 MiB device copy (three times): the known-size kernel "
                        "that scales rocprofv3's FETCH_SIZE / WRITE_SIZE readings")
    p.add_argument("--configs-only", action="store_true",
                   help="only time every BASELINE.json config (one JSON line)")
    p.add_argument("--phase-timeline", action="store_true",
                   help="only record the W8A8 ring kernel's per-workgroup tile phases on the two "
                        "north-star GEMMs (needs the timeline build: make -C omni-rs_amd timeline)")
    return p.parse_args()


def copy_calibration():
    import torch
    x = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": x.numel(), "copies": 3}))


def phase_timeline(runs=24):
    """Tile phases of the W8A8 ring kernel on the two north-star GEMMs
    (try_int8_gemm, f32 out, operands rotated past the MALL as in the timed
    bench), from the library built with OMNI_PHASE_TIMELINE: per unit (the
    workgroup's 1st, 2nd, ... tile), medians over the workgroups of the K
    loop's start (us from the first workgroup's start), its length and mean
    shader clock, the next unit's copy issue, the epilogue, and the spread of
    the epilogue's end (min / median / max), from the run of median length
    among `runs` eager calls. One JSON line per shape."""
    import ctypes
    import numpy as np
    here = os.path.dirname(os.path.abspath(__file__))
    lib_path = os.path.join(here, "omni-rs_amd", "_timeline", "libomni_int8.so")
    if not os.path.exists(lib_path):
        raise SystemExit("no timeline build: run make -C omni-rs_amd timeline")
    os.environ["OMNI_INT8_LIBRARY"] = lib_path
    import torch
    import omni_int8 as oi
    lib = ctypes.CDLL(lib_path)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    for M, K, N in GEMM_SHAPES:
        copies = max(4, -(-GEMV_ROTATION_BYTES // (2 * M * K + N * K + M * K)))
        xs = [torch.randn((M, K), generator=gen, device=dev).half() for _ in range(copies)]
        ws = [torch.randint(-127, 128, (N, K), generator=gen, device=dev, dtype=torch.int8)
              for _ in range(copies)]
        scale = torch.rand(N, generator=gen, device=dev) * 0.018 + 0.002
        zero = torch.zeros(N, dtype=torch.int32, device=dev)
        taken = []
        for it in range(copies + runs):
            k = it % copies
            assert lib.omni_phase_timeline_clear() == 0
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            oi.try_int8_gemm(xs[k], ws[k].view(torch.int32).reshape(-1), scale, zero)
            e1.record()
            torch.cuda.synchronize()
            if it >= copies:
                buf = np.zeros(1024 * 64, dtype=np.uint64)
                assert lib.omni_phase_timeline_read(buf.ctypes.data_as(ctypes.c_void_p),
                                                    ctypes.c_size_t(buf.nbytes)) == 0
                taken.append((e0.elapsed_time(e1) * 1e3, buf.reshape(1024, 64).astype(np.int64)))
        taken.sort(key=lambda r: r[0])
        op_us, ts = taken[len(taken) // 2]
        wg = np.nonzero(ts[:, 62] > 0)[0]       # workgroups that ran (index = blockIdx)
        ts = ts[wg]
        t0 = ts[:, 62].min()
        units = []
        for r in range(8):
            done = ts[:, 8 * r + 3] > 0
            if not done.any():
                break
            t = ts[done]
            ks, ke, es, ee = ((t[:, 8 * r + c] - t0) / 100.0 for c in range(4))
            mhz = (t[:, 8 * r + 5] - t[:, 8 * r + 4]) / np.maximum(ke - ks, 1e-3)
            units.append({"unit": r, "workgroups": int(done.sum()),
                          "k_start_us": round(float(np.median(ks)), 2),
                          "k_loop_us": round(float(np.median(ke - ks)), 2),
                          "k_loop_mhz": round(float(np.median(mhz))),
                          "next_copies_us": round(float(np.median(es - ke)), 2),
                          "epilogue_us": round(float(np.median(ee - es)), 2),
                          "epilogue_end_us": [round(float(np.min(ee)), 2), round(float(np.median(ee)), 2),
                                              round(float(np.max(ee)), 2)]})
        # Each workgroup's last epilogue end, median over the workgroups of
        # each XCD (dispatch places workgroup b on XCD b % 8).
        last = np.max(np.where(ts[:, [8 * r + 3 for r in range(8)]] > 0,
                               ts[:, [8 * r + 3 for r in range(8)]], 0), axis=1)
        xcd_end = [round(float(np.median((last[wg % 8 == x] - t0) / 100.0)), 2) if (wg % 8 == x).any() else None
                   for x in range(8)]
        print(json.dumps({"phase_timeline": {"M": M, "K": K, "N": N, "op_us": round(op_us, 1),
                                             "kernel_span_us": units[-1]["epilogue_end_us"][2] if units else None,
                                             "xcd_end_median_us": xcd_end, "units": units}}), flush=True)
        del xs, ws


PROFILE_MARKS = []


def mark(torch, key):
    """Launch a one-thread spin kernel (torch.cuda._sleep) on the current
    stream and record `key`. In a rocprofv3 trace of this command the marker
    sits between the dispatches of consecutive bench rows, and the bench line
    lists the keys in launch order (profile_markers), so the trace splits into
    one segment per row (rows whose kernels share a name and grid size stay
    apart). Always outside the timed regions."""
    PROFILE_MARKS.append(key)
    torch.cuda._sleep(1)


def graph_of(fn, iters):
    """Capture `iters` calls of fn into one HIP graph, so the timed region
    measures the GPU, not Python's launch rate. The library's launches go to
    torch's current stream, which is the capture stream here."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # first call outside capture (one-time attribute set-up)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(iters):
            fn()
    torch.cuda.synchronize()
    return g


def timed_graph(g, stream):
    """Seconds for one replay, bracketed by HIP events on `stream`, after one
    untimed replay (a graph's first replay runs measurably slower)."""
    import torch
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    g.replay()
    torch.cuda.synchronize()
    start.record(stream)
    g.replay()
    stop.record(stream)
    stop.synchronize()
    return start.elapsed_time(stop) / 1e3


def load_traffic():
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE and
    WRITE_SIZE, scaled by a copy-kernel calibration); null if not measured."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f)


def row_traffic(key):
    """Measured HBM bytes per launch of one bench row's kernel (None if the
    row was not profiled); profiles/bench_rows_counters.md lists them."""
    return load_traffic().get("rows", {}).get(key, {}).get("traffic_bytes")


def host_cpu():
    """The host this process runs on: logical CPUs, the CPUs this process may
    use, and the CPU model."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"nproc": os.cpu_count(), "usable_cpus": usable, "model": model}


def cpu_baseline(oracle, np, seconds):
    """Reference CPU path (C restatement of int8_host::gemm) on the first rows
    of the north_star GEMM, growing the sample until `seconds`: on one thread
    (the reference is single-threaded) and, for scale, on every CPU this
    process may use (at most 16, the box's share) with the same per-row code
    spread over OpenMP threads."""
    M, K, N = GEMM_SHAPES[0]
    rng = np.random.default_rng(0)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    scale = rng.uniform(0.002, 0.02, N).astype(np.float32)
    zero = np.zeros(N, np.int32)
    rows, elapsed = 0, 0.0
    while elapsed < seconds and rows < M:
        x = rng.standard_normal((2, K)).astype(np.float16).astype(np.float32)
        t0 = time.perf_counter()
        oracle.int8_gemm(x, w, scale, zero)
        elapsed += time.perf_counter() - t0
        rows += 2
    ops = 2.0 * rows * N * K
    host = host_cpu()
    threads = max(1, min(16, host["usable_cpus"]))
    mt_rows, mt_elapsed = 0, 0.0
    while mt_elapsed < seconds / 2 and mt_rows < M:
        x = rng.standard_normal((4 * threads, K)).astype(np.float16).astype(np.float32)
        t0 = time.perf_counter()
        oracle.int8_gemm_threads(x, w, scale, zero, threads)
        mt_elapsed += time.perf_counter() - t0
        mt_rows += x.shape[0]
    mt_ops = 2.0 * mt_rows * N * K
    return {"value": ops / elapsed / 1e12, "unit": "TOPS", "cores": 1, "kind": "port",
            "sample": f"{rows} rows of M={M},K={K},N={N} (f16 x -> int8 codes, int32 acc, "
                      f"f32 epilogue), {elapsed:.1f} s single-thread C restatement of "
                      f"int8_host.rs:19-53",
            "host": host,
            "all_cores": {"value": mt_ops / mt_elapsed / 1e12, "unit": "TOPS", "cores": threads,
                          "kind": "port",
                          "sample": f"{mt_rows} rows of the same GEMM, {mt_elapsed:.1f} s, the same "
                                    f"restatement with rows spread over {threads} OpenMP threads"}}


def cpu_gemv_baseline(oracle, np, seconds):
    """Reference-style CPU weight-only route (dequantise to f16, f32 dot) on
    the GEMV shape, columns sampled until `seconds`."""
    M, K, N = GEMV_SHAPE
    rng = np.random.default_rng(1)
    x = rng.standard_normal((M, K)).astype(np.float16)
    cols, elapsed = 0, 0.0
    while elapsed < seconds and cols < N:
        w = rng.integers(-127, 128, (256, K), dtype=np.int8)
        s = rng.uniform(0.002, 0.02, 256).astype(np.float16)
        t0 = time.perf_counter()
        oracle.w8a16_gemm(x, w, s)
        elapsed += time.perf_counter() - t0
        cols += 256
    return {"value": cols * K / elapsed / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{cols} of {N} output channels at M={M},K={K} (int8 weights streamed), "
                      f"{elapsed:.1f} s single-thread C restatement", "host": host_cpu()}


def step_parity(oracle, np, torch, cases, step_outs, rows_per_shape=6):
    """After timing: the f32 output of the last timed step, per shape, on
    sampled rows (first, last and random ones) against the CPU oracle's
    restatement of the reference CPU path, bit for bit."""
    rng = np.random.default_rng(123)
    res = []
    for c, (k, out) in zip(cases, step_outs):
        M = c["M"]
        idx = np.unique(np.concatenate([[0, M - 1], rng.choice(M, rows_per_shape, replace=False)]))
        it = torch.from_numpy(idx).to(out.device)
        x = c["xs"][k].index_select(0, it).float().cpu().numpy()
        got = out.index_select(0, it).cpu().numpy()
        want = oracle.int8_gemm(x, c["ws"][k].cpu().numpy(), c["scale"].cpu().numpy(),
                                c["zero"].cpu().numpy())
        equal = bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))
        res.append({"M": M, "K": c["K"], "N": c["N"], "rows_checked": int(idx.size),
                    "bit_exact": equal})
        if not equal:
            raise SystemExit(f"bench output differs from the oracle at M={M},K={c['K']},N={c['N']}")
    return res


def reference_shape_context(torch, oi, dev, stream, steps):
    """The reference's own published int8 GEMM shapes (m x n x k = 256 x
    4096 x 4096, 256 x 12288 x 4096, 256 x 4096 x 12288; its matmul2d on an
    Apple M5 Max: 0.171 / 0.943 / 0.595 ms, int32 out), timed through the
    reference operator try_int8_gemm (quantisation of the f16 activations +
    the W8A8 GEMM, f32 out) with the split-K workspace (``us``), with the
    plain workspace (``unsplit_us``: no split) and the GEMM alone on the
    codes (``gemm_us``), on the reference's own deterministic operands
    (scripts/bench_qwen_tensorops_int8.mm:46-47) as f16 activations and int8
    weights, with its sampled int32-dot exactness check (:65-79) on the
    accumulators. Cross-hardware context only: different chips, and this
    operator also quantises and applies the epilogue."""
    from omni_int8 import _lib
    L = _lib.lib()
    res = []
    for m, n, k, m5_ms in ((256, 4096, 4096, 0.171), (256, 12288, 4096, 0.943),
                           (256, 4096, 12288, 0.595)):
        a = ((torch.arange(m * k, device=dev, dtype=torch.int64) * 31 + 11) % 251 - 125)
        b = ((torch.arange(n * k, device=dev, dtype=torch.int64) * 17 + 3) % 241 - 120)
        a = a.to(torch.int8).reshape(m, k)
        b = b.to(torch.int8).reshape(n, k)
        x = a.to(torch.float16)
        wp = b.view(torch.int32).reshape(-1)
        ws = torch.ones(n, device=dev)
        zero = torch.zeros(n, dtype=torch.int32, device=dev)
        out = torch.empty((m, n), dtype=torch.float32, device=dev)
        split_bytes = L.omni_try_int8_gemm_split_workspace_size(m, n, k)
        plain_bytes = L.omni_try_int8_gemm_workspace_size(m, k)
        work = {nb: torch.empty(nb, dtype=torch.uint8, device=dev) for nb in {split_bytes, plain_bytes}}
        codes = oi.quantize_rows(x)

        def op(nbytes):
            st = L.omni_try_int8_gemm(x.data_ptr(), oi.OMNI_F16, m, k, wp.data_ptr(), wp.numel(), ws.data_ptr(),
                                      n, zero.data_ptr(), n, out.data_ptr(), work[nbytes].data_ptr(), nbytes,
                                      torch.cuda.current_stream(dev).cuda_stream)
            assert st == 0, _lib.last_error()

        times = {}
        for name, fn in (("us", lambda: op(split_bytes)), ("unsplit_us", lambda: op(plain_bytes)),
                         ("gemm_us", lambda: oi.w8a8_gemm(codes[0], codes[1], codes[2], b, ws, zero))):
            mark(torch, f"ref_{m}x{n}x{k}_{name}")
            for _ in range(3):
                fn()
            g = graph_of(fn, steps)
            times[name] = timed_graph(g, stream) / steps
            del g
        t = times["us"]
        _, acc = oi.w8a8_gemm(a, torch.ones(m, device=dev), None, b, ws, acc_dump=True)
        torch.cuda.synchronize()
        worst = 0
        for sidx in range(32):
            row = m - 1 if sidx == 31 else (sidx * 997) % m
            col = n - 1 if sidx == 31 else (sidx * 619) % n
            dot = int((a[row].to(torch.int64) * b[col].to(torch.int64)).sum().item())
            worst = max(worst, abs(int(acc[row, col].item()) - dot))
        del acc
        res.append({"m": m, "n": n, "k": k, "us": round(t * 1e6, 2),
                    "TOPS": round(2.0 * m * n * k / t / 1e12, 1),
                    "unsplit_us": round(times["unsplit_us"] * 1e6, 2),
                    "gemm_us": round(times["gemm_us"] * 1e6, 2),
                    "split": bool(split_bytes > plain_bytes),
                    "sampled_dot_max_abs_err": worst,
                    "reference_m5max_matmul2d_ms": m5_ms,
                    "note": "try_int8_gemm incl. quantisation; cross-hardware context "
                            "(Apple M5 Max, int32 out, no epilogue)"})
    return res


# Algorithmic bytes of the decode GEMV rows the read ceiling is measured for
# (M=1; weights + scales + activations + outputs): W8A16 4096 x 4096, W4A16
# 4096 -> 14336 (group 128), W8A16 4096 -> 14336 (the headline GEMV).
READ_CEILING_ROWS = (
    ("w8a16 M=1 4096x4096", 4096 * 4096 + 2 * 4096 + 2 * 4096 + 2 * 4096),
    ("w4a16 M=1 4096x14336", 14336 * 4096 // 2 + 2 * 14336 * 32 + 2 * 4096 + 2 * 14336),
    ("w8a16 M=1 4096x14336", 14336 * 4096 + 2 * 14336 + 2 * 4096 + 2 * 14336),
)


def hbm_read_ceiling(torch, gen, dev, stream, steps):
    """What one launch can stream from HBM at the decode GEMVs' byte counts:
    a bare read of the same number of bytes (libomni_read_ceiling.so: every
    nontemporal 16-byte load of a thread issued before any is used, nothing
    computed or written), over copies rotated past the 256 MB MALL like the
    GEMV rows, at nine launch shapes (1, 2 or 4 loads per thread; 256, 512 or
    1024 threads per block); the fastest shape is the ceiling. Outside every
    timed step."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "omni-rs_amd", "libomni_read_ceiling.so"))
    lib.omni_read_ceiling.restype = ctypes.c_int
    lib.omni_read_ceiling.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_uint32,
                                      ctypes.c_void_p, ctypes.c_void_p]
    shapes = [(u, t) for u in (1, 2, 4) for t in (256, 512, 1024)]
    assert lib.omni_read_ceiling_shapes() == len(shapes)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    rows = []
    for label, nbytes in READ_CEILING_ROWS:
        padded = -(-nbytes // 16) * 16
        copies = max(4, -(-GEMV_ROTATION_BYTES // padded))
        bufs = [torch.randint(-128, 128, (padded,), generator=gen, device=dev, dtype=torch.int8)
                for _ in range(copies)]
        times = []
        for shape in range(len(shapes)):
            idx = [0]

            def one(shape=shape):
                b = bufs[idx[0] % copies]
                idx[0] += 1
                st = lib.omni_read_ceiling(b.data_ptr(), padded, shape, 0x9E3779B9, sink.data_ptr(),
                                           torch.cuda.current_stream(dev).cuda_stream)
                assert st == 0, st

            for _ in range(copies):
                one()
            iters = copies * max(1, steps // 8)
            g = graph_of(one, iters)
            times.append(timed_graph(g, stream) / iters)
            del g
        del bufs
        best = min(range(len(shapes)), key=lambda i: times[i])
        t = times[best]
        rows.append({"row": label, "bytes": nbytes, "copies": copies, "us": round(t * 1e6, 3),
                     "GB/s": round(nbytes / t / 1e9, 1), "hbm_frac": round(nbytes / t / 1e9 / PEAK_HBM_GBS, 4),
                     "loads_per_thread": shapes[best][0], "block": shapes[best][1],
                     "all_shapes_us": [round(x * 1e6, 2) for x in times]})
    return rows


def read_ceiling_frac(ceiling, nbytes, us):
    """A GEMV row's time against the bare read of the same bytes (null when
    the ceiling was not measured at that byte count)."""
    for r in ceiling:
        if r["bytes"] == nbytes:
            return round(r["us"] / us, 4)
    return None


def w4a16_bench(torch, oi, gen, dev, stream, steps):
    """Weight-only int4 GEMV (group 128, bf16 scales) at M=1 on the W8A16
    headline shape K=4096, N=14336, over weight copies rotated past the MALL:
    HBM GB/s of its algorithmic bytes (N*K/2 codes + 2*N*K/128 scales +
    2*K activations + 2*N outputs)."""
    M, K, N = 1, 4096, 14336
    wbytes = N * K // 2 + 2 * N * (K // 128)
    copies = max(4, -(-GEMV_ROTATION_BYTES // wbytes))
    x = torch.randn((M, K), generator=gen, device=dev).half()
    ws = [torch.randint(0, 256, (N, K // 2), generator=gen, device=dev, dtype=torch.uint8)
          for _ in range(copies)]
    ss = [(torch.rand((N, K // 128), generator=gen, device=dev) * 0.02 + 0.002).to(torch.bfloat16)
          for _ in range(copies)]
    idx = [0]

    def gemv():
        i = idx[0] % copies
        oi.w4a16_linear(x, ws[i], ss[i])
        idx[0] += 1

    mark(torch, "w4a16_gemv")
    for _ in range(2 * copies):
        gemv()
    iters = copies * max(1, steps // 4)
    g = graph_of(gemv, iters)
    t = timed_graph(g, stream) / iters
    del g
    nbytes = wbytes + 2 * M * K + 2 * M * N
    res = {"M": M, "K": K, "N": N, "group": 128, "weight_copies": copies,
           "us_per_launch": round(t * 1e6, 3), "GB/s": round(nbytes / t / 1e9, 1),
           "roofline_frac": round(nbytes / t / 1e9 / PEAK_HBM_GBS, 4),
           "traffic": row_traffic("w4a16_gemv")}
    # The same weights at prefill (M=1024): the fp16-MFMA ring GEMM, packed
    # codes staged in LDS and dequantised to f16(q * s) in registers, in TFLOP/s.
    Mp = 1024
    xp = torch.randn((Mp, K), generator=gen, device=dev).half()

    def prefill():
        i = idx[0] % copies
        oi.w4a16_linear(xp, ws[i], ss[i])
        idx[0] += 1

    mark(torch, "w4a16_prefill")
    for _ in range(3):
        prefill()
    iters = max(copies, steps)
    g = graph_of(prefill, iters)
    tp = timed_graph(g, stream) / iters
    del g
    flops = 2.0 * Mp * N * K
    res["prefill"] = {"M": Mp, "K": K, "N": N, "us": round(tp * 1e6, 2),
                      "TFLOP/s": round(flops / tp / 1e12, 1),
                      "roofline_frac": round(flops / tp / 1e12 / PEAK_F16_TFLOPS, 4)}
    return res


def f16_bench(torch, gen, dev, stream, steps):
    """The fp16 analogs: the Breeze depth GEMV at its 8192 -> 1024 projection
    (M=1, over weight copies rotated past the MALL) in HBM GB/s of its
    algorithmic bytes (2*N*K weights + 2*K + 2*N), and the Qwen-Image DiT GEMM
    at 4096 x 4096 x 12288 (M x K x N) in TFLOP/s, with torch.matmul
    (hipBLASLt) on the same operands beside it."""
    from omni_int8.f16 import depth_try_linear, tensorops_try_linear
    M, K, N = 1, 8192, 1024
    wbytes = 2 * N * K
    copies = max(4, -(-GEMV_ROTATION_BYTES // wbytes))
    x = torch.randn((M, K), generator=gen, device=dev).half()
    ws = [(torch.randn((N, K), generator=gen, device=dev) * 0.02).half() for _ in range(copies)]
    idx = [0]

    def gemv():
        depth_try_linear(x, ws[idx[0] % copies].t())
        idx[0] += 1

    mark(torch, "f16_depth_gemv")
    for _ in range(2 * copies):
        gemv()
    iters = copies * max(1, steps // 4)
    g = graph_of(gemv, iters)
    t = timed_graph(g, stream) / iters
    del g
    nbytes = wbytes + 2 * M * K + 2 * M * N
    res = {"depth_gemv": {"M": M, "K": K, "N": N, "weight_copies": copies,
                          "us_per_launch": round(t * 1e6, 3), "GB/s": round(nbytes / t / 1e9, 1),
                          "roofline_frac": round(nbytes / t / 1e9 / PEAK_HBM_GBS, 4),
                          "traffic": row_traffic("f16_depth_gemv")}}
    M, K, N = 4096, 4096, 12288
    x = torch.randn((M, K), generator=gen, device=dev).half()
    w = (torch.randn((N, K), generator=gen, device=dev) * 0.02).half()
    wt = w.t()
    flops = 2.0 * M * N * K
    times = {}
    for name, fn in (("omni", lambda: tensorops_try_linear(x, wt)), ("torch_matmul", lambda: x @ wt)):
        mark(torch, f"f16_dit_{name}")
        for _ in range(3):
            fn()
        g = graph_of(fn, steps)
        times[name] = timed_graph(g, stream) / steps
        del g
    res["dit_gemm"] = {"M": M, "K": K, "N": N, "us": round(times["omni"] * 1e6, 2),
                       "TFLOP/s": round(flops / times["omni"] / 1e12, 1),
                       "roofline_frac": round(flops / times["omni"] / 1e12 / PEAK_F16_TFLOPS, 4),
                       "torch_matmul_TFLOP/s": round(flops / times["torch_matmul"] / 1e12, 1),
                       "traffic": row_traffic("f16_dit_gemm")}
    return res


def convrot_bench(torch, oi, gen, dev, stream, steps):
    """BASELINE config 4 (M=4352 = 4096 image + 256 text tokens): the fused
    ConvRot rotation + quantisation of the f16 activations at widths 3072
    (QKV / MLP-up input) and 12288 (MLP-down input), in HBM GB/s of its
    algorithmic bytes (2 B read + 1 B code written per element, 8 B per row),
    and one whole Int8Linear layer (QKV, N=9216, f16 out) in TOPS."""
    from omni_int8 import convrot
    M = 4352
    res = {"config": "BASELINE config 4, M=4352, f16 activations ~ N(0,1)"}
    kernels = []
    for K in (3072, 12288):
        x = torch.randn((M, K), generator=gen, device=dev).half()

        def fused(x=x):
            convrot.convrot_quantize_rows(x)

        mark(torch, f"convrot_{M}x{K}")
        for _ in range(3):
            fused()
        g = graph_of(fused, steps)
        t = timed_graph(g, stream) / steps
        del g
        nbytes = 3 * M * K + 8 * M
        kernels.append({"M": M, "K": K, "us": round(t * 1e6, 2), "GB/s": round(nbytes / t / 1e9, 1),
                        "roofline_frac": round(nbytes / t / 1e9 / PEAK_HBM_GBS, 4),
                        "traffic": row_traffic(f"convrot_{M}x{K}")})
    res["rotate_quantize"] = kernels
    K, N = 3072, 9216
    x = torch.randn((M, K), generator=gen, device=dev).half()
    w = torch.randint(-127, 128, (N, K), generator=gen, device=dev, dtype=torch.int8)
    layer = convrot.Int8Linear(K, N, w.view(torch.int32).reshape(-1),
                               torch.rand(N, generator=gen, device=dev) * 0.018 + 0.002,
                               torch.zeros(N, dtype=torch.int32, device=dev))

    def lin():
        layer(x)

    mark(torch, "convrot_layer")
    for _ in range(3):
        lin()
    g = graph_of(lin, steps)
    t = timed_graph(g, stream) / steps
    del g
    res["layer"] = {"M": M, "K": K, "N": N, "out": "f16", "us": round(t * 1e6, 2),
                    "tops": round(2.0 * M * N * K / t / 1e12, 1)}
    return res


def rotated_gemv_time(torch, gen, dev, stream, steps, M, K, N, wbytes_per_copy, make_w, run):
    """Per-launch seconds of run(x, w) at M x K -> N over enough weight copies
    (made by make_w) to exceed the 256 MB MALL, so every launch streams its
    weights from HBM."""
    copies = max(4, -(-GEMV_ROTATION_BYTES // wbytes_per_copy))
    x = torch.randn((M, K), generator=gen, device=dev).half()
    ws = [make_w() for _ in range(copies)]
    idx = [0]

    def one():
        run(x, ws[idx[0] % copies])
        idx[0] += 1

    for _ in range(2 * copies):
        one()
    iters = copies * max(1, steps // 8)
    g = graph_of(one, iters)
    t = timed_graph(g, stream) / iters
    del g, ws
    return t, copies


def configs_bench(torch, oi, gen, dev, stream, steps):
    """Every BASELINE.json config on the GPU, inputs resident in HBM, HIP-event
    timed graph replays. HBM-bound kernels report GB/s of algorithmic bytes,
    MFMA-bound ones TOPS / TFLOP/s (2*M*N*K)."""
    from omni_int8 import convrot
    res = {}

    def w8(N, K):
        return lambda: torch.randint(-127, 128, (N, K), generator=gen, device=dev, dtype=torch.int8)

    def s16(N):
        return (torch.rand(N, generator=gen, device=dev) * 0.018 + 0.002).half()

    # 1: weight-only GEMM M=16, K=N=4096 (the CPU-runnable case).
    M, K, N = 16, 4096, 4096
    sc = s16(N)
    mark(torch, "config1")
    t, copies = rotated_gemv_time(torch, gen, dev, stream, steps, M, K, N, N * K, w8(N, K),
                                  lambda x, w: oi.w8a16_linear(x, w, sc))
    nb = N * K + 2 * N + 2 * M * K + 2 * M * N
    res["1_w8a16_m16"] = {"M": M, "K": K, "N": N, "weight_copies": copies,
                          "us": round(t * 1e6, 3), "GB/s": round(nb / t / 1e9, 1),
                          "roofline_frac": round(nb / t / 1e9 / PEAK_HBM_GBS, 4),
                          "traffic": row_traffic("w8a16_m16")}

    # 2: decode GEMV sweep at 7B shapes, M = 1 and 4.
    sweep = []
    for K, N in ((4096, 4096), (4096, 14336), (14336, 4096), (4096, 128256)):
        sc = s16(N)
        for M in (1, 4):
            mark(torch, f"config2_m{M}_{K}x{N}")
            t, copies = rotated_gemv_time(torch, gen, dev, stream, steps, M, K, N, N * K,
                                          w8(N, K), lambda x, w: oi.w8a16_linear(x, w, sc))
            nb = N * K + 2 * N + 2 * M * K + 2 * M * N
            key = "w8a16_gemv" if (M, K, N) == GEMV_SHAPE else f"gemv_m{M}_{K}x{N}"
            sweep.append({"M": M, "K": K, "N": N, "weight_copies": copies,
                          "us": round(t * 1e6, 3), "GB/s": round(nb / t / 1e9, 1),
                          "roofline_frac": round(nb / t / 1e9 / PEAK_HBM_GBS, 4),
                          "traffic": row_traffic(key)})
    res["2_gemv_sweep"] = sweep

    def timed(fn, n=steps):
        for _ in range(3):
            fn()
        g = graph_of(fn, n)
        tt = timed_graph(g, stream) / n
        del g
        return tt

    # 3: W8A8 prefill, M=2048, K=4096: quantise + GEMM, f16 out + f32 bias.
    rows3 = []
    M, K = 2048, 4096
    x = torch.randn((M, K), generator=gen, device=dev).half()
    for N in (4096, 14336):
        w = w8(N, K)()
        scale = torch.rand(N, generator=gen, device=dev) * 0.018 + 0.002
        bias = torch.randn(N, generator=gen, device=dev)

        def layer(w=w, scale=scale, bias=bias):
            codes, rs, total = oi.quantize_rows(x)
            oi.w8a8_gemm(codes, rs, total, w, scale, None, bias, torch.float16)

        codes, rs, total = oi.quantize_rows(x)
        mark(torch, f"config3_n{N}")
        t = timed(layer)
        tg = timed(lambda w=w, scale=scale, bias=bias: oi.w8a8_gemm(
            codes, rs, total, w, scale, None, bias, torch.float16))
        ops = 2.0 * M * N * K
        rows3.append({"M": M, "K": K, "N": N, "out": "f16+bias", "us": round(t * 1e6, 2),
                      "TOPS": round(ops / t / 1e12, 1), "gemm_us": round(tg * 1e6, 2),
                      "gemm_TOPS": round(ops / tg / 1e12, 1),
                      "gemm_roofline_frac": round(ops / tg / 1e12 / PEAK_INT8_TOPS, 4),
                      "gemm_traffic": row_traffic(f"w8a8_cfg3_n{N}")})
    res["3_w8a8_prefill"] = rows3

    # 4: DiT linears at M=4352 with 1% outlier channels x20, as the production
    # Int8Linear (ConvRot rotation + quantisation, GEMM, f16 out).
    rows4 = []
    M = 4352
    for name, K, N in (("qkv", 3072, 9216), ("mlp_up", 3072, 12288), ("mlp_down", 12288, 3072)):
        x = torch.randn((M, K), generator=gen, device=dev)
        out_ch = torch.randperm(K, generator=gen, device=dev)[: max(1, K // 100)]
        x[:, out_ch] *= 20.0
        x = x.half()
        w = w8(N, K)()
        lin = convrot.Int8Linear(K, N, w.view(torch.int32).reshape(-1),
                                 torch.rand(N, generator=gen, device=dev) * 0.018 + 0.002,
                                 torch.zeros(N, dtype=torch.int32, device=dev))
        mark(torch, f"config4_{name}")
        t = timed(lambda lin=lin, x=x: lin(x))
        ops = 2.0 * M * N * K
        rows4.append({"layer": name, "M": M, "K": K, "N": N, "out": "f16", "us": round(t * 1e6, 2),
                      "TOPS": round(ops / t / 1e12, 1),
                      "gemm_traffic": row_traffic("w8a8_cfg4_" + {"qkv": "qkv", "mlp_up": "up",
                                                                  "mlp_down": "down"}[name]),
                      "convrot_traffic": row_traffic(f"convrot_{M}x{K}")})
    res["4_dit_convrot_layers"] = rows4

    # The floor under every launch: a graph of 400 launches of a 1 x 64 -> 1
    # GEMV (launch, dispatch and completion of an almost empty kernel).
    xt = torch.randn((1, 64), generator=gen, device=dev).half()
    wt = torch.ones((1, 64), device=dev, dtype=torch.int8)
    st = torch.ones(1, device=dev).half()
    mark(torch, "launch_floor")
    res["launch_floor_us"] = round(timed(lambda: oi.w8a16_linear(xt, wt, st), 400) * 1e6, 3)

    # 5: small-VLM mix: 28 layers of (q, kv, o, gate, up, down), W8A16.
    H, F, KV, L = 1536, 8960, 512, 28
    dims = ((H, H), (H, KV), (H, H), (H, F), (H, F), (F, H))  # (K, N) per linear
    layers = [[(w8(N, K)(), s16(N)) for K, N in dims] for _ in range(L)]
    wbytes = sum(N * K + 2 * N for K, N in dims) * L
    xp = {K: torch.randn((1024, K), generator=gen, device=dev).half() for K in (H, F)}
    xd = {K: torch.randn((1, K), generator=gen, device=dev).half() for K in (H, F)}

    def run_all(xs):
        for lay in layers:
            for (K, N), (w, sc) in zip(dims, lay):
                oi.w8a16_linear(xs[K], w, sc)

    mark(torch, "config5_prefill")
    t_pre = timed(lambda: run_all(xp), 3)
    mark(torch, "config5_decode")
    t_dec = timed(lambda: run_all(xd), 16)
    flops = 2.0 * 1024 * sum(N * K for K, N in dims) * L
    dbytes = wbytes + L * sum(2 * K + 2 * N for K, N in dims)
    # The same weights with the linears that read one input concatenated
    # along N (q with kv, gate with up), as inference engines store them:
    # 4 launches per layer instead of 6, identical outputs.
    fused_dims = ((H, H + KV), (H, H), (H, 2 * F), (F, H))
    fused = [[(torch.cat([lay[0][0], lay[1][0]]), torch.cat([lay[0][1], lay[1][1]])), lay[2],
              (torch.cat([lay[3][0], lay[4][0]]), torch.cat([lay[3][1], lay[4][1]])), lay[5]]
             for lay in layers]
    del layers

    def run_fused(xs):
        for lay in fused:
            for (K, N), (w, sc) in zip(fused_dims, lay):
                oi.w8a16_linear(xs[K], w, sc)

    mark(torch, "config5_fused_prefill")
    t_pre_f = timed(lambda: run_fused(xp), 3)
    mark(torch, "config5_fused_decode")
    t_dec_f = timed(lambda: run_fused(xd), 16)
    res["5_vlm_mix"] = {
        "layers": L, "hidden": H, "ffn": F, "kv_out": KV, "weight_bytes": wbytes,
        "prefill_kernel_traffic": {"gate_up": row_traffic("w8a16_cfg5_gateup"),
                                   "kv": row_traffic("w8a16_cfg5_kv")},
        "prefill_M": 1024, "prefill_ms": round(t_pre * 1e3, 3),
        "prefill_TFLOP/s": round(flops / t_pre / 1e12, 1),
        "decode_step_us": round(t_dec * 1e6, 2), "decode_GB/s": round(dbytes / t_dec / 1e9, 1),
        "decode_roofline_frac": round(dbytes / t_dec / 1e9 / PEAK_HBM_GBS, 4),
        "total_ms_prefill_plus_128_decode": round((t_pre + 128 * t_dec) * 1e3, 2),
        "fused_qkv_gateup": {
            "launches_per_layer": 4, "prefill_ms": round(t_pre_f * 1e3, 3),
            "prefill_TFLOP/s": round(flops / t_pre_f / 1e12, 1),
            "decode_step_us": round(t_dec_f * 1e6, 2),
            "decode_GB/s": round(dbytes / t_dec_f / 1e9, 1),
            "decode_roofline_frac": round(dbytes / t_dec_f / 1e9 / PEAK_HBM_GBS, 4),
            "total_ms_prefill_plus_128_decode": round((t_pre_f + 128 * t_dec_f) * 1e3, 2)}}
    del fused
    return res


def main():
    args = parse()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.phase_timeline:
        phase_timeline()
        return
    if args.configs_only:
        import torch
        import omni_int8 as oi
        dev = torch.device("cuda:0")
        torch.cuda.set_device(dev)
        gen = torch.Generator(device=dev)
        gen.manual_seed(0)
        print(json.dumps({"configs": configs_bench(torch, oi, gen, dev,
                                                   torch.cuda.current_stream(dev), args.steps)}))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(across GPUs the path would shard by output columns, one GPU's share being this "
              "same kernel at N/gpus columns)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import omni_int8 as oi

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if not oi.arch_supported(0):
        raise SystemExit("cuda:0 is not gfx950")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)

    # ---- W8A8: inputs resident in HBM, rotated past the MALL ---------------
    # Each shape keeps `copies` distinct activation/weight sets (>= 1 GiB in
    # all, >= 4 sets) and every step uses the next one, so no launch finds
    # its operands in the 256 MB Infinity Cache from an earlier launch.
    cases = []
    for M, K, N in GEMM_SHAPES:
        copies = max(4, -(-GEMV_ROTATION_BYTES // (2 * M * K + N * K + M * K)))
        xs, ws, codes = [], [], []
        for _ in range(copies):
            x = torch.randn((M, K), generator=gen, device=dev, dtype=torch.float32).half()
            w = torch.randint(-127, 128, (N, K), generator=gen, device=dev, dtype=torch.int8)
            xs.append(x)
            ws.append(w)
            codes.append(oi.quantize_rows(x))
        scale = torch.rand(N, generator=gen, device=dev) * 0.018 + 0.002
        zero = torch.zeros(N, dtype=torch.int32, device=dev)
        cases.append(dict(M=M, K=K, N=N, copies=copies, xs=xs, ws=ws, codes=codes, scale=scale,
                          zero=zero, next=0))

    outs = [None] * len(cases)
    used = [0] * len(cases)

    def step():
        for i, c in enumerate(cases):
            k = c["next"] % c["copies"]
            c["next"] += 1
            used[i] = k
            outs[i] = oi.try_int8_gemm(c["xs"][k], c["ws"][k].view(torch.int32).reshape(-1),
                                       c["scale"], c["zero"])

    mark(torch, "w8a8_step")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    g_steps = graph_of(step, args.steps)
    stream = torch.cuda.current_stream(dev)
    t_steps = timed_graph(g_steps, stream)
    # The replayed graph reproduces the eager result on the copies its last
    # step used.
    last = list(used)
    for i, c in enumerate(cases):
        k = last[i]
        eager = oi.try_int8_gemm(c["xs"][k], c["ws"][k].view(torch.int32).reshape(-1), c["scale"],
                                 c["zero"])
        assert torch.equal(outs[i].view(torch.int32), eager.view(torch.int32)), \
            "graph replay differs from eager try_int8_gemm"
    step_outs = [(last[i], outs[i].clone()) for i in range(len(cases))]
    del g_steps
    ops_per_step = sum(2.0 * c["M"] * c["N"] * c["K"] for c in cases)
    tops = ops_per_step * args.steps / t_steps / 1e12

    # Dominant kernel alone: the GEMM on pre-quantised codes, per orientation,
    # over the rotated copies (the roofline figure) and on one resident copy
    # (for comparison: what the MALL would add).
    gemm_time = 0.0
    per_shape = []
    for c in cases:
        def one(c=c):
            k = c["next"] % c["copies"]
            c["next"] += 1
            q, rs, total = c["codes"][k]
            oi.w8a8_gemm(q, rs, total, c["ws"][k], c["scale"], c["zero"])

        def resident(c=c):
            q, rs, total = c["codes"][0]
            oi.w8a8_gemm(q, rs, total, c["ws"][0], c["scale"], c["zero"])

        times = {}
        for name, fn in (("rotated", one), ("resident", resident)):
            mark(torch, f"w8a8_gemm_n{c['N']}_{name}")
            for _ in range(3):
                fn()
            g = graph_of(fn, args.steps)
            times[name] = timed_graph(g, stream) / args.steps
            del g
        t = times["rotated"]
        gemm_time += t
        per_shape.append({"M": c["M"], "K": c["K"], "N": c["N"], "copies": c["copies"],
                          "gemm_traffic": row_traffic(f"w8a8_gemm_n{c['N']}"),
                          "gemm_us": round(t * 1e6, 2),
                          "gemm_tops": round(2.0 * c["M"] * c["N"] * c["K"] / t / 1e12, 1),
                          "gemm_us_one_resident_copy": round(times["resident"] * 1e6, 2)})
    gemm_tops = ops_per_step / gemm_time / 1e12
    context = reference_shape_context(torch, oi, dev, stream, args.steps)
    traffic = load_traffic()

    # ---- W8A16 GEMV over rotating weight copies ---------------------------------
    gM, gK, gN = GEMV_SHAPE
    copies = max(4, -(-GEMV_ROTATION_BYTES // (gN * gK)))
    gx = torch.randn((gM, gK), generator=gen, device=dev).half()
    gws = [torch.randint(-127, 128, (gN, gK), generator=gen, device=dev, dtype=torch.int8)
           for _ in range(copies)]
    gs = (torch.rand(gN, generator=gen, device=dev) * 0.018 + 0.002).half()
    idx = [0]

    def gemv():
        oi.w8a16_linear(gx, gws[idx[0] % copies], gs)
        idx[0] += 1

    mark(torch, "w8a16_gemv")
    for _ in range(2 * copies):
        gemv()
    gemv_iters = copies * max(1, args.steps // 4)
    g = graph_of(gemv, gemv_iters)
    t_gemv = timed_graph(g, stream) / gemv_iters
    del g
    gemv_bytes = gN * gK + 2 * gN + 2 * gM * gK + 2 * gM * gN
    gemv_gbs = gemv_bytes / t_gemv / 1e9

    # ---- W4A16 GEMV (MiniCPM-V pack-quantized int4) --------------------------
    w4 = w4a16_bench(torch, oi, gen, dev, stream, args.steps)

    # ---- HBM read ceiling at the GEMV rows' byte counts ----------------------
    mark(torch, "hbm_read_ceiling")
    ceiling = hbm_read_ceiling(torch, gen, dev, stream, args.steps)
    w4["frac_of_read_ceiling"] = read_ceiling_frac(
        ceiling, READ_CEILING_ROWS[1][1], w4["us_per_launch"])

    # ---- fp16 analogs: depth GEMV and DiT GEMM -------------------------------
    f16_res = f16_bench(torch, gen, dev, stream, args.steps)

    # ---- ConvRot: fused rotation + quantisation, and one whole layer ---------
    convrot_res = convrot_bench(torch, oi, gen, dev, stream, args.steps)

    # ---- every BASELINE.json config ----------------------------------------------
    configs_res = configs_bench(torch, oi, gen, dev, stream, args.steps)
    for r in configs_res.get("2_gemv_sweep", []):
        nb = r["N"] * r["K"] + 2 * r["N"] + 2 * r["M"] * r["K"] + 2 * r["M"] * r["N"]
        r["frac_of_read_ceiling"] = read_ceiling_frac(ceiling, nb, r["us"])

    # ---- CPU baselines (oracle, bounded samples) -----------------------------
    import oracle_lib
    oracle = oracle_lib.Oracle()
    parity = step_parity(oracle, np, torch, cases, step_outs)
    cpu = cpu_baseline(oracle, np, args.cpu_seconds)
    cpu_gemv = cpu_gemv_baseline(oracle, np, max(2.0, args.cpu_seconds / 2))

    line = {
        "metric": "int8 GEMM TOPS + GEMV HBM GB/s (% of MI355X roofline), 1 GPU",
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_steps / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: x ~ N(0,1) f16, W ~ U[-127,127] int8, scales ~ U[0.002,0.02]; "
                "each step takes the next of >= 4 operand copies (>= 1 GiB per shape)",
        "config": {"workload": "try_int8_gemm (quantize_rows + W8A8 GEMM, f32 out) at "
                               "M=4096,K=3072,N=12288 and M=4096,K=12288,N=3072",
                   "gemm_shapes": per_shape},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tops, 1), "peak": PEAK_INT8_TOPS,
                     "unit": "TFLOP/s", "ops": "int8 MACs x2 (TOPS)",
                     "frac": round(gemm_tops / PEAK_INT8_TOPS, 4),
                     "traffic": traffic.get("w8a8_gemm")},
        "cpu_baseline": cpu,
        "parity": parity,
        "reference_shapes": context,
        "gemv": {
            "metric": "W8A16 GEMV HBM GB/s", "value": round(gemv_gbs, 1), "unit": "GB/s",
            "config": {"M": gM, "K": gK, "N": gN, "weight_copies": copies,
                       "rotation_bytes": copies * gN * gK},
            "us_per_launch": round(t_gemv * 1e6, 3),
            "frac_of_read_ceiling": read_ceiling_frac(ceiling, gemv_bytes, t_gemv * 1e6),
            "roofline": {"bound": "hbm", "achieved": round(gemv_gbs, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(gemv_gbs / PEAK_HBM_GBS, 4),
                         "traffic": traffic.get("w8a16_gemv")},
            "cpu_baseline": cpu_gemv,
        },
        "hbm_read_ceiling": ceiling,
        "convrot": convrot_res,
        "w4a16_gemv": w4,
        "f16": f16_res,
        "configs": configs_res,
        "profile_markers": PROFILE_MARKS,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
