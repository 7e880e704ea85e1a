"""Benchmark of the butterquant hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all|gemv|...]

Prints ONE JSON line.  Primary metric (value): decode GEMV HBM GB/s -- one
step is one per-row quantized GEMV (M=1 token, K=N=4096, weights rotated over
64 replicas = 1 GiB so every launch streams from HBM, not the 256 MB
Infinity Cache).  The same line carries the other headline numbers of the
metric: MoE-layer tokens/s at 32 and 2048 tokens, the prefill GEMM (M=512)
TOP/s and MFMA fraction, and the batch-16 decoder-layer time.

Kernel launches of each workload are captured once into a HIP graph
(torch.cuda.CUDAGraph records libbq's launches on its capture stream) and
replayed, so host launch overhead does not stretch the timed region.  After
at least 30 untimed replays, at least 600 replays are timed, each one a
sample: a HIP event is recorded on the replay stream before the first replay
and after every replay, and a sample is its replay's event time divided by
the launches the graph holds (64 rotated weight replicas for the GEMV).
Reported: p50 (the headline), min, mean, p90, p99; `steps` is the number of
launches timed.  Data: synthetic, bf16 N(0, 0.02) weights (seed 0)
quantized by libbq's own encoder, bf16 N(0,1) activations (seed 1),
N(0,1) router logits (seed 2); the vocabulary head uses uniform random int8
codes with per-block scales (seed 0).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mojo-gemma4-cpu_amd"))

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0     # dense int8 MFMA, published (no sparsity)
BF16_PEAK_TFLOPS = 2500.0   # dense bf16 MFMA, published
H, I, E, TOPK = 2816, 704, 128, 8   # Gemma-4-26B-A4B (modeling/gemma4_common.mojo)
MOE_LAYERS = []  # the timed MoE layers (inputs reused by the CPU baseline leg)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=128)
    ap.add_argument("--workload", default="all",
                    choices=["all", "gemv", "prefill", "moe32", "moe2048", "layer16", "head",
                             "attn", "load", "mfma", "stream_sweep"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a plain 256 MiB device copy (PMC calibration kernel)")
    ap.add_argument("--samples", type=int, default=600,
                    help="graph replays timed per workload (untimed warmup: min(30, samples)); "
                         "profiler runs use a few")
    ap.add_argument("--launch-histogram", metavar="KERNEL_TRACE_CSV",
                    help="no GPU: summarize the per-launch durations of the GEMV and the "
                         "streaming read in a rocprofv3 --kernel-trace CSV of --workload gemv")
    return ap.parse_args()


# ---------------------------------------------------------------------------
def graph_of(fn, n):
    """Capture n calls fn(i) into one graph (after one eager warm call each)."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(n):
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    torch.cuda.synchronize()
    return g


class Samples:
    """Per-launch times of one workload: each graph replay is one sample
    (its HIP-event time divided by the launches it holds)."""

    def __init__(self, ms, per_replay, wall):
        import numpy as np
        self.ms = np.asarray(ms, np.float64)
        self.per_replay, self.wall = per_replay, wall
        self.launches = len(self.ms) * per_replay
        self.p50 = float(np.median(self.ms))
        self.min = float(self.ms.min())
        self.mean = float(self.ms.mean())
        self.p90 = float(np.percentile(self.ms, 90))
        self.p99 = float(np.percentile(self.ms, 99))

    def summary(self, scale=1e3, unit="us"):
        """p50 / min / mean / p90 / p99 per launch (in `unit`), sample counts."""
        r = {f"p50_{unit}": self.p50 * scale, f"min_{unit}": self.min * scale,
             f"mean_{unit}": self.mean * scale, f"p90_{unit}": self.p90 * scale,
             f"p99_{unit}": self.p99 * scale}
        r = {k: round(v, 3) for k, v in r.items()}
        r.update(samples=len(self.ms), launches_per_sample=self.per_replay,
                 launches=self.launches)
        return r


SAMPLES = 600   # graph replays timed per workload (at least)
WARMUP = 30     # untimed replays before them (at least)


def n_samples(steps, per_replay):
    """Replays to time: >= SAMPLES, and enough for >= `steps` launches."""
    return max(SAMPLES, -(-steps // per_replay))


def time_graph(g, per_replay, steps, warmup):
    """Replay graph g max(WARMUP, warmup / per_replay) times untimed, then
    n_samples(steps, per_replay) times with a HIP event recorded on the replay
    stream before the first and after every replay -> Samples."""
    import torch
    for _ in range(max(WARMUP, -(-warmup // per_replay))):
        g.replay()
    torch.cuda.synchronize()
    n = n_samples(steps, per_replay)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    t0 = time.perf_counter()
    ev[0].record()
    for i in range(n):
        g.replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return Samples([ev[i].elapsed_time(ev[i + 1]) / per_replay for i in range(n)], per_replay, wall)


def quantized(bq, torch, n, k, block, gen):
    w = (torch.randn(n, k, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    codes, scales = bq.quantize_weight(w, block)
    tiled = bq.retile(codes.view(-1), n, k)
    return codes, scales, bq.ButterquantWeight(tiled, scales, n, k)


# ---------------------------------------------------------------------------
def calib_lib():
    """libbq_calib.so: the measurement kernels (streaming read of the GEMV's
    launch shape, int8 MFMA loop); built beside libbq.so."""
    import ctypes as C
    path = os.path.join(ROOT, "mojo-gemma4-cpu_amd", "libbq_calib.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (python __graft_entry__.py)")
    L = C.CDLL(path)
    L.bqc_stream_read.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    L.bqc_stream_sweep.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                   C.c_void_p]
    L.bqc_stream_shape.argtypes = [C.c_int, C.c_void_p]
    L.bqc_mfma_i8.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    L.bqc_mfma_i8_ops.argtypes = [C.c_int, C.c_int, C.c_int]
    L.bqc_mfma_i8_ops.restype = C.c_double
    L.bqc_lds_read.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    L.bqc_dma_l2.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                             C.c_void_p, C.c_void_p]
    L.bqc_mfma_chain.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    L.bqc_vmem_l2.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                              C.c_void_p, C.c_void_p, C.c_void_p]
    return L


def _stream(torch):
    return torch.cuda.current_stream().cuda_stream


def bench_gemv(bq, torch, steps, warmup, reps=64):
    """The decode GEMV over 64 weight replicas (1 GiB, one contiguous
    allocation), its activation prep, and the streaming-read kernel of the
    same launch shape over the same replicas (the measured per-launch
    ceiling of the GEMV)."""
    N = K = 4096
    gen = torch.Generator(device="cuda").manual_seed(0)
    codes, scales, W0 = quantized(bq, torch, N, K, 128, gen)
    pool = torch.empty(reps, N * K, dtype=torch.int8, device="cuda")
    pool.copy_(W0.data.view(1, -1).expand(reps, -1))
    replicas = [bq.ButterquantWeight(pool[i], scales if i == 0 else scales.clone(), N, K)
                for i in range(reps)]
    xg = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(1, K, generator=xg, device="cuda").to(torch.bfloat16)
    gamma = torch.ones(K, dtype=torch.bfloat16, device="cuda")
    xq, sa = bq.norm_quant(x, gamma, 128)
    out = torch.empty(1, N, dtype=torch.bfloat16, device="cuda")
    g = graph_of(lambda i: bq.linear(xq, sa, replicas[i], out=out), reps)
    smp = time_graph(g, reps, steps, warmup)
    alg_bytes = N * K + N * 4 + K + 4 + N * 2       # W + sw + x_i8 + sa + y
    # activation prep (norm-quant: RMS, FWHT128, int8) and the full decode linear
    gq = graph_of(lambda i: bq.norm_quant(x, gamma, 128, out=(xq, sa)), 64)
    s_nq = time_graph(gq, 64, 0, 0)
    gl = graph_of(lambda i: (bq.norm_quant(x, gamma, 128, out=(xq, sa)),
                             bq.linear(xq, sa, replicas[i], out=out)), reps)
    s_lin = time_graph(gl, reps, 0, 0)
    # the same in one launch (bq_norm_linear: every output tile quantizes the
    # row itself while its weights stream in)
    gf = graph_of(lambda i: bq.norm_linear(x, gamma, replicas[i], 128, out=out,
                                           act_out=(xq, sa)), reps)
    s_fused = time_graph(gf, reps, 0, 0)
    rd = bench_stream(torch, [r.data for r in replicas], N // 16, K // 64, steps, warmup)
    rd["sweep"] = bench_stream_sweep(torch, [r.data for r in replicas], N // 16)
    return dict(s=smp, alg_bytes=alg_bytes, gbs=alg_bytes / (smp.p50 * 1e-3) / 1e9,
                gbs_min=alg_bytes / (smp.min * 1e-3) / 1e9, s_nq=s_nq, s_lin=s_lin,
                s_fused=s_fused, rd=rd, codes=codes, scales=scales, xq=xq, sa=sa)


def _env_int(name):
    try:
        return int(os.environ.get(name, "0"))
    except ValueError:
        return 0


def gemv_kernel():
    """(kernel name, waves per workgroup) of the decode GEMV (M = 1, per-row,
    K = 4096, one output segment) as the library's launcher picks it:
    k_gemv_m1_1 with BQ_GEMV_M1_WAVES (2, 4, 8; default 4), or
    k_linear_skinny_1 when BQ_GEMV_WAVES (4, 8, 16) is set."""
    g = _env_int("BQ_GEMV_WAVES")
    if g:
        w = 16 if g >= 16 else 4 if g <= 4 else 8
        return f"k_linear_skinny_1<{w}, false, {64 // w}>", w
    m1 = _env_int("BQ_GEMV_M1_WAVES") or 4
    w = 2 if m1 <= 2 else 8 if m1 >= 8 else 4
    return f"k_gemv_m1_1<{w}, {64 // w}>", w


def gemv_waves():
    return gemv_kernel()[1]


def bench_stream(torch, bufs, tiles, K64, steps, warmup):
    """The streaming-read kernel (bqc_stream_read): the GEMV's launch shape
    (`tiles` workgroups x gemv_waves() waves, one-shot non-temporal 16-byte
    loads of each wave's K64/waves fragments) over the GEMV's own replicas -> the measured
    per-launch ceiling; the same grid reading nothing -> the fixed cost of a
    launch in a graph; and 256 MiB per launch (4096 workgroups) rotated over
    four windows of a 1 GiB buffer -> the sustained streaming rate."""
    L = calib_lib()
    sink = torch.empty(4096 * 16, dtype=torch.int16, device="cuda")

    def launcher(ptrs, t, k):
        def f(i):
            rc = L.bqc_stream_read(ptrs[i], t, k, gemv_waves(), sink.data_ptr(), _stream(torch))
            if rc != 0:
                raise RuntimeError(f"bqc_stream_read: hipError {rc}")
        return f

    ptrs = [b.data_ptr() for b in bufs]
    n = len(ptrs)
    same = time_graph(graph_of(launcher(ptrs, tiles, K64), n), n, steps, warmup)
    empty = time_graph(graph_of(launcher(ptrs, tiles, 0), n), n, 0, 0)
    big = torch.empty(4, 256 << 20, dtype=torch.int8, device="cuda")
    bptr = [big[i].data_ptr() for i in range(4)]
    large = time_graph(graph_of(launcher(bptr, 4096, 64), 4), 4, 0, 0)
    del big
    b16, b256 = tiles * K64 * 1024 + tiles * 32, (256 << 20) + 4096 * 32
    return dict(same=same, empty=empty, large=large, bytes=b16,
                gbs=b16 / (same.p50 * 1e-3) / 1e9, gbs_best=b16 / (same.min * 1e-3) / 1e9,
                large_gbs=b256 / (large.p50 * 1e-3) / 1e9,
                incr_gbs=(b256 - b16) / ((large.p50 - same.p50) * 1e-3) / 1e9)


def bench_stream_sweep(torch, bufs, tiles, samples=200):
    """The streaming read of the decode GEMV's bytes (tiles x 64 KiB of
    tile16x64 fragments per launch, over the GEMV's 64 replicas) in every
    launch shape of bqc_stream_sweep: workgroups, waves per workgroup, loads
    in flight per wave.  Each shape's p50 per launch with its bytes, and the
    same grid reading nothing (its fixed cost), graph-replayed as the GEMV."""
    import ctypes as C
    L = calib_lib()
    sink = torch.empty(tiles * 8 * 16, dtype=torch.int16, device="cuda")
    ptrs = [b.data_ptr() for b in bufs]
    n = len(ptrs)
    nbytes = tiles * 64 * 1024
    rows = []
    global SAMPLES
    keep, SAMPLES = SAMPLES, min(SAMPLES, samples)
    try:
        for i in range(L.bqc_stream_shapes()):
            desc = (C.c_int * 4)()
            L.bqc_stream_shape(i, desc)
            w, u, spw, ks = list(desc)

            def launcher(empty):
                def f(j):
                    rc = L.bqc_stream_sweep(ptrs[j], tiles, i, empty, sink.data_ptr(),
                                            _stream(torch))
                    if rc != 0:
                        raise RuntimeError(f"bqc_stream_sweep: hipError {rc}")
                return f
            full = time_graph(graph_of(launcher(0), n), n, 0, 0)
            empty = time_graph(graph_of(launcher(1), n), n, 0, 0)
            rows.append(dict(workgroups=tiles // spw * ks, waves=w, loads_per_wave=u * spw,
                             tiles_per_workgroup=spw, k_parts=ks,
                             p50_us=round(full.p50 * 1e3, 3), min_us=round(full.min * 1e3, 3),
                             GBs=round(nbytes / (full.p50 * 1e-3) / 1e9, 1),
                             empty_p50_us=round(empty.p50 * 1e3, 3)))
    finally:
        SAMPLES = keep
    best = min(rows, key=lambda r: r["p50_us"])
    return dict(bytes_per_launch=nbytes, shapes=rows, best=best)


def bench_mfma(torch):
    """int8 MFMA throughput from registers: 4 waves per workgroup, 4
    workgroups per CU, each wave 8 or 16 (16x16x64) or 4 (32x32x32)
    independent chains; the best and median of 20 launches timed with HIP
    events."""
    import numpy as np
    L = calib_lib()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks, iters = cus * 4, 2048
    out = torch.empty(blocks * 256, dtype=torch.int32, device="cuda")
    res = {}
    for shape, name in ((16, "v_mfma_i32_16x16x64_i8"), (17, "v_mfma_i32_16x16x64_i8 x16 chains"),
                        (32, "v_mfma_i32_32x32x32_i8")):
        ops = L.bqc_mfma_i8_ops(shape, blocks, iters)
        ts = []
        for i in range(23):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            rc = L.bqc_mfma_i8(shape, blocks, iters, out.data_ptr(), _stream(torch))
            b.record()
            torch.cuda.synchronize()
            if rc != 0:
                raise RuntimeError(f"bqc_mfma_i8: hipError {rc}")
            if i >= 3:
                ts.append(a.elapsed_time(b))
        ts = np.array(ts)
        res[name] = {"best_TOPs": round(ops / (ts.min() * 1e-3) / 1e12, 1),
                     "p50_TOPs": round(ops / (np.median(ts) * 1e-3) / 1e12, 1),
                     "ops_per_launch": ops}
    res["launch"] = f"{blocks} workgroups x 4 waves ({cus} CUs), {iters} iterations"
    return res


def bench_probes(torch):
    """The measured ceilings the tiled kernels are designed against
    (libbq_calib.so): LDS read bytes per clock per CU (ds_read_b128,
    conflict-free), L2-resident global -> LDS DMA (whole 128-byte lines vs
    the raw 16 x 64-byte MFMA fragment), the latency of a dependent
    v_mfma_i32_16x16x64_i8 chain, and the streaming read of 256 MiB per
    launch over the sweep's launch shapes (4 replicas, 1 GiB).  Cycle counts
    come from each workgroup's own shader clock; one workgroup per CU."""
    import numpy as np
    L = calib_lib()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    st = _stream(torch)
    cyc = torch.empty(cus, dtype=torch.int64, device="cuda")
    res = {}

    def timed(launch, reps=5):
        best = None
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            rc = launch()
            b.record()
            torch.cuda.synchronize()
            if rc != 0:
                raise RuntimeError(f"calib probe: hipError {rc}")
            ms, c = a.elapsed_time(b), float(cyc.float().median().item())
            if best is None or ms < best[0]:
                best = (ms, c)
        return best

    fold = torch.empty(cus * 1024, dtype=torch.int32, device="cuda")
    iters = 256
    lds = {}
    for waves in (4, 8, 16):
        ms, c = timed(lambda: L.bqc_lds_read(waves, cus, iters, cyc.data_ptr(), fold.data_ptr(), st))
        per_block = waves * 64 * 16 * 8 * iters
        lds[f"{waves}_waves"] = {"B_per_clk_per_cu": round(per_block / c, 1),
                                 "TBs": round(per_block * cus / (ms * 1e-3) / 1e12, 1)}
    res["lds_read_b128"] = lds
    rows, stride = 512, 4096  # a 2 MiB source every workgroup reads
    src = torch.randint(-127, 128, (rows * stride,), dtype=torch.int8, device="cuda")
    dma = {}
    for shape, name in ((0, "lines_8x128B"), (1, "fragments_16x64B")):
        for waves in (4, 8):  # 32 or 64 KiB in flight per CU
            ms, c = timed(lambda: L.bqc_dma_l2(shape, waves, src.data_ptr(), stride, rows, cus,
                                                64, cyc.data_ptr(), st))
            per_block = waves * 8 * 1024 * 64
            dma[f"{name}_{waves * 8}KiB_in_flight"] = {
                "B_per_clk_per_cu": round(per_block / c, 1),
                "TBs": round(per_block * cus / (ms * 1e-3) / 1e12, 1)}
    res["dma_l2_to_lds"] = dma
    vm = {}
    for waves in (4, 8, 16):
        ms, c = timed(lambda: L.bqc_vmem_l2(waves, src.data_ptr(), stride, rows, cus, 64,
                                             cyc.data_ptr(), fold.data_ptr(), st))
        per_block = waves * 8 * 1024 * 64
        vm[f"lines_8x128B_{waves * 8}KiB_in_flight"] = {
            "B_per_clk_per_cu": round(per_block / c, 1),
            "TBs": round(per_block * cus / (ms * 1e-3) / 1e12, 1)}
    res["vmem_l2_to_vgpr"] = vm
    n = 4096
    out = torch.empty(64, dtype=torch.int32, device="cuda")
    cyc1 = torch.empty(1, dtype=torch.int64, device="cuda")
    rc = L.bqc_mfma_chain(n, 1, cyc1.data_ptr(), out.data_ptr(), st)
    torch.cuda.synchronize()
    if rc != 0:
        raise RuntimeError(f"bqc_mfma_chain: hipError {rc}")
    res["mfma_16x16x64_i8_chain_cycles_per_link"] = round(int(cyc1.item()) / n, 1)
    big = torch.randint(-127, 128, (4, 256 << 20), dtype=torch.int8, device="cuda")
    sw = bench_stream_sweep(torch, [big[i] for i in range(4)], 4096, samples=50)
    res["stream_256MiB"] = {"best": sw["best"],
                            "shapes": [{k: r[k] for k in ("workgroups", "waves", "loads_per_wave",
                                                          "p50_us", "GBs")} for r in sw["shapes"]]}
    del big
    return res


def bench_prefill(bq, torch, steps, warmup, reps=32):
    M, N, K = 512, 4096, 4096
    gen = torch.Generator(device="cuda").manual_seed(0)
    codes, scales, W0 = quantized(bq, torch, N, K, 128, gen)
    replicas = [W0] + [bq.ButterquantWeight(W0.data.clone(), scales, N, K) for _ in range(reps - 1)]
    xg = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(M, K, generator=xg, device="cuda").to(torch.bfloat16)
    xq, sa = bq.norm_quant(x, torch.ones(K, dtype=torch.bfloat16, device="cuda"), 128)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    g = graph_of(lambda i: bq.linear(xq, sa, replicas[i], out=out), reps)
    smp = time_graph(g, reps, steps, warmup)
    ops = 2.0 * M * N * K
    tops = ops / (smp.p50 * 1e-3) / 1e12
    return dict(s=smp, ops=ops, tops=tops, int8_frac=tops / INT8_PEAK_TOPS,
                bf16_frac=tops / BF16_PEAK_TFLOPS,
                alg_bytes=N * K + N * 4 + M * K + M * 4 + M * N * 2,
                vendor=vendor_gemm(torch, M, N, K, reps),
                cpu_inputs=(codes, scales, xq, sa))


def vendor_gemm(torch, M, N, K, reps):
    """The same product through the vendor library (hipBLASLt behind torch),
    timed the same way over the same number of weight replicas: int8 x int8
    -> int32 (torch._int_mm, the weight as a transposed [K, N] view, its
    fastest layout here) and bf16 x bf16 -> bf16 (torch.mm).  Neither applies
    the butterquant scales: a reference point for the product alone."""
    g0 = torch.Generator(device="cuda").manual_seed(5)
    a = torch.randint(-127, 128, (M, K), generator=g0, dtype=torch.int8, device="cuda")
    ws = [torch.randint(-127, 128, (N, K), generator=g0, dtype=torch.int8, device="cuda")
          for _ in range(reps)]
    res = {}
    try:
        o = torch.empty(M, N, dtype=torch.int32, device="cuda")
        s = time_graph(graph_of(lambda i: torch._int_mm(a, ws[i].t(), out=o), reps), reps, 0, 0)
        res["int8_int_mm_p50_us"] = round(s.p50 * 1e3, 2)
    except Exception as e:  # an unsupported shape or build: report it, time the rest
        res["int8_int_mm_error"] = str(e)[:200]
    ab = a.to(torch.bfloat16)
    wb = [w.to(torch.bfloat16) for w in ws]
    ob = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    s = time_graph(graph_of(lambda i: torch.mm(ab, wb[i].t(), out=ob), reps), reps, 0, 0)
    res["bf16_mm_p50_us"] = round(s.p50 * 1e3, 2)
    res["library"] = "hipBLASLt via torch " + torch.__version__
    return res


class MoeLayer:
    """One quantized MoE expert layer from router logits and hidden states:
    top-8 + softmax routing and the CSR schedule (bq_moe_route_schedule),
    the norm-quant of the hidden states, phase 1 (gate/up + GELU) with the
    FWHT64 block-quant of the bucket fused, phase 2 (down + route-weighted,
    expert-ordered combine) -- the reference's MoE block,
    modeling/gemma_4_moe_bq.mojo:666-704, from its router logits on."""

    def __init__(self, bq, torch, T, Wgu, Wd, gen_seed=1):
        self.bq, self.T = bq, T
        xg = torch.Generator(device="cuda").manual_seed(gen_seed)
        self.x = torch.randn(T, H, generator=xg, device="cuda").to(torch.bfloat16)
        lg = torch.Generator(device="cuda").manual_seed(2)
        self.logits = torch.randn(T, E, generator=lg, device="cuda")
        self.pes = torch.ones(E, dtype=torch.bfloat16, device="cuda")  # per_expert_scale = 1
        self.gamma = torch.ones(H, dtype=torch.bfloat16, device="cuda")
        self.Wgu, self.Wd = Wgu, Wd
        d = "cuda"
        self.idx = torch.empty(T, TOPK, dtype=torch.int32, device=d)
        self.w = torch.empty(T, TOPK, dtype=torch.float32, device=d)
        self.xq = torch.empty(T, H, dtype=torch.int8, device=d)
        self.xsa = torch.empty(T, dtype=torch.float32, device=d)
        self.eo = torch.empty(E + 1, dtype=torch.int32, device=d)
        self.routes = torch.zeros(T * TOPK, 2, dtype=torch.int32, device=d)
        self.bucket = torch.empty(T * TOPK, I, dtype=torch.bfloat16, device=d)
        self.bi8 = torch.empty(T * TOPK, I, dtype=torch.int8, device=d)
        self.bsa = torch.empty(T * TOPK, I // 64, dtype=torch.float32, device=d)
        self.ws = torch.empty(max(bq.moe_phase2_workspace_size(T, TOPK, H), 256),
                              dtype=torch.uint8, device=d)
        self.accum = torch.empty(T, H, dtype=torch.float32, device=d)
        self.out = torch.empty(T, H, dtype=torch.bfloat16, device=d)
        self.side = torch.cuda.Stream()  # default priority

    def __call__(self, _i=0, fused=True, overlap=3, prep=True):
        # overlap 3: bq_moe_prep (top-k, schedule and norm-quant in one launch
        # up to 1024 route slots); 1: bq_moe_route_schedule then the
        # norm-quant; 2: the norm-quant on a second stream beside the routing
        # (measured slower: the graph's cross-stream joins cost more than the
        # overlap saves); 0: the reference's three calls.  prep=False: the
        # caller has already made idx/w/eo/routes/xq/xsa (bq_ffn_prep)
        import torch
        bq, T = self.bq, self.T
        if not prep:
            pass
        elif overlap == 3:
            bq.moe_prep(self.logits, self.x, self.gamma, TOPK, self.pes, 128,
                        out=(self.idx, self.w, self.eo, self.routes, self.xq, self.xsa))
        elif overlap == 2:
            main = torch.cuda.current_stream()
            self.side.wait_stream(main)
            with torch.cuda.stream(self.side):
                bq.norm_quant(self.x, self.gamma, 128, out=(self.xq, self.xsa))
            bq.route_schedule(self.logits, TOPK, self.pes,
                              out=(self.idx, self.w, self.eo, self.routes))
            main.wait_stream(self.side)
        elif overlap == 1:
            bq.route_schedule(self.logits, TOPK, self.pes,
                              out=(self.idx, self.w, self.eo, self.routes))
            bq.norm_quant(self.x, self.gamma, 128, out=(self.xq, self.xsa))
        else:
            bq.route_topk(self.logits, TOPK, self.pes, out=(self.idx, self.w))
            bq.norm_quant(self.x, self.gamma, 128, out=(self.xq, self.xsa))
            bq.build_schedule(self.idx, self.w, E, out=(self.eo, self.routes))
        if fused:  # phase 1 with the bucket's FWHT64 block-quant in its epilogue
            bq.moe_phase1_quant(self.xq, self.xsa, self.eo, self.routes, self.Wgu, E, T, TOPK, I,
                                out=(self.bi8, self.bsa, None))
        else:
            bq.moe_phase1(self.xq, self.xsa, self.eo, self.routes, self.Wgu, E, T, TOPK, I,
                          out=self.bucket)
            bq.block_quant(self.bucket, 64, True, out=(self.bi8, self.bsa))
        bq.moe_phase2(self.bi8, self.bsa, self.eo, self.routes, self.Wd, E, T, TOPK, H,
                      workspace=self.ws, out=(self.accum, self.out))


def bench_head(bq, torch, steps, rows_list=(1, 16)):
    """The tied vocabulary head at decode: head prep (per-block norm-quant of
    the final hidden rows) + flash sample over all 262144 vocabulary rows
    (per-block B = 128 int8 head, softcap 30, Gumbel sampling, top-256),
    graph-replayed.  The 761 MB head is larger than the Infinity Cache, so
    every replay streams it from HBM."""
    import numpy as np
    V, HH, B = 262144, H, 128
    gen = torch.Generator(device="cuda").manual_seed(0)
    codes = torch.randint(-127, 128, (V * HH,), generator=gen, dtype=torch.int8, device="cuda")
    W = bq.ButterquantWeight(bq.retile(codes, V, HH),
                             torch.rand(V, HH // B, generator=gen, device="cuda") / 127 / 30, V, HH)
    del codes
    gamma = torch.ones(HH, dtype=torch.bfloat16, device="cuda")
    alg = V * HH + V * (HH // B) * 4
    out = {}
    for R in rows_list:
        xg = torch.Generator(device="cuda").manual_seed(1)
        x = torch.randn(R, HH, generator=xg, device="cuda").to(torch.bfloat16)
        xq = torch.empty(R, HH, dtype=torch.int8, device="cuda")
        xsa = torch.empty(R, HH // B, dtype=torch.float32, device="cuda")
        p = np.zeros((R, 40), np.uint8)
        pv = p.view(np.dtype([("t", "<f4"), ("m", "<f4"), ("k", "<i8"), ("s", "<u8"),
                              ("n", "<i8"), ("g", "u1"), ("pad", "u1", 7)])).reshape(R)
        pv["t"], pv["n"], pv["s"], pv["k"], pv["m"] = 1.0, 256, np.arange(R) + 1, 64, 0.05
        pr = torch.from_numpy(p).cuda()
        ws = torch.empty(bq.flash_sample_workspace_size(R, V), dtype=torch.uint8, device="cuda")
        res = torch.empty(R, 2064, dtype=torch.uint8, device="cuda")

        def step(_i=0):
            bq.head_prep(x, gamma, B, out=(xq, xsa))
            bq.flash_sample(xq, xsa, W, W.scale, pr, block=B, workspace=ws, out=res)
        g = graph_of(step, 4)
        smp = time_graph(g, 4, 0, 0)
        out[R] = dict(s=smp, ms=smp.p50, gbs=alg / (smp.p50 * 1e-3) / 1e9)
    return dict(alg_bytes=alg, rows=out)


def bench_load(bq, torch):
    """The on-disk -> device path on the MoE gate/up tensor (128 experts x
    1408 x 2816 int8 + per-row scales, 507 MB) written as a safetensors file
    under $TMPDIR: bq_load_quantized (mmap, validate, host -> device copy
    through a 64 MiB staging buffer, re-tile), file in the page cache.
    Opt-in (--workload load): it writes a 0.5 GB file."""
    import tempfile

    import numpy as np
    from safetensors.numpy import save_file
    n, k = E * 2 * I, H
    rng = np.random.default_rng(0)
    codes = rng.integers(-127, 128, (E, 2 * I, k), dtype=np.int8)
    scales = rng.random((E, 2 * I)).astype(np.float32)
    d = tempfile.mkdtemp()
    path = os.path.join(d, "experts.safetensors")
    save_file({"experts.gate_up": codes, "experts.gate_up.scale": scales.reshape(-1)}, path)
    f = bq.SafetensorsFile(path)
    staging = torch.empty(64 << 20, dtype=torch.int8, device="cuda")
    w = torch.empty(n * k, dtype=torch.int8, device="cuda")
    s = torch.empty(n, dtype=torch.float32, device="cuda")
    ts = []
    for _ in range(6):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        bq.load_quantized([f], "experts.gate_up", n, k, staging=staging, out=(w, s))
        torch.cuda.synchronize()
        ts.append(time.perf_counter() - t0)
    ok = bool((bq.unpack(w[: 16 * k], 16, k).cpu().numpy().reshape(16, k) ==
               codes.reshape(n, k)[:16]).all())
    f.close()
    os.remove(path)
    os.rmdir(d)
    med = float(np.median(ts[1:]))
    return dict(ms=med * 1e3, gbs=(n * k + n * 4) / med / 1e9, checked=ok)


def moe_weights(bq, torch):
    gen = torch.Generator(device="cuda").manual_seed(0)
    _, _, Wgu = quantized(bq, torch, E * 2 * I, H, 128, gen)
    _, _, Wd = quantized(bq, torch, E * H, I, 64, gen)
    return Wgu, Wd


def bench_moe(bq, torch, T, weights, steps):
    """weights: list of (Wgu, Wd) replicas; consecutive steps alternate
    between them so each step's ~0.7 GB of experts is not resident in the
    256 MB Infinity Cache from the previous step."""
    layers = [MoeLayer(bq, torch, T, Wgu, Wd) for Wgu, Wd in weights]
    MOE_LAYERS.append(layers[0])
    g = graph_of(lambda i: layers[i](), len(layers))
    smp = time_graph(g, len(layers), steps, 0)
    ms = smp.p50
    layer = layers[0]
    eo = layer.eo.cpu().numpy()
    touched = int((eo[1:] - eo[:-1] > 0).sum())
    per_expert = 2 * I * H + 2 * I * 4 + H * I + H * 4
    wbytes = touched * per_expert
    return dict(T=T, s=smp, ms=ms, tokens_per_s=T / (ms * 1e-3), experts_touched=touched,
                weight_bytes=wbytes, hbm_gbs_weights=wbytes / (ms * 1e-3) / 1e9,
                ops=2.0 * T * TOPK * (2 * I * H + H * I))


def bench_layer16(bq, torch, Wgu, Wd, steps):
    """All quantized projections of one decoder layer at decode batch 16:
    sliding (q/k/v 4096/2048/2048, o B=256) and full (q 8192, k 1024, o
    B=512) attention projections, dense MLP (gate/up 2112, GELU-tanh(gate) *
    up, FWHT64 block-quant, down B=64) and the 128-expert MoE, each with its
    activation prep."""
    T = 16
    gen = torch.Generator(device="cuda").manual_seed(0)
    d = "cuda"
    host = {}

    def mk(n, k, b, name):
        codes, scales, w = quantized(bq, torch, n, k, b, gen)
        host[name] = (codes.cpu().numpy(), scales.cpu().numpy(), b)
        return w
    sq, sk, sv, so = (mk(4096, H, 128, "sq"), mk(2048, H, 128, "sk"), mk(2048, H, 128, "sv"),
                      mk(H, 4096, 256, "so"))
    fq, fk, fo = mk(8192, H, 128, "fq"), mk(1024, H, 128, "fk"), mk(H, 8192, 512, "fo")
    dg, du, dd = mk(2112, H, 128, "dg"), mk(2112, H, 128, "du"), mk(H, 2112, 64, "dd")
    xg = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(T, H, generator=xg, device=d).to(torch.bfloat16)
    gamma = torch.ones(H, dtype=torch.bfloat16, device=d)
    e = lambda *shape, dt=torch.bfloat16: torch.empty(*shape, dtype=dt, device=d)
    xq, xsa = e(T, H, dt=torch.int8), e(T, dt=torch.float32)
    # attention outputs feeding o_proj (the attention itself is not a bq op)
    attn_s = torch.randn(T, 4096, generator=xg, device=d).to(torch.bfloat16)
    attn_f = torch.randn(T, 8192, generator=xg, device=d).to(torch.bfloat16)
    oq_s, osa_s = e(T, 4096, dt=torch.int8), e(T, 16, dt=torch.float32)
    oq_f, osa_f = e(T, 8192, dt=torch.int8), e(T, 16, dt=torch.float32)
    q_s, k_s, v_s = e(T, 4096), e(T, 2048), e(T, 2048)
    q_f, k_f = e(T, 8192), e(T, 1024)
    o = e(T, H)
    gq_, gsa = e(T, 2112, dt=torch.int8), e(T, 2112 // 64, dt=torch.float32)
    moe = MoeLayer(bq, torch, T, Wgu, Wd)
    moe.x = x   # the dense MLP and the MoE both read the post-attention residual

    xqd, xsad = e(T, H, dt=torch.int8), e(T, dt=torch.float32)
    od = e(T, H)

    base = dict(q=sq, k=sk, v=sv, o=so, fq=fq, fk=fk, fo=fo, dg=dg, du=du, dd=dd, gu=Wgu, d=Wd)

    def ffn(L):
        # routing, schedule and both norm-quants of x (the MoE's gamma and the
        # dense MLP's) in one launch (bq_ffn_prep); the dense MLP's gate/up,
        # GELU and FWHT64 block-quant in the experts' gate/up launch
        # (bq_ffn_gate_up), its down projection in the experts' down launch
        # (bq_ffn_down)
        bq.ffn_prep(moe.logits, x, moe.gamma, gamma, TOPK, moe.pes, 128,
                    out=(moe.idx, moe.w, moe.eo, moe.routes, moe.xq, moe.xsa, xqd, xsad))
        bq.ffn_gate_up(moe.xq, moe.xsa, moe.eo, moe.routes, L["gu"], E, T, TOPK, I, xqd, xsad,
                       L["dg"], L["du"], out=(moe.bi8, moe.bsa, gq_, gsa))
        bq.ffn_down(moe.bi8, moe.bsa, moe.eo, moe.routes, L["d"], E, T, TOPK, H, gq_, gsa,
                    L["dd"], 64, workspace=moe.ws, out=(moe.accum, moe.out, od))

    def sliding_layer(L):
        bq.norm_quant(x, gamma, 128, out=(xq, xsa))
        bq.qkv(xq, xsa, L["q"], L["k"], L["v"], outs=(q_s, k_s, v_s))
        bq.block_quant(attn_s, 256, False, out=(oq_s, osa_s))
        bq.block_linear(oq_s, osa_s, L["o"], 256, out=o)
        ffn(L)

    def full_layer(L):
        bq.norm_quant(x, gamma, 128, out=(xq, xsa))
        # q and k (k_eq_v: one projection for K and V), the reference's two
        # dispatch_bq_linear on one activation, as one bq_linear_pair launch
        bq.linear_pair(xq, xsa, L["fq"], L["fk"], outs=(q_f, k_f))
        bq.block_quant(attn_f, 512, False, out=(oq_f, osa_f))
        bq.block_linear(oq_f, osa_f, L["fo"], 512, out=o)
        ffn(L)

    gs_ = graph_of(lambda _i: sliding_layer(base), 1)
    ms_s = time_graph(gs_, 1, steps, 0).p50
    gf_ = graph_of(lambda _i: full_layer(base), 1)
    ms_f = time_graph(gf_, 1, steps, 0).p50
    gm_ = graph_of(lambda _i: moe(), 1)
    ms_m = time_graph(gm_, 1, steps, 0).p50
    del gs_, gf_, gm_
    # The 30-layer stack as one graph, as a decode step runs it: five sliding
    # layers then a full one, five times, each layer on device copies of its
    # own (distinct addresses: no layer finds another's weights in L2 or the
    # Infinity Cache).  One graph launch per step instead of one per layer.
    cp = lambda W: bq.ButterquantWeight(W.data.clone(), W.scale.clone(), W.n_rows, W.k)
    layers = [("f" if j % 6 == 5 else "s", {k: cp(w) for k, w in base.items()
                                          if k in (("fq", "fk", "fo") if j % 6 == 5 else
                                                   ("q", "k", "v", "o")) + ("dg", "du", "dd",
                                                                            "gu", "d")})
              for j in range(30)]
    g_st = graph_of(lambda _i: [(sliding_layer if kd == "s" else full_layer)(L)
                                for kd, L in layers], 1)
    ms_graph = time_graph(g_st, 1, max(5, steps // 4), 0).p50
    del g_st, layers
    torch.cuda.empty_cache()
    stack_ms = 25 * ms_s + 5 * ms_f
    bf = lambda t: t.view(torch.int16).cpu().numpy().view("uint16")
    host.update(x=bf(x), attn_s=bf(attn_s), attn_f=bf(attn_f), moe=moe)
    # algorithmic bytes of one layer call: every weight (codes + per-row
    # scales) read once, the touched experts' weights, and each launch's
    # activations in and out
    wb = lambda n, k: n * k + 4 * n
    nq = lambda k: 2 * T * k + 2 * k + T * k + 4 * T            # norm-quant: bf16 in, int8 + scale out
    lin = lambda n, k, nb=1: T * k + 4 * T * nb + 2 * T * n     # linear: int8 + scales in, bf16 out
    bqz = lambda k, b: 2 * T * k + T * k + 4 * T * (k // b)     # block-quant
    # the dense MLP's norm-quant shares the MoE's read of x (one bq_ffn_prep
    # launch); its gate/up reads the int8 rows and writes the down
    # projection's block-quantized activation (bq_ffn_gate_up)
    mlp = (nq(H) - 2 * T * H + 2 * wb(2112, H) + T * H + 4 * T + T * 2112 + 4 * T * (2112 // 64) +
           wb(H, 2112) + lin(H, 2112, 2112 // 64))
    sliding_b = (nq(H) + wb(4096, H) + wb(2048, H) + wb(2048, H) + lin(8192, H) +
                 bqz(4096, 256) + wb(H, 4096) + lin(H, 4096, 16) + mlp)
    full_b = (nq(H) + wb(8192, H) + wb(1024, H) + lin(9216, H) + bqz(8192, 512) +
              wb(H, 8192) + lin(H, 8192, 16) + mlp)
    eo = moe.eo.cpu().numpy()
    touched = int((eo[1:] - eo[:-1] > 0).sum())
    R = T * TOPK
    moe_b = (touched * (2 * I * H + 2 * I * 4 + H * I + H * 4) + 4 * T * E + nq(H) +
             R * (I + 4 * (I // 64)) * 2 + R * H * 4 * 2 + T * H * (4 + 2))
    return dict(sliding_layer_ms=ms_s, full_layer_ms=ms_f, moe_ms=ms_m,
                stack_ms=stack_ms, stack_tokens_per_s=T / (stack_ms * 1e-3),
                stack_graph_ms=ms_graph, stack_graph_tokens_per_s=T / (ms_graph * 1e-3),
                cpu_inputs=host,
                experts_touched=touched, sliding_bytes=sliding_b + moe_b, full_bytes=full_b + moe_b,
                moe_bytes=moe_b)


def bench_attn(bq, torch, steps):
    """int8-KV attention at the model's shapes (modeling/gemma4_common.mojo):
    sliding layers (16 q heads, 8 kv heads, head_dim 256, window 1024, two
    1024-row ring pages per sequence) and full layers (16 q / 2 kv heads,
    head_dim 512).  Decode: a batch of 16 sequences, one token each, at a
    full window (sliding) or 4096 positions (full); prefill: one 2048-token
    chunk.  Caches are uniform random int8 codes with positive scales;
    every sequence owns its own pages, so a decode batch reads
    16 x L x kv_heads x (2 head_dim + 8) distinct bytes; decode calls rotate
    over cache replicas (>= 640 MB in total) so the KV streams from HBM.  The
    attention prep (per-head RMS, RoPE, FWHT, int8) is timed for the decode
    batch."""
    import numpy as np
    d = "cuda"
    g = torch.Generator(device=d).manual_seed(3)
    res = {}

    def make(nq, nkv, hd, window, seqs, page):
        runs, rows, buf, off, npg = [], [], 0, 0, 0
        for b, n in seqs:
            need = 2 if window else (b + n) // page + 1
            runs.append((buf, b, off, need))
            rows += list(range(npg, npg + need))
            npg, off, buf = npg + need, off + need, buf + n
        T, slots, kvs = buf, npg * page, nkv * hd
        ri = lambda *sh: torch.randint(-127, 128, sh, dtype=torch.int8, device=d, generator=g)
        c = dict(kc=ri(slots, kvs), vc=ri(slots, kvs),
                 ks=torch.rand(slots, nkv, device=d, generator=g) + 1,
                 vs=torch.rand(slots, nkv, device=d, generator=g) + 1,
                 q=ri(T, nq * hd), fq=torch.rand(T, nq, device=d, generator=g) + 1,
                 runs=torch.tensor(runs, dtype=torch.int32, device=d),
                 rows=torch.tensor([x * page for x in rows], dtype=torch.int32, device=d))
        c["qb"] = (c["q"].view(T, nq, hd).int().sum(-1) * 128).float()
        kvbytes = sum(min(window, b + t + 1) if window else b + t + 1
                      for b, n in seqs for t in range(n)) * nkv * (2 * hd + 8)
        return c, T, kvbytes

    shapes = {
        "sliding_decode_b16": (16, 8, 256, 1024, [(3000 + 37 * i, 1) for i in range(16)], 1024),
        "full_decode_b16_ctx4096": (16, 2, 512, 0, [(4095, 1)] * 16, 1024),
        "sliding_prefill_2048": (16, 8, 256, 1024, [(0, 2048)], 1024),
        "full_prefill_2048": (16, 2, 512, 0, [(0, 2048)], 1024),
    }
    for name, (nq, nkv, hd, window, seqs, page) in shapes.items():
        c, T, kvbytes = make(nq, nkv, hd, window, seqs, page)
        decode = T <= 16
        # decode: distinct cache replicas, one call each, so every call reads
        # its KV from HBM (past the 256 MB Infinity Cache) and the graph's
        # launch cost is spread over several calls
        nrep = min(8, max(1, -(-640_000_000 // (2 * c["kc"].numel())))) if decode else 1
        reps = [c] + [dict(c, kc=c["kc"].clone(), vc=c["vc"].clone()) for _ in range(nrep - 1)]
        maxlen = window if window else max(b + n for b, n in seqs)
        s_max = bq.attention_splits(T, nkv, maxlen)
        ws = bq.attention_workspace(T, nq, hd, s_max)
        out = torch.empty(T, nq * hd, dtype=torch.bfloat16, device=d)
        geo = (nq, nkv, hd, window, int(np.log2(page)), page - 1, 1 if window else -1)
        call = lambda i: bq.attention(
            reps[i]["q"], reps[i]["qb"], reps[i]["fq"], reps[i]["kc"], reps[i]["ks"],
            reps[i]["vc"], reps[i]["vs"], reps[i]["runs"], reps[i]["rows"], *geo, s_max=s_max,
            workspace=ws, out=out)
        gr = graph_of(call, nrep)
        ms = time_graph(gr, nrep, 0, 0).p50
        r = {"us": round(ms * 1e3, 2), "s_max": s_max}
        if decode:
            # one token per sequence, each with its own pages: every byte
            # counted is a distinct cache byte
            r.update(kv_bytes_read=kvbytes, kv_GBs=round(kvbytes / (ms * 1e-3) / 1e9, 1))
        else:
            # prefill: every query token reads its own window of the cache, so
            # the per-token sum counts each cache row many times; those
            # re-reads are served from L2 / LDS, not HBM, and the rate is not
            # an HBM bandwidth.  The distinct cache bytes are the HBM figure.
            distinct = T * nkv * (2 * hd + 8)
            r.update(kv_bytes_per_token_sum=kvbytes,
                     kv_GBs_per_token_sum_cache_served=round(kvbytes / (ms * 1e-3) / 1e9, 1),
                     kv_distinct_bytes=distinct,
                     kv_distinct_GBs=round(distinct / (ms * 1e-3) / 1e9, 1))
        if decode:
            r["hbm_frac"] = round(kvbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
            r["cache_replicas"] = nrep
            # the prep of the same batch: q/k/v projections' bf16 rows -> codes + cache rows
            bfr = lambda *sh: torch.randn(*sh, device=d, generator=g).to(torch.bfloat16)
            src = (bfr(T, nq * hd), bfr(T, nkv * hd), bfr(T, nkv * hd))
            gam = (bfr(hd), bfr(hd))
            rope_half = hd // 2 if window else 64
            maxpos = max(b + n for b, n in seqs) + 1
            cos = torch.rand(maxpos, rope_half, device=d, generator=g)
            sin = torch.rand(maxpos, rope_half, device=d, generator=g)
            qo = (torch.empty(T, nq * hd, dtype=torch.int8, device=d),
                  torch.empty(T, nq, device=d), torch.empty(T, nq, device=d))
            sqrt_n = float(np.sqrt(np.float32(hd), dtype=np.float32))
            n_eps = float(np.float32(hd) * np.float32(1e-6))
            gp = graph_of(lambda i: bq.attn_prep(*src, *gam, c["kc"], c["ks"], c["vc"], c["vs"],
                                                 cos, sin, c["runs"], c["rows"], nq, nkv, hd,
                                                 rope_half, hd // 2, int(np.log2(page)),
                                                 page - 1, 1 if window else -1, sqrt_n=sqrt_n,
                                                 n_eps=n_eps, out=qo), 8)
            pms = time_graph(gp, 8, 0, 0).p50
            r["prep_us"] = round(pms * 1e3, 2)
        else:
            # PV is an f32 fma per (position, column) on the vector ALUs
            flops = 2.0 * kvbytes / (2 * hd + 8) * (nq // nkv) * hd * 2
            r["tflops_qk_pv"] = round(flops / (ms * 1e-3) / 1e12, 1)
        res[name] = r
    return res


# ---------------------------------------------------------------------------
def cpu_topology(cap=16):
    """The host's CPUs as the CPU leg uses them: physical cores and NUMA nodes
    of the machine, the CPUs this process may run on, and two pin lists of at
    most `cap` CPUs (the box's CPU share): one CPU per physical core on the
    NUMA node holding most of the allowed cores (the reference's one pinned
    rank), and all allowed CPUs (SMT siblings included) across nodes."""
    import glob
    import re

    def rd(path):
        try:
            with open(path) as f:
                return f.read().strip()
        except OSError:
            return None

    def cpulist(txt):
        out = []
        for part in (txt or "").split(","):
            if "-" in part:
                lo, hi = part.split("-")
                out += range(int(lo), int(hi) + 1)
            elif part:
                out.append(int(part))
        return out

    allowed = sorted(os.sched_getaffinity(0))
    node_dirs = sorted(glob.glob("/sys/devices/system/node/node[0-9]*"),
                       key=lambda d: int(re.sub(r"\D", "", os.path.basename(d))))
    node_of = {}
    for d in node_dirs:
        for c in cpulist(rd(os.path.join(d, "cpulist"))):
            node_of[c] = int(re.sub(r"\D", "", os.path.basename(d)))
    online = cpulist(rd("/sys/devices/system/cpu/online")) or allowed
    core_of = {}
    for c in online:
        t = f"/sys/devices/system/cpu/cpu{c}/topology/"
        core_of[c] = (rd(t + "physical_package_id"), rd(t + "core_id"))
    by_node, seen = {}, set()
    for c in allowed:
        k = core_of.get(c, (None, c))
        if k in seen:
            continue
        seen.add(k)
        by_node.setdefault(node_of.get(c, 0), []).append(c)
    node = max(by_node, key=lambda n: len(by_node[n]))
    model = None
    for line in (rd("/proc/cpuinfo") or "").splitlines():
        if line.startswith("model name"):
            model = line.split(":", 1)[1].strip()
            break
    return dict(cpu_model=model, logical_cpus_online=len(online),
                physical_cores=len(set(core_of.values())), numa_nodes=max(1, len(node_dirs)),
                allowed_logical_cpus=len(allowed), allowed_physical_cores=len(seen),
                node=node, node_pin=by_node[node][:cap], all_pin=allowed[:cap])


def _cpu_samples(call, seconds, warm=30, cap=600):
    """30 warmup calls (fewer if one call is long), then up to 600 timed calls
    within about `seconds` (at least 2) -> (p50 s, min s, samples)."""
    import numpy as np
    t_end = time.perf_counter() + seconds / 4
    for i in range(warm):
        call()
        if time.perf_counter() > t_end:
            break
    ts = []
    t_end = time.perf_counter() + seconds
    while (time.perf_counter() < t_end and len(ts) < cap) or len(ts) < 2:
        t0 = time.perf_counter()
        call()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), float(min(ts)), len(ts)


def l3_bytes(cpus):
    """Total L3 of the distinct L3 instances serving `cpus` (sysfs cache
    index3: size and shared_cpu_list), or None if sysfs does not say."""
    seen, total = set(), 0
    for c in cpus:
        d = f"/sys/devices/system/cpu/cpu{c}/cache/index3/"
        try:
            with open(d + "shared_cpu_list") as f:
                key = f.read().strip()
            with open(d + "size") as f:
                txt = f.read().strip()
        except OSError:
            return None
        if key in seen:
            continue
        seen.add(key)
        mult = {"K": 1 << 10, "M": 1 << 20, "G": 1 << 30}.get(txt[-1:].upper(), 1)
        total += int(txt.rstrip("KMGkmg")) * mult
    return total or None


def cpu_baseline_gemv(codes, scales, xq, sa, seconds, topo):
    """The reference CPU path (VNNI u8 x i8 with colsums, 32-row tiles over
    worker_range, matmul_workers threads), ported to C in
    oracle/cpu_baseline.c, on the host cores: the same decode GEMV (M=1,
    K=N=4096) on the GPU run's own weight codes and quantized activation.
    Like the GPU leg, consecutive calls rotate over weight replicas, here
    enough that the bytes touched between two uses of a replica are at least
    twice the L3 that serves the pinned CPUs (read from sysfs), so each call
    streams its weights from DRAM.  First with threads pinned one per
    physical core of one NUMA node (the value), then on all allowed CPUs."""
    import ctypes as C

    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    lib = O.cpu()
    q = codes.cpu().numpy()
    s = scales.cpu().numpy().astype(np.float32)
    N, K = q.shape
    p, cs = O.pack_and_colsum(q)
    xq = xq.cpu().numpy().reshape(1, K)
    sa = sa.cpu().numpy().astype(np.float32).reshape(1)
    out = np.empty((1, N), np.uint16)
    ptr = lambda a: a.ctypes.data_as(C.c_void_p)
    alg_bytes = N * K + N * 4 + K + 4 + N * 2
    legs = {}
    for leg, pins in (("node", topo["node_pin"]), ("all", topo["all_pin"])):
        O.cpu_pin(pins)
        n = len(pins)
        l3 = l3_bytes(pins)
        reps = min(128, max(2, 1 + -(-2 * (l3 or (256 << 20)) // p.nbytes)))
        pool = np.empty((reps, p.size), np.int8)
        pool[:] = p
        wp = [ptr(pool[i]) for i in range(reps)]
        it = [0]

        def call():
            i = it[0] = (it[0] + 1) % reps
            lib.bqcpu_linear(ptr(xq), ptr(sa), 1, wp[i], ptr(s), ptr(cs), N, K, ptr(out), n)
        med, mn, cnt = _cpu_samples(call, seconds / 2)
        cached = _cpu_samples(
            lambda: lib.bqcpu_linear(ptr(xq), ptr(sa), 1, wp[0], ptr(s), ptr(cs), N, K, ptr(out),
                                     n), seconds / 4)
        del pool
        legs[leg] = dict(value=round(alg_bytes / med / 1e9, 2), p50_us=round(med * 1e6, 1),
                         min_us=round(mn * 1e6, 1), best_GBs=round(alg_bytes / mn / 1e9, 2),
                         samples=cnt, threads=n, cpus=pins, weight_replicas=reps,
                         l3_bytes_of_pinned_cpus=l3,
                         one_replica_GBs=round(alg_bytes / cached[0] / 1e9, 2))
    nd = legs["node"]
    return dict(value=nd["value"], unit="GB/s", cores=nd["threads"], kind="port",
                sample=f"decode GEMV M=1 K=N=4096 on the GPU run's codes and activation, "
                       f"rotated over {nd['weight_replicas']} weight replicas (>= 2x the "
                       f"{nd['l3_bytes_of_pinned_cpus']} B of L3 serving the pinned CPUs) so "
                       f"the weights stream from DRAM; p50 of {nd['samples']} calls after 30 "
                       f"warmups, {nd['threads']} threads pinned one per physical core on NUMA "
                       f"node {topo['node']}; ISA {lib.bqcpu_isa().decode()}; gcc -O3 -fopenmp, "
                       f"OMP_WAIT_POLICY={os.environ.get('OMP_WAIT_POLICY')}",
                p50_us=nd["p50_us"], min_us=nd["min_us"], all_cpus=legs["all"],
                topology={k: topo[k] for k in ("cpu_model", "physical_cores", "numa_nodes",
                                               "logical_cpus_online", "allowed_logical_cpus",
                                               "allowed_physical_cores")})


def cpu_baseline_prefill(codes, scales, xq, sa, seconds, topo):
    """The reference CPU path of the prefill linear (M=512, K=N=4096;
    dispatch_bq_linear's VNNI branch, the one an EPYC host takes: no AMX)
    on the GPU run's own weight codes and quantized activation, both legs as
    the GEMV's.  int8 TOP/s = 2*M*N*K / p50."""
    import ctypes as C

    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    lib = O.cpu()
    q = codes.cpu().numpy()
    s_ = scales.cpu().numpy().astype(np.float32)
    N, K = q.shape
    p, cs = O.pack_and_colsum(q)
    xq = np.ascontiguousarray(xq.cpu().numpy())
    sa = np.ascontiguousarray(sa.cpu().numpy().astype(np.float32))
    M = xq.shape[0]
    out = np.empty((M, N), np.uint16)
    ptr = lambda a: a.ctypes.data_as(C.c_void_p)
    ops = 2.0 * M * N * K
    legs = {}
    for leg, pins in (("node", topo["node_pin"]), ("all", topo["all_pin"])):
        O.cpu_pin(pins)
        med, mn, cnt = _cpu_samples(
            lambda: lib.bqcpu_linear(ptr(xq), ptr(sa), M, ptr(p), ptr(s_), ptr(cs), N, K,
                                     ptr(out), len(pins)), seconds / 2)
        legs[leg] = dict(tops=round(ops / med / 1e12, 3), p50_ms=round(med * 1e3, 3),
                         min_ms=round(mn * 1e3, 3), samples=cnt, threads=len(pins))
    nd = legs["node"]
    return dict(value=nd["tops"], unit="TOP/s", cores=nd["threads"], kind="port",
                sample=f"prefill linear M=512 K=N=4096 on the GPU run's codes and activation; "
                       f"p50 of {nd['samples']} calls, {nd['threads']} threads pinned one per "
                       f"physical core on NUMA node {topo['node']}; ISA "
                       f"{lib.bqcpu_isa().decode()}", p50_ms=nd["p50_ms"], all_cpus=legs["all"])


def cpu_baseline_layer16(bq, torch, host, Wgu, Wd, seconds, topo):
    """The reference CPU path of the batch-16 decoder layer's quantized
    projections, in the reference's calls (gemma_4_moe_bq.mojo:418-627,
    716-805): norm-quant, q|k|v as one linear over the concatenated tiles
    (dispatch_bq_qkv), block-quant + o_proj, norm-quant, gate|up, FWHT64
    block-quant + down, and the 128-expert MoE layer (bqcpu_moe_layer) -- on
    the GPU run's own weights and inputs; sliding and full layers, both legs
    as the GEMV's; stack = 25 sliding + 5 full layers."""
    import ctypes as C

    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    lib = O.cpu()
    T = 16
    ptr = lambda a: a.ctypes.data_as(C.c_void_p)

    def packed(*names):
        """VNNI-packed weights of one or more row-concatenated projections."""
        qs = [host[n][0] for n in names]
        q = np.concatenate(qs) if len(qs) > 1 else qs[0]
        b = host[names[0]][2]
        blk = q.shape[1] if b == 128 else b   # per-row weights carry one colsum block
        p, cs = O.pack_and_colsum(q, None if b == 128 else blk, b == 128)
        sc = np.concatenate([host[n][1] for n in names]).astype(np.float32)
        return p, sc, cs, q.shape[0], q.shape[1], b
    W = {k: packed(*v) for k, v in (("sqkv", ("sq", "sk", "sv")), ("so", ("so",)),
                                    ("fqk", ("fq", "fk")), ("fo", ("fo",)),
                                    ("dgu", ("dg", "du")), ("dd", ("dd",)))}
    gamma = np.full(H, 0x3F80, np.uint16)
    sqrt_n, n_eps = O.norm_consts(H)
    x, attn = host["x"], {"s": host["attn_s"], "f": host["attn_f"]}
    xq, xsa = np.empty((T, H), np.int8), np.empty(T, np.float32)
    bufs = {}

    def lin(key, act, sa, nt):
        p, sc, cs, n, k, b = W[key]
        out = bufs.setdefault(key, np.empty((T, n), np.uint16))
        if b == 128:
            lib.bqcpu_linear(ptr(act), ptr(sa), T, ptr(p), ptr(sc), ptr(cs), n, k, ptr(out), nt)
        else:
            lib.bqcpu_block_linear(ptr(act), ptr(sa), T, ptr(p), ptr(sc), ptr(cs), n, k, b,
                                   ptr(out), nt)
        return out

    def bquant(src, block, fwht, nt):
        rows, cols = src.shape
        q_ = bufs.setdefault(("q", cols, block), np.empty((rows, cols), np.int8))
        s_ = bufs.setdefault(("s", cols, block), np.empty((rows, cols // block), np.float32))
        lib.bqcpu_block_quant(ptr(src), ptr(q_), ptr(s_), rows, cols, block, int(fwht), nt)
        return q_, s_

    def nquant(nt):
        lib.bqcpu_norm_quant(ptr(x), ptr(gamma), ptr(xq), ptr(xsa), T, H, 128,
                             C.c_float(sqrt_n), C.c_float(n_eps), nt)

    moe = host["moe"]
    gu = bq.unpack(Wgu.data, Wgu.n_rows, Wgu.k).cpu().numpy().reshape(Wgu.n_rows, Wgu.k)
    dn = bq.unpack(Wd.data, Wd.n_rows, Wd.k).cpu().numpy().reshape(Wd.n_rows, Wd.k)
    gp, gcs = O.pack_and_colsum(gu)
    dp, dcs = O.pack_and_colsum(dn, 64, False)
    del gu, dn
    cl = O.CpuMoeLayer(T, E, TOPK, H, I, gp, Wgu.scale.cpu().numpy(), gcs, dp,
                       Wd.scale.cpu().numpy(), dcs)
    mx = moe.x.view(torch.int16).cpu().numpy().view(np.uint16)
    lg = moe.logits.cpu().numpy()
    pes = np.full(E, 0x3F80, np.uint16)

    def layer(kind, nt):
        nquant(nt)
        lin("sqkv" if kind == "s" else "fqk", xq, xsa, nt)
        oq, osa = bquant(attn[kind], 256 if kind == "s" else 512, False, nt)
        lin("so" if kind == "s" else "fo", oq, osa, nt)
        nquant(nt)                                  # the FFN's own norm-quant
        gu_out = lin("dgu", xq, xsa, nt)
        gq, gsa = bquant(np.ascontiguousarray(gu_out[:, :2112]), 64, True, nt)
        lin("dd", gq, gsa, nt)
        cl(lg, mx, gamma, pes, nt)
    legs = {}
    for leg, pins in (("node", topo["node_pin"]), ("all", topo["all_pin"])):
        O.cpu_pin(pins)
        r = {}
        for kind in ("s", "f"):
            med, mn, cnt = _cpu_samples(lambda: layer(kind, len(pins)), seconds / 4)
            r[kind] = (med, mn, cnt)
        stack = 25 * r["s"][0] + 5 * r["f"][0]
        legs[leg] = dict(sliding_p50_ms=round(r["s"][0] * 1e3, 3),
                         full_p50_ms=round(r["f"][0] * 1e3, 3), stack_ms=round(stack * 1e3, 2),
                         stack_tokens_per_s=round(T / stack, 1), samples=r["s"][2],
                         threads=len(pins))
    nd = legs["node"]
    return dict(value=nd["stack_tokens_per_s"], unit="tokens/s", cores=nd["threads"],
                kind="port",
                sample=f"all quantized projections + MoE of one decoder layer at decode batch 16 "
                       f"(sliding and full), the GPU run's weights and inputs; p50 of "
                       f"{nd['samples']} layers, {nd['threads']} threads pinned one per physical "
                       f"core on NUMA node {topo['node']}; stack = 25 sliding + 5 full",
                **{k: v for k, v in nd.items() if k not in ("samples", "threads")},
                all_cpus=legs["all"])


def cpu_baseline_moe(bq, torch, Wgu, Wd, layers, seconds, topo):
    """The reference CPU path of the whole MoE layer (bqcpu_moe_layer in
    oracle/cpu_baseline.c: router top-k + softmax merge, CSR schedule,
    norm-quant, phase 1 over intermediate tiles, FWHT64 block-quant, phase 2
    over hidden tiles; VNNI u8 x i8 with colsums; the reference's worker
    policies), on each timed GPU layer's own hidden states, router logits and
    expert weights, threads pinned one per physical core of one NUMA node,
    then on all allowed CPUs; about `seconds` per T and leg."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    lib = O.cpu()
    gu = bq.unpack(Wgu.data, Wgu.n_rows, Wgu.k).cpu().numpy().reshape(Wgu.n_rows, Wgu.k)
    dn = bq.unpack(Wd.data, Wd.n_rows, Wd.k).cpu().numpy().reshape(Wd.n_rows, Wd.k)
    gp, gcs = O.pack_and_colsum(gu)
    dp, dcs = O.pack_and_colsum(dn, 64, False)
    del gu, dn
    gsc = Wgu.scale.cpu().numpy()
    dsc = Wd.scale.cpu().numpy()
    gamma = np.full(H, 0x3F80, np.uint16)
    pes = np.full(E, 0x3F80, np.uint16)
    res = {}
    for layer in layers:
        T = layer.T
        x = layer.x.view(torch.int16).cpu().numpy().view(np.uint16)
        logits = layer.logits.cpu().numpy()
        cl = O.CpuMoeLayer(T, E, TOPK, H, I, gp, gsc, gcs, dp, dsc, dcs)
        r = {}
        for leg, pins in (("node", topo["node_pin"]), ("all", topo["all_pin"])):
            O.cpu_pin(pins)
            med, mn, cnt = _cpu_samples(lambda: cl(logits, x, gamma, pes, len(pins)), seconds / 2)
            r[leg] = {"tokens_per_s": round(T / med, 1), "p50_ms": round(med * 1e3, 3),
                      "min_ms": round(mn * 1e3, 3), "samples": cnt, "threads": len(pins)}
        res[f"T{T}"] = r
    res.update(unit="tokens/s", cores=len(topo["node_pin"]), kind="port",
               sample=f"whole MoE layer from router logits (128 experts, top-8, H={H}, I={I}) "
                      f"on the GPU run's inputs; p50 (and min) of up to 600 calls after up to 30 "
                      f"warmups, ~{seconds / 2:.0f} s per T and leg; 'node': threads pinned one "
                      f"per physical core of NUMA node {topo['node']}, 'all': every allowed CPU "
                      f"(at most 16, the box's CPU share); ISA {lib.bqcpu_isa().decode()}; "
                      f"OMP_WAIT_POLICY={os.environ.get('OMP_WAIT_POLICY')}")
    return res


def calib_copy(torch):
    """A plain device copy of 256 MiB (the PMC calibration kernel)."""
    a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()


def launch_histogram(path, reps=64):
    """Per-launch durations of the GEMV (k_gemv_m1 or k_linear_skinny) and
    k_stream_read from a rocprofv3 kernel trace of `bench.py --workload gemv`:
    for each kernel the longest run of back-to-back dispatches of it alone
    (the pure GEMV graph and the streaming-read graph, eager warm calls
    included), its
    percentiles, a histogram, the spread of per-replica medians (dispatch i
    of a run reads replica i mod 64) and the position of the slow launches
    inside each 64-launch replay."""
    import csv

    import numpy as np
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    out = []
    for key in ("k_gemv_m1", "k_linear_skinny", "k_stream_read"):
        best, cur = [], []
        for st, en, name in rows:
            if key in name:
                cur.append((st, en))
            else:
                if len(cur) > len(best):
                    best = cur
                cur = []
        if len(cur) > len(best):
            best = cur
        if not best:
            continue
        st = np.array([b[0] for b in best], np.float64)
        en = np.array([b[1] for b in best], np.float64)
        d = (en - st) / 1e3
        gap = (st[1:] - en[:-1]) / 1e3
        n = len(d) - len(d) % reps
        pos = np.arange(len(d)) % reps
        per_rep = np.array([np.median(d[:n][pos[:n] == i]) for i in range(reps)])
        pct = lambda q: float(np.percentile(d, q))
        out.append(f"== {key}: {len(d)} back-to-back launches")
        out.append(f"duration us: min {d.min():.2f}  p10 {pct(10):.2f}  p50 {pct(50):.2f}  "
                   f"mean {d.mean():.2f}  p90 {pct(90):.2f}  p99 {pct(99):.2f}  max {d.max():.2f}")
        out.append(f"gap to the previous launch us: p50 {np.median(gap):.2f}  "
                   f"p90 {np.percentile(gap, 90):.2f}  max {gap.max():.2f}")
        edges = np.arange(np.floor(d.min() * 4) / 4, d.max() + 0.25, 0.25)
        h, e = np.histogram(d, bins=edges)
        out.append("histogram (0.25 us bins):")
        for c, lo in zip(h, e):
            if c:
                out.append(f"  {lo:5.2f}-{lo + 0.25:5.2f} us  {c:7d}  {'#' * max(1, int(60 * c / h.max()))}")
        out.append(f"per-replica medians us: min {per_rep.min():.2f} (replica {per_rep.argmin()})  "
                   f"max {per_rep.max():.2f} (replica {per_rep.argmax()})  "
                   f"spread {per_rep.max() - per_rep.min():.2f}")
        slow = d >= np.sort(d)[int(0.9 * (len(d) - 1))]
        out.append("slowest decile by position in the 64-launch replay: first launch "
                   f"{(slow & (pos == 0)).sum()}, launches 1-7 {(slow & (pos >= 1) & (pos < 8)).sum()}, "
                   f"8-63 {(slow & (pos >= 8)).sum()}")
        out.append(f"first launch of a replay: p50 {np.median(d[pos == 0]):.2f} us; "
                   f"others p50 {np.median(d[pos != 0]):.2f} us")
    return "\n".join(out)


def main():
    args = parse()
    global SAMPLES, WARMUP
    SAMPLES = max(1, args.samples)
    WARMUP = min(WARMUP, SAMPLES)
    # the CPU legs' OpenMP team sleeps between parallel regions instead of
    # spinning: on a box whose CPU share equals the team size, spinning
    # threads exhaust the share and the process is throttled (the 32-token
    # MoE layer measured 290 ms spinning, 15.6 ms sleeping).  Read by libgomp
    # when the CPU port first loads, which is after this point.
    os.environ.setdefault("OMP_WAIT_POLICY", "PASSIVE")
    if args.launch_histogram:
        print(launch_histogram(args.launch_histogram))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not built)"}))
        sys.exit(2)
    import torch
    import bq
    bq.init(0)
    wl = args.workload
    res = {}
    if wl in ("all", "gemv"):
        res["gemv"] = bench_gemv(bq, torch, args.steps, args.warmup)
    if wl in ("all", "prefill"):
        res["prefill"] = bench_prefill(bq, torch, args.steps, args.warmup)
    if wl in ("all", "moe32", "moe2048", "layer16"):
        Wgu, Wd = moe_weights(bq, torch)
        moe_w = (Wgu, Wd)
        reps = [(Wgu, Wd), tuple(bq.ButterquantWeight(w.data.clone(), w.scale, w.n_rows, w.k)
                                 for w in (Wgu, Wd))]
        if wl in ("all", "moe32"):
            res["moe32"] = bench_moe(bq, torch, 32, reps, max(20, args.steps // 16))
        if wl in ("all", "moe2048"):
            res["moe2048"] = bench_moe(bq, torch, 2048, reps, max(10, args.steps // 32))
        if wl in ("all", "layer16"):
            res["layer16"] = bench_layer16(bq, torch, Wgu, Wd, max(10, args.steps // 32))
    if wl in ("all", "head"):
        res["head"] = bench_head(bq, torch, args.steps)
    if wl in ("all", "attn"):
        res["attn"] = bench_attn(bq, torch, args.steps)
    if wl == "load":
        res["load"] = bench_load(bq, torch)
    if wl == "stream_sweep":
        # the launch-shape sweep alone, over 64 replicas of the GEMV's 16 MiB
        pool = torch.randint(-127, 128, (64, 4096 * 4096), dtype=torch.int8, device="cuda")
        res["stream_sweep"] = bench_stream_sweep(torch, [pool[i] for i in range(64)], 256)
    if wl in ("all", "gemv", "mfma"):
        res["mfma"] = bench_mfma(torch)
    if wl in ("all", "mfma", "stream_sweep"):
        res["probes"] = bench_probes(torch)
    if args.calib_copy:
        calib_copy(torch)

    mf = res.get("mfma", {}).get("v_mfma_i32_16x16x64_i8", {}).get("best_TOPs")
    line = {
        "metric": "bq GEMV HBM GB/s (% peak); MoE-layer tokens/s at 32 and 2048 tokens",
        "unit": "GB/s", "n_gpus": 1, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
    }
    if "gemv" in res:
        gv = res["gemv"]
        smp = gv["s"]
        line.update(value=round(gv["gbs"], 1), steps=smp.launches, steps_requested=args.steps,
                    warmup=args.warmup, ms_per_step=round(smp.p50, 6),
                    config={"workload": "decode GEMV: per-row butterquant linear, M=1 token, "
                                        "K=4096, N=4096, int8 codes x int8 activation, "
                                        "fp32 accumulate -> bf16; 64 weight replicas (1 GiB) "
                                        "rotated", "global_batch": 1, "seq_len": 1,
                            "parallelism": "single GPU"},
                    pct_hbm_peak=round(100 * gv["gbs"] / HBM_PEAK_GBS, 1),
                    roofline={"bound": "hbm", "achieved": round(gv["gbs"], 1),
                              "peak": HBM_PEAK_GBS, "unit": "GB/s",
                              "frac": round(gv["gbs"] / HBM_PEAK_GBS, 4),
                              "traffic": _traffic("gemv_decode_k4096_n4096_traffic.txt"),
                              "measured_peak": round(gv["rd"]["gbs"], 1),
                              "frac_of_measured": round(gv["gbs"] / gv["rd"]["gbs"], 4),
                              "basis": "achieved = algorithmic bytes per launch (weights, "
                                       "scales, activation, output) / p50 launch time over "
                                       f"{len(smp.ms)} graph replays of 64 launches; "
                                       "measured_peak = the same-launch-shape streaming read "
                                       "of the same replicas (p50)"})
        line["gemv_detail"] = {"kernel": gemv_kernel()[0],
                               "alg_bytes_per_launch": gv["alg_bytes"],
                               "best_GBs": round(gv["gbs_min"], 1), **smp.summary(),
                               "norm_quant": gv["s_nq"].summary(),
                               "linear_with_prep": gv["s_lin"].summary(),
                               "linear_with_prep_fused": {
                                   "kernel": "k_norm_linear_skinny (bq_norm_linear)",
                                   **gv["s_fused"].summary()}}
        rd = gv["rd"]
        line["stream_read_same_shape"] = {
            "kernel": f"k_stream_read (256 workgroups x {gemv_waves()} waves, one-shot non-temporal 16-byte "
                      f"loads of each wave's {64 // gemv_waves()} KiB slice; the GEMV's launch without "
                      "arithmetic)",
            "bytes_per_launch": rd["bytes"], "p50_GBs": round(rd["gbs"], 1),
            "best_GBs": round(rd["gbs_best"], 1),
            "frac_of_datasheet": round(rd["gbs"] / HBM_PEAK_GBS, 4), **rd["same"].summary(),
            "empty_launch_p50_us": round(rd["empty"].p50 * 1e3, 3),
            "read_256MiB_per_launch": {"p50_us": round(rd["large"].p50 * 1e3, 2),
                                       "p50_GBs": round(rd["large_gbs"], 1),
                                       "incremental_GBs_16_to_256MiB": round(rd["incr_gbs"], 1)},
            "launch_shape_sweep": rd["sweep"]}
    else:
        line.update(value=None, steps=0, steps_requested=args.steps, warmup=args.warmup,
                    ms_per_step=None, config={"workload": wl})
    if "mfma" in res:
        line["mfma_i8_measured"] = res["mfma"]
    if "probes" in res:
        line["measured_ceilings"] = res["probes"]
    if "prefill" in res:
        p = res["prefill"]
        line["prefill_gemm_m512"] = {
            "tops": round(p["tops"], 1), "int8_mfma_frac": round(p["int8_frac"], 4),
            "bf16_mfma_frac": round(p["bf16_frac"], 4), **p["s"].summary(),
            "roofline": {"bound": "mfma", "achieved": round(p["tops"], 1),
                         "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
                         "frac": round(p["int8_frac"], 4),
                         "traffic": _traffic("prefill_gemm_m512_k4096_n4096_stats.txt"),
                         "measured_peak": mf,
                         "frac_of_measured": round(p["tops"] / mf, 4) if mf else None,
                         "basis": "2*M*N*K int8 ops / p50 launch time; peak = dense int8 MFMA"},
            "vendor_same_shape": p["vendor"]}
    for key in ("moe32", "moe2048"):
        if key in res:
            m = res[key]
            T = m["T"]
            ms = m["ms"]
            tops = m["ops"] / (ms * 1e-3) / 1e12
            wgbs = m["hbm_gbs_weights"]
            d = {"tokens_per_s": round(m["tokens_per_s"], 1), "ms": round(ms, 4),
                 "experts_touched": m["experts_touched"],
                 "weight_GBs": round(wgbs, 1), "hbm_frac_weights": round(wgbs / HBM_PEAK_GBS, 4),
                 "int8_tops": round(tops, 1), **m["s"].summary()}
            traffic = _traffic(f"moe_layer_t{T}_stats.txt")
            if T >= 2048:
                # this layer is judged as a fraction of the matching MFMA
                # peak; its weights are bf16 models computed at int8, so
                # dense bf16 is the declared matching peak
                d["roofline"] = {
                    "bound": "mfma", "achieved": round(tops, 1), "peak": BF16_PEAK_TFLOPS,
                    "unit": "TOP/s", "frac": round(tops / BF16_PEAK_TFLOPS, 4),
                    "traffic": traffic, "declared_matching_peak": "dense bf16 MFMA 2.5 PFLOP/s",
                    "int8_peak_frac": round(tops / INT8_PEAK_TOPS, 4),
                    "hbm_roof_TOPs": round(min(INT8_PEAK_TOPS, HBM_PEAK_GBS * 1e9 * m["ops"] /
                                               m["weight_bytes"] / 1e12), 1),
                    "basis": "2*T*top_k*(2*I*H + H*I) ops / p50 layer time"}
            else:
                d["roofline"] = {
                    "bound": "hbm", "achieved": round(wgbs, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(wgbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                    "basis": "touched experts' weight and scale bytes / p50 layer time"}
            line[f"moe_layer_T{T}"] = d
    if "layer16" in res:
        l16 = res["layer16"]
        line["decoder_layer_b16"] = {k: round(v, 4) for k, v in l16.items()
                                     if k not in ("cpu_inputs", "sliding_bytes", "full_bytes",
                                                  "moe_bytes", "experts_touched")}
        gbs = lambda b, ms: b / (ms * 1e-3) / 1e9
        s_gbs = gbs(l16["sliding_bytes"], l16["sliding_layer_ms"])
        line["decoder_layer_b16"]["experts_touched"] = l16["experts_touched"]
        line["decoder_layer_b16"]["roofline"] = {
            "bound": "hbm", "achieved": round(s_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(s_gbs / HBM_PEAK_GBS, 4),
            "traffic": _traffic("decoder_layer_b16_traffic.txt"),
            "alg_bytes": l16["sliding_bytes"],
            "full_layer_GBs": round(gbs(l16["full_bytes"], l16["full_layer_ms"]), 1),
            "full_layer_alg_bytes": l16["full_bytes"],
            "moe_GBs": round(gbs(l16["moe_bytes"], l16["moe_ms"]), 1),
            "basis": "sliding layer: every projection's weights once, the touched experts' "
                     "weights, each launch's activations in and out / p50 layer time"}
        if "attn" in res:
            # the same stack with each layer's attention step (prep + int8-KV
            # attention at decode batch 16: sliding layers at a full 1024
            # window, full layers at 4096 positions)
            a = res["attn"]
            sl = (a["sliding_decode_b16"]["us"] + a["sliding_decode_b16"]["prep_us"]) * 1e-3
            fl = (a["full_decode_b16_ctx4096"]["us"] + a["full_decode_b16_ctx4096"]["prep_us"]) * 1e-3
            l16 = res["layer16"]
            stack = 25 * (l16["sliding_layer_ms"] + sl) + 5 * (l16["full_layer_ms"] + fl)
            line["decoder_layer_b16"]["stack_with_attention_ms"] = round(stack, 4)
            line["decoder_layer_b16"]["stack_with_attention_tokens_per_s"] = round(16 / (stack * 1e-3), 1)
            # the one-graph stack plus each layer's attention step
            sg = l16["stack_graph_ms"] + 25 * sl + 5 * fl
            line["decoder_layer_b16"]["stack_graph_with_attention_ms"] = round(sg, 4)
            line["decoder_layer_b16"]["stack_graph_with_attention_tokens_per_s"] = round(16 / (sg * 1e-3), 1)
    if "stream_sweep" in res:
        line["launch_shape_sweep"] = res["stream_sweep"]
    if "load" in res:
        ld = res["load"]
        line["load_safetensors_gate_up_507MB"] = {"ms": round(ld["ms"], 2),
                                                  "GBs": round(ld["gbs"], 2),
                                                  "checked": ld["checked"]}
    if "head" in res:
        hd = res["head"]
        line["head_flash_sample_v262144"] = {
            f"rows{R}": {"us": round(v["ms"] * 1e3, 1), "weight_GBs": round(v["gbs"], 1),
                         "hbm_frac": round(v["gbs"] / HBM_PEAK_GBS, 4),
                         "min_us": round(v["s"].min * 1e3, 1), "samples": len(v["s"].ms)}
            for R, v in hd["rows"].items()}
        line["head_flash_sample_v262144"]["alg_bytes"] = hd["alg_bytes"]
    if "attn" in res:
        line["attention_int8_kv"] = res["attn"]
    if not args.no_cpu and ("gemv" in res or "prefill" in res or MOE_LAYERS):
        topo = cpu_topology()
        if "gemv" in res:
            gv = res["gemv"]
            line["cpu_baseline"] = cpu_baseline_gemv(gv["codes"], gv["scales"], gv["xq"], gv["sa"],
                                                     args.cpu_seconds, topo)
        if "prefill" in res:
            line["cpu_baseline_prefill"] = cpu_baseline_prefill(*res["prefill"]["cpu_inputs"],
                                                                args.cpu_seconds, topo)
        if MOE_LAYERS:
            line["cpu_baseline_moe"] = cpu_baseline_moe(bq, torch, *moe_w, MOE_LAYERS,
                                                        args.cpu_seconds, topo)
        if "layer16" in res:
            line["cpu_baseline_layer16"] = cpu_baseline_layer16(
                bq, torch, res["layer16"]["cpu_inputs"], *moe_w, args.cpu_seconds, topo)
    print(json.dumps(line))


def _traffic(name):
    """HBM bytes per launch (or layer call) from a committed rocprofv3 PMC
    summary under profiles/ (FETCH_SIZE + WRITE_SIZE, scaled by the
    plain-copy calibration), or None."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.startswith(("traffic_bytes_per_launch:", "traffic_bytes_per_call:")):
                return int(float(line.split(":")[1]))
    except OSError:
        pass
    return None


if __name__ == "__main__":
    main()
