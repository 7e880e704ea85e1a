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
replayed, so host launch overhead does not stretch the timed region.
Timing uses HIP events on the stream the kernels run on, bracketed by
device synchronizations.  Data: synthetic, bf16 N(0, 0.02) weights (seed 0)
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
                             "attn", "load"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a plain 256 MiB device copy (PMC calibration kernel)")
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


def time_graph(g, per_replay, steps, warmup):
    """Replay graph g until >= steps calls were timed; -> (ms per call, wall s)."""
    import torch
    reps = max(1, -(-steps // per_replay))
    wreps = max(1, -(-warmup // per_replay))
    for _ in range(wreps):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) / (reps * per_replay), wall, reps * per_replay


def quantized(bq, torch, n, k, block, gen):
    w = (torch.randn(n, k, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    codes, scales = bq.quantize_weight(w, block)
    tiled = bq.retile(codes.view(-1), n, k)
    return codes, scales, bq.ButterquantWeight(tiled, scales, n, k)


# ---------------------------------------------------------------------------
def bench_gemv(bq, torch, steps, warmup, reps=64):
    N = K = 4096
    gen = torch.Generator(device="cuda").manual_seed(0)
    codes, scales, W0 = quantized(bq, torch, N, K, 128, gen)
    replicas = [W0] + [bq.ButterquantWeight(W0.data.clone(), scales.clone(), N, K)
                       for _ in range(reps - 1)]
    xg = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(1, K, generator=xg, device="cuda").to(torch.bfloat16)
    gamma = torch.ones(K, dtype=torch.bfloat16, device="cuda")
    xq, sa = bq.norm_quant(x, gamma, 128)
    out = torch.empty(1, N, dtype=torch.bfloat16, device="cuda")
    g = graph_of(lambda i: bq.linear(xq, sa, replicas[i], out=out), reps)
    ms, wall, n = time_graph(g, reps, steps, warmup)
    alg_bytes = N * K + N * 4 + K + 4 + N * 2       # W + sw + x_i8 + sa + y
    # activation prep (norm-quant: RMS, FWHT128, int8) and the full decode linear
    gq = graph_of(lambda i: bq.norm_quant(x, gamma, 128, out=(xq, sa)), 64)
    ms_nq, _, _ = time_graph(gq, 64, 256, 64)
    gl = graph_of(lambda i: (bq.norm_quant(x, gamma, 128, out=(xq, sa)),
                             bq.linear(xq, sa, replicas[i], out=out)), reps)
    ms_lin, _, _ = time_graph(gl, reps, 256, 64)
    return dict(ms=ms, wall=wall, calls=n, alg_bytes=alg_bytes,
                gbs=alg_bytes / (ms * 1e-3) / 1e9, norm_quant_us=ms_nq * 1e3,
                linear_with_prep_us=ms_lin * 1e3, codes=codes, scales=scales)


def bench_prefill(bq, torch, steps, warmup, reps=32):
    M, N, K = 512, 4096, 4096
    gen = torch.Generator(device="cuda").manual_seed(0)
    _, scales, W0 = quantized(bq, torch, N, K, 128, gen)
    replicas = [W0] + [bq.ButterquantWeight(W0.data.clone(), scales, N, K) for _ in range(reps - 1)]
    xg = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(M, K, generator=xg, device="cuda").to(torch.bfloat16)
    xq, sa = bq.norm_quant(x, torch.ones(K, dtype=torch.bfloat16, device="cuda"), 128)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    g = graph_of(lambda i: bq.linear(xq, sa, replicas[i], out=out), reps)
    ms, wall, n = time_graph(g, reps, max(64, steps // 8), max(32, warmup // 4))
    ops = 2.0 * M * N * K
    tops = ops / (ms * 1e-3) / 1e12
    return dict(ms=ms, tops=tops, int8_frac=tops / INT8_PEAK_TOPS, bf16_frac=tops / BF16_PEAK_TFLOPS,
                alg_bytes=N * K + N * 4 + M * K + M * 4 + M * N * 2)


class MoeLayer:
    """One quantized MoE expert layer from router logits: top-8 + softmax
    routing -> norm-quant -> CSR schedule -> phase 1 (gate/up + GELU) with
    the FWHT64 block-quant of the bucket fused -> phase 2 (down +
    route-weighted, expert-ordered combine)."""

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

    def __call__(self, _i=0, fused=True):
        bq, T = self.bq, self.T
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
        ms, wall, n = time_graph(g, 4, max(8, steps // 64), 4)
        out[R] = dict(ms=ms, gbs=alg / (ms * 1e-3) / 1e9)
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
    ms, wall, n = time_graph(g, len(layers), steps, max(3, steps // 8))
    layer = layers[0]
    eo = layer.eo.cpu().numpy()
    touched = int((eo[1:] - eo[:-1] > 0).sum())
    per_expert = 2 * I * H + 2 * I * 4 + H * I + H * 4
    wbytes = touched * per_expert
    return dict(T=T, ms=ms, tokens_per_s=T / (ms * 1e-3), experts_touched=touched,
                weight_bytes=wbytes, hbm_gbs_weights=wbytes / (ms * 1e-3) / 1e9,
                ops=2.0 * T * TOPK * (2 * I * H + H * I))


def bench_layer16(bq, torch, Wgu, Wd, steps):
    """All quantized projections of one decoder layer at decode batch 16:
    sliding (q/k/v 4096/2048/2048, o B=256) and full (q 8192, k 1024, o
    B=512) attention projections, dense MLP (gate/up 2112, down B=64) and the
    128-expert MoE, each with its activation prep."""
    T = 16
    gen = torch.Generator(device="cuda").manual_seed(0)
    d = "cuda"
    mk = lambda n, k, b: quantized(bq, torch, n, k, b, gen)[2]
    sq, sk, sv, so = mk(4096, H, 128), mk(2048, H, 128), mk(2048, H, 128), mk(H, 4096, 256)
    fq, fk, fo = mk(8192, H, 128), mk(1024, H, 128), mk(H, 8192, 512)
    dg, du, dd = mk(2112, H, 128), mk(2112, H, 128), mk(H, 2112, 64)
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
    gt, up = e(T, 2112), e(T, 2112)
    gq_, gsa = e(T, 2112, dt=torch.int8), e(T, 2112 // 64, dt=torch.float32)
    moe = MoeLayer(bq, torch, T, Wgu, Wd)

    def dense_mlp():
        bq.norm_quant(x, gamma, 128, out=(xq, xsa))
        bq.linear(xq, xsa, dg, out=gt)
        bq.linear(xq, xsa, du, out=up)
        bq.block_quant(gt, 64, True, out=(gq_, gsa))   # GELU(gate)*up is elementwise (not a bq op)
        bq.block_linear(gq_, gsa, dd, 64, out=o)

    def sliding(_i=0):
        bq.norm_quant(x, gamma, 128, out=(xq, xsa))
        bq.qkv(xq, xsa, sq, sk, sv, outs=(q_s, k_s, v_s))
        bq.block_quant(attn_s, 256, False, out=(oq_s, osa_s))
        bq.block_linear(oq_s, osa_s, so, 256, out=o)
        dense_mlp()
        moe()

    def full(_i=0):
        bq.norm_quant(x, gamma, 128, out=(xq, xsa))
        bq.linear(xq, xsa, fq, out=q_f)
        bq.linear(xq, xsa, fk, out=k_f)               # k_eq_v: one projection for K and V
        bq.block_quant(attn_f, 512, False, out=(oq_f, osa_f))
        bq.block_linear(oq_f, osa_f, fo, 512, out=o)
        dense_mlp()
        moe()

    gs_ = graph_of(sliding, 1)
    ms_s, _, _ = time_graph(gs_, 1, steps, max(3, steps // 8))
    gf_ = graph_of(full, 1)
    ms_f, _, _ = time_graph(gf_, 1, steps, max(3, steps // 8))
    gm_ = graph_of(moe, 1)
    ms_m, _, _ = time_graph(gm_, 1, steps, max(3, steps // 8))
    stack_ms = 25 * ms_s + 5 * ms_f
    return dict(sliding_layer_ms=ms_s, full_layer_ms=ms_f, moe_ms=ms_m,
                stack_ms=stack_ms, stack_tokens_per_s=T / (stack_ms * 1e-3))


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
        n = max(64, steps // 4) if decode else max(5, steps // 128)
        ms, _, _ = time_graph(gr, nrep, n, max(8, n // 8))
        r = {"us": round(ms * 1e3, 2), "s_max": s_max, "kv_bytes_read": kvbytes,
             "kv_GBs": round(kvbytes / (ms * 1e-3) / 1e9, 1)}
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
            pms, _, _ = time_graph(gp, 8, n, max(8, n // 8))
            r["prep_us"] = round(pms * 1e3, 2)
        else:
            # PV is an f32 fma per (position, column) on the vector ALUs
            flops = 2.0 * kvbytes / (2 * hd + 8) * (nq // nkv) * hd * 2
            r["tflops_qk_pv"] = round(flops / (ms * 1e-3) / 1e12, 1)
        res[name] = r
    return res


# ---------------------------------------------------------------------------
def cpu_baseline_gemv(codes, scales, seconds):
    """The reference CPU path (VNNI u8 x i8, 32-row tiles over worker_range),
    ported to C in oracle/cpu_baseline.c, on the host cores: the same decode
    GEMV (M=1, K=N=4096), bounded to ~`seconds` of CPU work."""
    import ctypes as C

    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    lib = O.cpu()
    q = codes.cpu().numpy()
    s = scales.cpu().numpy().astype(np.float32)
    N, K = q.shape
    p, cs = O.pack_and_colsum(q)
    xq = np.random.default_rng(1).integers(-127, 128, (1, K), dtype=np.int8)
    sa = np.ones(1, np.float32)
    out = np.empty((1, N), np.uint16)
    nthreads = max(1, min(16, os.cpu_count() or 1))
    ptr = lambda a: a.ctypes.data_as(C.c_void_p)

    def call():
        lib.bqcpu_linear(ptr(xq), ptr(sa), 1, ptr(p), ptr(s), ptr(cs), N, K, ptr(out), nthreads)

    for _ in range(30):
        call()
    ts = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end and len(ts) < 600:
        t0 = time.perf_counter()
        call()
        ts.append(time.perf_counter() - t0)
    med = float(np.median(ts))
    alg_bytes = N * K + N * 4 + K + 4 + N * 2
    return dict(value=alg_bytes / med / 1e9, unit="GB/s", cores=nthreads, kind="port",
                sample=f"decode GEMV M=1 K=N=4096, {len(ts)} calls after 30 warmups, median "
                       f"{med * 1e6:.1f} us; ISA {lib.bqcpu_isa().decode()}")


def cpu_baseline_moe(bq, torch, Wgu, Wd, layers, seconds):
    """The reference CPU path of the MoE layer (router top-k + softmax merge,
    CSR schedule, norm-quant, phase 1 over intermediate tiles, FWHT64
    block-quant, phase 2 over hidden tiles; VNNI u8 x i8 with colsums) from
    oracle/cpu_baseline.c and the oracle's router / schedule, on the host
    cores, for each MoeLayer's inputs; bounded to about `seconds` per T."""
    import ctypes as C

    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    lib = O.cpu()
    nthreads = max(1, min(16, os.cpu_count() or 1))
    ptr = lambda a: a.ctypes.data_as(C.c_void_p)
    gu = bq.unpack(Wgu.data, Wgu.n_rows, Wgu.k).cpu().numpy().reshape(Wgu.n_rows, Wgu.k)
    dn = bq.unpack(Wd.data, Wd.n_rows, Wd.k).cpu().numpy().reshape(Wd.n_rows, Wd.k)
    gp, gcs = O.pack_and_colsum(gu)
    dp, dcs = O.pack_and_colsum(dn, 64, False)
    del gu, dn
    gsc = Wgu.scale.cpu().numpy()
    dsc = Wd.scale.cpu().numpy()
    sqrt_n, n_eps = O.norm_consts(H)
    res = {}
    for layer in layers:
        T = layer.T
        x = layer.x.view(torch.int16).cpu().numpy().view(np.uint16)
        logits = layer.logits.cpu().numpy()
        gamma = np.full(H, 0x3F80, np.uint16)
        pes = np.full(E, 0x3F80, np.uint16)
        xq = np.empty((T, H), np.int8)
        xsa = np.empty(T, np.float32)
        bucket = np.empty((T * TOPK, I), np.uint16)
        bi8 = np.empty((T * TOPK, I), np.int8)
        bsa = np.empty((T * TOPK, I // 64), np.float32)
        accum = np.empty((T, H), np.float32)
        out = np.empty((T, H), np.uint16)

        def call():
            idx, w = O.route_topk_softmax(logits, TOPK, pes)
            eo, routes = O.build_schedule(idx, w, E)
            lib.bqcpu_norm_quant(ptr(x), ptr(gamma), ptr(xq), ptr(xsa), T, H, 128,
                                 C.c_float(sqrt_n), C.c_float(n_eps), nthreads)
            lib.bqcpu_moe_phase1(ptr(xq), ptr(xsa), H, ptr(eo), ptr(routes), E, ptr(gp), ptr(gsc),
                                 ptr(gcs), I, ptr(bucket), nthreads)
            lib.bqcpu_block_quant(ptr(bucket), ptr(bi8), ptr(bsa), T * TOPK, I, 64, 1, nthreads)
            lib.bqcpu_moe_phase2(ptr(bi8), ptr(bsa), I, 64, ptr(eo), ptr(routes), E, T, ptr(dp),
                                 ptr(dsc), ptr(dcs), H, ptr(accum), ptr(out), nthreads)

        call()
        ts = []
        t_end = time.perf_counter() + seconds
        while (time.perf_counter() < t_end and len(ts) < 600) or len(ts) < 2:
            t0 = time.perf_counter()
            call()
            ts.append(time.perf_counter() - t0)
        med = float(np.median(ts))
        res[f"T{T}"] = {"tokens_per_s": round(T / med, 1), "ms": round(med * 1e3, 3),
                        "samples": len(ts)}
    res.update(unit="tokens/s", cores=nthreads, kind="port",
               sample=f"MoE layer from router logits, 128 experts, top-8, H={H}, I={I}; "
                      f"median of the calls in ~{seconds:.0f} s per T after one warm call; "
                      f"ISA {lib.bqcpu_isa().decode()}")
    return res


def calib_copy(torch):
    """A plain device copy of 256 MiB (the PMC calibration kernel)."""
    a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()


def main():
    args = parse()
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
    if args.calib_copy:
        calib_copy(torch)

    line = {
        "metric": "bq GEMV HBM GB/s (% peak); MoE-layer tokens/s at 32 and 2048 tokens",
        "unit": "GB/s", "n_gpus": 1, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
    }
    if "gemv" in res:
        gv = res["gemv"]
        line.update(value=round(gv["gbs"], 1), steps=gv["calls"], warmup=args.warmup,
                    ms_per_step=gv["ms"],
                    config={"workload": "decode GEMV: per-row butterquant linear, M=1 token, "
                                        "K=4096, N=4096, int8 codes x int8 activation, "
                                        "fp32 accumulate -> bf16; 64 weight replicas (1 GiB) "
                                        "rotated", "global_batch": 1, "seq_len": 1,
                            "parallelism": "single GPU"},
                    pct_hbm_peak=round(100 * gv["gbs"] / HBM_PEAK_GBS, 1),
                    roofline={"bound": "hbm", "achieved": round(gv["gbs"], 1),
                              "peak": HBM_PEAK_GBS, "unit": "GB/s",
                              "frac": round(gv["gbs"] / HBM_PEAK_GBS, 4),
                              "traffic": _traffic()})
        line["gemv_detail"] = {"kernel_us": round(gv["ms"] * 1e3, 3),
                               "alg_bytes_per_launch": gv["alg_bytes"],
                               "norm_quant_us": round(gv["norm_quant_us"], 3),
                               "linear_with_prep_us": round(gv["linear_with_prep_us"], 3)}
    else:
        line.update(value=None, steps=args.steps, warmup=args.warmup, ms_per_step=None,
                    config={"workload": wl})
    if "prefill" in res:
        p = res["prefill"]
        line["prefill_gemm_m512"] = {"us": round(p["ms"] * 1e3, 2), "tops": round(p["tops"], 1),
                                     "int8_mfma_frac": round(p["int8_frac"], 4),
                                     "bf16_mfma_frac": round(p["bf16_frac"], 4)}
    for key in ("moe32", "moe2048"):
        if key in res:
            m = res[key]
            line[f"moe_layer_T{m['T']}"] = {
                "tokens_per_s": round(m["tokens_per_s"], 1), "ms": round(m["ms"], 4),
                "experts_touched": m["experts_touched"],
                "weight_GBs": round(m["hbm_gbs_weights"], 1),
                "hbm_frac_weights": round(m["hbm_gbs_weights"] / HBM_PEAK_GBS, 4),
                "int8_tops": round(m["ops"] / (m["ms"] * 1e-3) / 1e12, 1)}
    if "layer16" in res:
        line["decoder_layer_b16"] = {k: round(v, 4) for k, v in res["layer16"].items()}
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
    if "load" in res:
        ld = res["load"]
        line["load_safetensors_gate_up_507MB"] = {"ms": round(ld["ms"], 2),
                                                  "GBs": round(ld["gbs"], 2),
                                                  "checked": ld["checked"]}
    if "head" in res:
        hd = res["head"]
        line["head_flash_sample_v262144"] = {
            f"rows{R}": {"us": round(v["ms"] * 1e3, 1), "weight_GBs": round(v["gbs"], 1),
                         "hbm_frac": round(v["gbs"] / HBM_PEAK_GBS, 4)}
            for R, v in hd["rows"].items()}
        line["head_flash_sample_v262144"]["alg_bytes"] = hd["alg_bytes"]
    if "attn" in res:
        line["attention_int8_kv"] = res["attn"]
    if "gemv" in res and not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_gemv(res["gemv"]["codes"], res["gemv"]["scales"],
                                                 args.cpu_seconds)
    if MOE_LAYERS and not args.no_cpu:
        line["cpu_baseline_moe"] = cpu_baseline_moe(bq, torch, *moe_w, MOE_LAYERS,
                                                    args.cpu_seconds / 2)
    print(json.dumps(line))


def _traffic():
    """HBM bytes per GEMV launch from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the plain-copy calibration), or None."""
    path = os.path.join(ROOT, "profiles", "gemv_decode_k4096_n4096_traffic.txt")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":")[1]))
    except OSError:
        pass
    return None


if __name__ == "__main__":
    main()
