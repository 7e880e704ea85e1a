"""numpy front-end of the C oracle (oracle/bq_oracle.c) and of the CPU baseline
(oracle/cpu_baseline.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the
checker, and by bench.py's cpu_baseline leg.  The HIP library never calls it.
Every wrapper names the reference lines its C function restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD = os.path.join(HERE, "_build")
_ORACLE = os.path.join(BUILD, "libbq_oracle.so")
_CPU = os.path.join(BUILD, "libbq_cpu_baseline.so")


def build() -> None:
    """Compile the oracle and the CPU baseline (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _load(path):
    if not os.path.exists(path):
        build()
    return C.CDLL(path)


_lib = None
_cpu = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load(_ORACLE)
        _declare(_lib)
    return _lib


def cpu():
    global _cpu
    if _cpu is None:
        _cpu = _load(_CPU)
        _declare(_cpu)
        _cpu.bqcpu_isa.restype = C.c_char_p
    return _cpu


def _declare(L):
    L.bqo_f32_to_bf16.restype = C.c_uint16
    L.bqo_f32_to_bf16.argtypes = [C.c_float]
    L.bqo_fwht_scale.restype = C.c_float
    L.bqo_fwht_scale.argtypes = [C.c_int]
    L.bqo_rms_reduce_row.restype = C.c_float
    for name in ("bqo_exp_f32_fast", "bqo_tanh_f32", "bqo_gelu_tanh_f32",
                 "bqo_fast_exp_softmax_biased"):
        getattr(L, name).restype = C.c_float
        getattr(L, name).argtypes = [C.c_float]
    for name in ("bqo_exp_f32", "bqo_log_f32"):
        getattr(L, name).restype = C.c_float
        getattr(L, name).argtypes = [C.c_float]
    L.bqo_mix64.restype = C.c_uint64
    L.bqo_mix64.argtypes = [C.c_uint64]
    L.bqo_gumbel_noise.restype = C.c_float
    L.bqo_gumbel_noise.argtypes = [C.c_uint64, C.c_int64, C.c_int64]
    L.bqo_softcap.restype = C.c_float
    L.bqo_softcap.argtypes = [C.c_float, C.c_float]
    L.bqo_vnni_offset.restype = C.c_size_t
    L.bqo_vnni_offset.argtypes = [C.c_int, C.c_int, C.c_int]


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a


ROUTE_DTYPE = np.dtype([("token", np.int32), ("weight", np.float32)])

# --------------------------------------------------------------------------
# bf16
# --------------------------------------------------------------------------


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """butterquant/convert.mojo:14-17 software RNE, vectorised in numpy
    (pinned against the C restatement in tests)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rne = b + ((b >> np.uint32(16)) & np.uint32(1))  # uint32 wraps like the reference's
    rne += np.uint32(0x7FFF)
    return (rne >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------------------
# FWHT + quant
# --------------------------------------------------------------------------


def fwht_rows(x: np.ndarray, block: int) -> np.ndarray:
    """butterquant/fwht.mojo:20-76 over every row (in a copy)."""
    x = _c(x, np.float32).copy()
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    for r in range(rows):
        rc = lib().bqo_fwht_row(C.c_void_p(x.ctypes.data + r * cols * 4), cols, block)
        if rc != 0:
            raise ValueError(f"unsupported FWHT block {block} for cols {cols}")
    return x


def fwht_scale(block: int) -> float:
    return float(lib().bqo_fwht_scale(block))


def quant_segment(x: np.ndarray, store_divided: bool):
    """butterquant/kernels.mojo:68-78 -> (codes int8, scale f32)."""
    x = _c(x, np.float32)
    q = np.empty(x.size, np.int8)
    s = np.zeros(1, np.float32)
    lib().bqo_quant_segment(_p(x), _p(q), _p(s), x.size, int(store_divided))
    return q, s[0]


def rotate_and_quant(w: np.ndarray, block: int, per_block: bool = False):
    """Weight encoding (butterquant/kernels.mojo:148-168): f32 [N,K] ->
    (int8 [N,K] row-major, scales [N] or [N, K/block])."""
    w = _c(w, np.float32).copy()
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty((rows, cols // block) if per_block else (rows,), np.float32)
    rc = lib().bqo_rotate_and_quant(block, _p(w), _p(q), _p(s), rows, cols, int(per_block))
    if rc != 0:
        raise ValueError("rotate_and_quant: bad block/cols")
    return q, s


def bake_split_gain(gamma_bf16: np.ndarray, eps: float = 1e-12) -> np.ndarray:
    g = _c(gamma_bf16, np.uint16).copy()
    lib().bqo_bake_split_gain(_p(g), g.size, C.c_float(eps))
    return g


def rms_reduce_row(x_bf16: np.ndarray) -> float:
    x = _c(x_bf16, np.uint16)
    lib().bqo_rms_reduce_row.argtypes = [C.c_void_p, C.c_int]
    return float(lib().bqo_rms_reduce_row(_p(x), x.size))


def norm_consts(hidden: int):
    """(sqrt_n, n_eps) as gemma_4_moe_bq.mojo:646-647 computes them in f32."""
    sqrt_n = np.sqrt(np.float32(hidden), dtype=np.float32)
    n_eps = np.float32(hidden) * np.float32(1e-6)
    return float(sqrt_n), float(n_eps)


def norm_quant(x_bf16: np.ndarray, gamma_bf16: np.ndarray, block: int = 128,
               sqrt_n=None, n_eps=None, per_block: bool = False):
    """dispatch_bq_norm_quant (butterquant_kernels/linear.mojo:58-82 ->
    runtime.mojo:11-37): bf16 [M,H] -> (int8 [M,H], sa [M]); with per_block
    the head prep (runtime.mojo:40-47): sa [M, H/block]."""
    x = _c(x_bf16, np.uint16)
    g = _c(gamma_bf16, np.uint16)
    m, h = x.shape
    if sqrt_n is None:
        sqrt_n, n_eps = norm_consts(h)
    q = np.empty((m, h), np.int8)
    nsa = h // block if per_block else 1
    sa = np.empty((m, nsa) if per_block else m, np.float32)
    f = lib().bqo_prepare_norm_activation
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                  C.c_float, C.c_float, C.c_int]
    for r in range(m):
        rc = f(C.c_void_p(x.ctypes.data + r * h * 2), _p(g),
               C.c_void_p(q.ctypes.data + r * h), C.c_void_p(sa.ctypes.data + r * nsa * 4),
               h, block, sqrt_n, n_eps, int(per_block))
        if rc != 0:
            raise ValueError("norm_quant: bad block/hidden")
    return q, sa


def block_quant(x_bf16: np.ndarray, block: int, apply_fwht: bool):
    """dispatch_bq_block_quant (linear.mojo:182-205 -> runtime.mojo:62-80):
    bf16 [R,cols] -> (int8 [R,cols], sa [R, cols/block])."""
    x = _c(x_bf16, np.uint16)
    r, cols = x.shape
    nb = cols // block
    q = np.empty((r, cols), np.int8)
    sa = np.empty((r, nb), np.float32)
    f = lib().bqo_prepare_block_activation
    for i in range(r):
        rc = f(C.c_void_p(x.ctypes.data + i * cols * 2), C.c_void_p(q.ctypes.data + i * cols),
               C.c_void_p(sa.ctypes.data + i * nb * 4), cols, block, int(apply_fwht))
        if rc != 0:
            raise ValueError("block_quant: bad block/cols")
    return q, sa


# --------------------------------------------------------------------------
# pack
# --------------------------------------------------------------------------


def vnni_offsets(rows: int, cols: int) -> np.ndarray:
    """The pack bijection (butterquant/vnni.mojo:146-163) as an index array:
    packed[off[n,k]] = W[n,k]."""
    n = np.arange(rows, dtype=np.int64)[:, None]
    k = np.arange(cols, dtype=np.int64)[None, :]
    return ((n // 32) * 32 * cols + (k // 64) * 2048 + ((n % 32) // 16) * 1024
            + ((k % 64) // 4) * 64 + (n % 16) * 4 + (k % 4))


def pack_and_colsum(w_i8: np.ndarray, block_cols: int | None = None,
                    colsum_row_major: bool = True):
    """butterquant/vnni.mojo:86-114 -> (packed int8 [rows*cols], colsum f32)."""
    w = _c(w_i8, np.int8)
    rows, cols = w.shape
    bc = cols if block_cols is None else block_cols
    nb = cols // bc
    dst = np.empty(rows * cols, np.int8)
    cs = np.empty(rows * nb, np.float32)
    rc = lib().bqo_pack_and_colsum_vnni(_p(w), _p(dst), rows, cols, bc, _p(cs),
                                        int(colsum_row_major))
    if rc != 0:
        raise ValueError("pack_and_colsum: contract violated")
    return dst, cs


# --------------------------------------------------------------------------
# GEMM
# --------------------------------------------------------------------------


def linear(act, sa, wpacked, wsc, colsum, n_rows: int):
    """VNNI per-row linear (butterquant/gemm.mojo:114-170) -> (bf16, f32)."""
    act = _c(act, np.int8); sa = _c(sa, np.float32)
    wpacked = _c(wpacked, np.int8); wsc = _c(wsc, np.float32); colsum = _c(colsum, np.float32)
    m, K = act.shape
    ob = np.empty((m, n_rows), np.uint16)
    of = np.empty((m, n_rows), np.float32)
    lib().bqo_gemm_i8_per_row(_p(act), _p(sa), m, _p(wpacked), _p(wsc), _p(colsum),
                              n_rows, K, _p(ob), _p(of))
    return ob, of


def block_linear(act, sa, wpacked, wsc, colsum, n: int, block: int):
    """VNNI per-block linear (butterquant/gemm.mojo:173-243) -> (bf16, f32)."""
    act = _c(act, np.int8); sa = _c(sa, np.float32)
    wpacked = _c(wpacked, np.int8); wsc = _c(wsc, np.float32); colsum = _c(colsum, np.float32)
    m, K = act.shape
    ob = np.empty((m, n), np.uint16)
    of = np.empty((m, n), np.float32)
    lib().bqo_gemm_i8_per_block(_p(act), _p(sa), m, _p(wpacked), _p(wsc), _p(colsum),
                                n, K, block, _p(ob), _p(of))
    return ob, of


def signed_linear(act, sa, wpacked, wsc, n_rows: int):
    """Signed (AMX-branch) per-row epilogue (butterquant/amx_gemm.mojo:28-44)."""
    act = _c(act, np.int8); sa = _c(sa, np.float32)
    wpacked = _c(wpacked, np.int8); wsc = _c(wsc, np.float32)
    m, K = act.shape
    ob = np.empty((m, n_rows), np.uint16)
    of = np.empty((m, n_rows), np.float32)
    lib().bqo_gemm_signed_per_row(_p(act), _p(sa), m, _p(wpacked), _p(wsc), n_rows, K,
                                  _p(ob), _p(of))
    return ob, of


def signed_block_linear(act, sa, wpacked, wsc, n: int, block: int):
    act = _c(act, np.int8); sa = _c(sa, np.float32)
    wpacked = _c(wpacked, np.int8); wsc = _c(wsc, np.float32)
    m, K = act.shape
    ob = np.empty((m, n), np.uint16)
    of = np.empty((m, n), np.float32)
    lib().bqo_gemm_signed_per_block(_p(act), _p(sa), m, _p(wpacked), _p(wsc), n, K, block,
                                    _p(ob), _p(of))
    return ob, of


def int_acc(act, wpacked, n: int, k_lo: int = 0, k_hi: int | None = None):
    act = _c(act, np.int8); wpacked = _c(wpacked, np.int8)
    m, K = act.shape
    k_hi = K if k_hi is None else k_hi
    out = np.empty((m, n), np.int64)
    lib().bqo_int_acc(_p(act), m, _p(wpacked), n, K, k_lo, k_hi, _p(out))
    return out


# --------------------------------------------------------------------------
# MoE
# --------------------------------------------------------------------------


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    f = lib().bqo_gelu_tanh_f32
    return np.array([f(float(v)) for v in np.ravel(x)], np.float32).reshape(np.shape(x))


def gelu_gate_up(gate_bf16: np.ndarray, up_bf16: np.ndarray) -> np.ndarray:
    """gelu_gate_up_row (kernels/elementwise.mojo:17-27), the dense MLP's step
    between its gate/up linears and the FWHT64 block-quant
    (modeling/gemma_4_moe_bq.mojo:763-764): bf16(gelu_tanh_f32(f32(gate)) *
    f32(up)) elementwise."""
    g = bf16_to_f32(_c(gate_bf16, np.uint16))
    u = bf16_to_f32(_c(up_bf16, np.uint16))
    return f32_to_bf16((gelu_tanh(g) * u).astype(np.float32))


def exp_fast(x):
    f = lib().bqo_exp_f32_fast
    return np.array([f(float(v)) for v in np.ravel(x)], np.float32).reshape(np.shape(x))


def router_logits(x_bf16: np.ndarray, router_proj_bf16: np.ndarray, router_scale_bf16: np.ndarray,
                  sqrt_n=None, n_eps=None) -> np.ndarray:
    """RouterExpertKernel up to the candidate insert (kernels/moe_router.mojo:
    164-187): bf16 x [T,H], router_proj [E,H], router_scale [H] -> f32 [T,E]."""
    x = _c(x_bf16, np.uint16)
    rp = _c(router_proj_bf16, np.uint16)
    rs = _c(router_scale_bf16, np.uint16)
    T, H = x.shape
    E = rp.shape[0]
    assert rp.shape == (E, H) and rs.shape == (H,)
    if sqrt_n is None:
        sqrt_n, n_eps = norm_consts(H)
    out = np.empty((T, E), np.float32)
    f = lib().bqo_router_logits
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_float,
                  C.c_float, C.c_void_p]
    f(_p(x), _p(rp), _p(rs), T, H, E, sqrt_n, n_eps, _p(out))
    return out


def route_topk_softmax(logits: np.ndarray, top_k: int = 8, per_expert_scale=None):
    """Top-k (moe_router.mojo:43-57) + softmax over the k (:276-293); optional
    bf16 [E] per-expert scale."""
    lg = _c(logits, np.float32)
    T, E = lg.shape
    idx = np.empty((T, top_k), np.int32)
    w = np.empty((T, top_k), np.float32)
    sc = None if per_expert_scale is None else _c(per_expert_scale, np.uint16)
    lib().bqo_route_topk_softmax(_p(lg), T, E, top_k, _p(sc) if sc is not None else None,
                                 _p(idx), _p(w))
    return idx, w


def build_schedule(route_idx: np.ndarray, route_w: np.ndarray, E: int):
    """kernels/moe_router.mojo:60-106 -> (expert_offset [E+1], routes)."""
    ri = _c(route_idx, np.int32); rw = _c(route_w, np.float32)
    T, k = ri.shape
    eo = np.empty(E + 1, np.int32)
    routes = np.zeros(T * k, ROUTE_DTYPE)
    lib().bqo_build_schedule(_p(ri), _p(rw), T, k, E, _p(eo), _p(routes))
    return eo, routes[: int(eo[E])]


def moe_phase1(x_i8, x_sa, expert_offset, routes, w_gu_packed, gu_scale, gu_colsum,
               inter: int):
    """butterquant_kernels/moe.mojo:25-164 -> bucket bf16 [n_routes, inter]."""
    x_i8 = _c(x_i8, np.int8); x_sa = _c(x_sa, np.float32)
    eo = _c(expert_offset, np.int32); routes = np.ascontiguousarray(routes, ROUTE_DTYPE)
    E = eo.size - 1
    hidden = x_i8.shape[1]
    bucket = np.zeros((max(int(eo[E]), 1), inter), np.uint16)
    lib().bqo_moe_phase1(_p(x_i8), _p(x_sa), hidden, _p(eo), _p(routes), E,
                         _p(_c(w_gu_packed, np.int8)), _p(_c(gu_scale, np.float32)),
                         _p(_c(gu_colsum, np.float32)), inter, _p(bucket))
    return bucket[: int(eo[E])]


def moe_phase2(bucket_i8, bucket_sa, expert_offset, routes, T: int, w_d_packed,
               d_scale, d_colsum, hidden: int, block: int = 64):
    """butterquant_kernels/moe.mojo:167-335 -> (accum f32 [T,H], out bf16)."""
    bi = _c(bucket_i8, np.int8); bs = _c(bucket_sa, np.float32)
    eo = _c(expert_offset, np.int32); routes = np.ascontiguousarray(routes, ROUTE_DTYPE)
    E = eo.size - 1
    inter = bi.shape[1]
    accum = np.empty((T, hidden), np.float32)
    out = np.empty((T, hidden), np.uint16)
    lib().bqo_moe_phase2(_p(bi), _p(bs), inter, block, _p(eo), _p(routes), E, T,
                         _p(_c(w_d_packed, np.int8)), _p(_c(d_scale, np.float32)),
                         _p(_c(d_colsum, np.float32)), hidden, _p(accum), _p(out))
    return accum, out


# --------------------------------------------------------------------------
# synthetic inputs
# --------------------------------------------------------------------------


def synth_normal_bf16(seed: int, sigma: float, shape) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.uint16)
    lib().bqo_synth_normal_bf16(C.c_uint64(seed), C.c_double(sigma), _p(out), C.c_size_t(n))
    return out.reshape(shape)


def synth_normal_f32(seed: int, sigma: float, shape) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    lib().bqo_synth_normal_f32(C.c_uint64(seed), C.c_double(sigma), _p(out), C.c_size_t(n))
    return out.reshape(shape)


# ---------------------------------------------------------------- bq head / embedding
SAMPLE_NMAX = 256  # continuous_batching/schedule.mojo:9
# kernels/flash_sample.mojo:21-28 SamplingParams, kernels/flash_sample.mojo:120-134 SampleOutcome
PARAMS_DT = np.dtype([("temperature", "<f4"), ("min_p", "<f4"), ("top_k", "<i8"), ("seed", "<u8"),
                      ("n_keep", "<i8"), ("greedy", "u1"), ("pad", "u1", 7)])
OUTCOME_DT = np.dtype([("token_id", "<i4"), ("logz", "<f4"), ("n", "<i8"),
                       ("topn_val", "<f4", SAMPLE_NMAX), ("topn_idx", "<i4", SAMPLE_NMAX)])


def sampling_params(rows, temperature=1.0, min_p=0.0, top_k=0, seed=0, n_keep=SAMPLE_NMAX,
                    greedy=False):
    """One SamplingParams per row; scalars broadcast, sequences per row."""
    p = np.zeros(rows, PARAMS_DT)
    for name, v in (("temperature", temperature), ("min_p", min_p), ("top_k", top_k),
                    ("seed", seed), ("n_keep", n_keep), ("greedy", greedy)):
        p[name] = v
    return p


def flash_sample(x_i8, x_sa, weight, wscales, params, block=128, cap=30.0, vocab_base=0):
    """BqFlashSampleKernel over the whole vocabulary as one worker +
    finalize_outcomes (butterquant_kernels/head.mojo:85-167,
    kernels/flash_sample.mojo:221-265).  weight int8 [V, H] row-major."""
    x = _c(x_i8, np.int8)
    sa = _c(x_sa, np.float32)
    w = _c(weight, np.int8)
    ws = _c(wscales, np.float32)
    pr = np.ascontiguousarray(params, PARAMS_DT)
    R, H = x.shape
    V = w.shape[0]
    assert sa.shape == (R, H // block) and ws.shape == (V, H // block) and pr.shape == (R,)
    out = np.zeros(R, OUTCOME_DT)
    f = lib().bqo_flash_sample
    f.argtypes = [C.c_void_p] * 4 + [C.c_int] * 4 + [C.c_float, C.c_int64, C.c_void_p, C.c_void_p]
    f(_p(x), _p(sa), _p(w), _p(ws), R, V, H, block, cap, vocab_base, _p(pr), _p(out))
    return out


def embed_lookup(token_ids, weight, wscales, block=128, scale=None, shard_rows=None, rank=0):
    """BqEmbedLookupKernel (butterquant_kernels/embedding.mojo:21-96):
    int8 [rows, H] per-block scales -> bf16 [T, H]."""
    tok = _c(token_ids, np.int32)
    w = _c(weight, np.int8)
    ws = _c(wscales, np.float32)
    rows, H = w.shape
    if scale is None:
        scale = embed_scale(H)
    if shard_rows is None:
        shard_rows = rows
    out = np.empty((tok.shape[0], H), np.uint16)
    f = lib().bqo_embed_lookup
    f.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                  C.c_int, C.c_float, C.c_void_p]
    f(_p(tok), tok.shape[0], _p(w), _p(ws), H, block, shard_rows, rank, scale, _p(out))
    return out


def embed_scale(hidden: int) -> float:
    """f32(bf16(sqrtf(hidden))) (gemma_4_moe_bq.mojo:965-966)."""
    s = np.sqrt(np.float32(hidden), dtype=np.float32)
    return float(bf16_to_f32(f32_to_bf16(np.array([s], np.float32)))[0])


# --------------------------------------------------------------------------
# int8-KV attention
# --------------------------------------------------------------------------

KV_RUN_DT = np.dtype([("buf_start", "<i4"), ("base_pos", "<i4"), ("rows_off", "<i4"),
                      ("page_count", "<i4")])   # kernels/attention_ops.mojo:54-58 KVRun


def kv_runs(runs) -> np.ndarray:
    """[(buf_start, base_pos, rows_off, page_count), ...] -> KV_RUN_DT array."""
    return np.array([tuple(int(v) for v in r) for r in runs], KV_RUN_DT)


def attn_prep(q_src, k_src, v_src, q_norm, k_norm, k_cache, k_scale, v_cache, v_scale,
              cos_table, sin_table, runs, base_rows, num_q, num_kv, head_dim, rope_half,
              pair_stride, page_shift, row_mask, page_mask, cache_degree=1, rank=0,
              sqrt_n=None, n_eps=None):
    """BqAttnPrepKernel (butterquant_kernels/attention.mojo:474-534): returns
    (q_i8 [T, num_q*hd], qi_bias [T, num_q], f_q [T, num_q]); writes the
    token's K/V rows and scales into the caches (numpy arrays, in place)."""
    T = q_src.shape[0]
    if sqrt_n is None:
        sqrt_n, n_eps = norm_consts(head_dim)
    q = _c(q_src, np.uint16); k = _c(k_src, np.uint16); v = _c(v_src, np.uint16)
    qn = _c(q_norm, np.uint16); kn = _c(k_norm, np.uint16)
    cs = _c(cos_table, np.float32); sn = _c(sin_table, np.float32)
    rr = np.ascontiguousarray(runs, KV_RUN_DT); br = _c(base_rows, np.int32)
    for a in (k_cache, k_scale, v_cache, v_scale):
        assert a.flags.c_contiguous
    qi = np.zeros((T, num_q * head_dim), np.int8)
    qb = np.zeros((T, num_q), np.float32)
    fq = np.zeros((T, num_q), np.float32)
    f = lib().bqo_attn_prep
    f.argtypes = ([C.c_void_p] * 15 + [C.c_int, C.c_void_p] + [C.c_int] * 6
                  + [C.c_float, C.c_float] + [C.c_int] * 5)
    f(_p(q), _p(k), _p(v), _p(qn), _p(kn), _p(qi), _p(qb), _p(fq), _p(k_cache), _p(k_scale),
      _p(v_cache), _p(v_scale), _p(cs), _p(sn), _p(rr), len(rr), _p(br), T, num_q, num_kv,
      head_dim, rope_half, pair_stride, sqrt_n, n_eps, cache_degree, rank, page_shift,
      row_mask, page_mask)
    return qi, qb, fq


def attn_num_splits(L: int, s_max: int, min_split: int) -> int:
    return int(lib().bqo_attn_num_splits(int(L), int(s_max), int(min_split)))


def flash_attention(q_i8, qi_bias, f_q, k_cache, k_scale, v_cache, v_scale, runs, base_rows,
                    num_q, num_kv, head_dim, window, page_shift, row_mask, page_mask,
                    s_max=1, min_split=32, degree=1, rank=0, with_f32=False):
    """int8-KV flash attention (butterquant_kernels/attention.mojo:32-327 with
    the merge of kernels/logsum_merge.mojo:29-122) -> bf16 [T, num_q*hd].
    window > 0: sliding; window == 0: full.  s_max / min_split fix the split
    of each token's KV range (and with it the f32 merge order).  with_f32:
    also return the f32 values before the bf16 cast."""
    qi = _c(q_i8, np.int8); qb = _c(qi_bias, np.float32); fq = _c(f_q, np.float32)
    kc = _c(k_cache, np.int8); ks = _c(k_scale, np.float32)
    vc = _c(v_cache, np.int8); vs = _c(v_scale, np.float32)
    rr = np.ascontiguousarray(runs, KV_RUN_DT); br = _c(base_rows, np.int32)
    T = qi.shape[0]
    out = np.zeros((T, num_q * head_dim), np.uint16)
    o32 = np.zeros((T, num_q * head_dim), np.float32)
    f = lib().bqo_flash_attention
    f.argtypes = [C.c_void_p] * 8 + [C.c_int, C.c_void_p] + [C.c_int] * 12 + [C.c_void_p] * 2
    f(_p(qi), _p(qb), _p(fq), _p(kc), _p(ks), _p(vc), _p(vs), _p(rr), len(rr), _p(br), T,
      num_q, num_kv, head_dim, window, degree, rank, page_shift, row_mask, page_mask, s_max,
      min_split, _p(out), _p(o32))
    return (out, o32) if with_f32 else out


# ---------------------------------------------------------------- CPU baseline (VNNI port)
# oracle/cpu_baseline.c: the reference's VNNI branch with OpenMP workers and the
# reference's worker policies; bench.py times it, tests pin it to the oracle.
def cpu_pin(cpus) -> None:
    """Pin the OpenMP team: thread i (0 = the caller) to CPU cpus[i]."""
    c = np.ascontiguousarray(cpus, np.int32)
    if cpu().bqcpu_pin(_p(c), int(c.size)) != 0:
        raise OSError(f"could not pin {c.size} OpenMP threads to CPUs {list(c)}")


def cpu_linear(act, sa, wpacked, wsc, colsum, n_rows: int, nthreads: int = 4):
    act = _c(act, np.int8); sa = _c(sa, np.float32)
    m, K = act.shape
    out = np.empty((m, n_rows), np.uint16)
    cpu().bqcpu_linear(_p(act), _p(sa), m, _p(_c(wpacked, np.int8)), _p(_c(wsc, np.float32)),
                       _p(_c(colsum, np.float32)), n_rows, K, _p(out), nthreads)
    return out


def cpu_block_linear(act, sa, wpacked, wsc, colsum, n: int, block: int, nthreads: int = 4):
    act = _c(act, np.int8); sa = _c(sa, np.float32)
    m, K = act.shape
    out = np.empty((m, n), np.uint16)
    cpu().bqcpu_block_linear(_p(act), _p(sa), m, _p(_c(wpacked, np.int8)),
                             _p(_c(wsc, np.float32)), _p(_c(colsum, np.float32)), n, K, block,
                             _p(out), nthreads)
    return out


def cpu_norm_quant(x_bf16, gamma_bf16, block: int = 128, nthreads: int = 4):
    x = _c(x_bf16, np.uint16); g = _c(gamma_bf16, np.uint16)
    m, hidden = x.shape
    sqrt_n, n_eps = norm_consts(hidden)
    q = np.empty((m, hidden), np.int8)
    sa = np.empty(m, np.float32)
    cpu().bqcpu_norm_quant(_p(x), _p(g), _p(q), _p(sa), m, hidden, block, C.c_float(sqrt_n),
                           C.c_float(n_eps), nthreads)
    return q, sa


def cpu_block_quant(x_bf16, block: int, apply_fwht: bool, nthreads: int = 4):
    x = _c(x_bf16, np.uint16)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.int8)
    sa = np.empty((rows, cols // block), np.float32)
    cpu().bqcpu_block_quant(_p(x), _p(q), _p(sa), rows, cols, block, int(apply_fwht), nthreads)
    return q, sa


def cpu_route_topk(logits, top_k: int = 8, per_expert_scale=None, nthreads: int = 4):
    lg = _c(logits, np.float32)
    T, E = lg.shape
    idx = np.empty((T, top_k), np.int32)
    w = np.empty((T, top_k), np.float32)
    sc = None if per_expert_scale is None else _c(per_expert_scale, np.uint16)
    cpu().bqcpu_route_topk(_p(lg), T, E, top_k, _p(sc) if sc is not None else None, _p(idx),
                           _p(w), nthreads)
    return idx, w


def cpu_moe_phase1(x_i8, x_sa, expert_offset, routes, w_gu_packed, gu_scale, gu_colsum,
                   inter: int, nthreads: int = 4):
    x_i8 = _c(x_i8, np.int8); x_sa = _c(x_sa, np.float32)
    eo = _c(expert_offset, np.int32); routes = np.ascontiguousarray(routes, ROUTE_DTYPE)
    E = eo.size - 1
    bucket = np.zeros((max(int(eo[E]), 1), inter), np.uint16)
    cpu().bqcpu_moe_phase1(_p(x_i8), _p(x_sa), x_i8.shape[1], _p(eo), _p(routes), E,
                           _p(_c(w_gu_packed, np.int8)), _p(_c(gu_scale, np.float32)),
                           _p(_c(gu_colsum, np.float32)), inter, _p(bucket), nthreads)
    return bucket[: int(eo[E])]


def cpu_moe_phase2(bucket_i8, bucket_sa, expert_offset, routes, T: int, w_d_packed, d_scale,
                   d_colsum, hidden: int, block: int = 64, nthreads: int = 4):
    bi = _c(bucket_i8, np.int8); bs = _c(bucket_sa, np.float32)
    eo = _c(expert_offset, np.int32); routes = np.ascontiguousarray(routes, ROUTE_DTYPE)
    E = eo.size - 1
    accum = np.empty((T, hidden), np.float32)
    out = np.empty((T, hidden), np.uint16)
    cpu().bqcpu_moe_phase2(_p(bi), _p(bs), bi.shape[1], block, _p(eo), _p(routes), E, T,
                           _p(_c(w_d_packed, np.int8)), _p(_c(d_scale, np.float32)),
                           _p(_c(d_colsum, np.float32)), hidden, _p(accum), _p(out), nthreads)
    return accum, out


class CpuMoeLayer:
    """The whole MoE layer of oracle/cpu_baseline.c (bqcpu_moe_layer) from
    router logits, with every buffer allocated once: route top-k + softmax,
    schedule, norm-quant, phase 1, FWHT64 block-quant, phase 2."""

    def __init__(self, T, E, top_k, hidden, inter, gp, gsc, gcs, dp, dsc, dcs):
        self.T, self.E, self.k, self.H, self.I = T, E, top_k, hidden, inter
        self.w = [_c(a, t) for a, t in ((gp, np.int8), (gsc, np.float32), (gcs, np.float32),
                                        (dp, np.int8), (dsc, np.float32), (dcs, np.float32))]
        R = T * top_k
        self.idx = np.empty((T, top_k), np.int32)
        self.rw = np.empty((T, top_k), np.float32)
        self.eo = np.empty(E + 1, np.int32)
        self.routes = np.zeros(R, ROUTE_DTYPE)
        self.xq = np.empty((T, hidden), np.int8)
        self.xsa = np.empty(T, np.float32)
        self.bucket = np.empty((R, inter), np.uint16)
        self.bi8 = np.empty((R, inter), np.int8)
        self.bsa = np.empty((R, inter // 64), np.float32)
        self.accum = np.empty((T, hidden), np.float32)
        self.out = np.empty((T, hidden), np.uint16)
        self.sqrt_n, self.n_eps = norm_consts(hidden)

    def __call__(self, logits, x_bf16, gamma_bf16, pes=None, nthreads: int = 4):
        lg = _c(logits, np.float32); x = _c(x_bf16, np.uint16); g = _c(gamma_bf16, np.uint16)
        assert lg.shape == (self.T, self.E) and x.shape == (self.T, self.H)
        sc = None if pes is None else _c(pes, np.uint16)
        gp, gsc, gcs, dp, dsc, dcs = self.w
        cpu().bqcpu_moe_layer(
            _p(lg), _p(sc) if sc is not None else None, _p(x), _p(g), self.T, self.E, self.k,
            self.H, self.I, C.c_float(self.sqrt_n), C.c_float(self.n_eps), _p(gp), _p(gsc),
            _p(gcs), _p(dp), _p(dsc), _p(dcs), _p(self.idx), _p(self.rw), _p(self.eo),
            _p(self.routes), _p(self.xq), _p(self.xsa), _p(self.bucket), _p(self.bi8),
            _p(self.bsa), _p(self.accum), _p(self.out), nthreads)
        return self.accum, self.out
