"""Python binding of libbq.so (the gfx950 butterquant library) for tests and
benchmarks.  torch supplies device memory and the current stream; every
computation runs in libbq.so through its C ABI (include/bq_api.h).  If the
library is missing this module raises on import -- there is no fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "libbq.so")

LAYOUT_ROWMAJOR = 0
LAYOUT_VNNI = 1


class BqError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"libbq error {code}: {msg}")
        self.code = code


_vp, _i, _f, _sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t

# symbol -> argtypes (restype int unless listed in _RESTYPES)
SIGNATURES = {
    "bq_init": [_i],
    "bq_last_error": [],
    "bq_stream_synchronize": [_vp],
    "bq_version": [],
    "bq_weight_retile": [_vp, _i, _vp, _i, _i, _vp],
    "bq_weight_unpack": [_vp, _vp, _i, _i, _vp],
    "bq_pack_colsum_vnni": [_vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "bq_quantize_weight": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "bq_norm_quant": [_vp, _vp, _vp, _vp, _i, _i, _i, _f, _f, _vp],
    "bq_block_quant": [_vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "bq_linear": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp],
    "bq_block_linear": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "bq_qkv": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "bq_norm_linear": [_vp] * 8 + [_i, _i, _i, _i, _f, _f, _vp],
    "bq_norm_qkv": [_vp] * 13 + [_i, _i, _i, _i, _i, _f, _f, _vp],
    "bq_linear_pair": [_vp] * 8 + [_i, _i, _i, _i, _vp],
    "bq_norm_linear_pair": [_vp] * 10 + [_i, _i, _i, _i, _i, _f, _f, _vp],
    "bq_moe_router_logits": [_vp, _vp, _vp, _vp, _i, _i, _i, _f, _f, _vp],
    "bq_moe_route_topk": [_vp, _vp, _i, _i, _i, _vp, _vp, _vp],
    "bq_moe_build_schedule": [_vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp],
    "bq_moe_route_schedule": [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp],
    "bq_moe_prep": [_vp] * 4 + [_i] * 5 + [_f, _f] + [_vp] * 7,
    "bq_ffn_prep": [_vp] * 5 + [_i] * 5 + [_f, _f] + [_vp] * 9,
    "bq_head_prep": [_vp, _vp, _vp, _vp, _i, _i, _i, _f, _f, _vp],
    "bq_flash_sample_workspace_size": [_i, _i],
    "bq_flash_sample": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, C.c_int64, _vp, _sz,
                        _vp],
    "bq_embed_lookup": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _vp],
    "bq_attn_prep": [_vp] * 15 + [_i, _vp] + [_i] * 5 + [_f, _f] + [_i] * 6 + [_vp],
    "bq_attention_splits": [_i, _i, _i],
    "bq_attention_workspace_size": [_i, _i, _i, _i],
    "bq_sliding_attention": [_vp] * 9 + [_sz, _vp, _i, _vp] + [_i] * 9 + [_vp],
    "bq_full_attention": [_vp] * 9 + [_sz, _vp, _i, _vp] + [_i] * 8 + [_vp],
    "bq_st_open": [C.c_char_p, C.POINTER(C.c_void_p)],
    "bq_st_close": [_vp],
    "bq_st_num_tensors": [_vp],
    "bq_st_tensor_info": [_vp, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_int),
                          C.POINTER(C.c_int64), C.POINTER(C.c_size_t), C.POINTER(C.c_void_p)],
    "bq_load_quantized": [C.POINTER(C.c_void_p), _i, C.c_char_p, _i, _i, _i, _vp, _vp, _vp, _sz,
                          _vp],
    "bq_moe_phase1_gate_up": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "bq_moe_phase1_gate_up_quant": [_vp] * 9 + [_i] * 5 + [_vp],
    "bq_moe_phase2_workspace_size": [_i, _i, _i],
    "bq_moe_phase2_down": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i,
                           _vp, _sz, _vp],
    "bq_moe_phase2_down_noalloc": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                   _i, _vp],
    "bq_ffn_gate_up": [_vp] * 8 + [_i] * 5 + [_vp] * 6 + [_i] + [_vp] * 3,
    "bq_ffn_down": [_vp] * 8 + [_i] * 6 + [_vp] * 4 + [_i, _vp, _vp, _sz, _vp],
}
_RESTYPES = {"bq_last_error": C.c_char_p, "bq_version": C.c_char_p,
             "bq_moe_phase2_workspace_size": C.c_size_t,
             "bq_flash_sample_workspace_size": C.c_size_t, "bq_st_close": None,
             "bq_attention_workspace_size": C.c_size_t}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run mojo-gemma4-cpu_amd/build.py "
                          "(or __graft_entry__.build())")
    lib = C.CDLL(LIB_PATH)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, C.c_int)
    return lib


_lib = _load()


def lib():
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        raise BqError(rc, _lib.bq_last_error().decode())


def _p(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dev(t: torch.Tensor, dtype=None):
    if not t.is_cuda:
        raise ValueError("libbq takes device tensors")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError("libbq takes contiguous tensors")
    return t


def init(device: int = 0) -> None:
    _check(_lib.bq_init(device))


def synchronize() -> None:
    _check(_lib.bq_stream_synchronize(_stream()))


def norm_consts(hidden: int):
    """(sqrt_n, n_eps) in f32 as gemma_4_moe_bq.mojo:646-647 computes them."""
    import numpy as np
    sqrt_n = np.sqrt(np.float32(hidden), dtype=np.float32)
    n_eps = np.float32(hidden) * np.float32(1e-6)
    return float(sqrt_n), float(n_eps)


@dataclass
class ButterquantWeight:
    """Device view of a quantized weight (butterquant/weight.mojo:50-64):
    codes in the tile16x64 layout + per-row scales."""
    data: torch.Tensor   # int8 [n_rows * k] tile16x64
    scale: torch.Tensor  # f32 [n_rows]
    n_rows: int
    k: int


# --------------------------------------------------------------------------
# weights
# --------------------------------------------------------------------------

def retile(codes: torch.Tensor, n_rows: int, k: int, layout: int = LAYOUT_ROWMAJOR) -> torch.Tensor:
    _dev(codes, torch.int8)
    out = torch.empty(n_rows * k, dtype=torch.int8, device=codes.device)
    _check(_lib.bq_weight_retile(_p(codes), layout, _p(out), n_rows, k, _stream()))
    return out


def unpack(tiled: torch.Tensor, n_rows: int, k: int) -> torch.Tensor:
    _dev(tiled, torch.int8)
    out = torch.empty((n_rows, k), dtype=torch.int8, device=tiled.device)
    _check(_lib.bq_weight_unpack(_p(tiled), _p(out), n_rows, k, _stream()))
    return out


def pack_colsum_vnni(codes: torch.Tensor, block_cols: int | None = None,
                     colsum_row_major: bool = True):
    _dev(codes, torch.int8)
    rows, cols = codes.shape
    bc = cols if block_cols is None else block_cols
    dst = torch.empty(rows * cols, dtype=torch.int8, device=codes.device)
    cs = torch.empty(rows * (cols // bc), dtype=torch.float32, device=codes.device)
    _check(_lib.bq_pack_colsum_vnni(_p(codes), _p(dst), _p(cs), rows, cols, bc,
                                    int(colsum_row_major), _stream()))
    return dst, cs


def quantize_weight(w: torch.Tensor, fwht_block: int, per_block: bool = False,
                    gamma: torch.Tensor | None = None):
    """bf16 [rows, cols] -> (int8 row-major codes, f32 scales)."""
    _dev(w, torch.bfloat16)
    rows, cols = w.shape
    codes = torch.empty((rows, cols), dtype=torch.int8, device=w.device)
    shape = (rows, cols // fwht_block) if per_block else (rows,)
    scales = torch.empty(shape, dtype=torch.float32, device=w.device)
    if gamma is not None:
        _dev(gamma, torch.float32)
    _check(_lib.bq_quantize_weight(_p(w), _p(gamma), _p(codes), _p(scales), rows, cols,
                                   fwht_block, int(per_block), _stream()))
    return codes, scales


def load_weight(w: torch.Tensor, fwht_block: int) -> ButterquantWeight:
    """Quantize a bf16 weight (per-row recipe) and re-tile it for the GPU."""
    codes, scales = quantize_weight(w, fwht_block)
    n, k = w.shape
    return ButterquantWeight(retile(codes, n, k), scales, n, k)


# --------------------------------------------------------------------------
# activations
# --------------------------------------------------------------------------

def norm_quant(x: torch.Tensor, gamma: torch.Tensor, block: int = 128, sqrt_n=None,
               n_eps=None, out=None):
    _dev(x, torch.bfloat16)
    _dev(gamma, torch.bfloat16)
    m, h = x.shape
    if sqrt_n is None:
        sqrt_n, n_eps = norm_consts(h)
    if out is None:
        xq = torch.empty((m, h), dtype=torch.int8, device=x.device)
        sa = torch.empty(m, dtype=torch.float32, device=x.device)
    else:
        xq, sa = out
    _check(_lib.bq_norm_quant(_p(x), _p(gamma), _p(xq), _p(sa), m, h, block, sqrt_n, n_eps,
                              _stream()))
    return xq, sa


def block_quant(x: torch.Tensor, block: int, apply_fwht: bool, out=None):
    _dev(x, torch.bfloat16)
    r, cols = x.shape
    if out is None:
        xq = torch.empty((r, cols), dtype=torch.int8, device=x.device)
        sa = torch.empty((r, cols // block), dtype=torch.float32, device=x.device)
    else:
        xq, sa = out
    _check(_lib.bq_block_quant(_p(x), _p(xq), _p(sa), cols, r, block, int(apply_fwht),
                               _stream()))
    return xq, sa


# --------------------------------------------------------------------------
# linears
# --------------------------------------------------------------------------

def linear(x_i8, x_sa, w: ButterquantWeight, want_f32: bool = False, out=None):
    m, k = x_i8.shape
    if out is None:
        out = torch.empty((m, w.n_rows), dtype=torch.bfloat16, device=x_i8.device)
    of = torch.empty((m, w.n_rows), dtype=torch.float32, device=x_i8.device) if want_f32 else None
    _check(_lib.bq_linear(_p(x_i8), _p(x_sa), _p(w.data), _p(w.scale), _p(out), _p(of),
                          w.n_rows, m, k, _stream()))
    return (out, of) if want_f32 else out


def block_linear(x_i8, x_sa, w: ButterquantWeight, block: int, want_f32: bool = False, out=None):
    m, k = x_i8.shape
    if out is None:
        out = torch.empty((m, w.n_rows), dtype=torch.bfloat16, device=x_i8.device)
    of = torch.empty((m, w.n_rows), dtype=torch.float32, device=x_i8.device) if want_f32 else None
    _check(_lib.bq_block_linear(_p(x_i8), _p(x_sa), _p(w.data), _p(w.scale), _p(out), _p(of),
                                w.n_rows, k, m, block, _stream()))
    return (out, of) if want_f32 else out


def qkv(x_i8, x_sa, q: ButterquantWeight, k: ButterquantWeight, v: ButterquantWeight, outs=None):
    m, hidden = x_i8.shape
    if v.n_rows != k.n_rows:
        raise ValueError(f"qkv: v has {v.n_rows} rows, k {k.n_rows}; they must match")
    if outs is None:
        outs = tuple(torch.empty((m, w.n_rows), dtype=torch.bfloat16, device=x_i8.device)
                     for w in (q, k, v))
    qo, ko, vo = outs
    _check(_lib.bq_qkv(_p(x_i8), _p(x_sa), _p(q.data), _p(q.scale), _p(k.data), _p(k.scale),
                       _p(v.data), _p(v.scale), _p(qo), _p(ko), _p(vo), q.n_rows, k.n_rows, m,
                       hidden, _stream()))
    return qo, ko, vo


def linear_pair(x_i8, x_sa, w0: ButterquantWeight, w1: ButterquantWeight, outs=None):
    """linear(x, w0) and linear(x, w1) in one launch (the dense FFN's gate and
    up projections)."""
    m, hidden = x_i8.shape
    if outs is None:
        outs = tuple(torch.empty((m, w.n_rows), dtype=torch.bfloat16, device=x_i8.device)
                     for w in (w0, w1))
    o0, o1 = outs
    _check(_lib.bq_linear_pair(_p(x_i8), _p(x_sa), _p(w0.data), _p(w0.scale), _p(w1.data),
                               _p(w1.scale), _p(o0), _p(o1), w0.n_rows, w1.n_rows, m, hidden,
                               _stream()))
    return o0, o1


def norm_linear(x: torch.Tensor, gamma: torch.Tensor, w: ButterquantWeight, block: int = 128,
                sqrt_n=None, n_eps=None, want_f32: bool = False, out=None, act_out=None):
    """norm_quant(x) then linear on its codes, fused into one launch for one
    token; returns out (and the f32 values) plus the activation (x_i8, x_sa)."""
    _dev(x, torch.bfloat16)
    _dev(gamma, torch.bfloat16)
    m, h = x.shape
    if sqrt_n is None:
        sqrt_n, n_eps = norm_consts(h)
    xq, sa = act_out if act_out is not None else (
        torch.empty((m, h), dtype=torch.int8, device=x.device),
        torch.empty(m, dtype=torch.float32, device=x.device))
    if out is None:
        out = torch.empty((m, w.n_rows), dtype=torch.bfloat16, device=x.device)
    of = torch.empty((m, w.n_rows), dtype=torch.float32, device=x.device) if want_f32 else None
    _check(_lib.bq_norm_linear(_p(x), _p(gamma), _p(xq), _p(sa), _p(w.data), _p(w.scale),
                               _p(out), _p(of), w.n_rows, m, h, block, sqrt_n, n_eps, _stream()))
    return ((out, of) if want_f32 else out), (xq, sa)


def norm_qkv(x: torch.Tensor, gamma: torch.Tensor, q: ButterquantWeight, k: ButterquantWeight,
             v: ButterquantWeight, block: int = 128, sqrt_n=None, n_eps=None, outs=None,
             act_out=None):
    """norm_quant(x) then qkv on its codes, fused into one launch for one token."""
    if v.n_rows != k.n_rows:
        raise ValueError(f"norm_qkv: v has {v.n_rows} rows, k {k.n_rows}; they must match")
    _dev(x, torch.bfloat16)
    _dev(gamma, torch.bfloat16)
    m, h = x.shape
    if sqrt_n is None:
        sqrt_n, n_eps = norm_consts(h)
    xq, sa = act_out if act_out is not None else (
        torch.empty((m, h), dtype=torch.int8, device=x.device),
        torch.empty(m, dtype=torch.float32, device=x.device))
    if outs is None:
        outs = tuple(torch.empty((m, wt.n_rows), dtype=torch.bfloat16, device=x.device)
                     for wt in (q, k, v))
    qo, ko, vo = outs
    _check(_lib.bq_norm_qkv(_p(x), _p(gamma), _p(xq), _p(sa), _p(q.data), _p(q.scale),
                            _p(k.data), _p(k.scale), _p(v.data), _p(v.scale), _p(qo), _p(ko),
                            _p(vo), q.n_rows, k.n_rows, m, h, block, sqrt_n, n_eps, _stream()))
    return (qo, ko, vo), (xq, sa)


def norm_linear_pair(x: torch.Tensor, gamma: torch.Tensor, w0: ButterquantWeight,
                     w1: ButterquantWeight, block: int = 128, sqrt_n=None, n_eps=None,
                     outs=None, act_out=None):
    """norm_quant(x) then linear_pair on its codes, one launch for one token."""
    _dev(x, torch.bfloat16)
    _dev(gamma, torch.bfloat16)
    m, h = x.shape
    if sqrt_n is None:
        sqrt_n, n_eps = norm_consts(h)
    xq, sa = act_out if act_out is not None else (
        torch.empty((m, h), dtype=torch.int8, device=x.device),
        torch.empty(m, dtype=torch.float32, device=x.device))
    if outs is None:
        outs = tuple(torch.empty((m, wt.n_rows), dtype=torch.bfloat16, device=x.device)
                     for wt in (w0, w1))
    o0, o1 = outs
    _check(_lib.bq_norm_linear_pair(_p(x), _p(gamma), _p(xq), _p(sa), _p(w0.data),
                                    _p(w0.scale), _p(w1.data), _p(w1.scale), _p(o0), _p(o1),
                                    w0.n_rows, w1.n_rows, m, h, block, sqrt_n, n_eps, _stream()))
    return (o0, o1), (xq, sa)


# --------------------------------------------------------------------------
# MoE
# --------------------------------------------------------------------------

def router_logits(x: torch.Tensor, router_proj: torch.Tensor, router_scale: torch.Tensor,
                  sqrt_n=None, n_eps=None, out=None):
    """bf16 x [T,H], router_proj [E,H], router_scale [H] -> f32 logits [T,E]."""
    _dev(x, torch.bfloat16)
    _dev(router_proj, torch.bfloat16)
    _dev(router_scale, torch.bfloat16)
    t, h = x.shape
    e = router_proj.shape[0]
    if sqrt_n is None:
        sqrt_n, n_eps = norm_consts(h)
    if out is None:
        out = torch.empty((t, e), dtype=torch.float32, device=x.device)
    _check(_lib.bq_moe_router_logits(_p(x), _p(router_proj), _p(router_scale), _p(out), t, h, e,
                                     sqrt_n, n_eps, _stream()))
    return out


def route_topk(logits: torch.Tensor, top_k: int, per_expert_scale: torch.Tensor | None = None,
               out=None):
    """f32 logits [T,E] -> (route_idx int32 [T,k], route_w f32 [T,k])."""
    _dev(logits, torch.float32)
    if per_expert_scale is not None:
        _dev(per_expert_scale, torch.bfloat16)
    t, e = logits.shape
    if out is None:
        idx = torch.empty((t, top_k), dtype=torch.int32, device=logits.device)
        w = torch.empty((t, top_k), dtype=torch.float32, device=logits.device)
    else:
        idx, w = out
    _check(_lib.bq_moe_route_topk(_p(logits), _p(per_expert_scale), t, e, top_k, _p(idx), _p(w),
                                  _stream()))
    return idx, w


def route_schedule(logits: torch.Tensor, top_k: int, per_expert_scale: torch.Tensor | None = None,
                   out=None):
    """route_topk then build_schedule (expert_base 0) in one call:
    f32 logits [T,E] -> (route_idx, route_w, expert_offset, routes)."""
    _dev(logits, torch.float32)
    if per_expert_scale is not None:
        _dev(per_expert_scale, torch.bfloat16)
    t, e = logits.shape
    d = logits.device
    if out is None:
        idx = torch.empty((t, top_k), dtype=torch.int32, device=d)
        w = torch.empty((t, top_k), dtype=torch.float32, device=d)
        eo = torch.empty(e + 1, dtype=torch.int32, device=d)
        routes = torch.zeros((t * top_k, 2), dtype=torch.int32, device=d)
    else:
        idx, w, eo, routes = out
    _check(_lib.bq_moe_route_schedule(_p(logits), _p(per_expert_scale), t, e, top_k, _p(idx), _p(w),
                                      _p(eo), _p(routes), _stream()))
    return idx, w, eo, routes


def moe_prep(logits: torch.Tensor, x: torch.Tensor, gamma: torch.Tensor, top_k: int,
             per_expert_scale: torch.Tensor | None = None, block: int = 128, sqrt_n=None,
             n_eps=None, out=None):
    """route_schedule and norm_quant of the MoE input in one call (one launch
    for decode-sized batches): f32 logits [T,E], bf16 x [T,H], gamma [H] ->
    (route_idx, route_w, expert_offset, routes, x_i8, x_sa)."""
    _dev(logits, torch.float32)
    _dev(x, torch.bfloat16)
    _dev(gamma, torch.bfloat16)
    if per_expert_scale is not None:
        _dev(per_expert_scale, torch.bfloat16)
    t, e = logits.shape
    h = x.shape[1]
    if sqrt_n is None:
        sqrt_n, n_eps = norm_consts(h)
    d = logits.device
    if out is None:
        idx = torch.empty((t, top_k), dtype=torch.int32, device=d)
        w = torch.empty((t, top_k), dtype=torch.float32, device=d)
        eo = torch.empty(e + 1, dtype=torch.int32, device=d)
        routes = torch.zeros((t * top_k, 2), dtype=torch.int32, device=d)
        xq = torch.empty((t, h), dtype=torch.int8, device=d)
        sa = torch.empty(t, dtype=torch.float32, device=d)
    else:
        idx, w, eo, routes, xq, sa = out
    _check(_lib.bq_moe_prep(_p(logits), _p(per_expert_scale), _p(x), _p(gamma), t, e, top_k, h,
                            block, sqrt_n, n_eps, _p(idx), _p(w), _p(eo), _p(routes), _p(xq),
                            _p(sa), _stream()))
    return idx, w, eo, routes, xq, sa


def ffn_prep(logits: torch.Tensor, x: torch.Tensor, gamma: torch.Tensor,
             dense_gamma: torch.Tensor, top_k: int, per_expert_scale: torch.Tensor | None = None,
             block: int = 128, sqrt_n=None, n_eps=None, out=None):
    """moe_prep plus the dense MLP's norm-quant of the same x with dense_gamma
    (bq_ffn_prep: one launch where moe_prep is one) ->
    (route_idx, route_w, expert_offset, routes, x_i8, x_sa, dense_i8, dense_sa)."""
    _dev(logits, torch.float32)
    _dev(x, torch.bfloat16)
    _dev(gamma, torch.bfloat16)
    _dev(dense_gamma, torch.bfloat16)
    if per_expert_scale is not None:
        _dev(per_expert_scale, torch.bfloat16)
    t, e = logits.shape
    h = x.shape[1]
    if sqrt_n is None:
        sqrt_n, n_eps = norm_consts(h)
    d = logits.device
    if out is None:
        idx = torch.empty((t, top_k), dtype=torch.int32, device=d)
        w = torch.empty((t, top_k), dtype=torch.float32, device=d)
        eo = torch.empty(e + 1, dtype=torch.int32, device=d)
        routes = torch.zeros((t * top_k, 2), dtype=torch.int32, device=d)
        xq = torch.empty((t, h), dtype=torch.int8, device=d)
        sa = torch.empty(t, dtype=torch.float32, device=d)
        dq = torch.empty((t, h), dtype=torch.int8, device=d)
        dsa = torch.empty(t, dtype=torch.float32, device=d)
    else:
        idx, w, eo, routes, xq, sa, dq, dsa = out
    _check(_lib.bq_ffn_prep(_p(logits), _p(per_expert_scale), _p(x), _p(gamma), _p(dense_gamma),
                            t, e, top_k, h, block, sqrt_n, n_eps, _p(idx), _p(w), _p(eo),
                            _p(routes), _p(xq), _p(sa), _p(dq), _p(dsa), _stream()))
    return idx, w, eo, routes, xq, sa, dq, dsa


def build_schedule(route_idx: torch.Tensor, route_w: torch.Tensor, experts: int,
                   expert_base: int = 0, out=None):
    """-> (expert_offset int32 [E+1], routes int32 [T*k, 2] = {token, weight bits})."""
    _dev(route_idx, torch.int32)
    _dev(route_w, torch.float32)
    t, k = route_idx.shape
    if out is None:
        eo = torch.empty(experts + 1, dtype=torch.int32, device=route_idx.device)
        routes = torch.zeros((t * k, 2), dtype=torch.int32, device=route_idx.device)
    else:
        eo, routes = out
    _check(_lib.bq_moe_build_schedule(_p(route_idx), _p(route_w), t, k, expert_base, experts,
                                      _p(eo), _p(routes), _stream()))
    return eo, routes


def moe_phase1(x_i8, x_sa, eo, routes, w_gu: ButterquantWeight, experts: int, seq_len: int,
               top_k: int, inter: int, out=None):
    hidden = x_i8.shape[1]
    if out is None:
        out = torch.empty((seq_len * top_k, inter), dtype=torch.bfloat16, device=x_i8.device)
    _check(_lib.bq_moe_phase1_gate_up(_p(x_i8), _p(x_sa), _p(eo), _p(routes), _p(w_gu.data),
                                      _p(w_gu.scale), _p(out), experts, seq_len, top_k, hidden,
                                      inter, _stream()))
    return out


def moe_phase1_quant(x_i8, x_sa, eo, routes, w_gu: ButterquantWeight, experts: int,
                     seq_len: int, top_k: int, inter: int, bucket=False, out=None):
    """bq_moe_phase1_gate_up_quant: phase 1 with the bucket's FWHT64
    block-quant fused -> (bucket_i8, bucket_sa[, bucket bf16 if bucket])."""
    hidden = x_i8.shape[1]
    dev = x_i8.device
    R = seq_len * top_k
    if out is None:
        bi8 = torch.empty((R, inter), dtype=torch.int8, device=dev)
        bsa = torch.empty((R, inter // 64), dtype=torch.float32, device=dev)
        bb = torch.empty((R, inter), dtype=torch.bfloat16, device=dev) if bucket else None
    else:
        bi8, bsa, bb = out
    _check(_lib.bq_moe_phase1_gate_up_quant(_p(x_i8), _p(x_sa), _p(eo), _p(routes),
                                            _p(w_gu.data), _p(w_gu.scale), _p(bb), _p(bi8),
                                            _p(bsa), experts, seq_len, top_k, hidden, inter,
                                            _stream()))
    return (bi8, bsa, bb) if bb is not None else (bi8, bsa)


def moe_phase2_workspace_size(seq_len: int, top_k: int, hidden: int) -> int:
    return int(_lib.bq_moe_phase2_workspace_size(seq_len, top_k, hidden))


def moe_phase2(b_i8, b_sa, eo, routes, w_d: ButterquantWeight, experts: int, seq_len: int,
               top_k: int, hidden: int, block: int = 64, workspace=None, out=None):
    inter = b_i8.shape[1]
    dev = b_i8.device
    if workspace is None:
        nbytes = max(moe_phase2_workspace_size(seq_len, top_k, hidden), 256)
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    if out is None:
        accum = torch.empty((seq_len, hidden), dtype=torch.float32, device=dev)
        o = torch.empty((seq_len, hidden), dtype=torch.bfloat16, device=dev)
    else:
        accum, o = out
    _check(_lib.bq_moe_phase2_down(_p(b_i8), _p(b_sa), _p(eo), _p(routes), _p(w_d.data),
                                   _p(w_d.scale), _p(accum), _p(o), experts, seq_len, top_k,
                                   hidden, inter, block, _p(workspace), workspace.numel(),
                                   _stream()))
    return accum, o


def moe_phase2_noalloc(b_i8, b_sa, eo, routes, w_d: ButterquantWeight, experts: int,
                       seq_len: int, top_k: int, hidden: int, block: int = 64, out=None):
    """bq_moe_phase2_down_noalloc: phase 2 on the library's static scratch
    (no workspace); seq_len * top_k * hidden * 4 bytes <= 24 MiB."""
    inter = b_i8.shape[1]
    dev = b_i8.device
    if out is None:
        accum = torch.empty((seq_len, hidden), dtype=torch.float32, device=dev)
        o = torch.empty((seq_len, hidden), dtype=torch.bfloat16, device=dev)
    else:
        accum, o = out
    _check(_lib.bq_moe_phase2_down_noalloc(_p(b_i8), _p(b_sa), _p(eo), _p(routes), _p(w_d.data),
                                           _p(w_d.scale), _p(accum), _p(o), experts, seq_len,
                                           top_k, hidden, inter, block, _stream()))
    return accum, o


def ffn_gate_up(x_i8, x_sa, eo, routes, w_gu: ButterquantWeight, experts: int, seq_len: int,
                top_k: int, inter: int, dense_x_i8, dense_x_sa, dense_gate: ButterquantWeight,
                dense_up: ButterquantWeight, out=None):
    """bq_ffn_gate_up: moe_phase1_quant plus the dense MLP's gate/up, GELU and
    FWHT64 block-quant of the same tokens in the experts' launch ->
    (bucket_i8, bucket_sa, dense_i8, dense_sa)."""
    hidden = x_i8.shape[1]
    dev = x_i8.device
    R, di = seq_len * top_k, dense_gate.n_rows
    if dense_up.n_rows != di or dense_gate.k != hidden or dense_up.k != hidden:
        raise ValueError("dense gate and up must both be [dense_inter, hidden]")
    if out is None:
        bi8 = torch.empty((R, inter), dtype=torch.int8, device=dev)
        bsa = torch.empty((R, inter // 64), dtype=torch.float32, device=dev)
        dq = torch.empty((seq_len, di), dtype=torch.int8, device=dev)
        dsa = torch.empty((seq_len, di // 64), dtype=torch.float32, device=dev)
    else:
        bi8, bsa, dq, dsa = out
    _check(_lib.bq_ffn_gate_up(_p(x_i8), _p(x_sa), _p(eo), _p(routes), _p(w_gu.data),
                               _p(w_gu.scale), _p(bi8), _p(bsa), experts, seq_len, top_k, hidden,
                               inter, _p(dense_x_i8), _p(dense_x_sa), _p(dense_gate.data),
                               _p(dense_gate.scale), _p(dense_up.data), _p(dense_up.scale), di,
                               _p(dq), _p(dsa), _stream()))
    return bi8, bsa, dq, dsa


def ffn_down(b_i8, b_sa, eo, routes, w_d: ButterquantWeight, experts: int, seq_len: int,
             top_k: int, hidden: int, dense_i8, dense_sa, dense_down: ButterquantWeight,
             block: int = 64, workspace=None, out=None):
    """bq_ffn_down: moe_phase2 plus the dense MLP's per-block down projection
    of the same tokens in the experts' launch -> (accum, out, dense_out)."""
    inter = b_i8.shape[1]
    dev = b_i8.device
    if dense_down.n_rows != hidden or dense_down.k != dense_i8.shape[1]:
        raise ValueError("dense down must be [hidden, dense_inter]")
    if workspace is None:
        nbytes = max(moe_phase2_workspace_size(seq_len, top_k, hidden), 256)
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    if out is None:
        accum = torch.empty((seq_len, hidden), dtype=torch.float32, device=dev)
        o = torch.empty((seq_len, hidden), dtype=torch.bfloat16, device=dev)
        do = torch.empty((seq_len, hidden), dtype=torch.bfloat16, device=dev)
    else:
        accum, o, do = out
    _check(_lib.bq_ffn_down(_p(b_i8), _p(b_sa), _p(eo), _p(routes), _p(w_d.data), _p(w_d.scale),
                            _p(accum), _p(o), experts, seq_len, top_k, hidden, inter, block,
                            _p(dense_i8), _p(dense_sa), _p(dense_down.data),
                            _p(dense_down.scale), dense_down.k, _p(do), _p(workspace),
                            workspace.numel(), _stream()))
    return accum, o, do


# --------------------------------------------------------------------------
# vocabulary head and embedding
# --------------------------------------------------------------------------
SAMPLE_NMAX = 256
PARAMS_BYTES, OUTCOME_BYTES = 40, 2064


def head_prep(x: torch.Tensor, gamma: torch.Tensor, block: int = 128, sqrt_n=None, n_eps=None,
              out=None):
    """dispatch_bq_head_prep: per-block norm-quant -> (int8 [R,H], sa [R, H/block])."""
    _dev(x, torch.bfloat16)
    _dev(gamma, torch.bfloat16)
    r, h = x.shape
    if sqrt_n is None:
        sqrt_n, n_eps = norm_consts(h)
    if out is None:
        xq = torch.empty((r, h), dtype=torch.int8, device=x.device)
        sa = torch.empty((r, h // block), dtype=torch.float32, device=x.device)
    else:
        xq, sa = out
    _check(_lib.bq_head_prep(_p(x), _p(gamma), _p(xq), _p(sa), r, h, block, sqrt_n, n_eps,
                             _stream()))
    return xq, sa


def flash_sample_workspace_size(rows: int, vocab: int) -> int:
    return int(_lib.bq_flash_sample_workspace_size(rows, vocab))


def flash_sample(x_i8, x_sa, weight: ButterquantWeight, wscales, params: torch.Tensor,
                 block: int = 128, cap: float = 30.0, vocab_base: int = 0, workspace=None,
                 out=None):
    """dispatch_bq_flash_sample.  params: uint8 device tensor [R, 40] holding
    SamplingParams; returns uint8 [R, 2064] SampleOutcome records."""
    r, h = x_i8.shape
    vocab = weight.n_rows
    if params.dtype != torch.uint8 or tuple(params.shape) != (r, PARAMS_BYTES):
        raise ValueError("params: uint8 [rows, 40] SamplingParams records")
    if workspace is None:
        workspace = torch.empty(max(flash_sample_workspace_size(r, vocab), 256),
                                dtype=torch.uint8, device=x_i8.device)
    if out is None:
        out = torch.empty((r, OUTCOME_BYTES), dtype=torch.uint8, device=x_i8.device)
    _check(_lib.bq_flash_sample(_p(x_i8), _p(x_sa), _p(weight.data), _p(wscales), _p(params),
                                _p(out), r, vocab, h, block, cap, vocab_base, _p(workspace),
                                workspace.numel(), _stream()))
    return out


def embed_lookup(token_ids: torch.Tensor, weight: ButterquantWeight, wscales: torch.Tensor,
                 block: int = 128, scale: float | None = None, shard_rows: int | None = None,
                 rank: int = 0, out=None):
    """dispatch_bq_embed_lookup -> bf16 [T, H]."""
    _dev(token_ids, torch.int32)
    t = token_ids.shape[0]
    h = weight.k
    if scale is None:
        import numpy as np
        s = np.sqrt(np.float32(h), dtype=np.float32)
        scale = float(torch.tensor(float(s)).to(torch.bfloat16).float())
    if shard_rows is None:
        shard_rows = weight.n_rows
    if out is None:
        out = torch.empty((t, h), dtype=torch.bfloat16, device=token_ids.device)
    _check(_lib.bq_embed_lookup(_p(token_ids), _p(weight.data), _p(wscales), _p(out), t, h, block,
                                shard_rows, rank, scale, _stream()))
    return out


# --------------------------------------------------------------------------
# int8-KV attention
# --------------------------------------------------------------------------
def attn_prep(q_src, k_src, v_src, q_norm, k_norm, k_cache, k_scale, v_cache, v_scale,
              cos_table, sin_table, runs, base_rows, num_q: int, num_kv: int, head_dim: int,
              rope_half: int, pair_stride: int, page_shift: int, row_mask: int,
              page_mask: int, sqrt_n: float | None = None, n_eps: float | None = None,
              cache_degree: int = 1, rank: int = 0, out=None):
    """dispatch_bq_attn_prep -> (q_i8 [T, num_q*hd], qi_bias [T, num_q],
    f_q [T, num_q]); K/V rows and scales are written into the caches.
    runs: int32 [num_runs, 4] (buf_start, base_pos, rows_off, page_count)."""
    for t in (q_src, k_src, v_src, q_norm, k_norm):
        _dev(t, torch.bfloat16)
    for t in (k_cache, v_cache):
        _dev(t, torch.int8)
    for t in (k_scale, v_scale, cos_table, sin_table):
        _dev(t, torch.float32)
    _dev(runs, torch.int32)
    _dev(base_rows, torch.int32)
    T = q_src.shape[0]
    if sqrt_n is None:
        import numpy as np
        sqrt_n = float(np.sqrt(np.float32(head_dim), dtype=np.float32))
        n_eps = float(np.float32(head_dim) * np.float32(1e-6))
    if out is None:
        d = q_src.device
        out = (torch.empty((T, num_q * head_dim), dtype=torch.int8, device=d),
               torch.empty((T, num_q), dtype=torch.float32, device=d),
               torch.empty((T, num_q), dtype=torch.float32, device=d))
    q_i8, qi_bias, f_q = out
    _check(_lib.bq_attn_prep(_p(q_src), _p(k_src), _p(v_src), _p(q_norm), _p(k_norm), _p(q_i8),
                             _p(qi_bias), _p(f_q), _p(k_cache), _p(k_scale), _p(v_cache),
                             _p(v_scale), _p(cos_table), _p(sin_table), _p(runs), runs.shape[0],
                             _p(base_rows), num_q, num_kv, head_dim, rope_half, pair_stride,
                             sqrt_n, n_eps, cache_degree, rank, page_shift, row_mask, page_mask,
                             T, _stream()))
    return q_i8, qi_bias, f_q


def attention_splits(seq_len: int, num_kv: int, max_kv_len: int) -> int:
    return int(_lib.bq_attention_splits(seq_len, num_kv, max_kv_len))


def attention_workspace(seq_len: int, num_q: int, head_dim: int, s_max: int, device="cuda"):
    n = int(_lib.bq_attention_workspace_size(seq_len, num_q, head_dim, s_max))
    return torch.empty(max(n, 16), dtype=torch.uint8, device=device)


def attention(q_i8, qi_bias, f_q, k_cache, k_scale, v_cache, v_scale, runs, base_rows,
              num_q: int, num_kv: int, head_dim: int, window: int, page_shift: int,
              row_mask: int, page_mask: int, s_max: int | None = None,
              max_kv_len: int | None = None, workspace=None, out=None):
    """dispatch_bq_sliding_attention (window > 0) or dispatch_bq_full_attention
    (window == 0) -> bf16 [T, num_q*hd].  Returns (out, s_max)."""
    _dev(q_i8, torch.int8)
    T = q_i8.shape[0]
    if s_max is None:
        s_max = attention_splits(T, num_kv, max_kv_len if max_kv_len else max(window, 1))
    if workspace is None:
        workspace = attention_workspace(T, num_q, head_dim, s_max, q_i8.device)
    if out is None:
        out = torch.empty((T, num_q * head_dim), dtype=torch.bfloat16, device=q_i8.device)
    common = (_p(q_i8), _p(qi_bias), _p(f_q), _p(k_cache), _p(k_scale), _p(v_cache),
              _p(v_scale), _p(out), _p(workspace), workspace.numel(), _p(runs), runs.shape[0],
              _p(base_rows), num_q, num_kv, head_dim)
    if window > 0:
        rc = _lib.bq_sliding_attention(*common, window, page_shift, row_mask, page_mask, s_max,
                                       T, _stream())
    else:
        rc = _lib.bq_full_attention(*common, page_shift, row_mask, page_mask, s_max, T,
                                    _stream())
    _check(rc)
    return out, s_max


# --------------------------------------------------------------------------
# on-disk weights (safetensors)
# --------------------------------------------------------------------------
DT_NAMES = ["BOOL", "U8", "I8", "I16", "U16", "F16", "BF16", "I32", "U32", "F32", "F64",
            "F8_E4M3", "F8_E5M2", "I64", "U64"]


class SafetensorsFile:
    """A memory-mapped safetensors shard parsed by libbq (host only)."""

    handle = None

    def __init__(self, path: str):
        h = C.c_void_p()
        _check(_lib.bq_st_open(os.fsencode(path), C.byref(h)))
        self.handle = h

    def close(self):
        if self.handle:
            _lib.bq_st_close(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def __len__(self):
        return _lib.bq_st_num_tensors(self.handle)

    def info(self, name: str):
        """-> (dtype tag, shape, nbytes, host address)."""
        dt, nd = C.c_int(), C.c_int()
        shape = (C.c_int64 * 8)()
        nbytes, data = C.c_size_t(), C.c_void_p()
        _check(_lib.bq_st_tensor_info(self.handle, name.encode(), C.byref(dt), C.byref(nd), shape,
                                      C.byref(nbytes), C.byref(data)))
        return DT_NAMES[dt.value], tuple(shape[i] for i in range(nd.value)), nbytes.value, data.value


def load_quantized(files, name: str, n_rows: int, k: int, scale_cols: int = 1,
                   staging: torch.Tensor | None = None, out=None) -> ButterquantWeight:
    """bq_load_quantized: codes "<name>" + scales "<name>.scale" from the
    shards -> ButterquantWeight (tile16x64 codes, f32 scales) on the device."""
    arr = (C.c_void_p * len(files))(*[f.handle for f in files])
    if staging is None:
        staging = torch.empty(min(n_rows * k, 64 << 20) // (16 * k) * 16 * k or 16 * k,
                              dtype=torch.int8, device="cuda")
    if out is None:
        w = torch.empty(n_rows * k, dtype=torch.int8, device="cuda")
        s = torch.empty((n_rows,) if scale_cols == 1 else (n_rows, scale_cols), dtype=torch.float32,
                        device="cuda")
    else:
        w, s = out
    _check(_lib.bq_load_quantized(arr, len(files), name.encode(), n_rows, k, scale_cols, _p(w),
                                  _p(s), _p(staging), staging.numel(), _stream()))
    return ButterquantWeight(w, s, n_rows, k)
