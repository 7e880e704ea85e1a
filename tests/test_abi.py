"""CPU-side checks of the C ABI: libbq.so loads, exports every entry point
include/bq_api.h declares, and rejects contract violations with the
documented status codes before touching the GPU (the reference enforces
these contracts with compile-time asserts / debug_assert / abort)."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "bq_api.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bq_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    import bq
    return bq.lib()


def test_header_symbols_exported(L):
    names = declared_functions()
    assert len(names) >= 17
    for n in names:
        assert hasattr(L, n), f"libbq.so does not export {n}"


def test_binding_covers_header():
    import bq
    assert set(declared_functions()) == set(bq.SIGNATURES)


def test_version(L):
    assert b"gfx950" in L.bq_version()


P = C.c_void_p(16)  # a non-null placeholder: validation fails before any use


def test_validation_errors(L):
    # null pointers
    assert L.bq_linear(None, P, P, P, P, None, 64, 1, 128, None) == 1
    assert b"null" in L.bq_last_error()
    # shape contracts (linear.mojo:132-136; vnni.mojo:91-99)
    assert L.bq_linear(P, P, P, P, P, None, 15, 1, 128, None) == 2
    assert L.bq_linear(P, P, P, P, P, None, 64, 1, 100, None) == 2
    assert L.bq_block_linear(P, P, P, P, P, None, 64, 256, 1, 96, None) == 2
    assert L.bq_block_linear(P, P, P, P, P, None, 64, 8192, 1, 64, None) == 4
    assert L.bq_weight_retile(P, 0, P, 24, 128, None) == 2
    assert L.bq_weight_retile(P, 7, P, 32, 128, None) == 1
    assert L.bq_weight_retile(P, 1, P, 48, 128, None) == 2
    assert L.bq_pack_colsum_vnni(P, C.c_void_p(32), P, 32, 100, 64, 1, None) == 2
    assert L.bq_pack_colsum_vnni(P, C.c_void_p(32), P, 32, 128, 24, 1, None) == 2
    assert L.bq_quantize_weight(P, None, P, P, 4, 256, 48, 0, None) == 2
    assert L.bq_quantize_weight(P, None, P, P, 4, 32768, 128, 0, None) == 4
    assert L.bq_norm_quant(P, P, P, P, 1, 2816, 48, C.c_float(1), C.c_float(1), None) == 2
    assert L.bq_norm_quant(P, P, P, P, 1, 2880, 128, C.c_float(1), C.c_float(1), None) == 2
    assert L.bq_block_quant(P, P, P, 704, 1, 256, 0, None) == 2
    assert L.bq_moe_build_schedule(P, P, 4, 8, 0, 512, P, P, None) == 4
    assert L.bq_moe_route_topk(P, None, 4, 128, 17, P, P, None) == 4
    assert L.bq_head_prep(P, P, P, P, 2, 2816, 96, C.c_float(1), C.c_float(1), None) == 2
    assert L.bq_head_prep(C.c_void_p(18), P, P, P, 2, 2816, 128, C.c_float(1), C.c_float(1),
                          None) == 1
    ws = C.c_void_p(256)
    assert L.bq_flash_sample(P, P, P, P, P, P, 33, 4096, 2816, 128, C.c_float(30), 0, ws,
                             1 << 30, None) == 4
    assert L.bq_flash_sample(P, P, P, P, P, P, 2, 4100, 2816, 128, C.c_float(30), 0, ws,
                             1 << 30, None) == 2
    assert L.bq_flash_sample(P, P, P, P, P, P, 2, 4096, 2816, 128, C.c_float(30), 0, ws,
                             16, None) == 2
    assert L.bq_flash_sample(P, P, P, P, P, P, 2, 4096, 2816, 128, C.c_float(30), 0,
                             C.c_void_p(272), 1 << 30, None) == 1
    assert L.bq_embed_lookup(P, P, P, P, 3, 2816, 100, 64, 0, C.c_float(1), None) == 2
    assert L.bq_moe_route_topk(P, None, 4, 2048, 8, P, P, None) == 4
    assert L.bq_moe_route_topk(P, None, 4, 128, 0, P, P, None) == 2
    assert L.bq_moe_route_topk(None, None, 4, 128, 8, P, P, None) == 1
    assert L.bq_moe_route_schedule(P, None, 4, 512, 8, P, P, P, P, None) == 4
    assert L.bq_moe_route_schedule(P, None, 4, 128, 17, P, P, P, P, None) == 4
    assert L.bq_moe_route_schedule(P, None, 4, 128, 0, P, P, P, P, None) == 2
    assert L.bq_moe_route_schedule(P, None, 4, 128, 8, P, P, None, P, None) == 1
    assert L.bq_moe_route_schedule(P, None, 0, 128, 8, None, None, None, None, None) == 0
    f1 = C.c_float(1)
    prep = lambda T, E, k, H, B, *ptrs: L.bq_moe_prep(P, None, P, P, T, E, k, H, B, f1, f1,
                                                      *ptrs, None)
    assert prep(0, 128, 8, 2816, 128, *([None] * 6)) == 0                 # empty batch
    assert prep(4, 128, 8, 2816, 128, P, P, None, P, P, P) == 1          # null expert_offset
    assert prep(4, 512, 8, 2816, 128, P, P, P, P, P, P) == 4             # experts > 256
    assert prep(4, 128, 0, 2816, 128, P, P, P, P, P, P) == 2             # top_k
    assert prep(4, 128, 8, 2816, 48, P, P, P, P, P, P) == 2              # FWHT block
    assert prep(4, 128, 8, 2880, 128, P, P, P, P, P, P) == 2             # hidden % block
    fprep = lambda T, E, k, H, B, *ptrs: L.bq_ffn_prep(P, None, P, P, P, T, E, k, H, B, f1, f1,
                                                       *ptrs, None)
    assert fprep(0, 128, 8, 2816, 128, *([None] * 8)) == 0               # empty batch
    assert fprep(4, 128, 8, 2816, 128, P, P, P, P, P, P, None, P) == 1   # null dense codes
    assert fprep(4, 512, 8, 2816, 128, *([P] * 8)) == 4                  # experts > 256
    assert fprep(4, 128, 0, 2816, 128, *([P] * 8)) == 2                  # top_k
    assert fprep(4, 128, 8, 2880, 128, *([P] * 8)) == 2                  # hidden % block
    assert L.bq_ffn_prep(P, None, P, P, None, 4, 128, 8, 2816, 128, f1, f1, *([P] * 8),
                         None) == 1                                       # null dense gain
    # bq_ffn_gate_up: bq_moe_phase1_gate_up_quant's checks plus the dense MLP's
    fgu = lambda E, T, k, H, I, DI, *dense: L.bq_ffn_gate_up(*([P] * 8), E, T, k, H, I, *dense,
                                                           DI, P, P, None)
    assert fgu(128, 0, 8, 2816, 704, 2112, *([None] * 6)) == 0          # empty batch
    assert fgu(128, 4, 8, 2816, 704, 2112, P, P, P, P, None, P) == 1    # null dense up
    assert fgu(128, 4, 8, 2816, 704, 2100, *([P] * 6)) == 2             # dense_inter % 64
    assert fgu(128, 4, 8, 2816, 700, 2112, *([P] * 6)) == 2             # inter % 64
    assert fgu(128, 4, 8, 2816, 704, 2112, C.c_void_p(24), *([P] * 5)) == 1  # alignment
    # bq_ffn_down: bq_moe_phase2_down's checks plus the dense MLP's
    fdn = lambda T, k, H, I, B, DI, *dense: L.bq_ffn_down(*([P] * 8), 128, T, k, H, I, B, *dense,
                                                          DI, P, C.c_void_p(256), 1 << 30, None)
    assert fdn(0, 8, 2816, 704, 64, 2112, *([None] * 4)) == 0           # empty batch
    assert fdn(4, 8, 2816, 704, 64, 2112, P, P, None, P) == 1           # null dense down
    assert fdn(4, 8, 2816, 704, 64, 2100, *([P] * 4)) == 2              # dense_inter % block
    assert fdn(4, 8, 2816, 704, 64, 8192, *([P] * 4)) == 4              # dense_inter / block
    assert fdn(4, 17, 2816, 704, 64, 2112, *([P] * 4)) == 4             # top_k
    assert fdn(4, 8, 2816, 704, 64, 2112, C.c_void_p(24), P, P, P) == 1  # alignment
    assert L.bq_moe_router_logits(P, P, P, P, 4, 2880 + 32, 128, C.c_float(1), C.c_float(1),
                                  None) == 2
    assert L.bq_moe_router_logits(P, C.c_void_p(18), P, P, 4, 2816, 128, C.c_float(1),
                                  C.c_float(1), None) == 1
    assert L.bq_moe_phase2_down(P, P, P, P, P, P, P, P, 128, 4, 8, 2816, 704, 64,
                                C.c_void_p(256), 0, None) == 2
    assert L.bq_moe_phase2_down(P, P, P, P, P, P, P, P, 128, 4, 8, 2816, 704, 64,
                                C.c_void_p(100), 1 << 30, None) == 1
    # the allocation-free phase 2 validates exactly as the workspace entry point
    ws = C.c_void_p(256)
    for args, code in (((128, 4, 8, 0, 704, 64), 2),        # hidden <= 0
                       ((128, 4, 8, 2816 + 8, 704, 64), 2),  # hidden % 16
                       ((128, 4, 0, 2816, 704, 64), 4),      # top_k
                       ((128, 4, 17, 2816, 704, 64), 4),
                       ((128, 4, 8, 2816, 700, 64), 2),      # inter % block
                       ((128, 4, 8, 2816, 704, 96), 2)):     # block
        assert L.bq_moe_phase2_down(*([P] * 8), *args, ws, 1 << 30, None) == code
        assert L.bq_moe_phase2_down_noalloc(*([P] * 8), *args, None) == code
    assert L.bq_moe_phase2_down_noalloc(*([P] * 7), None, 128, 4, 8, 2816, 704, 64, None) == 1
    f1 = C.c_float(1)
    nl = lambda *a: L.bq_norm_linear(*a, f1, f1, None)
    assert nl(P, P, P, P, P, P, P, None, 256, 1, 2816, 48) == 2        # FWHT block
    assert nl(P, P, P, P, P, P, P, None, 250, 1, 2816, 128) == 2       # n_rows % 16
    assert nl(P, P, P, P, P, P, P, None, 256, 1, 2880, 128) == 2       # hidden % block
    assert nl(P, P, None, P, P, P, P, None, 256, 1, 2816, 128) == 1    # x_i8
    assert nl(P, P, P, P, None, P, P, None, 256, 1, 2816, 128) == 1    # weights
    assert nl(P, P, C.c_void_p(264), P, P, P, P, None, 256, 1, 2816, 128) == 1  # alignment
    assert L.bq_norm_qkv(*([P] * 13), 4096, 2050, 1, 2816, 128, f1, f1, None) == 2
    assert L.bq_norm_qkv(*([P] * 12), None, 4096, 2048, 1, 2816, 128, f1, f1, None) == 1
    assert L.bq_linear_pair(*([P] * 8), 2112, 2100, 16, 2816, None) == 2   # n1 % 16
    assert L.bq_linear_pair(*([P] * 8), 2112, 2112, 16, 2880 + 8, None) == 2  # hidden % 64
    assert L.bq_linear_pair(*([P] * 7), None, 2112, 2112, 16, 2816, None) == 1
    assert L.bq_linear_pair(C.c_void_p(264), *([P] * 7), 2112, 2112, 16, 2816, None) == 1
    assert L.bq_norm_linear_pair(*([P] * 10), 2112, 2112, 1, 2816, 48, f1, f1, None) == 2
    assert L.bq_norm_linear_pair(*([P] * 9), None, 2112, 2112, 1, 2816, 128, f1, f1,
                                 None) == 1



def test_attention_validation(L):
    f1 = C.c_float(1)
    prep = lambda hd, rh, ps, deg=1, rank=0: L.bq_attn_prep(
        *([P] * 15), 1, P, 16, 8, hd, rh, ps, f1, f1, deg, rank, 10, 1023, 1, 4, None)
    assert prep(192, 64, 64) == 2                     # head_dim
    assert prep(256, 96, 128) == 2                    # rope_half % 64
    assert prep(256, 128, 192) == 2                   # pair_stride + rope_half > head_dim
    assert prep(512, 64, 256, deg=2, rank=2) == 2     # rank >= cache_degree
    assert L.bq_attn_prep(*([P] * 14), None, 1, P, 16, 8, 256, 128, 128, f1, f1, 1, 0, 10,
                          1023, 1, 4, None) == 1
    ws = C.c_void_p(256)
    need = L.bq_attention_workspace_size(4, 16, 256, 8)
    assert need == 4 * 16 * 8 * 258 * 4
    slide = lambda nq, nkv, hd, window, wsb, s_max=8, wsp=ws: L.bq_sliding_attention(
        *([P] * 8), wsp, wsb, P, 1, P, nq, nkv, hd, window, 10, 1023, 1, s_max, 4, None)
    assert slide(16, 8, 256, 0, need) == 2            # window
    assert slide(16, 6, 256, 1024, need) == 2         # num_q % num_kv
    assert slide(96, 3, 256, 1024, need) == 2         # gqa 32
    assert slide(16, 8, 320, 1024, need) == 2         # head_dim
    assert slide(16, 8, 256, 1024, need - 4) == 2     # workspace
    assert slide(16, 8, 256, 1024, need, wsp=C.c_void_p(264)) == 1
    assert L.bq_full_attention(*([P] * 8), ws, need, P, 1, P, 16, 2, 512, 10, 1023, -1, 0, 4,
                               None) == 2              # s_max
    assert L.bq_attention_splits(1, 8, 1024) == 32
    assert L.bq_attention_splits(2048, 8, 1024) == 1
    assert L.bq_attention_splits(16, 2, 100) == 4


def test_empty_batches_are_noops(L):
    # seq_len <= 0 returns early (linear.mojo:134-135, 255-256; moe.mojo:317-318)
    assert L.bq_linear(None, None, None, None, None, None, 64, 0, 128, None) == 0
    assert L.bq_block_linear(None, None, None, None, None, None, 64, 256, 0, 64, None) == 0
    assert L.bq_norm_quant(None, None, None, None, 0, 2816, 128, C.c_float(1), C.c_float(1), None) == 0
    assert L.bq_block_quant(None, None, None, 704, -1, 64, 1, None) == 0
    assert L.bq_moe_route_topk(None, None, 0, 128, 8, None, None, None) == 0
    assert L.bq_moe_router_logits(None, None, None, None, 0, 2816, 128, C.c_float(1),
                                  C.c_float(1), None) == 0
    assert L.bq_moe_phase2_down(None, None, None, None, None, None, None, None, 128, 0, 8, 2816,
                                704, 64, None, 0, None) == 0
    assert L.bq_full_attention(*([None] * 9), 0, None, 1, None, 16, 2, 512, 10, 1023, -1, 1, 0,
                               None) == 0
    assert L.bq_sliding_attention(*([None] * 9), 0, None, 1, None, 16, 8, 256, 1024, 10, 1023, 1,
                                  1, 0, None) == 0
    assert L.bq_qkv(*([None] * 11), 256, 128, 0, 2816, None) == 0
    assert L.bq_norm_linear(*([None] * 8), 256, 0, 2816, 128, C.c_float(1), C.c_float(1),
                            None) == 0
    assert L.bq_norm_qkv(*([None] * 13), 256, 128, 0, 2816, 128, C.c_float(1), C.c_float(1),
                         None) == 0
    assert L.bq_linear_pair(*([None] * 8), 2112, 2112, 0, 2816, None) == 0
    assert L.bq_norm_linear_pair(*([None] * 10), 2112, 2112, 0, 2816, 128, C.c_float(1),
                                 C.c_float(1), None) == 0
    assert L.bq_moe_build_schedule(None, None, 0, 8, 0, 128, None, None, None) == 0
    assert L.bq_moe_phase1_gate_up(*([None] * 7), 128, 0, 8, 2816, 704, None) == 0
    assert L.bq_head_prep(None, None, None, None, 0, 2816, 128, C.c_float(1), C.c_float(1),
                          None) == 0
    assert L.bq_flash_sample(*([None] * 6), 0, 262144, 2816, 128, C.c_float(30), 0, None, 0,
                             None) == 0
    assert L.bq_embed_lookup(None, None, None, None, 0, 2816, 128, 262144, 0, C.c_float(1),
                             None) == 0
    assert L.bq_attn_prep(*([None] * 15), 1, None, 16, 8, 256, 128, 128, C.c_float(16),
                          C.c_float(1), 1, 0, 10, 1023, 1, 0, None) == 0


def test_workspace_size(L):
    # per-route f32 down-projection rows
    T, k, H = 32, 8, 2816
    n = L.bq_moe_phase2_workspace_size(T, k, H)
    assert n >= T * k * H * 4 and n % 256 == 0
    assert L.bq_moe_phase2_workspace_size(0, 8, H) == 0


def test_calib_library_exports():
    """libbq_calib.so (the benchmark's streaming-read and MFMA measurement
    kernels) loads and rejects out-of-contract launches before any GPU call."""
    path = os.path.join(ROOT, "mojo-gemma4-cpu_amd", "libbq_calib.so")
    lib = C.CDLL(path)
    for n in ("bqc_stream_read", "bqc_stream_sweep", "bqc_stream_shapes", "bqc_stream_shape",
              "bqc_mfma_i8", "bqc_mfma_i8_ops", "bqc_lds_read", "bqc_dma_l2", "bqc_mfma_chain",
              "bqc_vmem_l2"):
        assert hasattr(lib, n)
    lib.bqc_stream_read.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                    C.c_void_p]
    lib.bqc_stream_sweep.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                     C.c_void_p]
    lib.bqc_stream_shape.argtypes = [C.c_int, C.c_void_p]
    n_shapes = lib.bqc_stream_shapes()
    assert n_shapes >= 10
    desc = (C.c_int * 4)()
    for i in range(n_shapes):   # every shape reads the 64 fragments of a 4096-wide tile
        assert lib.bqc_stream_shape(i, desc) == 0
        w, u, spw, ks = list(desc)
        assert w * u * ks == 64 and spw >= 1
    assert lib.bqc_stream_shape(n_shapes, desc) != 0
    assert lib.bqc_stream_sweep(P, 256, n_shapes, 0, P, None) != 0   # no such shape
    assert lib.bqc_stream_sweep(C.c_void_p(17), 256, 0, 0, P, None) != 0  # misaligned
    lib.bqc_mfma_i8.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    lib.bqc_mfma_i8_ops.argtypes = [C.c_int, C.c_int, C.c_int]
    lib.bqc_mfma_i8_ops.restype = C.c_double
    assert lib.bqc_stream_read(P, 256, 65, 16, P, None) != 0      # K64 beyond the one-shot shape
    assert lib.bqc_stream_read(C.c_void_p(17), 256, 64, 16, P, None) != 0  # misaligned
    assert lib.bqc_stream_read(P, 256, 64, 12, P, None) != 0      # waves
    assert lib.bqc_mfma_i8(24, 4, 8, P, None) != 0           # no such MFMA tile
    assert lib.bqc_mfma_i8(17, 4, 7, P, None) != 0           # odd iterations on 16 chains
    assert lib.bqc_mfma_i8_ops(32, 1024, 2048) == 262144.0 * 2048 * 1024 * 4
    # the probes' argument checks (no launch reaches the GPU)
    lib.bqc_lds_read.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    lib.bqc_dma_l2.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                               C.c_void_p, C.c_void_p]
    lib.bqc_mfma_chain.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    assert lib.bqc_lds_read(12, 4, 8, P, P, None) != 0            # waves
    assert lib.bqc_lds_read(8, 4, 0, P, P, None) != 0             # iterations
    assert lib.bqc_dma_l2(2, 8, P, 4096, 512, 4, 8, P, None) != 0   # no such shape
    assert lib.bqc_dma_l2(0, 8, P, 4000, 512, 4, 8, P, None) != 0   # stride not whole lines
    assert lib.bqc_dma_l2(0, 8, P, 4096, 500, 4, 8, P, None) != 0   # rows not whole blocks
    assert lib.bqc_dma_l2(0, 8, C.c_void_p(17), 4096, 512, 4, 8, P, None) != 0  # misaligned
    assert lib.bqc_mfma_chain(0, 1, P, P, None) != 0


def test_qkv_rejects_v_rows_unlike_k(L):
    """bq_qkv sizes v from k's row count, so the wrappers refuse a v of
    another row count before any launch (no GPU needed to reach the check)."""
    import bq
    import torch

    def w(n):
        return bq.ButterquantWeight(torch.empty(0, dtype=torch.int8), torch.empty(0), n, 256)

    x = torch.empty((1, 256), dtype=torch.int8)
    with pytest.raises(ValueError, match="must match"):
        bq.qkv(x, torch.empty(1), w(256), w(128), w(64))
    with pytest.raises(ValueError, match="must match"):
        bq.norm_qkv(torch.empty((1, 256), dtype=torch.bfloat16), torch.empty(256), w(256), w(128),
                    w(64))
