/*
 * bq_oracle.h -- CPU restatement of the butterquant hot path of
 * CoffeeVampir3/Mojo-Gemma4-CPU, used ONLY as test infrastructure (the parity
 * checker for the HIP library and the CPU baseline of bench.py).  Nothing in
 * the shipped library links or calls this code.
 *
 * Every function cites the reference file:line it restates.  All arithmetic is
 * IEEE f32 with no contraction (built with -ffp-contract=off), except where the
 * reference itself calls fma (`.fma(...)`), which is restated with fmaf().
 *
 * Parity status of each function (how it is pinned) is listed in
 * tests/test_oracle_pins.py; functions whose ulp-level behaviour depends on the
 * Mojo compiler are marked "ulp-unpinned" below.
 */
#ifndef BQ_ORACLE_H
#define BQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 ---------------------------------------------------------------- */
uint16_t bqo_f32_to_bf16(float v);                 /* butterquant/convert.mojo:14-17 */
float bqo_bf16_to_f32(uint16_t b);

/* ---- FWHT ---------------------------------------------------------------- */
float bqo_fwht_scale(int block);                   /* butterquant/fwht.mojo:55 */
int bqo_fwht_block(float* buf, int block);         /* butterquant/fwht.mojo:20-70 */
int bqo_fwht_row(float* buf, int cols, int block); /* butterquant/fwht.mojo:73-76 */

/* ---- quantization -------------------------------------------------------- */
float bqo_row_absmax(const float* x, int n);       /* butterquant/kernels.mojo:48-55 */
void bqo_quant_segment(const float* work, int8_t* qi, float* scale_slot, int n,
                       int store_divided);        /* butterquant/kernels.mojo:68-78 */
/* Weight encoding (offline quantizer): FWHT rows in K-blocks, then per-row
 * (scales[rows], amax/127) or per-block (scales[rows*cols/block]) int8.
 * butterquant/kernels.mojo:148-168, quant/quantizer.mojo:1019-1026. */
int bqo_rotate_and_quant(int block, float* work, int8_t* qi, float* scales,
                         int rows, int cols, int per_block);
void bqo_bake_split_gain(uint16_t* gamma, int cols, float eps); /* kernels.mojo:36-45 */

/* ---- activation prep ----------------------------------------------------- */
/* RMS sum of squares in the AVX-512BF16 accumulation order
 * (kernels/rmsnorm.mojo:16-17, kernels/dot_products.mojo:9-35,127-191);
 * the final 16-lane horizontal reduction is a halving tree (ulp-unpinned). */
float bqo_rms_reduce_row(const uint16_t* src, int hidden);
/* butterquant/runtime.mojo:11-37 (+ quantize.mojo:5-23). */
int bqo_prepare_norm_activation(const uint16_t* src, const uint16_t* gamma,
                                int8_t* x_i8, float* sa, int hidden, int block,
                                float sqrt_n, float n_eps, int per_block);
/* butterquant/runtime.mojo:62-80 */
int bqo_prepare_block_activation(const uint16_t* src, int8_t* x_i8, float* sa,
                                 int cols, int block, int apply_fwht);

/* ---- load-time pack ------------------------------------------------------ */
/* butterquant/vnni.mojo:31-114 (32x64 tiles, 16x16 dword transpose) + colsum */
int bqo_pack_and_colsum_vnni(const int8_t* src, int8_t* dst, int rows, int cols,
                             int block_cols, float* colsum, int colsum_row_major);
size_t bqo_vnni_offset(int n, int k, int cols);    /* the pack bijection */

/* ---- GEMM (packed weights, VNNI u8 x i8 form with colsum correction) ------ */
/* butterquant/gemm.mojo:114-170 (+ dot_products.mojo:7-73); out_bf16/out_f32
 * may be NULL.  act [m,K] row-major, sa[m]; W packed [n_rows,K]. */
void bqo_gemm_i8_per_row(const int8_t* act, const float* act_scale, int m,
                         const int8_t* wpacked, const float* wsc,
                         const float* colsum, int n_rows, int K,
                         uint16_t* out_bf16, float* out_f32);
/* butterquant/gemm.mojo:173-243; act_scale [m, K/block], colsum [K/block, N] */
void bqo_gemm_i8_per_block(const int8_t* act, const float* act_scale, int m,
                           const int8_t* wpacked, const float* wsc,
                           const float* colsum, int N, int k_dim, int block,
                           uint16_t* out_bf16, float* out_f32);
/* Signed i8 x i8 epilogues of the AMX branch (butterquant/amx_gemm.mojo:28-80):
 * per-row y = f32(acc)*(sa/127)*sw; per-block facc += f32(acc_b)*(sa_b/127). */
void bqo_gemm_signed_per_row(const int8_t* act, const float* act_scale, int m,
                             const int8_t* wpacked, const float* wsc, int n_rows,
                             int K, uint16_t* out_bf16, float* out_f32);
void bqo_gemm_signed_per_block(const int8_t* act, const float* act_scale, int m,
                               const int8_t* wpacked, const float* wsc, int N,
                               int k_dim, int block, uint16_t* out_bf16,
                               float* out_f32);
/* Exact integer accumulators acc[m*N+n] = sum_k x*w read through the packed
 * layout (for the int32 bit-exact checks). */
void bqo_int_acc(const int8_t* act, int m, const int8_t* wpacked, int N, int K,
                 int k_lo, int k_hi, int64_t* acc);

/* ---- MoE ----------------------------------------------------------------- */
typedef struct { int32_t token; float weight; } bqo_route; /* kernels/moe_router.mojo:33-36 */
float bqo_exp_f32_fast(float x);                 /* simd_math/ops.mojo:73-96 */
float bqo_tanh_f32(float x);                     /* simd_math/ops.mojo:128-141 */
float bqo_gelu_tanh_f32(float x);                /* simd_math/ops.mojo:145-156 */
float bqo_fast_exp_softmax_biased(float x);      /* simd_math/exponential.mojo:178-194 */
/* top-k (ties -> lower expert, moe_router.mojo:43-57) + softmax over the k
 * (moe_router.mojo:276-293) with per_expert_scale = 1. logits [T,E]. */
void bqo_router_logits(const uint16_t* x, const uint16_t* router_proj,
                       const uint16_t* router_scale, int T, int H, int E, float sqrt_n,
                       float n_eps, float* logits);   /* moe_router.mojo:164-187 */
void bqo_route_topk_softmax(const float* logits, int T, int E, int top_k,
                            const uint16_t* per_expert_scale, int32_t* route_idx,
                            float* route_w);
/* kernels/moe_router.mojo:60-106 (experts [0,E)) */
void bqo_build_schedule(const int32_t* route_idx, const float* route_w, int T,
                        int top_k, int E, int32_t* expert_offset,
                        bqo_route* routes);
/* butterquant_kernels/moe.mojo:25-129 ; bucket bf16 [T*top_k, inter] */
void bqo_moe_phase1(const int8_t* x_i8, const float* x_sa, int hidden,
                    const int32_t* expert_offset, const bqo_route* routes, int E,
                    const int8_t* w_gu_packed, const float* gu_scale,
                    const float* gu_colsum, int inter, uint16_t* bucket);
/* butterquant_kernels/moe.mojo:167-295 ; accum f32 [T,hidden], out bf16 */
void bqo_moe_phase2(const int8_t* bucket_i8, const float* bucket_sa, int inter,
                    int block, const int32_t* expert_offset,
                    const bqo_route* routes, int E, int T,
                    const int8_t* w_d_packed, const float* d_scale,
                    const float* d_colsum, int hidden, float* accum,
                    uint16_t* out);

/* ---- bq head and embedding --------------------------------------------------- */
#define BQO_SAMPLE_NMAX 256  /* continuous_batching/schedule.mojo:9 MAXIMUM_SAMPLING_LOGITS */
/* kernels/flash_sample.mojo:21-28 SamplingParams (Mojo field order and sizes) */
typedef struct {
    float temperature;
    float min_p;
    int64_t top_k;
    uint64_t seed;
    int64_t n_keep;
    uint8_t greedy;
    uint8_t pad_[7];
} bqo_sampling_params;
/* kernels/flash_sample.mojo:120-134 SampleOutcome[256] */
typedef struct {
    int32_t token_id;
    float logz;
    int64_t n;
    float topn_val[BQO_SAMPLE_NMAX];
    int32_t topn_idx[BQO_SAMPLE_NMAX];
} bqo_sample_outcome;
float bqo_exp_f32(float x);                       /* simd_math/ops.mojo:35-69 */
float bqo_log_f32(float x);                       /* simd_math/ops.mojo:100-124 */
uint64_t bqo_mix64(uint64_t x);                   /* simd_math/sampling_rng.mojo:10-21 */
float bqo_gumbel_noise(uint64_t seed, int64_t row, int64_t idx); /* sampling_rng.mojo:24-43 */
float bqo_softcap(float x, float cap);            /* simd_math/ops.mojo:160-167 */
float bqo_head_logit_row(const int8_t* x_i8, const float* sa, const int8_t* w,
                         const float* wscales, int cols, int block); /* dot_products.mojo:76-88 */
void bqo_flash_sample(const int8_t* x_i8, const float* x_sa, const int8_t* weight,
                      const float* wscales, int rows, int vocab, int cols, int block,
                      float cap, int64_t vocab_base, const bqo_sampling_params* params,
                      bqo_sample_outcome* out);   /* head.mojo:85-167 */
void bqo_embed_lookup(const int32_t* token_ids, int T, const int8_t* weight,
                      const float* wscales, int hidden, int block, int shard_rows,
                      int rank, float scale, uint16_t* dst); /* embedding.mojo:21-96 */

/* ---- int8-KV attention --------------------------------------------------- */
typedef struct {              /* kernels/attention_ops.mojo:54-58 KVRun */
    int32_t buf_start, base_pos, rows_off, page_count;
} bqo_kv_run;
void bqo_attn_prep(const uint16_t* q_src, const uint16_t* k_src, const uint16_t* v_src,
                   const uint16_t* q_norm, const uint16_t* k_norm, int8_t* q_i8,
                   float* qi_bias, float* f_q, int8_t* k_cache, float* k_scale,
                   int8_t* v_cache, float* v_scale, const float* cos_table,
                   const float* sin_table, const bqo_kv_run* runs, int num_runs,
                   const int32_t* base_rows, int seq_len, int num_q, int num_kv,
                   int head_dim, int rope_half, int pair_stride, float sqrt_n, float n_eps,
                   int cache_degree, int rank, int page_shift, int row_mask,
                   int page_mask);        /* butterquant_kernels/attention.mojo:474-534 */
int bqo_attn_num_splits(int L, int s_max, int min_split);
void bqo_flash_attention(const int8_t* q_i8, const float* qi_bias, const float* f_q,
                         const int8_t* k_cache, const float* k_scale, const int8_t* v_cache,
                         const float* v_scale, const bqo_kv_run* runs, int num_runs,
                         const int32_t* base_rows, int seq_len, int num_q, int num_kv,
                         int head_dim, int window, int degree, int rank, int page_shift,
                         int row_mask, int page_mask, int s_max, int min_split,
                         uint16_t* out, float* out_f32); /* attention.mojo:32-327 */

/* ---- synthetic inputs ---------------------------------------------------- */
uint64_t bqo_splitmix64(uint64_t* state);
/* splitmix64 -> Box-Muller (f64) -> *sigma -> f32 -> bf16 RNE */
void bqo_synth_normal_bf16(uint64_t seed, double sigma, uint16_t* out, size_t n);
void bqo_synth_normal_f32(uint64_t seed, double sigma, float* out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
