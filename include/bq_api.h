/*
 * bq_api.h -- C ABI of the MI355X (gfx950) butterquant library, libbq.so.
 *
 * This is the drop-in boundary for the reference's butterquant kernel entry
 * points (CoffeeVampir3/Mojo-Gemma4-CPU, butterquant_kernels/linear.mojo and
 * butterquant_kernels/moe.mojo) and for the load-time pack they consume
 * (butterquant/pack.mojo).  A Mojo caller binds these symbols with
 * `external_call` the way butterquant/amx_tiles.mojo:46-53 already calls C.
 *
 * Conventions (mapping the reference's Mojo conventions to C):
 *   - Every pointer is a DEVICE pointer unless marked (host).  bf16 values are
 *     passed as their uint16_t bit patterns.
 *   - `stream` is a hipStream_t (NULL = the null stream).  Entry points only
 *     enqueue work; the reference dispatchers join before returning
 *     (kernels/helpers.mojo:320-327), which a caller gets with
 *     bq_stream_synchronize().
 *   - seq_len <= 0 is a no-op returning BQ_OK, as the reference returns early
 *     (linear.mojo:134-135, 255-256; moe.mojo:317-318).
 *   - Contract violations the reference enforces with compile-time asserts or
 *     debug_assert (linear.mojo:132-133, vnni.mojo:91-99) or abort
 *     (kernels.mojo:82-83) return BQ_ERR_SHAPE / BQ_ERR_INVALID with a message
 *     in bq_last_error() and launch nothing.
 *   - No entry point allocates device memory; buffers are caller-owned, as the
 *     reference's arena-allocated bindings are (gemma_4_moe_bq.mojo:649-664).
 *
 * Weights: int8 codes in the GPU layout "tile16x64" (1 KiB fragments of 16
 * rows x 64 K; see bq_weight_retile), per-row f32 scales (amax/127).  The
 * colsum sidecar of the reference's VNNI layout is not needed: the GPU
 * multiplies signed codes directly, which yields the same integer sums.
 */
#ifndef BQ_API_H
#define BQ_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BQ_OK 0
#define BQ_ERR_INVALID 1      /* null pointer / bad enum */
#define BQ_ERR_SHAPE 2        /* shape contract violated */
#define BQ_ERR_HIP 3          /* HIP runtime error (launch failed) */
#define BQ_ERR_UNSUPPORTED 4  /* size beyond a kernel's stated limit */

#define BQ_LAYOUT_ROWMAJOR 0  /* on-disk int8 [N,K] (quant/quantizer.mojo:1028-1036) */
#define BQ_LAYOUT_VNNI 1      /* reference 32x64 tiles (butterquant/vnni.mojo:146-163) */

/* kernels/moe_router.mojo:33-36 SparseRoute {token:i32, weight:f32}, 8 bytes */
typedef struct bq_route {
  int32_t token;
  float weight;
} bq_route;

/* ---- runtime ------------------------------------------------------------ */
/* Select and warm the device; read the BQ_* tuning switches of the
 * environment.  The switches are published atomically: a launch on another
 * thread during bq_init runs with the old or the new values (each a valid
 * configuration with the same results). */
int bq_init(int device);
const char* bq_last_error(void);         /* message of the last failure (thread-local) */
int bq_stream_synchronize(void* stream); /* join, like fanout_dispatch's join_all */
const char* bq_version(void);

/* ---- weights (load time) -------------------------------------------------- */

/* Re-tile packed int8 codes [n_rows, k] once at load into tile16x64.
 * Replaces PackColsumKernel.execute / dispatch_pack_colsum
 * (butterquant/pack.mojo:29-99, called from gemma_4_moe_bq.mojo:872-892).
 * src_layout: BQ_LAYOUT_ROWMAJOR (quantizer output) or BQ_LAYOUT_VNNI.
 * n_rows % 16 == 0, k % 64 == 0; src and dst must not overlap. */
int bq_weight_retile(const int8_t* src, int src_layout, int8_t* dst, int n_rows, int k,
                     void* stream);

/* Inverse of bq_weight_retile to row-major (bit-exact unpack for tests and
 * for exporting weights). */
int bq_weight_unpack(const int8_t* tiled, int8_t* dst_rowmajor, int n_rows, int k, void* stream);

/* The reference's own load-time pack: row-major -> VNNI 32x64 tiles plus the
 * colsum sidecar (butterquant/vnni.mojo:86-114; task shape from
 * modeling/slot.mojo:263-301).  colsum may be NULL.  colsum_row_major=1 gives
 * [rows, cols/block_cols], 0 gives [cols/block_cols, rows].
 * rows % 32 == 0, cols % 64 == 0, block_cols % 16 == 0, cols % block_cols == 0. */
int bq_pack_colsum_vnni(const int8_t* src, int8_t* dst, float* colsum, int rows, int cols,
                        int block_cols, int colsum_row_major, void* stream);

/* Offline weight encoder (butterquant/kernels.mojo:148-168 rotate_and_quant
 * as driven by quant/quantizer.mojo:963-1051): bf16 [rows, cols] (x gamma,
 * f32 [cols] or NULL) -> FWHT(fwht_block) along K -> int8 row-major codes and
 * scales amax/127, per row [rows] or per block [rows, cols/fwht_block].
 * fwht_block in {16,32,64,128,256,512}; cols % 64 == 0; cols <= 16128. */
int bq_quantize_weight(const uint16_t* w_bf16, const float* gamma, int8_t* codes,
                       float* scales, int rows, int cols, int fwht_block, int per_block,
                       void* stream);

/* ---- activation prep ------------------------------------------------------ */

/* dispatch_bq_norm_quant[hidden, block, sqrt_n, n_eps] (butterquant_kernels/
 * linear.mojo:58-82 -> butterquant/runtime.mojo:11-37): per token,
 * inv_rms = sqrt_n / sqrt(sum(x^2) + n_eps); x*inv_rms*gamma -> FWHT(block)
 * -> per-row int8 with x_sa = amax.  gamma is the baked split gain (bf16).
 * hidden % 64 == 0, hidden % block == 0, hidden <= 16128. */
int bq_norm_quant(const uint16_t* src, const uint16_t* gamma, int8_t* x_i8, float* x_sa,
                  int seq_len, int hidden, int block, float sqrt_n, float n_eps, void* stream);

/* dispatch_bq_block_quant[block, apply_fwht] (linear.mojo:182-205 ->
 * runtime.mojo:62-80): bf16 [seq_len, cols] -> [FWHT(block)] -> per-block int8,
 * x_sa [seq_len, cols/block] = block amax.  cols % 64 == 0, cols % block == 0;
 * src and x_i8 16-byte aligned. */
int bq_block_quant(const uint16_t* src, int8_t* x_i8, float* x_sa, int cols, int seq_len,
                   int block, int apply_fwht, void* stream);

/* ---- linears ------------------------------------------------------------- */

/* dispatch_bq_linear[hidden] (linear.mojo:119-149; BqLinearKernel 85-116):
 * out[m, n] = bf16((f32(sum_k x*w) * (x_sa[m]/127)) * w_scale[n]).
 * out_f32 (optional, may be NULL) receives the pre-cast f32 values.
 * n_rows % 16 == 0, hidden % 64 == 0. */
int bq_linear(const int8_t* x_i8, const float* x_sa, const int8_t* w, const float* w_scale,
              uint16_t* out, float* out_f32, int n_rows, int seq_len, int hidden, void* stream);

/* dispatch_bq_block_linear[n_rows] (linear.mojo:240-270; gemm.mojo:173-243):
 * facc = fma(f32(sum_{k in b} x*w), x_sa[m,b]/127, facc) over blocks b in
 * order, out = bf16(facc * w_scale[n]).  block % 64 == 0 and a power of two,
 * k_dim % block == 0, k_dim/block <= 64. */
int bq_block_linear(const int8_t* x_i8, const float* x_sa, const int8_t* w, const float* w_scale,
                    uint16_t* out, float* out_f32, int n_rows, int k_dim, int seq_len, int block,
                    void* stream);

/* dispatch_bq_qkv[hidden, qn_full, kvn_full] (linear.mojo:273-326): three
 * per-row linears sharing one activation, in ONE launch over the
 * concatenated q|k|v output tiles (the reference's Chain split).  q has qn
 * rows; k and v both have kvn rows (v_out holds seq_len x kvn). */
int bq_qkv(const int8_t* x_i8, const float* x_sa, const int8_t* q_w, const float* q_scale,
           const int8_t* k_w, const float* k_scale, const int8_t* v_w, const float* v_scale,
           uint16_t* q_out, uint16_t* k_out, uint16_t* v_out, int qn, int kvn, int seq_len,
           int hidden, void* stream);

/* The dense FFN's gate_proj and up_proj on one activation
 * (gemma_4_moe_bq.mojo:756-761: two dispatch_bq_linear calls, linear.mojo:
 * 119-149), in ONE launch over the concatenated out0|out1 output tiles, as
 * bq_qkv does for three: out0 and out1 equal those of the two bq_linear
 * calls bit for bit.  n0, n1 % 16 == 0, hidden % 64 == 0. */
int bq_linear_pair(const int8_t* x_i8, const float* x_sa, const int8_t* w0, const float* w0_scale,
                   const int8_t* w1, const float* w1_scale, uint16_t* out0, uint16_t* out1,
                   int n0, int n1, int seq_len, int hidden, void* stream);

/* Fused decode prep: bq_norm_quant of src followed by bq_linear (resp.
 * bq_qkv) on its output, with the same results: x_i8 / x_sa receive the
 * norm-quant's codes and amax, out the linear's.  No single counterpart in
 * the reference, whose decoder calls dispatch_bq_norm_quant and then
 * dispatch_bq_linear / dispatch_bq_qkv on the activation it wrote
 * (butterquant_kernels/linear.mojo:58-82, 119-149, 273-326).  For seq_len 1,
 * hidden % 256 == 0 and hidden <= 4096 (the decode token) it is one launch,
 * in which every output tile quantizes the row itself while its weights
 * stream in; otherwise the two launches.  The checks of both calls apply
 * (src and x_i8 16-byte aligned). */
int bq_norm_linear(const uint16_t* src, const uint16_t* gamma, int8_t* x_i8, float* x_sa,
                   const int8_t* w, const float* w_scale, uint16_t* out, float* out_f32,
                   int n_rows, int seq_len, int hidden, int block, float sqrt_n, float n_eps,
                   void* stream);
int bq_norm_qkv(const uint16_t* src, const uint16_t* gamma, int8_t* x_i8, float* x_sa,
                const int8_t* q_w, const float* q_scale, const int8_t* k_w, const float* k_scale,
                const int8_t* v_w, const float* v_scale, uint16_t* q_out, uint16_t* k_out,
                uint16_t* v_out, int qn, int kvn, int seq_len, int hidden, int block,
                float sqrt_n, float n_eps, void* stream);
/* bq_norm_quant followed by bq_linear_pair (the dense FFN's prep, gate and
 * up: gemma_4_moe_bq.mojo:749-761), one launch for the decode token as
 * bq_norm_linear. */
int bq_norm_linear_pair(const uint16_t* src, const uint16_t* gamma, int8_t* x_i8, float* x_sa,
                        const int8_t* w0, const float* w0_scale, const int8_t* w1,
                        const float* w1_scale, uint16_t* out0, uint16_t* out1, int n0, int n1,
                        int seq_len, int hidden, int block, float sqrt_n, float n_eps,
                        void* stream);

/* ---- MoE ---------------------------------------------------------------- */

/* RouterExpertKernel (kernels/moe_router.mojo:149-193, dispatch_router_expert
 * :206-245; called at gemma_4_moe_bq.mojo:666-671)
 * up to the candidate insert, for all experts:
 * inv_rms = sqrt_n / sqrt(rms_reduce_row(x) + n_eps), scaled = (x *
 * router_scale) * inv_rms, logits[t, e] = dot_to_scalar(scaled,
 * router_proj[e]) in the reference's accumulator order (PU x 16 fma chains,
 * pairwise tree, 16-lane halving reduce), f32 [seq_len, experts].
 * x [seq_len, hidden], router_proj [experts, hidden], router_scale [hidden]
 * bf16, 4-byte aligned; hidden % 64 == 0. */
int bq_moe_router_logits(const uint16_t* x, const uint16_t* router_proj,
                         const uint16_t* router_scale, float* logits, int seq_len, int hidden,
                         int experts, float sqrt_n, float n_eps, void* stream);

/* insert_candidate top-k (kernels/moe_router.mojo:43-57) + the softmax of
 * RouterMergeKernel (:248-293; dispatch_merge_router_candidates, :333-389):
 * per token the top_k experts by (logit descending, lower expert first on
 * ties) among logits > -1e30, padded with {expert 0, logit -1e30};
 * w = fast_exp_softmax_biased(logit - max) * (1/sum) * f32(scale[expert]).
 * per_expert_scale: bf16 [experts], or NULL for scale 1.
 * experts <= 1024, top_k <= 16. */
int bq_moe_route_topk(const float* logits, const uint16_t* per_expert_scale, int seq_len,
                      int experts, int top_k, int32_t* route_idx, float* route_w, void* stream);

/* dispatch_build_expert_schedules (kernels/moe_router.mojo:60-145): routes
 * of experts [expert_base, expert_base+experts) into expert_offset[experts+1]
 * and routes[] sorted by (expert, token, k).  A token may list an expert more
 * than once (the router pads with expert 0); its records then sit in k order.
 * experts <= 256; routes holds seq_len*top_k. */
int bq_moe_build_schedule(const int32_t* route_idx, const float* route_w, int seq_len, int top_k,
                          int expert_base, int experts, int32_t* expert_offset, bq_route* routes,
                          void* stream);

/* dispatch_merge_router_candidates (kernels/moe_router.mojo:333-389)
 * followed by dispatch_build_expert_schedules (:60-145) over all experts
 * (expert_base 0) -- the two calls the reference's MoE block makes around
 * its norm-quant (modeling/gemma_4_moe_bq.mojo:673-688) -- in one call:
 * route_idx / route_w exactly as bq_moe_route_topk writes them, and
 * expert_offset[experts+1] / routes[] exactly as bq_moe_build_schedule.
 * Up to 8 tokens (and seq_len * top_k <= 1024) one workgroup keeps the
 * routes in LDS and builds the schedule from there (one launch); larger
 * calls run the two kernels.  experts <= 256, top_k <= 16; routes holds
 * seq_len*top_k. */
int bq_moe_route_schedule(const float* logits, const uint16_t* per_expert_scale, int seq_len,
                          int experts, int top_k, int32_t* route_idx, float* route_w,
                          int32_t* expert_offset, bq_route* routes, void* stream);

/* The three calls the reference's MoE block makes between its router and
 * phase 1 -- dispatch_merge_router_candidates, dispatch_bq_norm_quant of the
 * block input and dispatch_build_expert_schedules
 * (modeling/gemma_4_moe_bq.mojo:673-688; kernels/moe_router.mojo:333-389,
 * butterquant_kernels/linear.mojo:58-82, kernels/moe_router.mojo:60-145) --
 * in one call, with bq_moe_route_schedule's and bq_norm_quant's results:
 * route_idx / route_w / expert_offset / routes from logits, x_i8 / x_sa from
 * x and gamma.  For seq_len * top_k <= 1024 slots and the pair-layout
 * norm-quant's shapes (hidden % 256 == 0, hidden <= 4096) it is one launch,
 * in which workgroups quantize the rows while others take the top-k: up to
 * 16 tokens one workgroup takes every top-k and builds the schedule, above
 * that the last top-k workgroup to finish builds it, found through a
 * device-scope counter of the library's that its increment wraps back to 0.
 * Each stream of a device gets its own counter on first use (up to 256
 * streams per device; later streams take the separate launches), so calls
 * on different streams may overlap; calls on one stream run in order.
 * Above 1024 slots with block 128
 * the top-k and the norm-quant share one launch and the schedule follows;
 * otherwise the separate launches.  The checks of both calls apply. */
int bq_moe_prep(const float* logits, const uint16_t* per_expert_scale, const uint16_t* x,
                const uint16_t* gamma, int seq_len, int experts, int top_k, int hidden, int block,
                float sqrt_n, float n_eps, int32_t* route_idx, float* route_w,
                int32_t* expert_offset, bq_route* routes, int8_t* x_i8, float* x_sa,
                void* stream);

/* bq_moe_prep plus the decoder layer's dense-MLP norm-quant of the same
 * input: dispatch_bq_norm_quant(x_main, pre_ffn_norm) and the MoE block's
 * prep (modeling/gemma_4_moe_bq.mojo:749-753 and 673-688), which read the
 * same hidden states with different gains.  dense_i8 / dense_sa =
 * bq_norm_quant(x, dense_gamma, block); the other outputs are bq_moe_prep's.
 * Where bq_moe_prep is one launch, the dense rows are quantized by more
 * workgroups of that launch; otherwise the dense norm-quant runs first as a
 * launch of its own.  Both norm-quants use the same hidden, block, sqrt_n and
 * n_eps (the model's).  The checks of bq_moe_prep apply. */
int bq_ffn_prep(const float* logits, const uint16_t* per_expert_scale, const uint16_t* x,
                const uint16_t* gamma, const uint16_t* dense_gamma, int seq_len, int experts,
                int top_k, int hidden, int block, float sqrt_n, float n_eps, int32_t* route_idx,
                float* route_w, int32_t* expert_offset, bq_route* routes, int8_t* x_i8,
                float* x_sa, int8_t* dense_i8, float* dense_sa, void* stream);

/* dispatch_bq_phase1_gate_up[hidden, gate_up, inter] (moe.mojo:132-164):
 * for every route record rec of expert e (rows of w_gate_up: gate
 * [0,inter), up [inter, 2*inter) of expert e, expert stride 2*inter*hidden):
 * bucket[rec, i] = bf16(gelu_tanh(g)*u), g/u the per-row dequantized
 * projections of x_i8[token(rec)].  seq_len*top_k bounds the route count
 * (grid sizing; the reference sizes its loop from expert_offset alone).
 * inter % 16 == 0, hidden % 64 == 0. */
int bq_moe_phase1_gate_up(const int8_t* x_i8, const float* x_sa, const int32_t* expert_offset,
                          const bq_route* routes, const int8_t* w_gate_up,
                          const float* gate_up_scale, uint16_t* bucket, int experts_per_rank,
                          int seq_len, int top_k, int hidden, int inter, void* stream);

/* dispatch_bq_phase1_gate_up (moe.mojo:132-164) followed by
 * dispatch_bq_block_quant[block = 64, apply_fwht = True] of its bucket
 * (modeling/gemma_4_moe_bq.mojo:689-700), in one call: for every route record
 * rec of expert e, bucket[rec, i] = bf16(gelu_tanh(g)*u) as
 * bq_moe_phase1_gate_up computes it, then per 64-column block of the bf16
 * row FWHT(64) and per-block int8: bucket_i8 [seq_len*top_k, inter],
 * bucket_sa [seq_len*top_k, inter/64] = block amax -- bit for bit what the
 * two calls produce, for the rows of records [0, expert_offset[experts]).
 * The block-quant runs in the GEMM's epilogue on the tile's bucket values
 * kept in LDS; bucket (bf16) may be NULL, and is then never written to
 * memory.  inter % 64 == 0, hidden % 64 == 0; x_i8, w_gate_up and bucket
 * 16-byte, bucket_i8 8-byte, bucket_sa 4-byte aligned. */
int bq_moe_phase1_gate_up_quant(const int8_t* x_i8, const float* x_sa,
                                const int32_t* expert_offset, const bq_route* routes,
                                const int8_t* w_gate_up, const float* gate_up_scale,
                                uint16_t* bucket, int8_t* bucket_i8, float* bucket_sa,
                                int experts_per_rank, int seq_len, int top_k, int hidden,
                                int inter, void* stream);

/* Bytes of device workspace bq_moe_phase2_down needs (the per-route f32
 * down-projection rows, seq_len*top_k x hidden). */
size_t bq_moe_phase2_workspace_size(int seq_len, int top_k, int hidden);

/* dispatch_bq_phase2_down[hidden, inter] (moe.mojo:298-335): per-block
 * (block = 64) down projection of the block-quantized bucket, route-weighted
 * and accumulated per token in ascending expert order into moe_accum
 * f32 [seq_len, hidden]; moe_out = bf16(moe_accum).  w_down rows are
 * [experts_per_rank*hidden, inter] (expert stride hidden*inter).
 * Each expert's route records must be in ascending token order (the order
 * bq_moe_build_schedule and the reference's schedule produce); a token's
 * records within one expert are added in record order; top_k <= 16.
 * workspace: >= bq_moe_phase2_workspace_size() bytes, 256-byte aligned;
 * moe_accum and moe_out 16-byte aligned. */
int bq_moe_phase2_down(const int8_t* bucket_i8, const float* bucket_sa,
                       const int32_t* expert_offset, const bq_route* routes, const int8_t* w_down,
                       const float* down_scale, float* moe_accum, uint16_t* moe_out,
                       int experts_per_rank, int seq_len, int top_k, int hidden, int inter,
                       int block, void* workspace, size_t workspace_bytes, void* stream);

/* No counterpart in the reference: bq_moe_phase2_down for callers that
 * cannot allocate or pass a workspace (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  Same arguments and
 * results as bq_moe_phase2_down without workspace/workspace_bytes: the
 * per-route f32 rows live in the library's static per-GPU scratch of
 * 24 MiB, so seq_len * top_k * hidden * 4 <= 24 MiB (at hidden 2816 and
 * top_k 8: up to 279 tokens), else BQ_ERR_UNSUPPORTED.  Calls nothing that
 * allocates.  Every call on one GPU shares that GPU's scratch: calls that
 * overlap on one GPU (concurrent streams or threads) race. */
int bq_moe_phase2_down_noalloc(const int8_t* bucket_i8, const float* bucket_sa,
                               const int32_t* expert_offset, const bq_route* routes,
                               const int8_t* w_down, const float* down_scale, float* moe_accum,
                               uint16_t* moe_out, int experts_per_rank, int seq_len, int top_k,
                               int hidden, int inter, int block, void* stream);

/* The decoder layer's FFN gate/up: bq_moe_phase1_gate_up_quant (no bf16
 * bucket) plus the dense MLP's gate/up of the same seq_len tokens
 * (modeling/gemma_4_moe_bq.mojo:755-769: dispatch_bq_linear of gate and of
 * up on dense_x_i8 / dense_x_sa, dispatch_gelu_gate_up, then
 * dispatch_bq_block_quant[64, apply_fwht=True]).  dense_i8 [seq_len,
 * dense_inter] and dense_sa [seq_len, dense_inter / 64] equal
 * bq_block_quant(bf16(gelu_tanh(bf16(gate)) * bf16(up)), 64, FWHT) with gate
 * and up the bq_linear outputs (kernels/elementwise.mojo:17-27).  dense_gate
 * and dense_up are [dense_inter, hidden] per-row (B = 128) weights.  While
 * the experts use the 16-row kernel (few routes per expert, decode) the
 * dense rows are more workgroups of its launch; otherwise they are a launch
 * of their own after the experts', in 64-token tiles (2048 tokens: 135 us
 * for the dense rows, against 68 us for bq_linear_pair of gate and up
 * alone, which leaves the GELU and the block-quant to further calls).  The checks of bq_moe_phase1_gate_up_quant apply;
 * dense_inter % 64 == 0; dense_x_i8, dense_gate, dense_up 16-byte, dense_i8
 * 8-byte, dense_sa 4-byte aligned. */
int bq_ffn_gate_up(const int8_t* x_i8, const float* x_sa, const int32_t* expert_offset,
                   const bq_route* routes, const int8_t* w_gate_up, const float* gate_up_scale,
                   int8_t* bucket_i8, float* bucket_sa, int experts_per_rank, int seq_len,
                   int top_k, int hidden, int inter, const int8_t* dense_x_i8,
                   const float* dense_x_sa, const int8_t* dense_gate,
                   const float* dense_gate_scale, const int8_t* dense_up,
                   const float* dense_up_scale, int dense_inter, int8_t* dense_i8,
                   float* dense_sa, void* stream);

/* The decoder layer's FFN down: bq_moe_phase2_down plus the dense MLP's down
 * projection of the same seq_len tokens (gemma_4_moe_bq.mojo:774-778:
 * dispatch_bq_block_linear of dense_i8 / dense_sa, per-block activations of
 * the same block): dense_out [seq_len, hidden] bf16 = bq_block_linear(
 * dense_i8, dense_sa, dense_down, block).  dense_down is [hidden,
 * dense_inter].  While the experts use the 16-row kernel the dense rows are
 * more workgroups of its launch; otherwise they are bq_block_linear's own
 * (tiled) launch.  The checks
 * of bq_moe_phase2_down apply; dense_inter % block == 0, dense_inter / block
 * <= 64; dense_i8 and dense_down 16-byte, dense_out 8-byte aligned. */
int bq_ffn_down(const int8_t* bucket_i8, const float* bucket_sa, const int32_t* expert_offset,
                const bq_route* routes, const int8_t* w_down, const float* down_scale,
                float* moe_accum, uint16_t* moe_out, int experts_per_rank, int seq_len, int top_k,
                int hidden, int inter, int block, const int8_t* dense_i8, const float* dense_sa,
                const int8_t* dense_down, const float* dense_down_scale, int dense_inter,
                uint16_t* dense_out, void* workspace, size_t workspace_bytes, void* stream);

/* ---- vocabulary head and embedding ----------------------------------------- */

#define BQ_SAMPLE_NMAX 256 /* continuous_batching/schedule.mojo:9 MAXIMUM_SAMPLING_LOGITS */

/* kernels/flash_sample.mojo:21-28 SamplingParams, in the Mojo struct's field
 * order and sizes (Int = int64, Bool = one byte), 40 bytes. */
typedef struct bq_sampling_params {
  float temperature;
  float min_p;
  int64_t top_k;
  uint64_t seed;
  int64_t n_keep;
  uint8_t greedy;
  uint8_t pad_[7];
} bq_sampling_params;

/* kernels/flash_sample.mojo:120-134 SampleOutcome[256], 2064 bytes.
 * Entries k >= n of topn_val / topn_idx hold -1e30 / -1. */
typedef struct bq_sample_outcome {
  int32_t token_id;
  float logz;
  int64_t n;
  float topn_val[BQ_SAMPLE_NMAX];
  int32_t topn_idx[BQ_SAMPLE_NMAX];
} bq_sample_outcome;

/* dispatch_bq_head_prep[hidden, block, sqrt_n, n_eps] (butterquant_kernels/
 * head.mojo:57-78 -> runtime.mojo:40-47): bq_norm_quant with per-block
 * activation scales, x_sa [num_rows, hidden/block] = block amax.
 * block in {64, 128, 256, 512}; hidden % block == 0; src 4-byte aligned. */
int bq_head_prep(const uint16_t* src, const uint16_t* gamma, int8_t* x_i8, float* x_sa,
                 int num_rows, int hidden, int block, float sqrt_n, float n_eps, void* stream);

/* Bytes of device workspace bq_flash_sample needs (bf16 logits [rows, vocab]
 * plus per-workgroup partials). */
size_t bq_flash_sample_workspace_size(int num_rows, int vocab);

/* dispatch_bq_flash_sample[cols, cap, n_max = 256] (butterquant_kernels/
 * head.mojo:127-167) + finalize_outcomes (kernels/flash_sample.mojo:221-265)
 * over vocabulary rows [vocab_base, vocab_base + vocab): per (row, v)
 * y = bf16(softcap(head_logit_row)), score = y/T + gumbel(seed, row, v)
 * (0 when greedy); outcome = score argmax (or the min_p / top_k pick among
 * the top 256), logz = log-sum-exp of y/T, the top n_keep (y, v) by y
 * descending, lower v first.  weight: the per-block head in tile16x64
 * [vocab, hidden], wscales [vocab, hidden/block]; x_i8 [num_rows, hidden]
 * and x_sa [num_rows, hidden/block] from bq_head_prep.  params and outcome
 * are device arrays of num_rows.  num_rows <= 32, vocab % 16 == 0, vocab <= 2^20,
 * block in {64, 128, 256, 512}, hidden/block <= 64; x_i8 and weight 16-byte
 * aligned; workspace >= bq_flash_sample_workspace_size(), 256-byte aligned. */
int bq_flash_sample(const int8_t* x_i8, const float* x_sa, const int8_t* weight,
                    const float* wscales, const bq_sampling_params* params,
                    bq_sample_outcome* outcome, int num_rows, int vocab, int hidden, int block,
                    float cap, int64_t vocab_base, void* workspace, size_t workspace_bytes,
                    void* stream);

/* dispatch_bq_embed_lookup[hidden, scale] (butterquant_kernels/embedding.mojo:
 * 65-96; BqEmbedLookupKernel 21-62): per token id (device int32 [seq_len]),
 * the row of this shard (rows [rank*shard_rows, (rank+1)*shard_rows)) is
 * dequantized per block (q * wscales[row, b]), FWHT(block)-rotated and
 * written as bf16(x * scale); a token of another shard gives a zero row.
 * weight: the per-block table in tile16x64 [shard_rows, hidden] (the head's
 * own buffer when the embedding is tied); block in {64, 128, 256, 512}. */
int bq_embed_lookup(const int32_t* token_ids, const int8_t* weight, const float* wscales,
                    uint16_t* dst, int seq_len, int hidden, int block, int shard_rows, int rank,
                    float scale, void* stream);

/* ---- int8-KV attention -------------------------------------------------------- */

/* One run of buffer rows that share a page table (kernels/attention_ops.mojo:
 * 54-58 KVRun): rows [buf_start, next run's buf_start) hold positions
 * base_pos, base_pos + 1, ...; page j of the run is physical row base
 * base_rows[rows_off + j].  Device arrays: the KVRunTable's runs and
 * base_rows lists (attention_ops.mojo:61-91) copied as they are. */
typedef struct {
    int32_t buf_start, base_pos, rows_off, page_count;
} bq_kv_run;

/* dispatch_bq_attn_prep[head_dim, rope_half, pair_stride, sqrt_n, n_eps]
 * (butterquant_kernels/attention.mojo:537-583; BqAttnPrepKernel 474-534,
 * prep_head_qk_i8 / prep_head_v_i8 butterquant/head_prep.mojo:39-92): per
 * token (position = run.base_pos + row - run.buf_start) and q head: per-head
 * RMS (sqrt_n / sqrt(ssq + n_eps)) x q_norm, RoPE (cos/sin_table
 * [position, rope_half] on pairs (i, pair_stride + i), i < rope_half), FWHT
 * (head_dim), absmax int8 -> q_i8 [seq_len, num_q*head_dim], qi_bias =
 * 128 * sum(codes), f_q = amax [seq_len, num_q].  K heads (k_norm, RoPE) and V
 * heads (no gain, no RoPE) the same way into the paged caches
 * (k_cache/v_cache [slots, num_kv*head_dim] int8, k_scale/v_scale
 * [slots, num_kv]) at slot base_rows[rows_off + ((p >> page_shift) &
 * page_mask)] + (p & row_mask), p = position / cache_degree, for positions
 * with position % cache_degree == rank.  v_src may equal k_src (K = V
 * layers).  cos/sin_table may be NULL when rope_half is 0.  head_dim in
 * {64, 128, 256, 512}; rope_half and pair_stride
 * multiples of 64 with rope_half <= pair_stride, pair_stride + rope_half <=
 * head_dim. */
int bq_attn_prep(const uint16_t* q_src, const uint16_t* k_src, const uint16_t* v_src,
                 const uint16_t* q_norm, const uint16_t* k_norm, int8_t* q_i8, float* qi_bias,
                 float* f_q, int8_t* k_cache, float* k_scale, int8_t* v_cache, float* v_scale,
                 const float* cos_table, const float* sin_table, const bq_kv_run* runs,
                 int num_runs, const int32_t* base_rows, int num_q, int num_kv, int head_dim,
                 int rope_half, int pair_stride, float sqrt_n, float n_eps, int cache_degree,
                 int rank, int page_shift, int row_mask, int page_mask, int seq_len,
                 void* stream);

/* The split count s_max the attention entry points are sized for: each
 * token's KV range of L positions is cut into min(s_max, ceil(L / 32))
 * contiguous parts (worker_range, kernels/helpers.mojo:182-190) processed in
 * parallel and merged in order.  max_kv_len: the longest range any token
 * has (the window for sliding layers). */
int bq_attention_splits(int seq_len, int num_kv, int max_kv_len);

/* Bytes of device workspace the attention entry points need for s_max
 * splits (f32 partials [seq_len, num_q, s_max] x (head_dim + 2)). */
size_t bq_attention_workspace_size(int seq_len, int num_q, int head_dim, int s_max);

/* dispatch_bq_sliding_attention[head_dim, max_q, gqa_ratio, window,
 * cache_size, page_len] (butterquant_kernels/attention.mojo:330-403; decode
 * kernel 83-146, sliding prefill 149-247, bq_process_kv_tile 32-80): per
 * token and q head h (kv head h / (num_q/num_kv)), softmax attention over the
 * cached positions [max(0, pos - window + 1), pos]: score =
 * (f32(sum (k ^ 0x80) * q) - qi_bias) * f_q * ks / 127^2, tiles of 16
 * positions with online_softmax_tile (kernels/attention_ops.mojo:166-182),
 * acc += (w * vs / 127) * v; output bf16 [seq_len, num_q*head_dim] =
 * acc / l (zeros if l = 0), or the logsum merge of the splits
 * (kernels/logsum_merge.mojo:29-122).  Page addressing as bq_attn_prep with
 * p = position.  num_q % num_kv == 0 with num_q/num_kv in {1, 2, 4, 8, 16};
 * head_dim in {64, 128, 256, 512}; q_i8, k_cache, v_cache 16-byte aligned;
 * workspace >= bq_attention_workspace_size(seq_len, num_q, head_dim, s_max),
 * 16-byte aligned. */
int bq_sliding_attention(const int8_t* q_i8, const float* qi_bias, const float* f_q,
                         const int8_t* k_cache, const float* k_scale, const int8_t* v_cache,
                         const float* v_scale, uint16_t* output, void* workspace,
                         size_t workspace_bytes, const bq_kv_run* runs, int num_runs,
                         const int32_t* base_rows, int num_q, int num_kv, int head_dim,
                         int window, int page_shift, int row_mask, int page_mask, int s_max,
                         int seq_len, void* stream);

/* dispatch_bq_full_attention[head_dim, num_q, num_kv, gqa_ratio, kv_stride,
 * partial_stride, page_len] (butterquant_kernels/attention.mojo:406-471; full
 * prefill 250-327) at one cache rank: every token attends to positions
 * [0, pos]; the per-token result goes through the logsum merge as the
 * reference's does.  Same layout and limits as bq_sliding_attention
 * (page_mask -1 for an unbounded page table). */
int bq_full_attention(const int8_t* q_i8, const float* qi_bias, const float* f_q,
                      const int8_t* k_cache, const float* k_scale, const int8_t* v_cache,
                      const float* v_scale, uint16_t* output, void* workspace,
                      size_t workspace_bytes, const bq_kv_run* runs, int num_runs,
                      const int32_t* base_rows, int num_q, int num_kv, int head_dim,
                      int page_shift, int row_mask, int page_mask, int s_max, int seq_len,
                      void* stream);

/* ---- on-disk weights (safetensors) -------------------------------------------- */

/* safetensors dtype tags (safetensors/parser.mojo:19-54) */
#define BQ_DT_BOOL 0
#define BQ_DT_U8 1
#define BQ_DT_I8 2
#define BQ_DT_I16 3
#define BQ_DT_U16 4
#define BQ_DT_F16 5
#define BQ_DT_BF16 6
#define BQ_DT_I32 7
#define BQ_DT_U32 8
#define BQ_DT_F32 9
#define BQ_DT_F64 10
#define BQ_DT_F8_E4M3 11
#define BQ_DT_F8_E5M2 12
#define BQ_DT_I64 13
#define BQ_DT_U64 14

/* A memory-mapped safetensors shard (host). */
typedef struct bq_st_file bq_st_file;

/* parse_safetensors_header (safetensors/parser.mojo:270-320) on a mapped
 * file: the same validation (header <= 100 MiB, required fields, supported
 * dtypes, byte size = dtype size x numel, offsets inside the payload, no
 * overlapping ranges or duplicate names, payload fully indexed, no trailing
 * content); BQ_ERR_INVALID with the reason otherwise.  Host only. */
int bq_st_open(const char* path, bq_st_file** out);
void bq_st_close(bq_st_file* f);
int bq_st_num_tensors(const bq_st_file* f);
/* Metadata of one tensor (shape: up to 8 dims) and a host pointer to its
 * bytes inside the mapping; BQ_ERR_INVALID "missing tensor" if absent. */
int bq_st_tensor_info(const bq_st_file* f, const char* name, int* dtype, int* ndim,
                      int64_t* shape, size_t* nbytes, const void** host_data);

/* Load one quantized weight straight from its on-disk members
 * (quant/manifest.mojo:69-199: int8 codes "<name>" row-major [n_rows, k],
 * f32 scales "<name>.scale" [n_rows] (scale_cols = 1) or [n_rows,
 * scale_cols]) located across shards (modeling/loader.mojo:151-186) and
 * validated like validate_weight (loader.mojo:52-96: dtype, 1-D / 2-D / 3-D
 * folded shapes), into device buffers: codes re-tiled to tile16x64 through a
 * device staging buffer of at least 16*k bytes (whole 16-row strips per
 * chunk), scales copied as they are.  Replaces the loader's host reads plus
 * the VNNI pack at init.  n_rows % 16 == 0, k % 64 == 0. */
int bq_load_quantized(const bq_st_file* const* files, int n_files, const char* name, int n_rows,
                      int k, int scale_cols, int8_t* w_tiled, float* scales, int8_t* staging,
                      size_t staging_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* BQ_API_H */
