// bq_kernels.hpp -- host-side launch interface of the butterquant HIP kernels
// (internal to the library; the public C ABI is include/bq_api.h).
#pragma once

#include <stdarg.h>

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bq {

// Tuning switches (BQ_* environment variables, 0 = the launcher's default)
// and the device's compute-unit count, read once: at bq_init, or at the
// first launch of a process that never called it.
struct Tune {
  int gemv_waves;   // BQ_GEMV_WAVES: waves per workgroup of the general M <= 16 kernel (4, 8, 16;
                   // default 16); set, it also takes M = 1 per-row from k_gemv_m1
  int gemv_m1_waves;  // BQ_GEMV_M1_WAVES: waves per k_gemv_m1 workgroup (2, 4, 8)
  int tile_bm;      // BQ_TILE_BM: rows per tiled prefill tile (32, 64, 128)
  int tile_bn;      // BQ_TILE_BN: columns per tiled tile (128, 256)
  int ring;         // BQ_RING: LDS ring stages of the tiled kernels
  int tile_ksp;     // BQ_TILE_KSP: K groups per 64 x 128 prefill tile (1, 2)
  int moe_bm;       // BQ_MOE_BM: MoE m-tile records (16 = skinny kernels)
  int moe_bm_down;  // BQ_MOE_BM_DOWN: the down projection's m-tile alone
  int moe_order;    // BQ_MOE_ORDER: MoE work order of the LDS-ring kernels (0, 1, 2)
  int down_breg;    // BQ_DOWN_BREG: 0 disables the register-streamed down kernel
  int nq_pair;      // BQ_NQ_PAIR: 0 disables the pair-layout norm-quant
  int nq_v8;        // BQ_NQ_V8: 0 disables the 8-values-per-lane norm-quant and head prep (block 128)
  int moe_prep;     // BQ_MOE_PREP: 0 runs bq_moe_prep as separate launches
  int mf;           // BQ_MF: MFMA tile of the LDS-ring kernels (16: 16x16x64, 32: 32x32x32)
  int down_skinny;  // BQ_DOWN_SKINNY: skinny MoE down, 10 x k-steps per slot + strips per wave (32; 12, 14, 21, 22, 42)
  int gu_skinny;    // BQ_GU_SKINNY: skinny MoE gate/up, k-steps per register slot (4; 2, 6)
  int head_grid;    // BQ_HEAD_GRID: vocabulary-head workgroups (one per CU)
  int sel_fused;    // BQ_SEL_FUSED: 0 keeps the head selection's two threshold launches
  int attn_waves;   // BQ_ATTN_WAVES: waves the attention split plan aims for (2048)
  int prep_one;     // BQ_PREP_ONE: MoE prep's top-k + schedule in one workgroup (up to 16 tokens)
  int skinny2;      // BQ_SKINNY2: 0 keeps one n-tile per workgroup for 2..16-row per-row linears; 2 or 3 caps the tiles per workgroup (default 4)
  int cus;          // compute units of the device
};
const Tune& tune();
void tune_init(int device);

// the allocation-free phase 2's static device scratch (bytes) and its
// address on a device
constexpr size_t kNoallocScratchBytes = size_t(24) << 20;
hipError_t scratch_address(int device, void** out);

// One output segment of a (possibly fused) per-row / per-block linear: the
// fused q/k/v projection (butterquant_kernels/linear.mojo:273-326) runs as
// three segments of one launch sharing the activation.
struct LinSeg {
  const int8_t* w;   // tile16x64 codes [n, K]
  const float* ws;   // per-row weight scale [n]
  uint16_t* out;     // bf16 [M, n]
  float* out_f32;    // optional f32 [M, n] (pre-cast values)
  int n;             // output rows of this segment
  int tile0;         // first global n-tile (16 rows) of this segment
};

struct LinArgs {
  LinSeg seg[3];
  int nseg;
  const int8_t* act;  // int8 [M, K] row-major
  const float* sa;    // per-row [M] or per-block [M, K/block] activation scales
  int M, K;
  int block;          // per-block K block (multiple of 64); K for per-row
};

hipError_t launch_retile(const int8_t* src, int layout, int8_t* dst, int N, int K, hipStream_t st);
hipError_t launch_unpack(const int8_t* src, int8_t* dst, int N, int K, hipStream_t st);
hipError_t launch_pack_colsum(const int8_t* src, int8_t* dst, float* colsum, int N, int K,
                              int block_cols, int row_major, hipStream_t st);
hipError_t launch_quantize_weight(const uint16_t* w, const float* gamma, int8_t* q, float* scales,
                                  int rows, int cols, int block, int per_block, hipStream_t st);

int pick_port_unroll(int cols);
hipError_t launch_norm_quant(const uint16_t* src, const uint16_t* gamma, int8_t* xq, float* sa,
                             int seq_len, int hidden, int block, float sqrt_n, float n_eps,
                             hipStream_t st);
hipError_t launch_block_quant(const uint16_t* src, int8_t* xq, float* sa, int rows, int cols,
                              int block, int apply_fwht, hipStream_t st);

// per_block = 0: y = f32(acc) * (sa[m]/127) * ws[n]
// per_block = 1: y = ws[n] * sum_b fma-chain f32(acc_b) * (sa[m,b]/127)
hipError_t launch_linear(const LinArgs& a, int per_block, hipStream_t st);
// bq_norm_quant of a.act's source rows followed by the per-row linear a
// (a.act / a.sa are nq.xq / nq.sa): one fused launch for one token, else the
// two launches
struct NormArgs {
  const uint16_t* src;    // bf16 [M, K]
  const uint16_t* gamma;  // bf16 [K]
  int8_t* xq;             // int8 [M, K] codes (written)
  float* sa;              // [M] amax (written)
  int block;              // FWHT block
  float sqrt_n, n_eps, fwht_scale;  // fwht_scale: set by the launcher
};
hipError_t launch_norm_linear(const LinArgs& a, const NormArgs& nq, hipStream_t st);

struct Route { int32_t token; float weight; };

hipError_t launch_linear_tiled(const LinArgs& a, int per_block, int bm, hipStream_t st);
hipError_t launch_moe_gate_up_tiled(const int8_t* x_i8, const float* x_sa, const int32_t* eo,
                                    const Route* routes, const int8_t* w_gu, const float* gu_scale,
                                    uint16_t* bucket, int8_t* bi8, float* bsa, int experts,
                                    int max_routes, int hidden, int inter, int bm, hipStream_t st);
hipError_t launch_moe_down_tiled(const int8_t* b_i8, const float* b_sa, const int32_t* eo,
                                 const Route* routes, const int8_t* w_d, const float* d_scale,
                                 float* y, int experts, int max_routes, int hidden, int inter,
                                 int block, int bm, hipStream_t st);
int moe_tile_bm(int max_routes, int experts);

// kernels/flash_sample.mojo:21-28 SamplingParams and :120-134
// SampleOutcome[256], laid out as the Mojo structs are (bq_api.h mirrors them)
constexpr int kSampleNmax = 256;
struct SamplingParams {
  float temperature;
  float min_p;
  int64_t top_k;
  uint64_t seed;
  int64_t n_keep;
  uint8_t greedy;
  uint8_t pad_[7];
};
struct SampleOutcome {
  int32_t token_id;
  float logz;
  int64_t n;
  float topn_val[kSampleNmax];
  int32_t topn_idx[kSampleNmax];
};
hipError_t launch_head_prep(const uint16_t* src, const uint16_t* gamma, int8_t* xq, float* sa,
                            int rows, int hidden, int block, float sqrt_n, float n_eps,
                            hipStream_t st);
hipError_t launch_embed(const int32_t* tokens, const int8_t* w, const float* ws, uint16_t* dst,
                        int T, int hidden, int block, int shard_rows, int rank, float scale,
                        hipStream_t st);
size_t head_workspace_bytes(int rows, int vocab);
hipError_t launch_flash_sample(const int8_t* x, const float* xsa, const int8_t* w, const float* ws,
                               const SamplingParams* params, SampleOutcome* out, int R, int V,
                               int H, int block, float cap, int64_t vbase, void* workspace,
                               hipStream_t st);
int api_failv(int code, const char* fmt, va_list ap);  // sets bq_last_error()
hipError_t launch_router_logits(const uint16_t* x, const uint16_t* proj, const uint16_t* rscale,
                                float* logits, int T, int H, int E, float sqrt_n, float n_eps,
                                hipStream_t st);
hipError_t launch_route_schedule(const float* logits, const uint16_t* pes, int T, int E,
                                 int top_k, int32_t* route_idx, float* route_w,
                                 int32_t* expert_offset, Route* routes, hipStream_t st);
hipError_t launch_route_topk(const float* logits, const uint16_t* pes, int T, int E, int top_k,
                             int32_t* route_idx, float* route_w, hipStream_t st);
hipError_t launch_moe_prep(const float* logits, const uint16_t* pes, const uint16_t* src,
                           const uint16_t* gamma, int T, int E, int top_k, int hidden, int block,
                           float sqrt_n, float n_eps, int32_t* route_idx, float* route_w,
                           int32_t* expert_offset, Route* routes, int8_t* xq, float* sa,
                           hipStream_t st, const uint16_t* gamma2 = nullptr,
                           int8_t* xq2 = nullptr, float* sa2 = nullptr);
hipError_t launch_build_schedule(const int32_t* route_idx, const float* route_w, int seq_len,
                                 int top_k, int expert_base, int experts, int32_t* expert_offset,
                                 Route* routes, hipStream_t st);
// The decoder layer's dense MLP carried by the MoE launches (bq_ffn_gate_up,
// bq_ffn_down): T tokens' gate and up projections (per-row weights, the
// linears' bf16 outputs, GELU-tanh(gate) * up, FWHT64 block-quant) in extra
// workgroups of the MoE gate/up launch, and their down projection (per-block
// activations, bf16 out) in extra workgroups of the MoE down launch.
struct DenseGateUp {
  const int8_t* wg;    // gate [inter, hidden], tile16x64
  const int8_t* wu;    // up [inter, hidden], tile16x64
  const float* sg;     // gate per-row scales [inter]
  const float* su;     // up per-row scales [inter]
  const int8_t* x_i8;  // [T, hidden]
  const float* x_sa;   // [T]
  int8_t* out_i8;      // [T, inter]
  float* out_sa;       // [T, inter / 64]
  int T, inter;
  int ytiles, cpg, gx;  // the launcher's: grid rows taken, 64-column chunks per row, grid x
};
struct DenseDown {
  const int8_t* w;     // down [hidden, inter], tile16x64
  const float* ws;     // per-row scales [hidden]
  const int8_t* x_i8;  // [T, inter]
  const float* x_sa;   // [T, inter / block]
  uint16_t* out;       // [T, hidden] bf16
  int T, inter;
  int ytiles;          // the launcher's: grid rows taken
};
// bi8 / bsa non-null: the bucket's FWHT64 block-quant fused into the
// epilogue (bucket may then be null); inter % 64 == 0 for that.  dn: the
// dense MLP's gate/up in the same launch (bi8 required, dn->inter % 64 == 0).
hipError_t launch_moe_phase1(const int8_t* x_i8, const float* x_sa, const int32_t* expert_offset,
                             const Route* routes, const int8_t* w_gu, const float* gu_scale,
                             uint16_t* bucket, int8_t* bi8, float* bsa, int experts,
                             int max_routes, int hidden, int inter, hipStream_t st,
                             const DenseGateUp* dn = nullptr);
size_t moe_phase2_workspace(int max_routes, int seq_len, int hidden);
// dn: the dense MLP's down projection in the down launch (dn->inter % block
// == 0, dn->inter / block <= 64)
hipError_t launch_moe_phase2(const int8_t* bucket_i8, const float* bucket_sa,
                             const int32_t* expert_offset, const Route* routes,
                             const int8_t* w_down, const float* down_scale, float* accum,
                             uint16_t* out, int experts, int seq_len, int max_routes, int hidden,
                             int inter, int block, void* workspace, hipStream_t st,
                             const DenseDown* dn = nullptr);

// int8-KV attention (bq_attn.hip)
struct KvRun {  // kernels/attention_ops.mojo:54-58 KVRun
  int32_t buf_start, base_pos, rows_off, page_count;
};
constexpr int kAttnMinSplit = 32;  // fewest KV positions per split
struct PrepArgs {
  const uint16_t *q_src, *k_src, *v_src, *q_norm, *k_norm;
  int8_t* q_i8;
  float *qi_bias, *f_q;
  int8_t* k_cache;
  float* k_scale;
  int8_t* v_cache;
  float* v_scale;
  const float *cos_table, *sin_table;
  const KvRun* runs;
  const int32_t* base_rows;
  int num_runs, T, num_q, num_kv, rope_half, pair_stride;
  float sqrt_n, n_eps, fwht_scale;  // fwht_scale: set by launch_attn_prep
  int cache_degree, rank, page_shift, row_mask, page_mask;
};
struct AttnArgs {
  const int8_t* q_i8;
  const float *qi_bias, *f_q;
  const int8_t* k_cache;
  const float* k_scale;
  const int8_t* v_cache;
  const float* v_scale;
  const KvRun* runs;
  const int32_t* base_rows;
  uint16_t* out;
  float *ws_acc, *ws_ml;
  int num_runs, T, num_q, num_kv, window, page_shift, row_mask, page_mask, s_max;
};
hipError_t launch_attn_prep(const PrepArgs& a, int head_dim, hipStream_t st);
hipError_t launch_flash_attn(const AttnArgs& a, int head_dim, hipStream_t st);
int attn_splits(int seq_len, int num_kv, int max_kv_len);

}  // namespace bq
