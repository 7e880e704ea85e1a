// bq_moe.hip -- the quantized MoE expert layer (butterquant_kernels/moe.mojo)
// and its CSR schedule (kernels/moe_router.mojo:60-106).
//
// Schedule: expert_offset[E+1] (exclusive prefix of per-expert route counts)
//   and routes[] sorted by (expert, token, k) -- the reference's order -- built
//   by one workgroup with LDS counters and per-expert token bitmasks (a route's
//   rank = number of earlier tokens routed to the same expert).
// Phase 1 (moe.mojo:25-164): grouped GEMM over (expert m-tile, intermediate
//   tile); each wave accumulates the gate and up 16x16 tiles of the same
//   intermediate columns, so the epilogue bucket = bf16(gelu(g)*u) is
//   element-wise in registers.  A rows are gathered by route token.
// Phase 2 (moe.mojo:167-335): grouped per-block GEMM (B = 64) producing the
//   per-route f32 results y = (facc*ws)*route_w, then a combine that adds each
//   token's routes in ascending expert order -- the reference's accumulation
//   order (experts ascending, moe.mojo:259-282) -- so accum is bit-identical.
#include "bq_device.hpp"
#include "bq_kernels.hpp"

#include <stdlib.h>

namespace bq {

constexpr int kMaxExperts = 256;

__global__ __launch_bounds__(1024) void k_build_schedule(
    const int32_t* __restrict__ route_idx, const float* __restrict__ route_w, int T, int top_k,
    int ebase, int E, int32_t* __restrict__ expert_offset, Route* __restrict__ routes) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int running[kMaxExperts];
  __shared__ uint32_t bits[kMaxExperts][32];
  __shared__ int wpre[kMaxExperts][32];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  const int slots = T * top_k;
  for (int s = tid; s < slots; s += blockDim.x) {
    const int e = route_idx[s] - ebase;
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int e = 0; e < E; ++e) {
      expert_offset[e] = run;
      running[e] = run;
      run += cnt[e];
    }
    expert_offset[E] = run;
  }
  __syncthreads();
  for (int c0 = 0; c0 < T; c0 += 1024) {
    for (int i = tid; i < E * 32; i += blockDim.x) bits[i >> 5][i & 31] = 0u;
    __syncthreads();
    const int t = c0 + tid;
    if (t < T) {
      for (int kk = 0; kk < top_k; ++kk) {
        const int e = route_idx[(size_t)t * top_k + kk] - ebase;
        if (e >= 0 && e < E) atomicOr(&bits[e][tid >> 5], 1u << (tid & 31));
      }
    }
    __syncthreads();
    for (int e = tid; e < E; e += blockDim.x) {
      int run = 0;
      for (int w = 0; w < 32; ++w) {
        wpre[e][w] = run;
        run += __popc(bits[e][w]);
      }
    }
    __syncthreads();
    if (t < T) {
      const int w = tid >> 5;
      const uint32_t below = (1u << (tid & 31)) - 1u;
      for (int kk = 0; kk < top_k; ++kk) {
        const size_t slot = (size_t)t * top_k + kk;
        const int e = route_idx[slot] - ebase;
        if (e >= 0 && e < E) {
          const int pos = running[e] + wpre[e][w] + __popc(bits[e][w] & below);
          routes[pos].token = t;
          routes[pos].weight = route_w[slot];
        }
      }
    }
    __syncthreads();
    for (int e = tid; e < E; e += blockDim.x) running[e] += wpre[e][31] + __popc(bits[e][31]);
    __syncthreads();
  }
}

// Phase 1, 16-record m-tiles: blockIdx.y = m-tile, blockIdx.x = group of 4
// intermediate 16-column subtiles (one per wave).
template <int U>
__global__ __launch_bounds__(256) void k_moe_gate_up_skinny(
    const int8_t* __restrict__ x_i8, const float* __restrict__ x_sa,
    const int32_t* __restrict__ eo, const Route* __restrict__ routes,
    const int8_t* __restrict__ w_gu, const float* __restrict__ gu_scale,
    uint16_t* __restrict__ bucket, int E, int hidden, int inter, int max_routes) {
  int e, r0, r1;
  if (!find_mtile(eo, E, 16, blockIdx.y, max_routes, e, r0, r1)) return;
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int isub = blockIdx.x * 4 + wave;
  if (isub * 16 >= inter) return;
  const int K = hidden, K64 = K >> 6;
  const size_t gate_up = (size_t)2 * inter;
  const int8_t* we = w_gu + (size_t)e * gate_up * K;
  const int8_t* wg = we + (size_t)isub * K64 * 1024 + lane * 16;
  const int8_t* wu = we + (size_t)((inter >> 4) + isub) * K64 * 1024 + lane * 16;
  const int arow = r0 + (lane & 15);
  const bool aval = arow < r1;
  const int8_t* ab = x_i8 + (size_t)routes[aval ? arow : r0].token * K + (lane >> 4) * 16;
  const v4i zero = {0, 0, 0, 0};
  v4i cg = zero, cu = zero;
  int kt = 0;
  for (; kt + U <= K64; kt += U) {
    v4i bg[U], bu[U], af[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      bg[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wg + (size_t)(kt + u) * 1024));
      bu[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wu + (size_t)(kt + u) * 1024));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) af[u] = ld16(ab + (kt + u) * 64);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      cg = mfma16x16x64(af[u], bg[u], cg);
      cu = mfma16x16x64(af[u], bu[u], cu);
    }
  }
  for (; kt < K64; ++kt) {
    const v4i bgf = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wg + (size_t)kt * 1024));
    const v4i buf = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wu + (size_t)kt * 1024));
    const v4i af = ld16(ab + kt * 64);
    cg = mfma16x16x64(af, bgf, cg);
    cu = mfma16x16x64(af, buf, cu);
  }
  const float* ws = gu_scale + (size_t)e * gate_up;
  const int col = isub * 16 + (lane & 15);
  const int g4[4] = {cg.x, cg.y, cg.z, cg.w};
  const int u4[4] = {cu.x, cu.y, cu.z, cu.w};
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int rec = r0 + 4 * (lane >> 4) + v;
    if (rec >= r1) continue;
    const float ad = x_sa[routes[rec].token] * kInv127;
    const float gv = (float)g4[v] * ad * ws[col];
    const float uv = (float)u4[v] * ad * ws[inter + col];
    bucket[(size_t)rec * inter + col] = f32_to_bf16(gelu_tanh_f32(gv) * uv);
  }
}

// Phase 2 GEMM, 16-record m-tiles: y[rec, n] = (facc * ws[n]) * route_w[rec]
// with facc the fma chain over K blocks (moe.mojo:198-223).
template <int U>
__global__ __launch_bounds__(256) void k_moe_down_skinny(
    const int8_t* __restrict__ b_i8, const float* __restrict__ b_sa,
    const int32_t* __restrict__ eo, const Route* __restrict__ routes,
    const int8_t* __restrict__ w_d, const float* __restrict__ d_scale, float* __restrict__ y,
    int E, int hidden, int inter, int block, int max_routes) {
  int e, r0, r1;
  if (!find_mtile(eo, E, 16, blockIdx.y, max_routes, e, r0, r1)) return;
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int nsub = blockIdx.x * 4 + wave;
  if (nsub * 16 >= hidden) return;
  const int K = inter, K64 = K >> 6, fpb = block >> 6, nb = K / block;
  const int8_t* wb = w_d + (size_t)e * hidden * K + (size_t)nsub * K64 * 1024 + lane * 16;
  const int arow = r0 + (lane & 15);
  const bool aval = arow < r1;
  const int8_t* ab = b_i8 + (size_t)(aval ? arow : r0) * K + (lane >> 4) * 16;
  const v4i zero = {0, 0, 0, 0};
  float facc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  int rec4[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) rec4[v] = r0 + 4 * (lane >> 4) + v;
  v4i c = zero;
  for (int kt0 = 0; kt0 < K64; kt0 += U) {
    v4i bf[U], af[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (kt0 + u < K64) {
        bf[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wb + (size_t)(kt0 + u) * 1024));
        af[u] = ld16(ab + (kt0 + u) * 64);
      }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kt = kt0 + u;
      if (kt >= K64) break;
      c = mfma16x16x64(af[u], bf[u], c);
      if (((kt + 1) & (fpb - 1)) == 0) {
        const int b = kt / fpb;
        const int cc[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float adv = rec4[v] < r1 ? b_sa[(size_t)rec4[v] * nb + b] * kInv127 : 0.0f;
          facc[v] = fmaf((float)cc[v], adv, facc[v]);
        }
        c = zero;
      }
    }
  }
  const float* ws = d_scale + (size_t)e * hidden;
  const int col = nsub * 16 + (lane & 15);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    if (rec4[v] >= r1) continue;
    y[(size_t)rec4[v] * hidden + col] = facc[v] * ws[col] * routes[rec4[v]].weight;
  }
}

__global__ void k_fill_i32(int32_t* p, int n, int v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// per-token record lists (unordered; the combine sorts them)
__global__ void k_token_lists(const int32_t* __restrict__ eo, int E, const Route* __restrict__ routes,
                              int32_t* __restrict__ tok_cnt, int32_t* __restrict__ tok_recs,
                              int cap, int T, int max_routes) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= eo[E] || r >= max_routes) return;
  const int t = routes[r].token;
  if (t < 0 || t >= T) return;
  const int p = atomicAdd(&tok_cnt[t], 1);
  if (p < cap) tok_recs[(size_t)t * cap + p] = r;
}

// Same lists built by one workgroup with LDS counters (seq_len <= 16384):
// no separate clearing pass over global memory.
__global__ __launch_bounds__(1024) void k_token_lists_lds(
    const int32_t* __restrict__ eo, int E, const Route* __restrict__ routes,
    int32_t* __restrict__ tok_cnt, int32_t* __restrict__ tok_recs, int cap, int T,
    int max_routes) {
  extern __shared__ int cnt[];
  for (int t = threadIdx.x; t < T; t += blockDim.x) cnt[t] = 0;
  __syncthreads();
  const int n = min(eo[E], max_routes);
  for (int r = threadIdx.x; r < n; r += blockDim.x) {
    const int t = routes[r].token;
    if (t < 0 || t >= T) continue;
    const int p = atomicAdd(&cnt[t], 1);
    if (p < cap) tok_recs[(size_t)t * cap + p] = r;
  }
  __syncthreads();
  for (int t = threadIdx.x; t < T; t += blockDim.x) tok_cnt[t] = cnt[t];
}

// accum[t, n] = (((0 + y[r1,n]) + y[r2,n]) + ...) over t's records in
// ascending record order (= ascending expert order); out = bf16(accum).
__global__ __launch_bounds__(256) void k_combine(
    const float* __restrict__ y, const int32_t* __restrict__ tok_cnt,
    const int32_t* __restrict__ tok_recs, int cap, int T, int hidden,
    float* __restrict__ accum, uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= hidden) return;
  int recs[16];
  int cnt = tok_cnt[t];
  cnt = cnt < cap ? cnt : cap;
  for (int j = 0; j < cnt; ++j) {
    const int r = tok_recs[(size_t)t * cap + j];
    int p = j;
    while (p > 0 && recs[p - 1] > r) { recs[p] = recs[p - 1]; --p; }
    recs[p] = r;
  }
  float acc = 0.0f;
  for (int j = 0; j < cnt; ++j) acc = acc + y[(size_t)recs[j] * hidden + n];
  accum[(size_t)t * hidden + n] = acc;
  out[(size_t)t * hidden + n] = f32_to_bf16(acc);
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
hipError_t launch_build_schedule(const int32_t* route_idx, const float* route_w, int seq_len,
                                 int top_k, int expert_base, int experts, int32_t* expert_offset,
                                 Route* routes, hipStream_t st) {
  if (seq_len <= 0) return hipSuccess;
  if (experts > kMaxExperts) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_build_schedule, dim3(1), dim3(1024), 0, st, route_idx, route_w, seq_len,
                     top_k, expert_base, experts, expert_offset, routes);
  return hipGetLastError();
}

static inline int mtile_bound(int max_routes, int experts, int bm) {
  // sum_e ceil(n_e/bm) <= max_routes/bm + experts
  long b = (long)(max_routes + bm - 1) / bm + experts;
  return (int)b;
}

// m-tile height for the grouped kernels from the mean routes per expert:
// 16-row skinny tiles while experts see a handful of tokens (decode), LDS-
// tiled 64/128-row tiles once each expert's weights can be reused.
int moe_tile_bm(int max_routes, int experts) {
  if (const char* s = getenv("BQ_MOE_BM")) return atoi(s);
  const int per = max_routes / (experts > 0 ? experts : 1);
  if (per >= 96) return 128;
  if (per >= 24) return 64;
  return 16;
}

hipError_t launch_moe_phase1(const int8_t* x_i8, const float* x_sa, const int32_t* eo,
                             const Route* routes, const int8_t* w_gu, const float* gu_scale,
                             uint16_t* bucket, int experts, int max_routes, int hidden,
                             int inter, hipStream_t st) {
  if (max_routes <= 0) return hipSuccess;
  const int bm = moe_tile_bm(max_routes, experts);
  if (bm >= 64 && inter % 64 == 0)
    return launch_moe_gate_up_tiled(x_i8, x_sa, eo, routes, w_gu, gu_scale, bucket, experts,
                                    max_routes, hidden, inter, bm, st);
  dim3 g((inter / 16 + 3) / 4, mtile_bound(max_routes, experts, 16)), b(256);
  hipLaunchKernelGGL(k_moe_gate_up_skinny<4>, g, b, 0, st, x_i8, x_sa, eo, routes, w_gu,
                     gu_scale, bucket, experts, hidden, inter, max_routes);
  return hipGetLastError();
}

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t moe_phase2_workspace(int max_routes, int seq_len, int hidden) {
  if (seq_len <= 0) return 0;
  const size_t cap = ((size_t)max_routes + seq_len - 1) / seq_len;
  return align256((size_t)max_routes * hidden * sizeof(float)) +
         align256((size_t)seq_len * sizeof(int32_t)) +
         align256((size_t)seq_len * cap * sizeof(int32_t));
}

hipError_t launch_moe_phase2(const int8_t* bucket_i8, const float* bucket_sa, const int32_t* eo,
                             const Route* routes, const int8_t* w_down, const float* down_scale,
                             float* accum, uint16_t* out, int experts, int seq_len,
                             int max_routes, int hidden, int inter, int block, void* workspace,
                             hipStream_t st) {
  if (seq_len <= 0) return hipSuccess;
  const int cap = (max_routes + seq_len - 1) / seq_len;
  if (cap > 16) return hipErrorInvalidValue;
  char* ws = (char*)workspace;
  float* y = (float*)ws;
  int32_t* tok_cnt = (int32_t*)(ws + align256((size_t)max_routes * hidden * sizeof(float)));
  int32_t* tok_recs = (int32_t*)((char*)tok_cnt + align256((size_t)seq_len * sizeof(int32_t)));
  if (seq_len <= 16384) {
    hipLaunchKernelGGL(k_token_lists_lds, dim3(1), dim3(1024), (size_t)seq_len * sizeof(int), st,
                       eo, experts, routes, tok_cnt, tok_recs, cap, seq_len, max_routes);
  } else {
    hipLaunchKernelGGL(k_fill_i32, dim3((seq_len + 255) / 256), dim3(256), 0, st, tok_cnt, seq_len, 0);
    hipLaunchKernelGGL(k_token_lists, dim3((max_routes + 255) / 256), dim3(256), 0, st, eo,
                       experts, routes, tok_cnt, tok_recs, cap, seq_len, max_routes);
  }
  if (max_routes > 0) {
    const int bm = moe_tile_bm(max_routes, experts);
    if (bm >= 64 && hidden % 128 == 0) {
      hipError_t e = launch_moe_down_tiled(bucket_i8, bucket_sa, eo, routes, w_down, down_scale, y,
                                           experts, max_routes, hidden, inter, block, bm, st);
      if (e != hipSuccess) return e;
    } else {
      dim3 g((hidden / 16 + 3) / 4, mtile_bound(max_routes, experts, 16)), b(256);
      hipLaunchKernelGGL(k_moe_down_skinny<4>, g, b, 0, st, bucket_i8, bucket_sa, eo, routes,
                         w_down, down_scale, y, experts, hidden, inter, block, max_routes);
    }
  }
  hipLaunchKernelGGL(k_combine, dim3((hidden + 255) / 256, seq_len), dim3(256), 0, st, y, tok_cnt,
                     tok_recs, cap, seq_len, hidden, accum, out);
  return hipGetLastError();
}

}  // namespace bq
