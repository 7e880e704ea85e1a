// bq_router.hip -- the MoE router ahead of the expert schedule
// (kernels/moe_router.mojo:148-298): router logits, top-k with the
// reference's candidate order, and the softmax merge.
//
// Logits (RouterExpertKernel, moe_router.mojo:164-187): every logit is an f32
//   dot product whose rounding the reference fixes through its SIMD
//   accumulator order, so each one is computed in exactly that order: chain
//   c = p*16 + j (PU accumulators of 16 lanes) is an fma chain over elements
//   i*PU*16 + c; lanes own adjacent chains, the chains of a logit are merged
//   with cross-lane adds in the reference's tree order.  Vector fp32 (an MFMA
//   would reassociate the sums).
// Top-k + softmax (insert_candidate :43-57 and RouterMergeKernel :248-293):
//   one wave per token.  insert_candidate keeps the k best candidates under
//   a strict total order (logit descending, lower expert first on ties)
//   among logits above the sentinel -1e30, padding with {expert 0, -1e30}.
//   The wave takes k successive maxima of a 64-bit key that encodes that
//   order, so the selected list is the reference's list entry for entry.
#include <mutex>
#include <unordered_map>

#include "bq_device.hpp"
#include "bq_kernels.hpp"
#include "bq_sched.hpp"

namespace bq {

constexpr float kRouterSentinel = -1.0e30f;

// A workgroup computes TT tokens x (4 waves x EE experts).  Lane l owns the
// CPL adjacent chains c = l*CPL + r of the PU = CPL*4 accumulator bank
// (64*CPL chains); per step i it scales its TT x values on the fly
// ((x * router_scale) * inv_rms, :177-181) and runs TT*EE*CPL fma chains.
template <int TT, int EE, int CPL>
__global__ __launch_bounds__(256) void k_router_logits(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ proj,
    const uint16_t* __restrict__ rscale, float* __restrict__ logits, int T, int H, int E,
    int pu_bf16, float sqrt_n, float n_eps) {
  __shared__ float s_inv[TT];
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int t0 = blockIdx.x * TT, e0 = (blockIdx.y * 4 + wave) * EE;
  for (int tt = wave; tt < TT; tt += 4) {
    const int t = min(t0 + tt, T - 1);
    const float ssq =
        wave_row_ssq(reinterpret_cast<const uint32_t*>(x + (size_t)t * H), H, pu_bf16);
    if (lane == 0) s_inv[tt] = sqrt_n / __builtin_sqrtf(ssq + n_eps);
  }
  __syncthreads();
  float inv[TT];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) inv[tt] = s_inv[tt];

  const uint16_t* xr[TT];
  const uint16_t* wr[EE];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) xr[tt] = x + (size_t)min(t0 + tt, T - 1) * H;
#pragma unroll
  for (int ee = 0; ee < EE; ++ee) wr[ee] = proj + (size_t)min(e0 + ee, E - 1) * H;

  constexpr int C = 64 * CPL;  // chains = PU*16 elements per step
  float acc[TT][EE][CPL];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int ee = 0; ee < EE; ++ee)
#pragma unroll
      for (int r = 0; r < CPL; ++r) acc[tt][ee][r] = 0.0f;

  const int iters = H / C;
  for (int i = 0; i < iters; ++i) {
    const int off = i * C + lane * CPL;
    float sv[CPL], xs[TT][CPL], wv[EE][CPL];
    if constexpr (CPL == 2) {
      const uint32_t s2 = *reinterpret_cast<const uint32_t*>(rscale + off);
      sv[0] = __uint_as_float(s2 << 16);
      sv[1] = __uint_as_float(s2 & 0xFFFF0000u);
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(xr[tt] + off);
        xs[tt][0] = __uint_as_float(v << 16);
        xs[tt][1] = __uint_as_float(v & 0xFFFF0000u);
      }
#pragma unroll
      for (int ee = 0; ee < EE; ++ee) {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(wr[ee] + off);
        wv[ee][0] = __uint_as_float(v << 16);
        wv[ee][1] = __uint_as_float(v & 0xFFFF0000u);
      }
    } else {
      sv[0] = bf16_to_f32(rscale[off]);
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) xs[tt][0] = bf16_to_f32(xr[tt][off]);
#pragma unroll
      for (int ee = 0; ee < EE; ++ee) wv[ee][0] = bf16_to_f32(wr[ee][off]);
    }
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int r = 0; r < CPL; ++r) xs[tt][r] = xs[tt][r] * sv[r] * inv[tt];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int ee = 0; ee < EE; ++ee)
#pragma unroll
        for (int r = 0; r < CPL; ++r) acc[tt][ee][r] = fmaf(xs[tt][r], wv[ee][r], acc[tt][ee][r]);
  }

  // chain c = l*CPL + r is (p, j) = (c >> 4, c & 15).  tree_merge_accs
  // (simd_math/matrixops.mojo:265-283): acc[p] += acc[p + s] for s = 1, 2,
  // 4 -> partner lane + s*16/CPL; then the 16-lane halving reduce_add: lane
  // + h/CPL for h >= CPL, in-lane r + 1 for h = 1 < CPL.  Lane 0, r = 0 ends
  // with the logit; lane tt*EE + ee stores it.
  constexpr int PU = 4 * CPL;
  float mine = 0.0f;
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int ee = 0; ee < EE; ++ee) {
      float v[CPL];
#pragma unroll
      for (int r = 0; r < CPL; ++r) v[r] = acc[tt][ee][r];
#pragma unroll
      for (int q = 0; (1 << q) < PU; ++q)
#pragma unroll
        for (int r = 0; r < CPL; ++r) v[r] = v[r] + __shfl_down(v[r], (16 << q) / CPL, kWave);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int h = 8 >> q;
        if (h >= CPL) {
#pragma unroll
          for (int r = 0; r < CPL; ++r) v[r] = v[r] + __shfl_down(v[r], h / CPL, kWave);
        } else if constexpr (CPL == 2) {
          v[0] = v[0] + v[1];
        }
      }
      const float total = __shfl(v[0], 0, kWave);
      if (lane == tt * EE + ee) mine = total;
    }
  static_assert(TT * EE <= 64, "one logit per lane");
  const int tt = lane / EE, ee = lane % EE;
  if (lane < TT * EE && t0 + tt < T && e0 + ee < E) logits[(size_t)(t0 + tt) * E + e0 + ee] = mine;
}

// 64-bit key ordering candidates like insert_candidate: high word = the
// logit mapped to an unsigned order (-0.0 taken as +0.0, since the reference
// compares floats), low word = (1023 - expert) << 1 so lower experts win
// ties, plus bit 0 remembering a -0.0 logit.  Candidates at or below the
// sentinel (and NaN) get key 0 and are never selected.
__device__ inline uint64_t cand_key(float lg, int e) {
  const uint32_t b = __float_as_uint(lg);
  const uint32_t negzero = (b == 0x80000000u) ? 1u : 0u;
  const uint32_t cb = negzero ? 0u : b;
  const uint32_t ord = (cb & 0x80000000u) ? ~cb : (cb | 0x80000000u);
  return ((uint64_t)ord << 32) | ((uint32_t)(1023 - e) << 1) | negzero;
}

__device__ inline uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// One step of a wave max through a DPP lane move (a VALU op, no LDS round
// trip).  Rows outside ROW_MASK keep their own value.
template <int CTRL, int ROW_MASK>
__device__ inline uint32_t dpp_max_step32(uint32_t v) {
  const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, ROW_MASK, 0xF, false);
  return v > o ? v : o;
}

// Wave-uniform maximum: quad swaps (xor 1, xor 2), half-row and row
// mirrors leave every lane of a 16-lane row with the row maximum; the
// row_bcast15 / row_bcast31 steps carry it up so lane 63 holds the wave's.
__device__ inline uint32_t wave_max_u32(uint32_t v) {
  v = dpp_max_step32<0xB1, 0xF>(v);
  v = dpp_max_step32<0x4E, 0xF>(v);
  v = dpp_max_step32<0x141, 0xF>(v);
  v = dpp_max_step32<0x140, 0xF>(v);
  v = dpp_max_step32<0x142, 0xA>(v);
  v = dpp_max_step32<0x143, 0xC>(v);
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// The wave maximum of 64-bit candidate keys (0 when every key is 0):
// the maximum of the high words first (32-bit), then the low word of the
// one lane holding it, or -- only when several lanes tie on the high word
// -- the maximum of those lanes' low words.
__device__ inline uint64_t wave_max_key(uint64_t v) {
  const uint32_t hi = (uint32_t)(v >> 32), lo = (uint32_t)v;
  const uint32_t m = wave_max_u32(hi);
  if (m == 0u) return 0ull;  // no candidate left anywhere (uniform)
  const uint64_t tie = __ballot(hi == m);
  uint32_t l;
  if (__popcll(tie) == 1)  // uniform
    l = (uint32_t)__builtin_amdgcn_readlane((int)lo, (int)__builtin_ctzll(tie));
  else
    l = wave_max_u32(hi == m ? lo : 0u);
  return ((uint64_t)m << 32) | l;
}

// TPW tokens' top_k routes on one wave, their candidate chains interleaved:
// lane k < top_k gets route k's expert and weight of token i in out_e[i],
// out_w[i].  rows[i] points at token i's logits (all TPW rows are loaded
// before any selection starts).
template <int NE, int TPW>
__device__ inline void topk_tokens(const float* const (&rows)[TPW],
                                   const uint16_t* __restrict__ pes, int E, int top_k, int lane,
                                   int (&out_e)[TPW], float (&out_w)[TPW]) {
  uint64_t key[TPW][NE];
  float lgv[TPW][NE];
#pragma unroll
  for (int i = 0; i < TPW; ++i)
#pragma unroll
    for (int q = 0; q < NE; ++q) lgv[i][q] = rows[i][min(lane + 64 * q, E - 1)];
  // the per-expert scales of this lane's experts, loaded beside the logits:
  // the winners' scales are then a lane exchange, not a second dependent
  // global load after the top-k
  float pev[NE];
#pragma unroll
  for (int q = 0; q < NE; ++q) pev[q] = pes ? bf16_to_f32(pes[min(lane + 64 * q, E - 1)]) : 1.0f;
  uint64_t local[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
#pragma unroll
    for (int q = 0; q < NE; ++q) {
      const int e = lane + 64 * q;
      key[i][q] = (e < E && lgv[i][q] > kRouterSentinel) ? cand_key(lgv[i][q], e) : 0ull;
    }
    local[i] = key[i][0];
#pragma unroll
    for (int q = 1; q < NE; ++q) local[i] = umax64(local[i], key[i][q]);
  }
  // lane k keeps route k's logit and expert; the softmax follows the loop
  float my_lg[TPW], sum[TPW], my_ev[TPW];
  int my_e[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    my_lg[i] = kRouterSentinel;
    my_e[i] = 0;
  }
  for (int k = 0; k < top_k; ++k) {
    uint64_t best[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) best[i] = wave_max_key(local[i]);
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      float lg = kRouterSentinel;
      int e = 0;
      if (best[i] != 0ull) {
        const uint32_t hi = (uint32_t)(best[i] >> 32), lo = (uint32_t)best[i];
        e = 1023 - (int)(lo >> 1);
        const uint32_t b = (hi & 0x80000000u) ? (hi & 0x7FFFFFFFu) : ~hi;
        lg = __uint_as_float((lo & 1u) ? 0x80000000u : b);
#pragma unroll
        for (int q = 0; q < NE; ++q) key[i][q] = key[i][q] == best[i] ? 0ull : key[i][q];
        local[i] = key[i][0];
#pragma unroll
        for (int q = 1; q < NE; ++q) local[i] = umax64(local[i], key[i][q]);
      }
      if (lane == k) {
        my_lg[i] = lg;
        my_e[i] = e;
      }
    }
  }
  // RouterMergeKernel (:276-293): max = merged[0].logit, exp of the
  // difference, sum in slot order -- every route's exp at once (lane k),
  // then the sum over k in order
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const float mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_lg[i]), 0));
    const float ev = fast_exp_softmax_biased(my_lg[i] - mx);
    float s = 0.0f;
    for (int k = 0; k < top_k; ++k)
      s = s + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), k));
    sum[i] = s;
    my_ev[i] = lane < top_k ? ev : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const float inv_sum = 1.0f / sum[i];
    // expert my_e's scale sits in lane my_e % 64, slot my_e / 64
    float sc = 1.0f;
#pragma unroll
    for (int q = 0; q < NE; ++q) {
      const float v = __shfl(pev[q], my_e[i] & 63, kWave);
      if ((my_e[i] >> 6) == q) sc = v;
    }
    if (!(lane < top_k && pes)) sc = 1.0f;
    out_e[i] = my_e[i];
    out_w[i] = my_ev[i] * inv_sum * sc;
  }
}

template <int NE>
__global__ __launch_bounds__(256) void k_route_topk(
    const float* __restrict__ logits, const uint16_t* __restrict__ pes, int T, int E, int top_k,
    int32_t* __restrict__ route_idx, float* __restrict__ route_w) {
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;  // whole waves; no block synchronization below
  const float* rows[1] = {logits + (size_t)t * E};
  int e[1];
  float w[1];
  topk_tokens<NE, 1>(rows, pes, E, top_k, lane, e, w);
  if (lane < top_k) {
    route_idx[(size_t)t * top_k + lane] = e[0];
    route_w[(size_t)t * top_k + lane] = w[0];
  }
}

// Route top-k + the CSR schedule in one workgroup (used up to 8 tokens;
// seq_len * top_k <= kSchedSmallSlots, experts <= kMaxExperts): wave w takes tokens w, w + 16,
// ... (TPW <= 8 at a time, their logits loaded at once and their selections
// interleaved), writes route_idx / route_w and keeps each slot's expert and
// weight in LDS, and the schedule is built from there (schedule_small) --
// what k_route_topk followed by k_build_schedule_small write, in one launch.
template <int NE, int TPW>
__device__ inline void route_schedule_block(
    const float* __restrict__ logits, const uint16_t* __restrict__ pes, int T, int E, int top_k,
    int32_t* __restrict__ route_idx, float* __restrict__ route_w,
    int32_t* __restrict__ expert_offset, Route* __restrict__ routes) {
  constexpr int NWV = kSchedSmallSlots / 64;
  __shared__ int s_e[kSchedSmallSlots];
  __shared__ float s_w[kSchedSmallSlots];
  __shared__ int s_wc[kSchedWavesSmall][kMaxExperts];
  __shared__ int s_cnt[kMaxExperts];
  const int tid = threadIdx.x, wave = tid >> 6, lane = lane_id();
  for (int t0 = wave; t0 < T; t0 += NWV * TPW) {  // wave-uniform
    const float* rows[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) rows[i] = logits + (size_t)min(t0 + NWV * i, T - 1) * E;
    int e[TPW];
    float w[TPW];
    topk_tokens<NE, TPW>(rows, pes, E, top_k, lane, e, w);
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int t = t0 + NWV * i;
      if (t < T && lane < top_k) {
        const int slot = t * top_k + lane;
        route_idx[slot] = e[i];
        route_w[slot] = w[i];
        s_e[slot] = e[i];
        s_w[slot] = w[i];
      }
    }
  }
  __syncthreads();
  const bool live = tid < T * top_k;
  const int e = live ? s_e[tid] : -1;
  const float w = live ? s_w[tid] : 0.0f;
  schedule_small(e, w, top_k, E, T * top_k, s_wc, s_cnt, expert_offset, routes);
}

template <int NE, int TPW>
__global__ __launch_bounds__(kSchedSmallSlots) void k_route_schedule_small(
    const float* __restrict__ logits, const uint16_t* __restrict__ pes, int T, int E, int top_k,
    int32_t* __restrict__ route_idx, float* __restrict__ route_w,
    int32_t* __restrict__ expert_offset, Route* __restrict__ routes) {
  route_schedule_block<NE, TPW>(logits, pes, T, E, top_k, route_idx, route_w, expert_offset,
                                routes);
}

// The MoE block's prep for a decode-sized batch in one launch: the route
// top-k + softmax merge, the norm-quant of the hidden states and the CSR
// schedule -- the reference's dispatch_merge_router_candidates,
// dispatch_bq_norm_quant and dispatch_build_expert_schedules
// (modeling/gemma_4_moe_bq.mojo:673-688) -- with the same results.
// Workgroups [0, nq_blocks) norm-quantize two tokens each (the pair layout of
// k_norm_quant_pair: a token over WPT <= 8 waves of SPW segments, the row's
// amax through LDS); with a second gain (gamma2, the decoder's dense-MLP
// input norm, gemma_4_moe_bq.mojo:749-753) the second half of them quantizes
// the same rows into xq2 / sa2.  The others take 16 tokens' top-k each, one
// wave per token.  The last top-k workgroup to finish builds the schedule from every
// workgroup's routes (schedule_small, one thread per slot): each top-k
// workgroup fences its route stores at device scope before it counts itself
// done on *done, and the last one fences again before it reads them.  The
// count wraps to 0 on the last workgroup's increment (atomicInc), ready for
// the next launch on the same counter.  Each stream of a device has its own
// counter (prep_counter), so launches that overlap on different streams do
// not share one, and launches on one stream run in order.  With ONE > 0 (up to 16 tokens) a single
// workgroup after the norm-quant ones takes every token's top-k and builds
// the schedule from LDS (route_schedule_block), with no hand-off.
constexpr int kPrepThreads = kSchedSmallSlots;   // 16 waves
constexpr int kPrepTopkTokens = kPrepThreads / 64;
constexpr int kPrepCounters = 256;  // streams per device with a counter of their own
__device__ unsigned g_prep_done[kPrepCounters];  // zero-initialized at load

template <int NE, int NSEG, int SPW, int ONE = 0>  // ONE: tokens per wave of the one route workgroup
__global__ __launch_bounds__(kPrepThreads) void k_moe_prep(
    const float* __restrict__ logits, const uint16_t* __restrict__ pes,
    const uint16_t* __restrict__ src, const uint16_t* __restrict__ gamma,
    int8_t* __restrict__ xq, float* __restrict__ sa, int32_t* __restrict__ route_idx,
    float* __restrict__ route_w, int32_t* __restrict__ expert_offset, Route* __restrict__ routes,
    int T, int E, int top_k, int hidden, int block, float sqrt_n, float n_eps, float fwht_scale,
    int nq_blocks, unsigned* done, int nq_per, const uint16_t* __restrict__ gamma2,
    int8_t* __restrict__ xq2, float* __restrict__ sa2) {
  __shared__ float s_max[kPrepThreads / 64];
  __shared__ int s_wc[kSchedWavesSmall][kMaxExperts];
  __shared__ int s_cnt[kMaxExperts];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if ((int)blockIdx.x < nq_blocks) {
    // ---- norm-quant: token 2 b + g on waves 8 g .. 8 g + WPT - 1.  Blocks
    // [nq_per, 2 nq_per) quantize the same rows with a second gain into
    // xq2 / sa2 (the dense MLP's input beside the experts')
    const bool second = (int)blockIdx.x >= nq_per;  // workgroup-uniform
    if (second) { gamma = gamma2; xq = xq2; sa = sa2; }
    const int nseg = hidden >> 7, wpt = (nseg + SPW - 1) / SPW;
    const int g = wave >> 3, wv = wave & 7;
    const int t = ((int)blockIdx.x - (second ? nq_per : 0)) * 2 + g, q0 = wv * SPW;
    const bool live = t < T && wv < wpt;  // wave-uniform
    float v[SPW][2];
    if (live) {
      const uint32_t* xr = reinterpret_cast<const uint32_t*>(src + (size_t)t * hidden) + lane;
      const uint32_t* gr = reinterpret_cast<const uint32_t*>(gamma) + lane;
      // (loads return in issue order: the row first, which the sum of
      // squares needs first; the wave's own segments again, into x)
      uint32_t xp[NSEG], x[SPW], gp[SPW];
#pragma unroll
      for (int q = 0; q < NSEG; ++q)
        if (q < nseg) xp[q] = xr[64 * q];
#pragma unroll
      for (int i = 0; i < SPW; ++i) {
        if (q0 + i < nseg) {
          x[i] = xr[64 * (q0 + i)];
          gp[i] = gr[64 * (q0 + i)];
        }
      }
      const float total = nq_pair_sumsq<NSEG>(xp, nseg);
      const float inv_rms = sqrt_n / __builtin_sqrtf(total + n_eps);
      const float m = nq_pair_transform<SPW>(x, gp, inv_rms, q0, nseg, block, fwht_scale, v);
      const float am = wave_max(m);
      if (lane == 0) s_max[wave] = am;
    }
    __syncthreads();
    if (!live) return;
    float amax = s_max[8 * g];
    for (int w = 1; w < wpt; ++w) amax = fmaxf(amax, s_max[8 * g + w]);
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    uint16_t* qrow = reinterpret_cast<uint16_t*>(xq + (size_t)t * hidden) + lane;
#pragma unroll
    for (int i = 0; i < SPW; ++i)
      if (q0 + i < nseg) qrow[64 * (q0 + i)] = nq_pair_code(v[i], inv);
    if (lane == 0 && wv == 0) sa[t] = amax;
    return;
  }
  if constexpr (ONE > 0) {
    // one workgroup: every token's top-k (ONE per wave at a time) and the
    // schedule from LDS, no cross-workgroup hand-off
    route_schedule_block<NE, ONE>(logits, pes, T, E, top_k, route_idx, route_w, expert_offset,
                                  routes);
    return;
  }
  // ---- top-k + softmax merge: token 16 b' + wave
  const int t = ((int)blockIdx.x - nq_blocks) * kPrepTopkTokens + wave;
  if (t < T) {  // wave-uniform
    const float* rows[1] = {logits + (size_t)t * E};
    int e[1];
    float w[1];
    topk_tokens<NE, 1>(rows, pes, E, top_k, lane, e, w);
    if (lane < top_k) {
      route_idx[(size_t)t * top_k + lane] = e[0];
      route_w[(size_t)t * top_k + lane] = w[0];
    }
  }
  // ---- the last top-k workgroup builds the schedule.  Every wave waits
  // for its route stores to reach L2; after the barrier one thread makes
  // them visible device-wide (a device-scope fence writes the XCD's L2 back)
  // and counts the workgroup done.  The last one invalidates its caches
  // (the fence again, one thread) before any of its waves reads the routes.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    // top-k workgroups less one (from T, not gridDim: reading gridDim would
    // add the runtime's implicit arguments to the kernel's argument block)
    const unsigned last = (unsigned)((T + kPrepTopkTokens - 1) / kPrepTopkTokens) - 1u;
    s_last = atomicInc(done, last) == last;  // the last increment wraps the count to 0
    if (s_last) __threadfence();
  }
  __syncthreads();
  if (!s_last) return;
  const int slots = T * top_k, sc = min(tid, slots - 1);
  const int ex = route_idx[sc];
  const float wx = route_w[sc];
  schedule_small(tid < slots ? ex : -1, wx, top_k, E, slots, s_wc, s_cnt, expert_offset, routes);
}

template <int NE>
static void launch_rss(int T, int E, int top_k, const float* logits, const uint16_t* pes,
                       int32_t* route_idx, float* route_w, int32_t* eo, Route* routes,
                       hipStream_t st) {
  // one token per wave (T <= kRouteScheduleFusedTokens <= kSchedWavesSmall)
  hipLaunchKernelGGL((k_route_schedule_small<NE, 1>), dim3(1), dim3(kSchedSmallSlots), 0, st,
                     logits, pes, T, E, top_k, route_idx, route_w, eo, routes);
}

static int pick_port_unroll(int width, int cols) {
  if (cols % (8 * width) == 0) return 8;
  if (cols % (4 * width) == 0) return 4;
  if (cols % (2 * width) == 0) return 2;
  return 1;
}

template <int TT, int EE>
static hipError_t launch_logits_tile(const uint16_t* x, const uint16_t* proj,
                                     const uint16_t* rscale, float* logits, int T, int H, int E,
                                     float sqrt_n, float n_eps, hipStream_t st) {
  const dim3 grid((T + TT - 1) / TT, (E + 4 * EE - 1) / (4 * EE));
  const int pu_bf16 = pick_port_unroll(32, H);
  if (pick_port_unroll(16, H) == 8)
    hipLaunchKernelGGL((k_router_logits<TT, EE, 2>), grid, dim3(256), 0, st, x, proj, rscale,
                       logits, T, H, E, pu_bf16, sqrt_n, n_eps);
  else
    hipLaunchKernelGGL((k_router_logits<TT, EE, 1>), grid, dim3(256), 0, st, x, proj, rscale,
                       logits, T, H, E, pu_bf16, sqrt_n, n_eps);
  return hipGetLastError();
}

hipError_t launch_router_logits(const uint16_t* x, const uint16_t* proj, const uint16_t* rscale,
                                float* logits, int T, int H, int E, float sqrt_n, float n_eps,
                                hipStream_t st) {
  if (T >= 256) return launch_logits_tile<8, 8>(x, proj, rscale, logits, T, H, E, sqrt_n, n_eps, st);
  return launch_logits_tile<2, 4>(x, proj, rscale, logits, T, H, E, sqrt_n, n_eps, st);
}

constexpr int kRouteScheduleFusedTokens = 8;
static_assert(kRouteScheduleFusedTokens <= kSchedWavesSmall, "a wave per token");

hipError_t launch_route_schedule(const float* logits, const uint16_t* pes, int T, int E,
                                 int top_k, int32_t* route_idx, float* route_w,
                                 int32_t* expert_offset, Route* routes, hipStream_t st) {
  if (T <= 0) return hipSuccess;
  if (E > kMaxExperts) return hipErrorInvalidValue;
  // one workgroup for the whole call up to 8 tokens (one wave each: 1 token
  // 5.8 -> 5.1 us, 8 tokens 9.3 -> 8.5 us); from 12 tokens the top-k spread
  // over the chip and the schedule kernel are as fast or faster (16 tokens
  // 9.3 vs 10.0 us)
  if (T > kRouteScheduleFusedTokens || T * top_k > kSchedSmallSlots) {
    const hipError_t r = launch_route_topk(logits, pes, T, E, top_k, route_idx, route_w, st);
    if (r != hipSuccess) return r;
    return launch_build_schedule(route_idx, route_w, T, top_k, 0, E, expert_offset, routes, st);
  }
  if (E <= 64) launch_rss<1>(T, E, top_k, logits, pes, route_idx, route_w, expert_offset, routes, st);
  else if (E <= 128) launch_rss<2>(T, E, top_k, logits, pes, route_idx, route_w, expert_offset, routes, st);
  else launch_rss<4>(T, E, top_k, logits, pes, route_idx, route_w, expert_offset, routes, st);
  return hipGetLastError();
}

// The completion counter of stream `st` on the current device: slot i of
// g_prep_done, the slots handed out to streams in order of first use (the
// array's address looked up once per device).  *out is null once every slot
// of the device is taken; the caller then runs the prep as separate launches,
// which need no counter.
static hipError_t prep_counter(hipStream_t st, unsigned** out) {
  constexpr int kDevices = 64;
  static unsigned* addr[kDevices] = {};
  static std::unordered_map<hipStream_t, int> slot[kDevices];
  static std::mutex mu;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_prep_done));
    if (e != hipSuccess) return e;
    addr[dev] = static_cast<unsigned*>(p);
  }
  auto it = slot[dev].find(st);
  if (it == slot[dev].end()) {
    if ((int)slot[dev].size() >= kPrepCounters) {
      *out = nullptr;
      return hipSuccess;
    }
    it = slot[dev].emplace(st, (int)slot[dev].size()).first;
  }
  *out = addr[dev] + it->second;
  return hipSuccess;
}

// The prep's route top-k and norm-quant for larger batches in one launch
// (the schedule follows as its own launch): workgroups [0, tk_blocks) take
// four tokens' top-k + softmax merge (one wave per token, as k_route_topk),
// the others four tokens' norm-quant with FWHT block 128 (one wave per token,
// nq_v8_token, as k_norm_quant_v8).  The two are independent, so the
// norm-quant's waves fill the issue slots the top-k's leave.
template <int NE, int NSEG>
__global__ __launch_bounds__(256) void k_topk_norm_quant(
    const float* __restrict__ logits, const uint16_t* __restrict__ pes,
    const uint16_t* __restrict__ src, const uint16_t* __restrict__ gamma,
    int8_t* __restrict__ xq, float* __restrict__ sa, int32_t* __restrict__ route_idx,
    float* __restrict__ route_w, int T, int E, int top_k, int hidden, float sqrt_n, float n_eps,
    float fwht_scale, int tk_blocks) {
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const bool tk = (int)blockIdx.x < tk_blocks;
  const int t = ((int)blockIdx.x - (tk ? 0 : tk_blocks)) * 4 + wave;
  if (t >= T) return;  // whole waves; no block synchronization below
  if (!tk) {
    nq_v8_token<NSEG>(src, gamma, xq, sa, t, hidden, sqrt_n, n_eps, fwht_scale);
    return;
  }
  const float* rows[1] = {logits + (size_t)t * E};
  int e[1];
  float w[1];
  topk_tokens<NE, 1>(rows, pes, E, top_k, lane, e, w);
  if (lane < top_k) {
    route_idx[(size_t)t * top_k + lane] = e[0];
    route_w[(size_t)t * top_k + lane] = w[0];
  }
}

// The prep in one launch (k_moe_prep) for T * top_k <= 1024 slots, E <= 256
// and the pair-layout norm-quant's shapes (hidden % 256 == 0, <= 4096, FWHT
// block <= 512, 2-byte aligned codes); above 1024 slots with FWHT block 128,
// the top-k and the norm-quant in one launch (k_topk_norm_quant) and the
// schedule in a second; otherwise the route top-k + schedule and the
// norm-quant as separate launches.  Same results either way.
hipError_t launch_moe_prep(const float* logits, const uint16_t* pes, const uint16_t* src,
                           const uint16_t* gamma, int T, int E, int top_k, int hidden, int block,
                           float sqrt_n, float n_eps, int32_t* route_idx, float* route_w,
                           int32_t* expert_offset, Route* routes, int8_t* xq, float* sa,
                           hipStream_t st, const uint16_t* gamma2, int8_t* xq2, float* sa2) {
  if (T <= 0) return hipSuccess;
  if (E > kMaxExperts) return hipErrorInvalidValue;
  const int ns = hidden >> 7;
  const int unit = block > 128 ? block / 128 : 1;
  int spw = (ns + 7) / 8;
  spw = (spw + unit - 1) / unit * unit;
  const bool one = tune().prep_one && T <= kPrepTopkTokens;
  unsigned* done = nullptr;
  bool fused = T * top_k <= kSchedSmallSlots && hidden % 256 == 0 && hidden <= 4096 &&
               tune().nq_pair && tune().moe_prep && !(reinterpret_cast<uintptr_t>(xq) & 1u) &&
               !(reinterpret_cast<uintptr_t>(xq2) & 1u) && (ns + spw - 1) / spw <= 8;
  if (fused && !one) {  // the spread form's hand-off needs the stream's counter
    const hipError_t ra = prep_counter(st, &done);
    if (ra != hipSuccess) return ra;
    fused = done != nullptr;
  }
  // larger batches with FWHT block 128: top-k and norm-quant in one launch,
  // then the schedule (the conditions of launch_norm_quant's v8 path)
  const bool wide = !fused && T * top_k > kSchedSmallSlots && block == 128 && hidden % 256 == 0 &&
                    hidden <= 4096 && tune().nq_pair && tune().nq_v8 && tune().moe_prep &&
                    !(reinterpret_cast<uintptr_t>(gamma) & 15u) &&
                    !(reinterpret_cast<uintptr_t>(xq) & 7u);
  // the second norm-quant (gamma2) runs in the k_moe_prep launch; on the
  // other paths it is a launch of its own, first
  if (gamma2 && !fused) {
    const hipError_t r2 = launch_norm_quant(src, gamma2, xq2, sa2, T, hidden, block, sqrt_n, n_eps, st);
    if (r2 != hipSuccess) return r2;
  }
  if (wide) {
    const int tk_blocks = (T + 3) / 4;
    const dim3 g(2 * tk_blocks), b(256);
    const float sc = fwht_scale_host(block);
    const int ne = (E + 63) / 64;
    bool launched = false;
#define BQ_TNQ(NEV, N)                                                                           \
  if (!launched && ne <= NEV && ns <= N) {                                                       \
    hipLaunchKernelGGL((k_topk_norm_quant<NEV, N>), g, b, 0, st, logits, pes, src, gamma, xq, sa, \
                       route_idx, route_w, T, E, top_k, hidden, sqrt_n, n_eps, sc, tk_blocks);   \
    launched = true;                                                                             \
  }
#define BQ_TNQ_NS(NEV) BQ_TNQ(NEV, 8) BQ_TNQ(NEV, 16) BQ_TNQ(NEV, 22) BQ_TNQ(NEV, 24) BQ_TNQ(NEV, 32)
    BQ_TNQ_NS(1) BQ_TNQ_NS(2) BQ_TNQ_NS(4)
#undef BQ_TNQ_NS
#undef BQ_TNQ
    if (!launched) return hipErrorInvalidValue;
    const hipError_t r = hipGetLastError();
    if (r != hipSuccess) return r;
    return launch_build_schedule(route_idx, route_w, T, top_k, 0, E, expert_offset, routes, st);
  }
  if (!fused) {
    const hipError_t r = launch_route_schedule(logits, pes, T, E, top_k, route_idx, route_w,
                                               expert_offset, routes, st);
    if (r != hipSuccess) return r;
    return launch_norm_quant(src, gamma, xq, sa, T, hidden, block, sqrt_n, n_eps, st);
  }
  const int nq_per = (T + 1) / 2, nq_blocks = gamma2 ? 2 * nq_per : nq_per;
  // up to 16 tokens one workgroup takes every top-k (one token per wave) and
  // builds the schedule from LDS, with no cross-workgroup hand-off: the
  // batch-16 decoder layer's MoE 106.6 -> 105.1 us.  At 32 tokens (two per
  // wave) the spread top-k with the last-workgroup schedule is faster (the
  // prep alone 9.2 vs 13.2 us, the layer 125.4 vs 129.3 us).  BQ_PREP_ONE=0
  // keeps the spread form.
  const dim3 g(nq_blocks + (one ? 1 : (T + kPrepTopkTokens - 1) / kPrepTopkTokens)), b(kPrepThreads);
  const float sc = fwht_scale_host(block);
  const int ne = (E + 63) / 64;
#define BQ_PREP(NEV, N, S)                                                                        \
  if (ne <= NEV && ns <= N && spw == S) {                                                        \
    if (one)                                                                                      \
      hipLaunchKernelGGL((k_moe_prep<NEV, N, S, 1>), g, b, 0, st, logits, pes, src, gamma, xq, sa, \
                         route_idx, route_w, expert_offset, routes, T, E, top_k, hidden, block,  \
                         sqrt_n, n_eps, sc, nq_blocks, done, nq_per, gamma2, xq2, sa2);           \
    else                                                                                          \
      hipLaunchKernelGGL((k_moe_prep<NEV, N, S>), g, b, 0, st, logits, pes, src, gamma, xq, sa,   \
                         route_idx, route_w, expert_offset, routes, T, E, top_k, hidden, block,  \
                         sqrt_n, n_eps, sc, nq_blocks, done, nq_per, gamma2, xq2, sa2);           \
    return hipGetLastError();                                                                     \
  }
#define BQ_PREP_NQ(NEV) \
  BQ_PREP(NEV, 8, 1) BQ_PREP(NEV, 8, 2) BQ_PREP(NEV, 8, 4) BQ_PREP(NEV, 16, 2) BQ_PREP(NEV, 16, 4) \
  BQ_PREP(NEV, 24, 3) BQ_PREP(NEV, 24, 4) BQ_PREP(NEV, 32, 4)
  BQ_PREP_NQ(1) BQ_PREP_NQ(2) BQ_PREP_NQ(4)
#undef BQ_PREP_NQ
#undef BQ_PREP
  return hipErrorInvalidValue;
}

hipError_t launch_route_topk(const float* logits, const uint16_t* pes, int T, int E, int top_k,
                             int32_t* route_idx, float* route_w, hipStream_t st) {
  const dim3 grid((T + 3) / 4), block(256);
  const int ne = (E + 63) / 64;
  if (ne <= 1)
    hipLaunchKernelGGL(k_route_topk<1>, grid, block, 0, st, logits, pes, T, E, top_k, route_idx, route_w);
  else if (ne <= 2)
    hipLaunchKernelGGL(k_route_topk<2>, grid, block, 0, st, logits, pes, T, E, top_k, route_idx, route_w);
  else if (ne <= 4)
    hipLaunchKernelGGL(k_route_topk<4>, grid, block, 0, st, logits, pes, T, E, top_k, route_idx, route_w);
  else if (ne <= 8)
    hipLaunchKernelGGL(k_route_topk<8>, grid, block, 0, st, logits, pes, T, E, top_k, route_idx, route_w);
  else
    hipLaunchKernelGGL(k_route_topk<16>, grid, block, 0, st, logits, pes, T, E, top_k, route_idx, route_w);
  return hipGetLastError();
}

}  // namespace bq
