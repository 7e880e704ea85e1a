// bq_sched.hpp -- the one-workgroup CSR expert schedule of up to
// kSchedSmallSlots route slots (kernels/moe_router.mojo:60-106), shared by
// bq_moe_build_schedule's decode-sized kernel and the fused route + schedule
// kernel.
#pragma once
#include "bq_device.hpp"
#include "bq_kernels.hpp"

namespace bq {

constexpr int kMaxExperts = 256;
constexpr int kSchedSmallSlots = 1024;

// Called by all kSchedSmallSlots threads of the workgroup; thread tid owns
// route slot tid = token * top_k + k, with e its expert (0..E-1, or -1 for
// no slot) and w its weight; threads tid >= slots hold no slot, so only the
// first ceil(slots / 64) waves take part in the counts.  A slot's record is
// its expert's offset plus the number of earlier slots routed to the same
// expert -- the (expert, token, k) order.  Earlier slots of the same wave
// are counted from the wave's experts staged in LDS (each lane compares the
// lanes below it: no serial pass per distinct expert); earlier waves' slots
// through an exclusive prefix over the waves' per-expert counts (s_wc, LDS
// atomics), and the experts' offsets through a scan of their totals
// (s_cnt).
constexpr int kSchedWavesSmall = kSchedSmallSlots / 64;

__device__ inline void schedule_small(int e, float w, int top_k, int E, int slots,
                                      int (*s_wc)[kMaxExperts], int* s_cnt,
                                      int32_t* __restrict__ expert_offset,
                                      Route* __restrict__ routes) {
  __shared__ __attribute__((aligned(16))) int s_key[kSchedSmallSlots];
  const int tid = threadIdx.x, lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = min(max((slots + 63) >> 6, 1), kSchedWavesSmall);  // waves holding slots
  for (int i = tid; i < nw * kMaxExperts; i += kSchedSmallSlots)
    s_wc[i / kMaxExperts][i % kMaxExperts] = 0;
  s_key[tid] = e;
  __syncthreads();
  // rank among the wave's earlier lanes with the same expert; four keys per
  // 16-byte LDS read (every lane reads the same address: a broadcast)
  int rank = 0;
  if (wave < nw) {  // wave-uniform: the other waves hold no slot
    const int* wk = &s_key[wave * 64];
#pragma unroll
    for (int j0 = 0; j0 < 64; j0 += 4) {
      const int4 k4 = *reinterpret_cast<const int4*>(wk + j0);
      rank += (j0 + 0 < lane && k4.x == e) ? 1 : 0;
      rank += (j0 + 1 < lane && k4.y == e) ? 1 : 0;
      rank += (j0 + 2 < lane && k4.z == e) ? 1 : 0;
      rank += (j0 + 3 < lane && k4.w == e) ? 1 : 0;
    }
    if (e >= 0) atomicAdd(&s_wc[wave][e], 1);
  }
  __syncthreads();
  for (int x = tid; x < E; x += kSchedSmallSlots) {  // prefix over the waves, per expert
    int run = 0;
    for (int q = 0; q < nw; ++q) {
      const int v = s_wc[q][x];
      s_wc[q][x] = run;
      run += v;
    }
    s_cnt[x] = run;
  }
  __syncthreads();
  if (wave == 0) {  // exclusive scan of the E <= 256 totals, 4 per lane
    int v[4], sum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ex = lane * 4 + j;
      v[j] = ex < E ? s_cnt[ex] : 0;
      sum += v[j];
    }
    int inc = wave_incl_scan(sum);
    int off = inc - sum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ex = lane * 4 + j;
      if (ex < E) {
        s_cnt[ex] = off;
        expert_offset[ex] = off;
      }
      off += v[j];
    }
    if (lane == 63) expert_offset[E] = inc;
  }
  __syncthreads();
  if (e >= 0) {
    const int pos = s_cnt[e] + s_wc[wave][e] + rank;
    routes[pos].token = tid / top_k;
    routes[pos].weight = w;
  }
}

}  // namespace bq
