// bq_moe.hip -- the quantized MoE expert layer (butterquant_kernels/moe.mojo)
// and its CSR schedule (kernels/moe_router.mojo:60-106).
//
// Schedule: expert_offset[E+1] (exclusive prefix of per-expert route counts)
//   and routes[] sorted by (expert, token, k) -- the reference's order -- one
//   workgroup per expert, ranks from a block scan over route slots.
// Phase 1 (moe.mojo:25-164): grouped GEMM over (expert m-tile, intermediate
//   tile); each wave accumulates the gate and up 16x16 tiles of the same
//   intermediate columns, so the epilogue bucket = bf16(gelu(g)*u) is
//   element-wise in registers.  A rows are gathered by route token.
// Phase 2 (moe.mojo:167-335): grouped per-block GEMM (B = 64) producing the
//   per-route f32 results y = (facc*ws)*route_w, then a combine that adds each
//   token's routes in ascending expert order -- the reference's accumulation
//   order (experts ascending, moe.mojo:259-282) -- so accum is bit-identical.
//   The combine relies on each expert's records being in ascending token
//   order, as the schedule (and the reference's) produces them.
#include "bq_device.hpp"
#include "bq_kernels.hpp"
#include "bq_sched.hpp"

namespace bq {

// One workgroup per expert e.  The (expert, token, k) order puts route slot
// s = t*top_k + kk of expert e at expert_offset[e] + (number of earlier slots
// routed to e) -- slot order is (token, k) order, also for a token that lists
// an expert twice -- and
// expert_offset[e] = number of slots routed to experts below e.  Both counts
// come from scanning route_idx: a chunk of kRows x 1024 slots is read
// coalesced (thread tid takes slots j*1024 + tid, row j = 0..kRows-1), so
// slot order is (row, wave, lane): per-row wave ballots plus one exclusive
// scan over the kRows x 16 (row, wave) counts give every hit its rank.
constexpr int kSchedThreads = 1024, kSchedWaves = kSchedThreads / 64, kRows = 16;

__global__ __launch_bounds__(kSchedThreads) void k_build_schedule(
    const int32_t* __restrict__ route_idx, const float* __restrict__ route_w, int slots,
    int top_k, int ebase, int E, int32_t* __restrict__ expert_offset, Route* __restrict__ routes) {
  __shared__ int cnt[kRows * kSchedWaves];  // per (row, wave) counts, then their exclusive prefix
  __shared__ int red[2 * kSchedWaves];
  __shared__ int chunk_total;
  const int e = blockIdx.x, target = ebase + e, tid = threadIdx.x;
  const int lane = lane_id(), wave = tid >> 6;
  constexpr int kChunk = kRows * kSchedThreads;
  // pass 1: slots routed to experts below e, and to e.  The first chunk's
  // experts and weights stay in registers for pass 2 (with up to kChunk
  // slots -- 2048 tokens x top-8 -- pass 2 then loads nothing).
  int below = 0, mine = 0;
  int x0[kRows];
  float w0[kRows];
  for (int c0 = 0; c0 < slots; c0 += kChunk) {
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
      const int s = c0 + j * kSchedThreads + tid;
      const int x = route_idx[min(s, slots - 1)];  // unmasked: loads stay batched
      if (c0 == 0) {
        x0[j] = x;
        w0[j] = route_w[min(s, slots - 1)];
      }
      below += (s < slots && x >= ebase && x < target) ? 1 : 0;
      mine += (s < slots && x == target) ? 1 : 0;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    below += __shfl_xor(below, o, kWave);
    mine += __shfl_xor(mine, o, kWave);
  }
  if (lane == 0) { red[wave] = below; red[kSchedWaves + wave] = mine; }
  __syncthreads();
  int offset = 0, count = 0;
#pragma unroll
  for (int w = 0; w < kSchedWaves; ++w) { offset += red[w]; count += red[kSchedWaves + w]; }
  if (tid == 0) {
    expert_offset[e] = offset;
    if (e == E - 1) expert_offset[E] = offset + count;
  }
  // pass 2: ranks in slot order
  int run = offset;
  for (int c0 = 0; c0 < slots; c0 += kChunk) {
    unsigned long long m[kRows];
    float wts[kRows];
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
      const int s = c0 + j * kSchedThreads + tid;
      const int sc = min(s, slots - 1);
      const int x = c0 == 0 ? x0[j] : route_idx[sc];
      wts[j] = c0 == 0 ? w0[j] : route_w[sc];
      m[j] = __ballot(s < slots && x == target);
      if (lane == 0) cnt[j * kSchedWaves + wave] = __popcll(m[j]);
    }
    __syncthreads();
    if (wave == 0) {  // exclusive scan of the kRows*16 (row, wave) counts, 4 per lane
      int v[4], sum = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) { v[i] = cnt[lane * 4 + i]; sum += v[i]; }
      int inc = wave_incl_scan(sum);
      int ex = inc - sum;
#pragma unroll
      for (int i = 0; i < 4; ++i) { cnt[lane * 4 + i] = ex; ex += v[i]; }
      if (lane == 63) chunk_total = inc;
    }
    __syncthreads();
    const unsigned long long below_lane = (1ull << lane) - 1ull;
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
      if ((m[j] >> lane) & 1ull) {
        const int pos = run + cnt[j * kSchedWaves + wave] + __popcll(m[j] & below_lane);
        const int s = c0 + j * kSchedThreads + tid;
        routes[pos].token = s / top_k;
        routes[pos].weight = wts[j];
      }
    }
    run += chunk_total;
    __syncthreads();  // cnt / chunk_total are rewritten by the next chunk
  }
}

// Decode-sized schedules (at most 1024 slots): one workgroup, one thread per
// slot (schedule_small) -- one load, per-wave matching, two scans and one
// scatter replace the per-expert passes over every slot.
__global__ __launch_bounds__(kSchedSmallSlots) void k_build_schedule_small(
    const int32_t* __restrict__ route_idx, const float* __restrict__ route_w, int slots,
    int top_k, int ebase, int E, int32_t* __restrict__ expert_offset, Route* __restrict__ routes) {
  __shared__ int s_wc[kSchedWavesSmall][kMaxExperts];
  __shared__ int s_cnt[kMaxExperts];
  const int tid = threadIdx.x;
  const int sc = min(tid, slots - 1);  // unmasked loads (slots >= 1)
  const int x = route_idx[sc];
  const float w = route_w[sc];
  const int e = (tid < slots && x >= ebase && x < ebase + E) ? x - ebase : -1;
  schedule_small(e, w, top_k, E, slots, s_wc, s_cnt, expert_offset, routes);
}

// Skinny (16-record m-tile) kernels for decode-sized batches.  Each wave owns
// one 16-column output subtile and streams its weight rows in chunks of U
// k-steps through two register slots: chunk c+1's loads are in flight while
// chunk c is multiplied.  Loads are never masked (indices are clamped, work
// past K is skipped by a uniform test), and every epilogue operand is loaded
// at kernel start.

// Phase 1: blockIdx.y = m-tile, blockIdx.x = group of 4 intermediate subtiles
// (64 columns).  With bi8 the workgroup's 16 x 64 bf16 bucket block goes
// through LDS to the fused FWHT64 block-quant (inter % 64 == 0: no wave of
// the group is idle).  The first dn.ytiles rows of the grid are the dense
// MLP's (16 tokens x 64 columns of its gate and up each): the same products,
// with the dense linears' bf16 rounding of gate and up before the GELU
// (gemma_4_moe_bq.mojo:755-769: two dispatch_bq_linear, dispatch_gelu_gate_up,
// dispatch_bq_block_quant[64, True]).
template <int U>
// (the scalars the m-tile lookup and the first addresses need come first:
// the dispatch preloads the first 14 argument dwords into SGPRs)
__global__ __launch_bounds__(256) void k_moe_gate_up_skinny(
    int E, int hidden, int inter, int max_routes, const int32_t* __restrict__ eo,
    const Route* __restrict__ routes, const int8_t* __restrict__ w_gu,
    const int8_t* __restrict__ x_i8, const float* __restrict__ gu_scale,
    const float* __restrict__ x_sa, uint16_t* __restrict__ bucket, int8_t* __restrict__ bi8,
    float* __restrict__ bsa, float fwht64, DenseGateUp dn) {
  __shared__ __attribute__((aligned(16))) uint16_t qtile[16 * 64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = lane_id();
  const int K = hidden, K64 = K >> 6;
  const bool dense = (int)blockIdx.y < dn.ytiles;  // uniform
  int r0, r1, grp = blockIdx.x, n_inter = inter;
  const int8_t *wg, *wu, *xa;
  const float *sg, *su, *xs;
  int8_t* oq;
  float* os;
  if (dense) {
    const int ty = blockIdx.y / dn.cpg;
    grp = ((int)blockIdx.y - ty * dn.cpg) * dn.gx + blockIdx.x;
    if (grp * 64 >= dn.inter) return;  // whole workgroup
    r0 = ty * 16;
    r1 = min(dn.T, r0 + 16);
    n_inter = dn.inter;
    wg = dn.wg; wu = dn.wu; sg = dn.sg; su = dn.su;
    xa = dn.x_i8; xs = dn.x_sa; oq = dn.out_i8; os = dn.out_sa;
  } else {
    int e;
    if (!find_mtile(eo, E, 16, blockIdx.y - dn.ytiles, max_routes, e, r0, r1)) return;
    const size_t gate_up = (size_t)2 * inter;
    wg = w_gu + (size_t)e * gate_up * K;
    wu = wg + (size_t)inter * K;  // the up rows follow the expert's inter gate rows
    sg = gu_scale + (size_t)e * gate_up;
    su = sg + inter;
    xa = x_i8; xs = x_sa; oq = bi8; os = bsa;
  }
  const int isub = grp * 4 + wave;
  if (isub * 16 >= n_inter) return;  // never with bi8 (inter % 64 == 0)
  const int8_t* wgp = wg + (size_t)isub * K64 * 1024 + lane * 16;
  const int8_t* wup = wu + (size_t)isub * K64 * 1024 + lane * 16;
  v4i bg[2][U], bu[2][U], af[2][U];
  auto load_w = [&](int s, int c) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kt = min(c * U + u, K64 - 1);
      bg[s][u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wgp + (size_t)kt * 1024));
      bu[s][u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wup + (size_t)kt * 1024));
    }
  };
  // this lane's activation row and its four epilogue rows: the records'
  // tokens (their routes' for the experts, the records themselves for the
  // dense MLP), requested together; then the weight stream, which depends
  // only on the expert, goes out while they are in flight (loads return in
  // issue order, so the activation loads wait for the tokens alone).  Rows
  // past the tile's last record read that record: accumulator row i depends
  // only on A row i, and those rows are never stored.
  int tk[5];
  tk[0] = min(r0 + (lane & 15), r1 - 1);
#pragma unroll
  for (int v = 0; v < 4; ++v) tk[1 + v] = min(r0 + 4 * (lane >> 4) + v, r1 - 1);
  if (!dense) {
#pragma unroll
    for (int i = 0; i < 5; ++i) tk[i] = routes[tk[i]].token;
  }
  asm volatile("" ::: "memory");  // keep the three groups of loads in this order
  load_w(0, 0);
  asm volatile("" ::: "memory");
  const int8_t* ab = xa + (size_t)tk[0] * K + (lane >> 4) * 16;
  auto load_a = [&](int s, int c) {
#pragma unroll
    for (int u = 0; u < U; ++u) af[s][u] = ld16(ab + min(c * U + u, K64 - 1) * 64);
  };
  auto load = [&](int s, int c) {
    load_w(s, c);
    load_a(s, c);
  };
  load_a(0, 0);
  // epilogue operands
  const int col = isub * 16 + (lane & 15);
  const float wsg = sg[col], wsu = su[col];
  float ad[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) ad[v] = xs[tk[1 + v]] * kInv127;
  const v4i zero = {0, 0, 0, 0};
  v4i cg = zero, cu = zero;
  auto mul = [&](int s, int c) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (c * U + u < K64) {
        cg = mfma16x16x64(af[s][u], bg[s][u], cg);
        cu = mfma16x16x64(af[s][u], bu[s][u], cu);
      }
  };
  const int nch = (K64 + U - 1) / U;
  for (int c = 0; c < nch; c += 2) {  // (chunk 0 is in flight)
    if (c + 1 < nch) load(1, c + 1);
    mul(0, c);
    if (c + 1 >= nch) break;
    if (c + 2 < nch) load(0, c + 2);
    mul(1, c + 1);
  }
  const int g4[4] = {cg.x, cg.y, cg.z, cg.w};
  const int u4[4] = {cu.x, cu.y, cu.z, cu.w};
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int rec = r0 + 4 * (lane >> 4) + v;
    if (rec >= r1) continue;
    float gv = (float)g4[v] * ad[v] * wsg;
    float uv = (float)u4[v] * ad[v] * wsu;
    if (dense) {  // the dense linears write bf16 gate and up
      gv = bf16_to_f32(f32_to_bf16(gv));
      uv = bf16_to_f32(f32_to_bf16(uv));
    }
    const uint16_t hb = f32_to_bf16(gelu_tanh_f32(gv) * uv);
    if (oq) qtile[(rec - r0) * 64 + wave * 16 + (lane & 15)] = hb;
    else bucket[(size_t)rec * inter + col] = hb;
  }
  if (!oq) return;  // uniform
  __syncthreads();
  // 16 records x one 64-column block: 8 lanes per record (waves 0 and 1)
  if (wave >= 2) return;
  const int r = wave * 8 + (lane >> 3), i = lane & 7;
  const v4i raw = *reinterpret_cast<const v4i*>(&qtile[r * 64 + i * 8]);
  float v[8];
  bf16x8_to_f32(raw, v);
  uint32_t w[2];
  const float m = block_quant_lanes<8>(v, true, fwht64, w);
  if (r0 + r < r1) {
    const size_t rec = (size_t)(r0 + r), c0 = (size_t)grp * 64 + i * 8;
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u2*>(oq + rec * n_inter + c0) = u2{w[0], w[1]};
    if (i == 0) os[rec * (n_inter / 64) + grp] = m;
    if (bucket && !dense) *reinterpret_cast<v4i*>(bucket + rec * inter + c0) = raw;
  }
}

// The dense MLP's gate/up alone at many tokens (the experts on the tiled
// kernels): as the dense rows of k_moe_gate_up_skinny, but a workgroup takes
// RT 16-token tiles of its 64-column group, so every weight fragment feeds
// RT tiles' products (the 16-token form re-reads the dense weights once per
// 16 tokens).  Each tile's epilogue is the skinny kernel's: the linears'
// bf16 gate and up, GELU-tanh(gate) * up, FWHT64 block-quant through LDS.
template <int RT, int U>  // U: k-steps per register slot
__global__ __launch_bounds__(256) void k_dense_gate_up(int hidden, float fwht64, DenseGateUp dn) {
  __shared__ __attribute__((aligned(16))) uint16_t qtile[16 * 64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = lane_id();
  const int K = hidden, K64 = K >> 6;
  const int grp = blockIdx.x, t0 = blockIdx.y * 16 * RT;  // grid x = inter / 64
  const int isub = grp * 4 + wave;
  const int8_t* wgp = dn.wg + (size_t)isub * K64 * 1024 + lane * 16;
  const int8_t* wup = dn.wu + (size_t)isub * K64 * 1024 + lane * 16;
  v4i bg[2][U], bu[2][U], af[2][U][RT];
  const int8_t* ab[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r)  // rows past the batch read its last row, never stored
    ab[r] = dn.x_i8 + (size_t)min(t0 + 16 * r + (lane & 15), dn.T - 1) * K + (lane >> 4) * 16;
  auto load = [&](int s, int c) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kt = min(c * U + u, K64 - 1);
      bg[s][u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wgp + (size_t)kt * 1024));
      bu[s][u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wup + (size_t)kt * 1024));
#pragma unroll
      for (int r = 0; r < RT; ++r) af[s][u][r] = ld16(ab[r] + kt * 64);
    }
  };
  load(0, 0);
  const int col = isub * 16 + (lane & 15);
  const float wsg = dn.sg[col], wsu = dn.su[col];
  const v4i zero = {0, 0, 0, 0};
  v4i cg[RT], cu[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) cg[r] = cu[r] = zero;
  auto mul = [&](int s, int c) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (c * U + u < K64) {
#pragma unroll
        for (int r = 0; r < RT; ++r) {
          cg[r] = mfma16x16x64(af[s][u][r], bg[s][u], cg[r]);
          cu[r] = mfma16x16x64(af[s][u][r], bu[s][u], cu[r]);
        }
      }
  };
  const int nch = (K64 + U - 1) / U;
  for (int c = 0; c < nch; c += 2) {  // (chunk 0 is in flight)
    if (c + 1 < nch) load(1, c + 1);
    mul(0, c);
    if (c + 1 >= nch) break;
    if (c + 2 < nch) load(0, c + 2);
    mul(1, c + 1);
  }
  typedef uint32_t u2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int r0 = t0 + 16 * r;
    if (r0 >= dn.T) break;  // workgroup-uniform
    const int r1 = min(dn.T, r0 + 16);
    const int g4[4] = {cg[r].x, cg[r].y, cg[r].z, cg[r].w};
    const int u4[4] = {cu[r].x, cu[r].y, cu[r].z, cu[r].w};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int rec = r0 + 4 * (lane >> 4) + v;
      if (rec >= r1) continue;
      const float ad = dn.x_sa[rec] * kInv127;
      const float gv = bf16_to_f32(f32_to_bf16((float)g4[v] * ad * wsg));  // the linears' bf16
      const float uv = bf16_to_f32(f32_to_bf16((float)u4[v] * ad * wsu));
      qtile[(rec - r0) * 64 + wave * 16 + (lane & 15)] = f32_to_bf16(gelu_tanh_f32(gv) * uv);
    }
    __syncthreads();
    if (wave < 2) {  // 16 records x one 64-column block: 8 lanes per record
      const int rr = wave * 8 + (lane >> 3), i = lane & 7;
      const v4i raw = *reinterpret_cast<const v4i*>(&qtile[rr * 64 + i * 8]);
      float vv[8];
      bf16x8_to_f32(raw, vv);
      uint32_t w[2];
      const float m = block_quant_lanes<8>(vv, true, fwht64, w);
      if (r0 + rr < r1) {
        const size_t rec = (size_t)(r0 + rr), c0 = (size_t)grp * 64 + i * 8;
        *reinterpret_cast<u2*>(dn.out_i8 + rec * dn.inter + c0) = u2{w[0], w[1]};
        if (i == 0) dn.out_sa[rec * (dn.inter / 64) + grp] = m;
      }
    }
    __syncthreads();  // qtile is refilled by the next tile
  }
}

// Phase 2 GEMM: y[rec, n] = (facc * ws[n]) * route_w[rec] with facc the fma
// chain over K blocks (moe.mojo:198-223).  The m-tile's per-block activation
// scales (16 records x K/block <= 64) are staged in LDS up front.  A wave
// owns NS 16-row strips of the output: the records' activation fragments
// are loaded once per k-step for all of them, and NS weight fragments per
// k-step are in flight.  The product is taken transposed, D = W x A^T (the
// weight strip as the MFMA's A operand, the 16 records as its B): lane L
// holds columns 4 (L/16) .. +3 of a strip for record L % 16, so a drain
// reads one activation scale per lane and a record's four y values are one
// 16-byte store; the integer dot of each (record, column) is the same.
// With up to two weight fragments per k-step slot the kernel fits 64
// registers, eight waves per SIMD (waves_per_eu(8)), so a 16-token batch's
// 86 experts x 22 workgroups fit in one round on 256 CUs; the default, three
// k-steps x two strips, has more weight bytes in flight per wave instead,
// which measured faster once the dense rows (K = 2112) joined the launch.
// The first dn.ytiles rows of the grid are the
// dense MLP's down projection (16 tokens each, K = dn.inter): the same fma
// chain over blocks, out = bf16(facc * ws) with no route weight
// (dispatch_bq_block_linear, gemma_4_moe_bq.mojo:774-778).
template <int U, int NS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(U * NS <= 2 ? 8 : 1)))
void k_moe_down_skinny(
    int E, int hidden, int inter, int block, int max_routes, const int32_t* __restrict__ eo,
    const Route* __restrict__ routes, const float* __restrict__ b_sa,
    const int8_t* __restrict__ w_d, const int8_t* __restrict__ b_i8,
    const float* __restrict__ d_scale, float* __restrict__ y, DenseDown dn) {
  __shared__ float s_sa[16 * 64];
  const bool dense = (int)blockIdx.y < dn.ytiles;  // uniform
  int r0, r1, K;
  const int8_t *wbase, *xa;
  const float *dsc, *xsa;
  if (dense) {
    r0 = blockIdx.y * 16;
    r1 = min(dn.T, r0 + 16);
    K = dn.inter;
    wbase = dn.w; dsc = dn.ws; xa = dn.x_i8; xsa = dn.x_sa;
  } else {
    int e;
    if (!find_mtile(eo, E, 16, blockIdx.y - dn.ytiles, max_routes, e, r0, r1)) return;  // whole workgroup
    K = inter;
    wbase = w_d + (size_t)e * hidden * K;
    dsc = d_scale + (size_t)e * hidden;
    xa = b_i8; xsa = b_sa;
  }
  const int K64 = K >> 6, fpb = block >> 6, nb = K / block;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = lane_id();
  const int nsub0 = (blockIdx.x * 4 + wave) * NS;
  const int nstrips = hidden / 16;
  const bool active = nsub0 < nstrips;  // wave-uniform; idle waves still meet the barrier
  const int8_t* wb[NS];
  float wsc[NS][4];
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int ns = min(nsub0 + j, nstrips - 1);  // a strip past the end is never stored
    wb[j] = wbase + (size_t)ns * K64 * 1024 + lane * 16;
#pragma unroll
    for (int v = 0; v < 4; ++v) wsc[j][v] = dsc[ns * 16 + 4 * (lane >> 4) + v];
  }
  // this lane's record: its activation fragment row and its result row
  const int arow = r0 + (lane & 15);
  const int8_t* ab = xa + (size_t)(arow < r1 ? arow : r0) * K + (lane >> 4) * 16;
  const float rw = dense ? 1.0f : routes[arow < r1 ? arow : r0].weight;
  const v4i zero = {0, 0, 0, 0};
  float facc[NS][4];
  v4i c[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    c[j] = zero;
#pragma unroll
    for (int v = 0; v < 4; ++v) facc[j][v] = 0.0f;
  }
  v4i bf[2][NS][U], af[2][U];
  auto load = [&](int s, int ch) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kt = min(ch * U + u, K64 - 1);
#pragma unroll
      for (int j = 0; j < NS; ++j)
        bf[s][j][u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wb[j] + (size_t)kt * 1024));
      af[s][u] = ld16(ab + kt * 64);
    }
  };
  auto mul = [&](int s, int ch) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kt = ch * U + u;
      if (kt < K64) {
#pragma unroll
        for (int j = 0; j < NS; ++j) c[j] = mfma16x16x64(bf[s][j][u], af[s][u], c[j]);
        if (((kt + 1) & (fpb - 1)) == 0) {
          const int b = kt / fpb;
          const float sc = s_sa[(lane & 15) * nb + b];
#pragma unroll
          for (int j = 0; j < NS; ++j) {
            const int cc[4] = {c[j].x, c[j].y, c[j].z, c[j].w};
#pragma unroll
            for (int v = 0; v < 4; ++v) facc[j][v] = fmaf((float)cc[v], sc, facc[j][v]);
            c[j] = zero;
          }
        }
      }
    }
  };
  const int nch = (K64 + U - 1) / U;
  // the first weight and activation fragments go out before the block
  // scales are staged: the staging's loads and barrier overlap them
  if (active) load(0, 0);
  for (int i = threadIdx.x; i < 16 * nb; i += 256) {  // 256-thread blocks
    const int row = r0 + i / nb;
    s_sa[i] = xsa[(size_t)(row < r1 ? row : r0) * nb + i % nb] * kInv127;
  }
  __syncthreads();
  if (!active) return;
  for (int ch = 0; ch < nch; ch += 2) {
    if (ch + 1 < nch) load(1, ch + 1);
    mul(0, ch);
    if (ch + 1 >= nch) break;
    if (ch + 2 < nch) load(0, ch + 2);
    mul(1, ch + 1);
  }
  if (arow >= r1) return;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    if (nsub0 + j >= nstrips) continue;
    const int col = (nsub0 + j) * 16 + 4 * (lane >> 4);
    if (dense) {
      typedef uint32_t u2 __attribute__((ext_vector_type(2)));
      const uint32_t lo = (uint32_t)f32_to_bf16(facc[j][0] * wsc[j][0]) |
                          ((uint32_t)f32_to_bf16(facc[j][1] * wsc[j][1]) << 16);
      const uint32_t hi = (uint32_t)f32_to_bf16(facc[j][2] * wsc[j][2]) |
                          ((uint32_t)f32_to_bf16(facc[j][3] * wsc[j][3]) << 16);
      *reinterpret_cast<u2*>(dn.out + (size_t)arow * hidden + col) = u2{lo, hi};
    } else {
      *reinterpret_cast<float4*>(&y[(size_t)arow * hidden + col]) =
          float4{facc[j][0] * wsc[j][0] * rw, facc[j][1] * wsc[j][1] * rw,
                 facc[j][2] * wsc[j][2] * rw, facc[j][3] * wsc[j][3] * rw};
    }
  }
}

// Ordered combine, one workgroup per token t: accum[t, :] = (((0 + y[r1]) +
// y[r2]) + ...) over t's records in ascending expert order (moe.mojo:259-282),
// out = bf16(accum).  t's records in expert e's segment are a run that starts
// where a binary search for t lands (segments are in ascending token order);
// a token that lists an expert twice (the router's padding repeats expert 0)
// has a run of two, added in record order as the reference adds its routes.
// A scan over experts lists the runs in ascending expert order.  At most
// kMaxTopK records.  Workgroup (t, c) takes columns [c * chunk, + chunk) of
// token t (a small batch spreads over more CUs; each repeats the scan).
constexpr int kMaxTopK = 16;

__global__ __launch_bounds__(256) void k_combine(
    const float* __restrict__ y, const int32_t* __restrict__ eo, const Route* __restrict__ routes,
    int E, int max_routes, int hidden, int chunk, float* __restrict__ accum,
    uint16_t* __restrict__ out) {
  __shared__ int recs[kMaxTopK];
  __shared__ int wsum[4];
  const int t = blockIdx.x, tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  int cnt = 0;
  for (int e0 = 0; e0 < E; e0 += 256) {
    const int e = e0 + tid;
    int first = 0, run = 0;
    if (e < E) {
      const int lo0 = max(0, min(eo[e], max_routes)), hi0 = max(0, min(eo[e + 1], max_routes));
      int lo = lo0, hi = hi0;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (routes[mid].token < t) lo = mid + 1; else hi = mid;
      }
      first = lo;
      while (lo + run < hi0 && run < kMaxTopK && routes[lo + run].token == t) ++run;
    }
    // exclusive prefix of the run lengths over this chunk's experts
    int inc = wave_incl_scan(run);
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    int base = cnt, total = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      base += w < wave ? wsum[w] : 0;
      total += wsum[w];
    }
    base += inc - run;
    for (int j = 0; j < run; ++j)
      if (base + j < kMaxTopK) recs[base + j] = first + j;
    cnt += total;
    __syncthreads();
  }
  cnt = min(cnt, kMaxTopK);
  int rr[kMaxTopK];
#pragma unroll
  for (int j = 0; j < kMaxTopK; ++j) rr[j] = j < cnt ? recs[j] : 0;
  typedef float f4 __attribute__((ext_vector_type(4)));
  const int c1 = min(hidden, ((int)blockIdx.y + 1) * chunk);
  for (int c = (int)blockIdx.y * chunk + tid * 4; c < c1; c += 1024) {
    f4 v[kMaxTopK];
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j)
      if (j < cnt)  // each y row is read once: non-temporal
        v[j] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(y + (size_t)rr[j] * hidden + c));
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j)
      if (j < cnt) acc = acc + v[j];
    __builtin_nontemporal_store(acc, reinterpret_cast<f4*>(accum + (size_t)t * hidden + c));
    const uint32_t lo = (uint32_t)f32_to_bf16(acc.x) | ((uint32_t)f32_to_bf16(acc.y) << 16);
    const uint32_t hi = (uint32_t)f32_to_bf16(acc.z) | ((uint32_t)f32_to_bf16(acc.w) << 16);
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u2*>(out + (size_t)t * hidden + c) = u2{lo, hi};
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
hipError_t launch_build_schedule(const int32_t* route_idx, const float* route_w, int seq_len,
                                 int top_k, int expert_base, int experts, int32_t* expert_offset,
                                 Route* routes, hipStream_t st) {
  if (seq_len <= 0) return hipSuccess;
  if (experts > kMaxExperts) return hipErrorInvalidValue;
  if (seq_len * top_k <= kSchedSmallSlots) {
    hipLaunchKernelGGL(k_build_schedule_small, dim3(1), dim3(kSchedSmallSlots), 0, st, route_idx,
                       route_w, seq_len * top_k, top_k, expert_base, experts, expert_offset, routes);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(k_build_schedule, dim3(experts), dim3(kSchedThreads), 0, st, route_idx,
                     route_w, seq_len * top_k, top_k, expert_base, experts, expert_offset, routes);
  return hipGetLastError();
}

static inline int mtile_bound(int max_routes, int experts, int bm) {
  // sum_e ceil(n_e/bm) <= max_routes/bm + experts
  long b = (long)(max_routes + bm - 1) / bm + experts;
  return (int)b;
}

// m-tile height for the grouped kernels from the mean routes per expert:
// 16-row skinny tiles while experts see a handful of tokens (decode), LDS-
// tiled tiles once each expert's weights can be reused.  The tile is sized
// so that nearly every expert fits in one m-tile (mean + 4 standard
// deviations of a binomial count): then each expert's weights stream from
// HBM once instead of once per m-tile.
int moe_tile_bm(int max_routes, int experts) {
  if (tune().moe_bm) return tune().moe_bm;
  const int per = max_routes / (experts > 0 ? experts : 1);
  if (per < 24) return 16;
  const double hi = per + 4.0 * __builtin_sqrt((double)per);
  if (hi > 192.0) return 256;
  if (hi > 128.0) return 192;  // 2048 tokens x top-8 / 128 experts: 128 + 45
  if (hi > 64.0) return 128;
  return 64;
}

hipError_t launch_moe_phase1(const int8_t* x_i8, const float* x_sa, const int32_t* eo,
                             const Route* routes, const int8_t* w_gu, const float* gu_scale,
                             uint16_t* bucket, int8_t* bi8, float* bsa, int experts,
                             int max_routes, int hidden, int inter, hipStream_t st,
                             const DenseGateUp* dense) {
  const bool has_dense = dense && dense->T > 0;
  if (max_routes <= 0 && !has_dense) return hipSuccess;
  if (bi8 && inter % 64) return hipErrorInvalidValue;
  if (has_dense && (!bi8 || dense->inter <= 0 || dense->inter % 64)) return hipErrorInvalidValue;
  const int gx = (inter / 16 + 3) / 4;
  DenseGateUp dn{};  // ytiles 0: no dense rows
  if (has_dense) {
    dn = *dense;
    dn.gx = gx;
    dn.cpg = (dn.inter / 64 + gx - 1) / gx;
    dn.ytiles = (dn.T + 15) / 16 * dn.cpg;
  }
  const int moe_rows = max_routes > 0 ? mtile_bound(max_routes, experts, 16) : 0;
  if (max_routes > 0) {
    const int bm = moe_tile_bm(max_routes, experts);
    if (bm >= 64 && inter % 64 == 0) {
      const hipError_t r = launch_moe_gate_up_tiled(x_i8, x_sa, eo, routes, w_gu, gu_scale, bucket,
                                                    bi8, bsa, experts, max_routes, hidden, inter,
                                                    bm, st);
      if (r != hipSuccess || !has_dense) return r;
      // the dense rows alone: 64 tokens per workgroup share each weight
      // fragment (2048 tokens: 135 us for them, against 229 us in 16-token
      // tiles and 306 us with 128 tokens and one k-step per slot)
      constexpr int RT = 4, U = 2;
      hipLaunchKernelGGL((k_dense_gate_up<RT, U>), dim3(dn.inter / 64, (dn.T + 16 * RT - 1) / (16 * RT)),
                         dim3(256), 0, st, hidden, fwht_scale_host(64), dn);
      return hipGetLastError();
    }
  }
  dim3 g(gx, dn.ytiles + moe_rows), b(256);
#define BQ_GU(U)                                                                                  \
  case U:                                                                                         \
    hipLaunchKernelGGL(k_moe_gate_up_skinny<U>, g, b, 0, st, experts, hidden, inter, max_routes,  \
                       eo, routes, w_gu, x_i8, gu_scale, x_sa, bucket, bi8, bsa,                  \
                       fwht_scale_host(64), dn);                                                  \
    break;
  switch (tune().gu_skinny) {  // 2 or 6 k-steps per register slot; 4 measured best
    BQ_GU(2) BQ_GU(6)
    default: BQ_GU(4)
  }
#undef BQ_GU
  return hipGetLastError();
}

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t moe_phase2_workspace(int max_routes, int seq_len, int hidden) {
  if (seq_len <= 0) return 0;
  return align256((size_t)max_routes * hidden * sizeof(float));
}

hipError_t launch_moe_phase2(const int8_t* bucket_i8, const float* bucket_sa, const int32_t* eo,
                             const Route* routes, const int8_t* w_down, const float* down_scale,
                             float* accum, uint16_t* out, int experts, int seq_len,
                             int max_routes, int hidden, int inter, int block, void* workspace,
                             hipStream_t st, const DenseDown* dense) {
  if (seq_len <= 0) return hipSuccess;
  const bool has_dense = dense && dense->T > 0;
  DenseDown dn{};  // ytiles 0: no dense rows
  if (has_dense) {
    if (dense->inter <= 0 || dense->inter % 64 || dense->inter % block || dense->inter / block > 64)
      return hipErrorInvalidValue;
    dn = *dense;
    dn.ytiles = (dn.T + 15) / 16;
  }
  float* y = (float*)workspace;
  // three k-steps per register slot and two strips per wave (BQ_DOWN_SKINNY).
  // The 30-layer batch-16 decode stack, whose dense down rows run K = 2112:
  // 1 / 2 k-steps 3.587 / 3.512 ms on one box, 2 / 3 / 4 k-steps 3.522 /
  // 3.501 / 3.524 ms on another; the 32-token MoE layer 2 / 3 k-steps 122.8 /
  // 122.6 us.  Four strips or one were slower.
  auto skinny = [&](int E, int moe_rows) {
#define BQ_DS(U, NS)                                                                              \
  case U * 10 + NS: {                                                                             \
    dim3 g((hidden / 16 + 4 * NS - 1) / (4 * NS), dn.ytiles + moe_rows), b(256);                 \
    hipLaunchKernelGGL((k_moe_down_skinny<U, NS>), g, b, 0, st, E, hidden, inter, block,          \
                       max_routes, eo, routes, bucket_sa, w_down, bucket_i8, down_scale, y, dn);  \
    break;                                                                                        \
  }
    switch (tune().down_skinny) {
      BQ_DS(1, 2) BQ_DS(1, 4) BQ_DS(2, 1) BQ_DS(2, 2) BQ_DS(4, 2)
      default: BQ_DS(3, 2)
    }
#undef BQ_DS
    return hipGetLastError();
  };
  bool dense_done = !has_dense;
  if (max_routes > 0) {
    const int bm = moe_tile_bm(max_routes, experts);
    if (bm >= 64 && hidden % 128 == 0) {
      // see launch_moe_down_tiled; BQ_MOE_BM_DOWN overrides the down tile alone
      const int bm_down = tune().moe_bm_down ? tune().moe_bm_down : tune().moe_bm ? bm : 64;
      hipError_t e = launch_moe_down_tiled(bucket_i8, bucket_sa, eo, routes, w_down, down_scale, y,
                                           experts, max_routes, hidden, inter, block, bm_down, st);
      if (e != hipSuccess) return e;
    } else {
      const hipError_t e = skinny(experts, mtile_bound(max_routes, experts, 16));
      if (e != hipSuccess) return e;
      dense_done = true;
    }
  }
  if (!dense_done) {
    // the experts took the tiled kernels (many tokens): the dense down
    // projection is the per-block linear's own launch (bq_block_linear), whose
    // tiles reuse each weight block across many tokens
    LinArgs la{};
    la.seg[0] = {dn.w, dn.ws, dn.out, nullptr, hidden, 0};
    la.nseg = 1;
    la.act = dn.x_i8;
    la.sa = dn.x_sa;
    la.M = dn.T;
    la.K = dn.inter;
    la.block = block;
    const hipError_t e = launch_linear(la, 1, st);
    if (e != hipSuccess) return e;
  }
  // below 256 tokens each workgroup takes 256 columns of its token (32
  // tokens: 32 workgroups -> 352, the layer ~130 -> 128.7 us), else the
  // whole row
  const int chunk = seq_len < 256 ? 256 : (hidden + 3) / 4 * 4;
  hipLaunchKernelGGL(k_combine, dim3(seq_len, (hidden + chunk - 1) / chunk), dim3(256), 0, st, y,
                     eo, routes, experts, max_routes, hidden, chunk, accum, out);
  return hipGetLastError();
}

}  // namespace bq
