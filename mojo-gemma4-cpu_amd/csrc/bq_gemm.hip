// bq_gemm.hip -- quantized linear kernels on v_mfma_i32_16x16x64_i8.
//
// Both operands are the signed int8 codes, so every 16x16 int32 accumulator
// is the exact sum_k x*w (the reference's AMX branch works the same way,
// butterquant/amx_gemm.mojo:36-44; its VNNI branch gets the same integer as
// sum (x^0x80)*w - 128*colsum, butterquant/dot_products.mojo:53-73).
//
// Epilogues follow the reference's f32 op order:
//   per-row  (gemm.mojo:133-142):  y = (f32(acc) * (sa[m]*(1/127))) * ws[n]
//   per-block(gemm.mojo:194-215):  facc = fma(f32(acc_b), sa[m,b]*(1/127), facc)
//                                  for b ascending;  y = facc * ws[n]
//
// k_linear_skinny (M <= 16, decode): one workgroup per 16-row n-tile, waves
//   split K; each step streams one 1 KiB weight fragment per wave (HBM-bound,
//   no LDS staging of weights).  Partial int32 tiles are reduced exactly in LDS.
// M > 16 (prefill) runs the LDS-tiled kernel of bq_tiled.hip.
#include "bq_device.hpp"
#include "bq_kernels.hpp"

namespace bq {

// The segment of global n-tile nt_global, selected by value: the fields of
// all three segments are read in one batch of scalar loads, so the first
// weight load waits for one kernel-argument round trip.  (Indexing a.seg[s]
// by address makes the compiler load nseg and the boundaries first and the
// chosen segment's fields after them: two dependent round trips.)
__device__ inline LinSeg pick_seg(const LinArgs& a, int nt_global, int& nt_local) {
  const LinSeg s0 = a.seg[0], s1 = a.seg[1], s2 = a.seg[2];
  const bool in1 = a.nseg > 1 && nt_global >= s1.tile0;
  const bool in2 = a.nseg > 2 && nt_global >= s2.tile0;
  LinSeg r;
  r.w = in2 ? s2.w : in1 ? s1.w : s0.w;
  r.ws = in2 ? s2.ws : in1 ? s1.ws : s0.ws;
  r.out = in2 ? s2.out : in1 ? s1.out : s0.out;
  r.out_f32 = in2 ? s2.out_f32 : in1 ? s1.out_f32 : s0.out_f32;
  r.n = in2 ? s2.n : in1 ? s1.n : s0.n;
  r.tile0 = in2 ? s2.tile0 : in1 ? s1.tile0 : s0.tile0;
  nt_local = nt_global - r.tile0;
  return r;
}

// A one-segment call's arguments: 64 bytes, one scalar-cache line (the
// three-segment LinArgs spans three).  They are read before any address is
// known, and a smaller argument block measured shorter launches (the decode
// GEMV 4.545 -> 4.447 us).
struct Seg1Args {
  const int8_t* w;    // tile16x64 codes [n, K]
  const float* ws;    // per-row weight scale [n]
  const int8_t* act;  // int8 [M, K] row-major
  const float* sa;    // per-row [M] or per-block [M, K/block] activation scales
  uint16_t* out;      // bf16 [M, n]
  float* out_f32;     // optional f32 [M, n]
  int n, M, K, block;  // output rows; rows, K and the activation block
};

static Seg1Args seg1_args(const LinArgs& a) {
  const LinSeg& s0 = a.seg[0];
  return Seg1Args{s0.w, s0.ws, a.act, a.sa, s0.out, s0.out_f32, s0.n, a.M, a.K, a.block};
}

__device__ inline LinSeg seg_of(const LinArgs& a, int& nt) { return pick_seg(a, blockIdx.x, nt); }
__device__ inline LinSeg seg_of(const Seg1Args& a, int& nt) {
  LinSeg r;
  r.w = a.w; r.ws = a.ws; r.out = a.out; r.out_f32 = a.out_f32; r.n = a.n; r.tile0 = 0;
  nt = blockIdx.x;
  return r;
}

// ---------------------------------------------------------------------------
// skinny: M <= 16
// ---------------------------------------------------------------------------
template <int WAVES, bool PER_BLOCK, int U, class Args>
__device__ __forceinline__ void linear_skinny(const Args& args) {
  extern __shared__ int lds[];  // per-row: WAVES*256 ints; per-block: nb*256 ints
  int nt;
  const LinSeg seg = seg_of(args, nt);
  const int K = args.K, K64 = K >> 6, M = args.M;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int fpb = args.block >> 6;  // fragments per K block (power of two)
  const int nb = K / args.block;
  int kt0, kt1;
  if (PER_BLOCK) {  // waves own whole blocks, so block partials need no atomics
    const int per_b = (nb + WAVES - 1) / WAVES;
    const int b0 = min(nb, wave * per_b), b1 = min(nb, b0 + per_b);
    kt0 = b0 * fpb;
    kt1 = b1 * fpb;
  } else {
    const int per = (K64 + WAVES - 1) / WAVES;
    kt0 = min(K64, wave * per);
    kt1 = min(K64, kt0 + per);
  }
  const int8_t* wb = seg.w + (size_t)nt * K64 * 1024 + lane * 16;
  // the weight stream goes out first: a K slice of at most U fragments per
  // wave (K <= 64*U*WAVES) is requested before anything else
  v4i bf0[U];
  const bool one_shot = kt1 - kt0 <= U;
  if (one_shot) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      bf0[u] = __builtin_nontemporal_load(
          reinterpret_cast<const v4i*>(wb + (size_t)min(kt0 + u, max(kt1 - 1, 0)) * 1024));
  }
  // epilogue operands, fetched before the weights arrive (thread t < 256
  // owns accumulator element t of the tile)
  const int t = threadIdx.x;
  const int ev = (t & 255) >> 6, eL = t & 63;
  const int ei = 4 * (eL >> 4) + ev;
  const int en = nt * 16 + (eL & 15);
  const bool eact = t < 256 && ei < M;
  // unmasked loads (clamped index): a masked load would make the compiler
  // wait for the whole weight stream at the branch join
  const float ews = seg.ws[en];
  const float ead = PER_BLOCK ? 0.0f : args.sa[min(ei, M - 1)] * kInv127;
  // rows >= M load row 0 instead: accumulator row i depends only on A row i
  // and rows >= M are never stored, so the loads need no mask (a branch
  // around them would force the compiler to wait for every outstanding load)
  const bool arow = (lane & 15) < M;
  const int8_t* ab = args.act + (size_t)(arow ? (lane & 15) : 0) * K + (lane >> 4) * 16;
  const v4i zero = {0, 0, 0, 0};
  v4i c = zero;

  int kt = kt0;
  if (one_shot) {
    v4i af[U];
#pragma unroll
    for (int u = 0; u < U; ++u) af[u] = ld16(ab + min(kt0 + u, max(kt1 - 1, 0)) * 64);
    if constexpr (!PER_BLOCK) {
      // two independent accumulator chains (exact int32 sums, added at the end)
      v4i c1 = zero;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (kt0 + u < kt1) {
          if (u & 1) c1 = mfma16x16x64(af[u], bf0[u], c1);
          else c = mfma16x16x64(af[u], bf0[u], c);
        }
      }
      c += c1;
    } else {
      // one chain, drained at block ends
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (kt0 + u < kt1) {
          c = mfma16x16x64(af[u], bf0[u], c);
          if (((kt0 + u + 1) & (fpb - 1)) == 0) {
            const int b = (kt0 + u) / fpb;
            lds[b * 256 + 0 * 64 + lane] = c.x;
            lds[b * 256 + 1 * 64 + lane] = c.y;
            lds[b * 256 + 2 * 64 + lane] = c.z;
            lds[b * 256 + 3 * 64 + lane] = c.w;
            c = zero;
          }
        }
      }
    }
    kt = kt1;
  }
  for (; kt + U <= kt1; kt += U) {
    v4i bf[U], af[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      bf[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wb + (size_t)(kt + u) * 1024));
#pragma unroll
    for (int u = 0; u < U; ++u) af[u] = ld16(ab + (kt + u) * 64);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      c = mfma16x16x64(af[u], bf[u], c);
      if (PER_BLOCK && (((kt + u + 1) & (fpb - 1)) == 0)) {
        const int b = (kt + u) / fpb;
        lds[b * 256 + 0 * 64 + lane] = c.x;
        lds[b * 256 + 1 * 64 + lane] = c.y;
        lds[b * 256 + 2 * 64 + lane] = c.z;
        lds[b * 256 + 3 * 64 + lane] = c.w;
        c = zero;
      }
    }
  }
  for (; kt < kt1; ++kt) {
    v4i bfr = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wb + (size_t)kt * 1024));
    v4i afr = ld16(ab + kt * 64);
    c = mfma16x16x64(afr, bfr, c);
    if (PER_BLOCK && (((kt + 1) & (fpb - 1)) == 0)) {
      const int b = kt / fpb;
      lds[b * 256 + 0 * 64 + lane] = c.x;
      lds[b * 256 + 1 * 64 + lane] = c.y;
      lds[b * 256 + 2 * 64 + lane] = c.z;
      lds[b * 256 + 3 * 64 + lane] = c.w;
      c = zero;
    }
  }
  if (!PER_BLOCK) {
    lds[wave * 256 + 0 * 64 + lane] = c.x;
    lds[wave * 256 + 1 * 64 + lane] = c.y;
    lds[wave * 256 + 2 * 64 + lane] = c.z;
    lds[wave * 256 + 3 * 64 + lane] = c.w;
  }
  __syncthreads();

  // epilogue: thread t <-> accumulator element (v = t/64, L = t%64):
  // row 4*(L/16)+v, column L%16 of the 16x16 tile.
  if (!eact) return;
  const int i = ei, n = en;
  float y;
  if (PER_BLOCK) {
    float facc = 0.0f;
    for (int b = 0; b < nb; ++b) {
      const float adv = args.sa[(size_t)i * nb + b] * kInv127;
      facc = fmaf((float)lds[b * 256 + t], adv, facc);
    }
    y = facc * ews;
  } else {
    int acc = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) acc += lds[w * 256 + t];
    y = (float)acc * ead * ews;
  }
  seg.out[(size_t)i * seg.n + n] = f32_to_bf16(y);
  if (seg.out_f32) seg.out_f32[(size_t)i * seg.n + n] = y;
}

// A one-segment call's arguments as the kernel's own scalars: the dispatch
// preloads the first 14 dwords into SGPRs (the build's kernarg preload), so
// everything the addresses need -- K, M, block and the weight, activation and
// scale pointers, in that order -- is there at the first instruction; only
// out_f32 and n, read by the epilogue, are loaded.
#define BQ_SEG1_PARAMS                                                                          \
  int K, int M, int block, const int8_t *w, const int8_t *act, const float *ws, const float *sa, \
      uint16_t *out, float *out_f32, int n
#define BQ_SEG1_FIELDS w, ws, act, sa, out, out_f32, n, M, K, block
#define BQ_SEG1_ARGS(s) \
  s.K, s.M, s.block, s.w, s.act, s.ws, s.sa, s.out, s.out_f32, s.n

template <int WAVES, bool PER_BLOCK, int U>
__global__ __launch_bounds__(WAVES * 64) void k_linear_skinny(LinArgs args) {
  linear_skinny<WAVES, PER_BLOCK, U>(args);
}
template <int WAVES, bool PER_BLOCK, int U>
__global__ __launch_bounds__(WAVES * 64) void k_linear_skinny_1(BQ_SEG1_PARAMS) {
  linear_skinny<WAVES, PER_BLOCK, U>(Seg1Args{BQ_SEG1_FIELDS});
}

// NT 16-row n-tiles per workgroup (per-row, 2 <= M <= 16, K <= 4096): each
// of the 16 waves takes the same one-shot K slice of every tile, so the
// slice's activation fragments (the whole M x K activation per workgroup,
// as much as one tile's weights at M = 16) are read once for NT tiles.  The
// tiles are global n-tiles NT b .. NT b + NT - 1 and may lie in different
// segments (q | k | v); a short last group has fewer.  The same exact int32
// sums and y = (f32(acc) * (sa*(1/127))) * ws[n] epilogue as
// k_linear_skinny.
template <int NT, int U>
__global__ __launch_bounds__(1024) void k_linear_skinny2(LinArgs args) {
  constexpr int WAVES = 16;
  __shared__ int lds[NT * WAVES * 256];
  const LinSeg& last_seg = args.seg[args.nseg - 1];
  const int tiles = last_seg.tile0 + last_seg.n / 16;
  const int g0 = NT * blockIdx.x;
  const int ntl = min(NT, tiles - g0);  // tiles of this workgroup
  LinSeg sg[NT];
  int ntt[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) sg[j] = pick_seg(args, j < ntl ? g0 + j : g0, ntt[j]);
  const int K = args.K, K64 = K >> 6, M = args.M;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int per = (K64 + WAVES - 1) / WAVES;
  const int kt0 = min(K64, wave * per), kt1 = min(K64, kt0 + per);
  const int last = max(kt1 - 1, 0);  // loads past the wave's range read this k-step
  // every tile's weight slice goes out first
  v4i b[NT][U];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int8_t* wb = sg[j].w + (size_t)ntt[j] * K64 * 1024 + lane * 16;
#pragma unroll
    for (int u = 0; u < U; ++u)
      b[j][u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wb + (size_t)min(kt0 + u, last) * 1024));
  }
  // epilogue operands: thread t < 256 NT owns element t % 256 of tile t / 256
  const int t = threadIdx.x, tile = min(t >> 8, NT - 1);
  const int ev = (t & 255) >> 6, eL = t & 63;
  const int ei = 4 * (eL >> 4) + ev;
  LinSeg es = sg[0];
  int ent = ntt[0];
#pragma unroll
  for (int j = 1; j < NT; ++j)
    if (tile == j) { es = sg[j]; ent = ntt[j]; }
  const int en = ent * 16 + (eL & 15);
  const bool eact = t < 256 * NT && ei < M && tile < ntl;
  const float ews = es.ws[en];
  const float ead = args.sa[min(ei, M - 1)] * kInv127;
  // rows >= M read row 0 (accumulator row i depends only on A row i; rows
  // >= M are never stored)
  const int8_t* ab = args.act + (size_t)((lane & 15) < M ? (lane & 15) : 0) * K + (lane >> 4) * 16;
  v4i af[U];
#pragma unroll
  for (int u = 0; u < U; ++u) af[u] = ld16(ab + min(kt0 + u, last) * 64);
  const v4i zero = {0, 0, 0, 0};
  v4i c[NT], cb[NT];  // two chains per tile
#pragma unroll
  for (int j = 0; j < NT; ++j) c[j] = cb[j] = zero;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (kt0 + u < kt1) {
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        if (u & 1) cb[j] = mfma16x16x64(af[u], b[j][u], cb[j]);
        else c[j] = mfma16x16x64(af[u], b[j][u], c[j]);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    c[j] += cb[j];
    int* l = lds + (j * WAVES + wave) * 256 + lane;
    l[0] = c[j].x; l[64] = c[j].y; l[128] = c[j].z; l[192] = c[j].w;
  }
  __syncthreads();
  if (!eact) return;
  int acc = 0;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) acc += lds[(tile * WAVES + w) * 256 + (t & 255)];
  const float y = (float)acc * ead * ews;
  es.out[(size_t)ei * es.n + en] = f32_to_bf16(y);
  if (es.out_f32) es.out_f32[(size_t)ei * es.n + en] = y;
}

// ---------------------------------------------------------------------------
// M = 1, per-row (the decode GEMV)
// ---------------------------------------------------------------------------
// f(std::integral_constant<int, I>{}) for I = I0 .. I1 - 1, in order
template <int I0, int I1, typename F>
__device__ inline void static_for(F&& f) {
  if constexpr (I0 < I1) {
    f(std::integral_constant<int, I0>{});
    static_for<I0 + 1, I1>(f);
  }
}

// the four dwords of x as lane (lane + R) of the same 16-lane row holds them
// (DPP row_shl:R); R = 0 is x itself
template <int R>
__device__ inline v4i row_shl_v4(const v4i& x) {
  if constexpr (R == 0) {
    return x;
  } else {
    v4i r;
    r.x = __builtin_amdgcn_update_dpp(x.x, x.x, 0x100 + R, 0xF, 0xF, false);
    r.y = __builtin_amdgcn_update_dpp(x.y, x.y, 0x100 + R, 0xF, 0xF, false);
    r.z = __builtin_amdgcn_update_dpp(x.z, x.z, 0x100 + R, 0xF, 0xF, false);
    r.w = __builtin_amdgcn_update_dpp(x.w, x.w, 0x100 + R, 0xF, 0xF, false);
    return r;
  }
}

// One workgroup of WAVES waves per 16-row n-tile; wave w owns k-steps
// [w*per, (w+1)*per), per = ceil(K/64 / WAVES) <= U.  At M = 1 only row 0 of
// the MFMA's A operand is stored, and row 0 is lane 16c's 16-byte chunk c of
// the k-step.  So one 16-byte load per lane brings 16 k-steps' activation
// (lane 16c + r: chunk c of k-step r), and a DPP row_shl:r moves k-step r's
// chunks to lanes 16c when it is multiplied (the other rows are never
// stored).  The activation and the scales are requested before the weights;
// loads return in issue order, so the MFMA of k-step u waits only for
// weight fragments 0..u and the products overlap the stream.  NC independent
// chains of exact int32 sums: after the last fragment lands one MFMA, three
// adds and the cross-wave sum remain.  Same y = (f32(acc) * (sa*(1/127))) *
// ws[n] epilogue as k_linear_skinny (gemm.mojo:133-142).
// (one workgroup per CU at the model's widths: waves_per_eu(1, 2) lets the
// compiler hold every fragment in registers instead of sinking the loads)
template <int WAVES, int U, class Args>
__device__ __forceinline__ void gemv_m1(const Args& args) {
  constexpr int NC = U >= 4 ? 4 : U;  // accumulator chains
  constexpr int NA = (U + 15) / 16;   // activation loads per lane
  __shared__ int part[WAVES * 16];
  int nt;
  const LinSeg seg = seg_of(args, nt);
  const int K64 = args.K >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int per = (K64 + WAVES - 1) / WAVES;
  const int kt0 = min(K64, wave * per), kt1 = min(K64, kt0 + per);
  const int last = max(kt1 - 1, 0);  // loads past the wave's range read this k-step
  v4i xa[NA];
#pragma unroll
  for (int g = 0; g < NA; ++g)
    xa[g] = ld16(args.act + (size_t)min(kt0 + 16 * g + (lane & 15), last) * 64 + (lane >> 4) * 16);
  const float ews = seg.ws[nt * 16 + (lane & 15)];
  const float ead = args.sa[0] * kInv127;
  asm volatile("" ::: "memory");  // the weight loads go out after these
  const int8_t* wb = seg.w + (size_t)nt * K64 * 1024 + lane * 16;
  v4i bf[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    bf[u] = __builtin_nontemporal_load(
        reinterpret_cast<const v4i*>(wb + (size_t)min(kt0 + u, last) * 1024));
  asm volatile("" ::: "memory");  // all of them before any product
  const v4i zero = {0, 0, 0, 0};
  v4i c[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) c[j] = zero;
  static_for<0, U>([&](auto uc) {
    constexpr int u = decltype(uc)::value;
    const v4i a = kt0 + u < kt1 ? row_shl_v4<u % 16>(xa[u / 16]) : zero;
    c[u % NC] = mfma16x16x64(a, bf[u], c[u % NC]);
  });
  int s = c[0].x;
#pragma unroll
  for (int j = 1; j < NC; ++j) s += c[j].x;  // row 0, column lane (lanes 0..15)
  if (lane < 16) part[wave * 16 + lane] = s;
  __syncthreads();
  if (threadIdx.x >= 16) return;
  int acc = 0;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) acc += part[w * 16 + lane];
  const float y = (float)acc * ead * ews;
  const int n = nt * 16 + lane;
  seg.out[n] = f32_to_bf16(y);
  if (seg.out_f32) seg.out_f32[n] = y;
}

template <int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(1, 2)))
void k_gemv_m1(LinArgs args) {
  gemv_m1<WAVES, U>(args);
}
template <int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(1, 2)))
void k_gemv_m1_1(BQ_SEG1_PARAMS) {
  gemv_m1<WAVES, U>(Seg1Args{BQ_SEG1_FIELDS});
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------
hipError_t launch_linear(const LinArgs& a, int per_block, hipStream_t st) {
  if (a.M <= 0) return hipSuccess;
  if (a.M <= 16) {
    int tiles = 0;
    for (int q = 0; q < a.nseg; ++q) tiles += a.seg[q].n / 16;
    // M = 1 per-row up to K = 4096: k_gemv_m1 (BQ_GEMV_WAVES sends it to the
    // general kernel below)
    if (a.M == 1 && !per_block && !tune().gemv_waves && a.K <= 4096) {
      const int w1 = tune().gemv_m1_waves ? tune().gemv_m1_waves : 4;
      dim3 g1(tiles);
      if (a.nseg == 1) {
        const Seg1Args s1 = seg1_args(a);
#define BQ_GO(W, U_, B) \
  hipLaunchKernelGGL((k_gemv_m1_1<W, U_>), g1, dim3(B), 0, st, BQ_SEG1_ARGS(s1))
        if (w1 <= 2) BQ_GO(2, 32, 128);
        else if (w1 >= 8) BQ_GO(8, 8, 512);
        else BQ_GO(4, 16, 256);
#undef BQ_GO
      } else {
        if (w1 <= 2) hipLaunchKernelGGL((k_gemv_m1<2, 32>), g1, dim3(128), 0, st, a);
        else if (w1 >= 8) hipLaunchKernelGGL((k_gemv_m1<8, 8>), g1, dim3(512), 0, st, a);
        else hipLaunchKernelGGL((k_gemv_m1<4, 16>), g1, dim3(256), 0, st, a);
      }
      return hipGetLastError();
    }
    // ceil(tiles / CUs) n-tiles per workgroup (at most 4, or BQ_SKINNY2 when
    // that is 2 or 3) while there are >= 2 per CU: one workgroup per CU, each
    // activation read shared by its tiles
    if (!per_block && a.M >= 2 && !tune().gemv_waves && a.K <= 4096 && tune().skinny2 &&
        tiles >= 2 * tune().cus) {
      const int cap = tune().skinny2 >= 2 ? min(tune().skinny2, 4) : 4;
      const int nt = min(cap, (tiles + tune().cus - 1) / tune().cus);
      if (nt <= 2) hipLaunchKernelGGL((k_linear_skinny2<2, 4>), dim3((tiles + 1) / 2), dim3(1024), 0, st, a);
      else if (nt == 3) hipLaunchKernelGGL((k_linear_skinny2<3, 4>), dim3((tiles + 2) / 3), dim3(1024), 0, st, a);
      else hipLaunchKernelGGL((k_linear_skinny2<4, 4>), dim3((tiles + 3) / 4), dim3(1024), 0, st, a);
      return hipGetLastError();
    }
    // 16 waves split K so that each wave's whole slice (<= 4 fragments for
    // K <= 4096) is requested at once: the full weight is in flight within
    // the first memory latency.  K = N = 4096, M = 1: 4.86 -> 4.72 us against
    // 8 waves of 8 fragments (5.20 us with 4 of 16); the batch-16 decoder
    // layer 147.4 -> 145.8 us.
    const int waves = tune().gemv_waves ? tune().gemv_waves : 16;
    const int nb = a.K / a.block;
    dim3 g(tiles);
    const Seg1Args s1 = seg1_args(a);
    const bool one = a.nseg == 1;
#define BQ_GO(W, PB, U_)                                                                        \
  do {                                                                                          \
    const size_t lds = (size_t)(PB ? nb : W) * 256 * sizeof(int);                              \
    if (one)                                                                                    \
      hipLaunchKernelGGL((k_linear_skinny_1<W, PB, U_>), g, dim3(64 * W), lds, st,              \
                         BQ_SEG1_ARGS(s1));                                                      \
    else                                                                                        \
      hipLaunchKernelGGL((k_linear_skinny<W, PB, U_>), g, dim3(64 * W), lds, st, a);            \
  } while (0)
    if (waves >= 16) {
      if (per_block) BQ_GO(16, true, 4); else BQ_GO(16, false, 4);
    } else if (waves <= 4) {
      if (per_block) BQ_GO(4, true, 16); else BQ_GO(4, false, 16);
    } else {
      if (per_block) BQ_GO(8, true, 8); else BQ_GO(8, false, 8);
    }
#undef BQ_GO
    return hipGetLastError();
  }
  // prefer the largest M tile that still yields >= 256 workgroups (one per CU)
  int gn128 = 0;
  for (int q = 0; q < a.nseg; ++q) gn128 += (a.seg[q].n + 127) / 128;
  int bm = 32;
  if (a.M > 64 && ((a.M + 127) / 128) * gn128 >= 256) bm = 128;
  else if (a.M > 32) bm = 64;
  if (tune().tile_bm) bm = tune().tile_bm;
  return launch_linear_tiled(a, per_block, bm, st);
}

// ---------------------------------------------------------------------------
// norm-quant + per-row linear of one token (decode) in one launch
// ---------------------------------------------------------------------------
// What bq_norm_quant followed by bq_linear / bq_qkv on its output computes,
// for seq_len 1.  Each workgroup of 8 waves loads the token's row, requests
// its weight fragments (k_linear_skinny<8, false, 8>'s one-shot slices,
// K <= 4096) and quantizes the row itself while they are in flight: every
// wave takes the sum of squares over the whole row (nq_pair_sumsq's chain
// order) and transforms its SPW segments (nq_pair_transform), the amax is
// exchanged through LDS, and the int8 codes land in LDS, where the A operand
// is read from.  Every workgroup
// computes the same codes and scale; workgroup 0 also writes them to
// x_i8 / x_sa.  Two launches become one, and the norm-quant's memory round
// trips overlap the weight stream instead of preceding it.
// V8 (FWHT block 128): wave w transforms values 512 w .. 512 w + 511 with 8
// consecutive values per lane (nq_v8_transform), the codes one 8-byte store
// per lane; otherwise the pair layout's SPW segments per wave.
template <int NSEG, int SPW, bool V8, class Args>
__device__ __forceinline__ void norm_linear_skinny(const Args& args, const NormArgs& nq) {
  constexpr int WAVES = 8, U = 8;
  __shared__ __attribute__((aligned(16))) int8_t s_x[64 * WAVES * U];  // the row's codes
  __shared__ int lds[WAVES * 256];
  __shared__ float s_f[WAVES];  // per-wave amax
  int nt;
  const LinSeg seg = seg_of(args, nt);
  const int K = args.K, K64 = K >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int per = (K64 + WAVES - 1) / WAVES;
  const int kt0 = min(K64, wave * per), kt1 = min(K64, kt0 + per);
  // The row's loads go out before the weights: loads return in issue order,
  // so the norm-quant's operands must not queue behind the weight stream.
  // Every wave loads the whole row and takes its sum of squares (as
  // k_norm_quant_pair does: no barrier before the transform).
  const int nseg = K >> 7, q0 = wave * SPW, wpt = (nseg + SPW - 1) / SPW;
  const uint32_t* xr = reinterpret_cast<const uint32_t*>(nq.src) + lane;
  const uint32_t* gr = reinterpret_cast<const uint32_t*>(nq.gamma) + lane;
  // (the wave's own segments are loaded again, into x: cheaper than picking
  // them out of xp by a run-time index)
  uint32_t xp[NSEG], x[SPW], g[SPW];
  v4i xv, gv;
#pragma unroll
  for (int q = 0; q < NSEG; ++q)  // first: the sum of squares needs it first
    if (q < nseg) xp[q] = xr[64 * q];
  const int e0 = 512 * wave + 8 * lane;  // V8: this lane's run
  if constexpr (V8) {
    const int ec = min(e0, K - 8);  // runs past the row are read, never used
    xv = *reinterpret_cast<const v4i*>(nq.src + ec);
    gv = *reinterpret_cast<const v4i*>(nq.gamma + ec);
  } else {
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      const bool in = q0 + i < nseg;
      x[i] = in ? xr[64 * (q0 + i)] : 0u;
      g[i] = in ? gr[64 * (q0 + i)] : 0u;
    }
  }
  // epilogue: thread t < 16 owns row 0's column t (accumulator element v = 0
  // of lanes 0..15); its weight scale is fetched now
  const int t = threadIdx.x;
  const float ews = seg.ws[nt * 16 + (t & 15)];
  asm volatile("" ::: "memory");  // keep the weight loads after these
  const int8_t* wb = seg.w + (size_t)nt * K64 * 1024 + lane * 16;
  v4i bf[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    bf[u] = __builtin_nontemporal_load(
        reinterpret_cast<const v4i*>(wb + (size_t)min(kt0 + u, max(kt1 - 1, 0)) * 1024));

  // ---- the row's norm-quant ------------------------------------------------
  const float total = nq_pair_sumsq<NSEG>(xp, nseg);
  const float inv_rms = nq.sqrt_n / __builtin_sqrtf(total + nq.n_eps);
  float v[SPW][2], v8[8];
  float m;
  if constexpr (V8) {
    m = nq_v8_transform(xv, gv, inv_rms, nq.fwht_scale, v8);
    if (e0 >= K) m = 0.0f;
  } else {
    m = nq_pair_transform<SPW>(x, g, inv_rms, q0, nseg, nq.block, nq.fwht_scale, v);
  }
  const float wmax = wave_max(m);
  if (lane == 0) s_f[wave] = wmax;
  __syncthreads();
  float amax = s_f[0];
  for (int w = 1; w < (V8 ? WAVES : wpt); ++w) amax = fmaxf(amax, s_f[w]);
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  if constexpr (V8) {
    if (e0 < K) {
      uint32_t w[2];
      nq_v8_codes(v8, inv, w);
      typedef uint32_t u2 __attribute__((ext_vector_type(2)));
      *reinterpret_cast<u2*>(&s_x[e0]) = u2{w[0], w[1]};
      if (blockIdx.x == 0) *reinterpret_cast<u2*>(nq.xq + e0) = u2{w[0], w[1]};
    }
  } else {
    uint16_t* sx = reinterpret_cast<uint16_t*>(s_x) + lane;
    uint16_t* gx = reinterpret_cast<uint16_t*>(nq.xq) + lane;
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      if (q0 + i < nseg) {
        const uint16_t c = nq_pair_code(v[i], inv);
        sx[64 * (q0 + i)] = c;
        if (blockIdx.x == 0) gx[64 * (q0 + i)] = c;
      }
    }
  }
  if (blockIdx.x == 0 && t == 0) nq.sa[0] = amax;
  __syncthreads();

  // ---- the product (k_linear_skinny's per-row one-shot path, M = 1) ---------
  const v4i zero = {0, 0, 0, 0};
  v4i c = zero, c1 = zero;  // two independent chains of exact int32 sums
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (kt0 + u < kt1) {
      const v4i af = *reinterpret_cast<const v4i*>(&s_x[(kt0 + u) * 64 + (lane >> 4) * 16]);
      if (u & 1) c1 = mfma16x16x64(af, bf[u], c1);
      else c = mfma16x16x64(af, bf[u], c);
    }
  }
  c += c1;
  lds[wave * 256 + lane] = c.x;  // element v = 0: row 0 for lanes 0..15
  __syncthreads();
  if (t >= 16) return;
  int acc = 0;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) acc += lds[w * 256 + t];
  const float y = (float)acc * (amax * kInv127) * ews;
  const int n = nt * 16 + t;
  seg.out[n] = f32_to_bf16(y);
  if (seg.out_f32) seg.out_f32[n] = y;
}

template <int NSEG, int SPW, bool V8>
__global__ __launch_bounds__(512) void k_norm_linear_skinny(LinArgs args, NormArgs nq) {
  norm_linear_skinny<NSEG, SPW, V8>(args, nq);
}
// one segment, scalar arguments: the first 14 dwords (preloaded) hold what
// the row loads and the weight stream need first -- K, the FWHT block, the
// row and gain, the weights and their scales, sqrt_n, n_eps, the FWHT scale
template <int NSEG, int SPW, bool V8>
__global__ __launch_bounds__(512) void k_norm_linear_skinny_1(
    int K, int block, const uint16_t* src, const uint16_t* gamma, const int8_t* w, const float* ws,
    float sqrt_n, float n_eps, float fwht_scale, int8_t* xq, float* sa, uint16_t* out,
    float* out_f32, int n) {
  norm_linear_skinny<NSEG, SPW, V8>(Seg1Args{w, ws, nullptr, nullptr, out, out_f32, n, 1, K, K},
                                    NormArgs{src, gamma, xq, sa, block, sqrt_n, n_eps, fwht_scale});
}

// the fused kernel's shapes: one token, the pair-layout norm-quant's shapes
// (hidden % 256 == 0, hidden <= 4096), per-row weights
static bool launch_norm_linear_fused(const LinArgs& a, const NormArgs& nq, hipStream_t st) {
  if (a.M != 1 || a.K % 256 || a.K > 4096 || !tune().nq_pair ||
      (reinterpret_cast<uintptr_t>(nq.xq) & 1u))
    return false;
  int tiles = 0;
  for (int q = 0; q < a.nseg; ++q) tiles += a.seg[q].n / 16;
  const int ns = a.K >> 7;
  const int unit = nq.block > 128 ? nq.block / 128 : 1;
  int spw = (ns + 7) / 8;
  spw = (spw + unit - 1) / unit * unit;
  const dim3 g(tiles), b(512);
  // FWHT block 128 (the model's): 8 values per lane for the transform
  // (16-byte aligned gain, 8-byte aligned codes)
  const bool v8 = nq.block == 128 && tune().nq_v8 && !(reinterpret_cast<uintptr_t>(nq.gamma) & 15u) &&
                  !(reinterpret_cast<uintptr_t>(nq.xq) & 7u);
  const Seg1Args s1 = seg1_args(a);
  const bool one = a.nseg == 1;
#define BQ_NLL(N, S, V)                                                                          \
  do {                                                                                           \
    if (one)                                                                                     \
      hipLaunchKernelGGL((k_norm_linear_skinny_1<N, S, V>), g, b, 0, st, s1.K, nq.block, nq.src, \
                         nq.gamma, s1.w, s1.ws, nq.sqrt_n, nq.n_eps, nq.fwht_scale, nq.xq, nq.sa, \
                         s1.out, s1.out_f32, s1.n);                                              \
    else                                                                                         \
      hipLaunchKernelGGL((k_norm_linear_skinny<N, S, V>), g, b, 0, st, a, nq);                   \
    return true;                                                                                 \
  } while (0)
  if (v8) {
#define BQ_NL8(N) if (ns <= N) BQ_NLL(N, 1, true);
    BQ_NL8(8) BQ_NL8(16) BQ_NL8(22) BQ_NL8(24) BQ_NL8(32)
#undef BQ_NL8
  }
#define BQ_NL(N, S) if (ns <= N && spw == S) BQ_NLL(N, S, false);
  BQ_NL(8, 1) BQ_NL(8, 2) BQ_NL(8, 4) BQ_NL(16, 2) BQ_NL(16, 4)
  BQ_NL(24, 3) BQ_NL(24, 4) BQ_NL(32, 4)
#undef BQ_NL
#undef BQ_NLL
  return false;
}

hipError_t launch_norm_linear(const LinArgs& a, const NormArgs& nq_in, hipStream_t st) {
  if (a.M <= 0) return hipSuccess;
  NormArgs nq = nq_in;
  nq.fwht_scale = fwht_scale_host(nq.block);
  if (launch_norm_linear_fused(a, nq, st)) return hipGetLastError();
  const hipError_t e = launch_norm_quant(nq.src, nq.gamma, nq.xq, nq.sa, a.M, a.K, nq.block,
                                         nq.sqrt_n, nq.n_eps, st);
  if (e != hipSuccess) return e;
  return launch_linear(a, 0, st);
}

}  // namespace bq
