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
// k_linear_tiled (M > 16, prefill): BMxBN tile per workgroup, 2x2 waves,
//   A and B staged through double-buffered LDS in MFMA fragment order,
//   XCD-aware tile order (all m-tiles of an n-panel on one XCD's L2).
#include "bq_device.hpp"
#include "bq_kernels.hpp"

namespace bq {

__device__ inline const LinSeg& pick_seg(const LinArgs& a, int nt_global, int& nt_local) {
  int s = 0;
  if (a.nseg > 1 && nt_global >= a.seg[1].tile0) s = 1;
  if (a.nseg > 2 && nt_global >= a.seg[2].tile0) s = 2;
  nt_local = nt_global - a.seg[s].tile0;
  return a.seg[s];
}

// ---------------------------------------------------------------------------
// skinny: M <= 16
// ---------------------------------------------------------------------------
template <int WAVES, bool PER_BLOCK, int U>
__global__ __launch_bounds__(WAVES * 64) void k_linear_skinny(LinArgs args) {
  extern __shared__ int lds[];  // per-row: WAVES*256 ints; per-block: nb*256 ints
  int nt;
  const LinSeg& seg = pick_seg(args, blockIdx.x, nt);
  const int K = args.K, K64 = K >> 6, M = args.M;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
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
  const bool arow = (lane & 15) < M;
  const int8_t* ab = args.act + (size_t)(lane & 15) * K + (lane >> 4) * 16;
  const v4i zero = {0, 0, 0, 0};
  v4i c = zero;

  int kt = kt0;
  for (; kt + U <= kt1; kt += U) {
    v4i bf[U], af[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      bf[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wb + (size_t)(kt + u) * 1024));
#pragma unroll
    for (int u = 0; u < U; ++u) af[u] = arow ? ld16(ab + (kt + u) * 64) : zero;
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
    v4i afr = arow ? ld16(ab + kt * 64) : zero;
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
  const int t = threadIdx.x;
  if (t >= 256) return;
  const int v = t >> 6, L = t & 63;
  const int i = 4 * (L >> 4) + v;
  const int n = nt * 16 + (L & 15);
  if (i >= M) return;
  float y;
  if (PER_BLOCK) {
    float facc = 0.0f;
    for (int b = 0; b < nb; ++b) {
      const float adv = args.sa[(size_t)i * nb + b] * kInv127;
      facc = fmaf((float)lds[b * 256 + t], adv, facc);
    }
    y = facc * seg.ws[n];
  } else {
    int acc = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) acc += lds[w * 256 + t];
    const float ad = args.sa[i] * kInv127;
    y = (float)acc * ad * seg.ws[n];
  }
  seg.out[(size_t)i * seg.n + n] = f32_to_bf16(y);
  if (seg.out_f32) seg.out_f32[(size_t)i * seg.n + n] = y;
}

// ---------------------------------------------------------------------------
// tiled: M > 16
// ---------------------------------------------------------------------------
template <int BM, int BN, bool PER_BLOCK>
__global__ __launch_bounds__(256) void k_linear_tiled(LinArgs args, int gm, int gn) {
  constexpr int WM = BM / 2, WN = BN / 2, MI = WM / 16, NI = WN / 16;
  __shared__ __attribute__((aligned(16))) int8_t lds_a[2][BM * 64];
  __shared__ __attribute__((aligned(16))) int8_t lds_b[2][BN * 64];

  // XCD-aware order: hardware deals workgroups round-robin over 8 XCDs; give
  // XCD x a contiguous range of work so all m-tiles of an n-panel share one
  // L2 and each weight panel is fetched from HBM once.
  const int total = gm * gn;
  int work = blockIdx.x;
  if ((total & 7) == 0) work = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
  const int mt = work % gm, ntg = work / gm;

  // n-tiles of BN rows over the concatenated segments
  int s = 0, nt_in = ntg;
  for (int q = 0; q < args.nseg; ++q) {
    const int tiles = (args.seg[q].n + BN - 1) / BN;
    if (nt_in < tiles) { s = q; break; }
    nt_in -= tiles;
  }
  const LinSeg& seg = args.seg[s];
  const int N = seg.n, K = args.K, K64 = K >> 6, M = args.M;
  const int m0 = mt * BM, n0 = nt_in * BN;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int fpb = args.block >> 6, nb = K / args.block;
  const v4i zero = {0, 0, 0, 0};

  constexpr int CA = (BM * 4 + 255) / 256;  // 16-byte A chunks per thread
  constexpr int CB = (BN * 4 + 255) / 256;
  v4i ra[CA], rb[CB];

  auto gload = [&](int kt) {
#pragma unroll
    for (int j = 0; j < CA; ++j) {
      const int c = tid + j * 256;
      if (c < BM * 4) {
        const int m = c >> 2, kc = c & 3;
        const int row = m0 + m;
        ra[j] = row < M ? ld16(args.act + (size_t)row * K + kt * 64 + kc * 16) : zero;
      }
    }
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const int c = tid + j * 256;
      if (c < BN * 4) {
        const int f = c >> 6, l = c & 63;
        const int nrow = n0 + f * 16;
        rb[j] = nrow < N ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(
                               seg.w + ((size_t)(nrow >> 4) * K64 + kt) * 1024 + l * 16))
                         : zero;
      }
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < CA; ++j) {
      const int c = tid + j * 256;
      if (c < BM * 4) {
        const int m = c >> 2, kc = c & 3;
        *reinterpret_cast<v4i*>(&lds_a[buf][((m >> 4) * 64 + kc * 16 + (m & 15)) * 16]) = ra[j];
      }
    }
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const int c = tid + j * 256;
      if (c < BN * 4) *reinterpret_cast<v4i*>(&lds_b[buf][c * 16]) = rb[j];
    }
  };

  v4i acc[MI][NI];
  float facc[MI][NI][4];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      acc[mi][ni] = zero;
#pragma unroll
      for (int v = 0; v < 4; ++v) facc[mi][ni][v] = 0.0f;
    }

  gload(0);
  lstore(0);
  __syncthreads();
  int buf = 0;
  for (int kt = 0; kt < K64; ++kt) {
    if (kt + 1 < K64) gload(kt + 1);
    v4i a[MI], b[NI];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
      a[mi] = *reinterpret_cast<const v4i*>(&lds_a[buf][((wm * MI + mi) * 64 + lane) * 16]);
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
      b[ni] = *reinterpret_cast<const v4i*>(&lds_b[buf][((wn * NI + ni) * 64 + lane) * 16]);
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = mfma16x16x64(a[mi], b[ni], acc[mi][ni]);
    if (PER_BLOCK && (((kt + 1) & (fpb - 1)) == 0)) {
      const int blk = kt / fpb;
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = m0 + (wm * MI + mi) * 16 + 4 * (lane >> 4) + v;
          const float adv = row < M ? args.sa[(size_t)row * nb + blk] * kInv127 : 0.0f;
#pragma unroll
          for (int ni = 0; ni < NI; ++ni) facc[mi][ni][v] = fmaf((float)acc[mi][ni][v], adv, facc[mi][ni][v]);
        }
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = zero;
      }
    }
    if (kt + 1 < K64) lstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }

#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = m0 + (wm * MI + mi) * 16 + 4 * (lane >> 4) + v;
      if (row >= M) continue;
      const float ad = PER_BLOCK ? 0.0f : args.sa[row] * kInv127;
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        const int col = n0 + (wn * NI + ni) * 16 + (lane & 15);
        if (col >= N) continue;
        float y;
        if (PER_BLOCK) y = facc[mi][ni][v] * seg.ws[col];
        else y = (float)acc[mi][ni][v] * ad * seg.ws[col];
        seg.out[(size_t)row * N + col] = f32_to_bf16(y);
        if (seg.out_f32) seg.out_f32[(size_t)row * N + col] = y;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------
template <int BM, int BN>
static hipError_t launch_tiled(const LinArgs& a, int per_block, hipStream_t st) {
  int gn = 0;
  for (int q = 0; q < a.nseg; ++q) gn += (a.seg[q].n + BN - 1) / BN;
  const int gm = (a.M + BM - 1) / BM;
  dim3 g(gm * gn), b(256);
  if (per_block) hipLaunchKernelGGL((k_linear_tiled<BM, BN, true>), g, b, 0, st, a, gm, gn);
  else hipLaunchKernelGGL((k_linear_tiled<BM, BN, false>), g, b, 0, st, a, gm, gn);
  return hipGetLastError();
}

hipError_t launch_linear(const LinArgs& a, int per_block, hipStream_t st) {
  if (a.M <= 0) return hipSuccess;
  if (a.M <= 16) {
    int tiles = 0;
    for (int q = 0; q < a.nseg; ++q) tiles += a.seg[q].n / 16;
    constexpr int WAVES = 4;
    const int nb = a.K / a.block;
    const size_t lds = (size_t)(per_block ? nb : WAVES) * 256 * sizeof(int);
    dim3 g(tiles), b(WAVES * 64);
    if (per_block) hipLaunchKernelGGL((k_linear_skinny<WAVES, true, 8>), g, b, lds, st, a);
    else hipLaunchKernelGGL((k_linear_skinny<WAVES, false, 8>), g, b, lds, st, a);
    return hipGetLastError();
  }
  // prefer the largest M tile that still yields >= 256 workgroups (one per CU)
  int gn128 = 0;
  for (int q = 0; q < a.nseg; ++q) gn128 += (a.seg[q].n + 127) / 128;
  const int g128 = ((a.M + 127) / 128) * gn128;
  const int g64 = ((a.M + 63) / 64) * gn128;
  if (a.M > 64 && g128 >= 256) return launch_tiled<128, 128>(a, per_block, st);
  if (a.M > 32 && g64 >= 128) return launch_tiled<64, 128>(a, per_block, st);
  return launch_tiled<32, 128>(a, per_block, st);
}

}  // namespace bq
