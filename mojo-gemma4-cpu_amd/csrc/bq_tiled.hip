// bq_tiled.hip -- LDS-tiled v_mfma_i32_16x16x64_i8 GEMM for many rows:
// dense prefill linears (butterquant/gemm.mojo:114-243 at large M) and the
// grouped MoE projections at prefill (butterquant_kernels/moe.mojo:25-295).
//
// One template, three modes sharing the main loop:
//   DENSE   : C = act[M,K] x W[N,K]^T, per-row or per-block epilogue
//   GATE_UP : rows gathered by route token, B tile = 64 gate + 64 up rows of
//             the expert, epilogue bucket = bf16(gelu(g) * u)
//   DOWN    : rows = the expert's bucket records, per-block drains (B = 64),
//             epilogue y[rec, n] = (facc * ws[n]) * route_w
//
// Pipeline: WM x WN waves, K advanced in stages of 64 bytes.
// Operands move global -> LDS directly (global_load_lds_dwordx4, no VGPR
// staging) into a ring of LDS stages: loads for the next ring-1 stages are
// in flight while one stage is multiplied.  Every DMA instruction moves one 1 KiB
// MFMA fragment (lane L's 16 bytes land at L*16): A fragments gather 16 rows
// x 64 K of the activation, B fragments are contiguous 1 KiB runs of the
// tile16x64 weight layout.
#include <type_traits>

#include "bq_device.hpp"
#include "bq_kernels.hpp"

namespace bq {

enum { MODE_DENSE = 0, MODE_GATE_UP = 1, MODE_DOWN = 2 };

struct TiledArgs {
  LinArgs lin;              // DENSE: segments, activation, scales, M, K, block
  // MoE modes
  const int8_t* a;          // GATE_UP: x_i8 [T, K]; DOWN: bucket_i8 [routes, K]
  const float* a_scale;     // GATE_UP: x_sa [T];   DOWN: bucket_sa [routes, K/block]
  const int32_t* eo;        // expert_offset [E+1]
  const Route* routes;
  const int8_t* w;          // expert weights, tile16x64, expert stride N*K
  const float* ws;          // per-row weight scales, expert stride N
  uint16_t* bucket;         // GATE_UP output [routes, inter] (or null with bi8)
  int8_t* bi8;              // GATE_UP fused block-quant: [routes, inter] codes ...
  float* bsa;               // ... and [routes, inter / 64] block scales (or null)
  float fwht64;             // f32(1/f64(sqrtf(64)))
  float* y;                 // DOWN output [routes, N]
  int E, max_routes, N, K, inter, block;
  int gm, gn;               // grid decomposition: m-tiles, n-tiles
  int order;                // MoE work order (0: n-tile fastest, 1: XCD ranges, 2: m-tile per XCD)
};

// Wait until at most `later` stages of this wave's fragment DMAs (D each)
// are outstanding: s_waitcnt takes an immediate, so dispatch on the count.
template <int D, int NBUF>
__device__ inline void wait_dma(int later) {
  static_assert((NBUF - 2) * D <= 63, "vmcnt field holds 6 bits");
  switch (later) {
#define BQ_WAIT_CASE(n) \
    case n: if constexpr (n <= NBUF - 2) { asm volatile("s_waitcnt vmcnt(%0)" :: "n"(n * D) : "memory"); break; }
    BQ_WAIT_CASE(12) BQ_WAIT_CASE(11) BQ_WAIT_CASE(10) BQ_WAIT_CASE(9) BQ_WAIT_CASE(8)
    BQ_WAIT_CASE(7) BQ_WAIT_CASE(6) BQ_WAIT_CASE(5) BQ_WAIT_CASE(4)
    BQ_WAIT_CASE(3) BQ_WAIT_CASE(2) BQ_WAIT_CASE(1)
#undef BQ_WAIT_CASE
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

// The same, for a wave that issues n (0..DMAX) DMAs per stage.
template <int DMAX, int NBUF>
__device__ inline void wait_dma_n(int later, int n) {
  if constexpr (DMAX > 0) {
    if (n == DMAX) { wait_dma<DMAX, NBUF>(later); return; }
    wait_dma_n<DMAX - 1, NBUF>(later, n);
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

// 32-bit LDS address of a __shared__ object (what M0 takes for LDS DMA)
__device__ inline uint32_t lds_addr(const int8_t* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) int8_t*)p;
}

// The (m-tile, n-tile) item of this workgroup in the grouped MoE launches
// (grid from moe_grid); false past the last item.  XCD-aware orders: the
// hardware places workgroup b on XCD b % 8.  Order 1: XCD x takes the
// contiguous work range [x*G/8, (x+1)*G/8) of (m-tile major, n-tile minor)
// items, so the n-tiles sharing one gathered activation tile, and the
// consecutive m-tiles of one expert sharing its weight tiles, meet in the
// same L2.  Order 2: an m-tile's n-tiles on one XCD, consecutive m-tiles on
// different XCDs.  Order 0: workgroup order.
__device__ inline bool moe_item(const TiledArgs& args, int& mt, int& nt) {
  const int total = args.gm * args.gn, per_xcd = (int)gridDim.x >> 3;
  if (args.order == 1) {
    const int work = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
    mt = work / args.gn; nt = work % args.gn;
    return work < total;
  }
  if (args.order == 2) {
    const int xcd = (int)(blockIdx.x & 7), k = (int)(blockIdx.x >> 3);
    mt = xcd + 8 * (k / args.gn); nt = k % args.gn;
    return mt < args.gm;
  }
  const int work = (int)blockIdx.x;
  mt = work / args.gn; nt = work % args.gn;
  return work < total;
}

// A stage covers 128 bytes of K (two MFMA k-steps of 64).
//   A: BM/8 DMAs, each 8 rows x 128 B, so every DMA reads whole 128-byte
//      lines (a DMA of 16 rows x 64 B -- the raw MFMA fragment -- moves a
//      third as fast).  Inside a 1 KiB block (rows 8b..8b+7) the 16-byte
//      chunk c of row r sits at slot r*8 + (c ^ r ^ (b & 1)): the swizzle
//      keeps the MFMA operand reads (16 rows x one chunk) free of LDS bank
//      conflicts.
//   B: two contiguous 1 KiB tile16x64 fragments per 16-row strip.
// When K/64 is odd the last stage holds one k-step; its second-half DMAs are
// pointed at the first half (valid memory, never read).
// KSP = 2 (dense per-row tiles only): the workgroup holds two groups of WM x WN
// waves, each with its own LDS ring, taking the first and the second half of
// the K stages; the second group's exact int32 accumulators are added to the
// first's through LDS before the epilogue.  Twice the waves and bytes in
// flight per CU for the same tile, so one group computes while the other
// waits for its operands.
template <int MODE, int BM, int BN, int WM, int WN, bool PER_BLOCK, int NBUF, int KSP = 1,
          int MF = 16>
__global__ __launch_bounds__(64 * WM * WN * KSP) void k_tiled(TiledArgs args) {
  static_assert(KSP == 1 || (KSP == 2 && MODE == MODE_DENSE && !PER_BLOCK), "split-K: dense per-row");
  static_assert(MF == 16 || MF == 32, "MFMA tile: 16x16x64 or 32x32x32");
  constexpr int KS = 2;                                     // k-steps per stage
  constexpr int NW = WM * WN, NT = 64 * NW * KSP;           // waves per K group, threads
  constexpr int MI = BM / (MF * WM), NI = BN / (MF * WN);   // MF x MF tiles per wave
  constexpr int EV = MF * MF / 64;                          // accumulator elements per lane
  constexpr int KH = MF == 32 ? 2 : 1;                      // MFMAs per tile and k-step of 64
  constexpr int SPT = MF / 16;                              // 16-row weight strips per tile
  using acc_t = std::conditional_t<MF == 32, v16i, v4i>;
  static_assert(MI >= 1 && NI >= 1 && MI * MF * WM == BM && NI * MF * WN == BN &&
                (MODE != MODE_GATE_UP || NI % 2 == 0), "tile shape");
  constexpr int FA = BM / 8, FB = (BN / 16) * KS;           // 1 KiB DMAs per stage
  constexpr int D = (FA + FB + NW - 1) / NW;                // DMAs per wave per stage
  constexpr int REM = (FA + FB) % NW;  // when nonzero, waves >= REM issue D - 1
  constexpr int A_STAGE = FA * 1024, B_STAGE = FB * 1024;
  // ring of NBUF LDS stages (NBUF-1 stages of DMA in flight)
  __shared__ __attribute__((aligned(16))) int8_t abuf_all[KSP][NBUF][A_STAGE];
  __shared__ __attribute__((aligned(16))) int8_t bbuf_all[KSP][NBUF][B_STAGE];
  static_assert(KSP == 1 || BM * BN * 4 <= NBUF * B_STAGE, "split-K partials fit the B ring");
  // per-block activation scales of the tile's rows, times 1/127 (dynamic
  // LDS of BM * K/block floats, sized at launch)
  extern __shared__ float lds_sa[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int gwave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = gwave / NW;       // K group (0 unless KSP = 2)
  const int wave = gwave % NW;     // wave within the K group
  const int wm = wave / WN, wn = wave % WN;
  auto& abuf_ = abuf_all[kg];
  auto& bbuf_ = bbuf_all[kg];
  const bool full_d = REM == 0 || wave < REM;  // wave-uniform

  // ---- work item -------------------------------------------------------
  int K, n0 = 0, r0 = 0, r1 = 0, e = 0;
  LinSeg segv{};
  const LinSeg* seg = &segv;
  const int8_t* wbase;
  if constexpr (MODE == MODE_DENSE) {
    const int total = args.gm * args.gn;
    int work = blockIdx.x;
    if ((total & 7) == 0) work = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
    const int mt = work % args.gm;
    int nt_in = work / args.gm;
    // the segment selected by value: the three segments' fields are read in
    // one batch of scalar loads (indexing seg[s] by address would take a
    // second, dependent kernel-argument round trip)
    const LinSeg s0 = args.lin.seg[0], s1 = args.lin.seg[1], s2 = args.lin.seg[2];
    const int t0 = (s0.n + BN - 1) / BN, t1 = (s1.n + BN - 1) / BN;
    const bool in1 = args.lin.nseg > 1 && nt_in >= t0;
    const bool in2 = args.lin.nseg > 2 && nt_in >= t0 + t1;
    nt_in -= in2 ? t0 + t1 : in1 ? t0 : 0;
    segv.w = in2 ? s2.w : in1 ? s1.w : s0.w;
    segv.ws = in2 ? s2.ws : in1 ? s1.ws : s0.ws;
    segv.out = in2 ? s2.out : in1 ? s1.out : s0.out;
    segv.out_f32 = in2 ? s2.out_f32 : in1 ? s1.out_f32 : s0.out_f32;
    segv.n = in2 ? s2.n : in1 ? s1.n : s0.n;
    segv.tile0 = in2 ? s2.tile0 : in1 ? s1.tile0 : s0.tile0;
    K = args.lin.K;
    r0 = mt * BM;
    r1 = min(args.lin.M, r0 + BM);
    n0 = nt_in * BN;
    wbase = seg->w;
  } else {
    int mt, nt;
    if (!moe_item(args, mt, nt)) return;
    if (!find_mtile(args.eo, args.E, BM, mt, args.max_routes, e, r0, r1)) return;
    K = args.K;
    n0 = nt * (MODE == MODE_GATE_UP ? BN / 2 : BN);
    wbase = args.w + (size_t)e * args.N * K;
  }
  const int K64 = K >> 6;
  const int blk = MODE == MODE_DENSE ? args.lin.block : args.block;
  const int fpb = blk >> 6, nb = K / blk;
  const int nstages = (K64 + 1) / 2;
  const int tail = nstages - 1;  // the stage that may hold one k-step
  const bool odd = K64 & 1;

  // ---- this wave's DMAs: DMA wave + NW*d, d < D (or D - 1) ---------------
  const int8_t* src[D];
  int dst_off[D];
  bool is_a[D], hi[D];  // hi: reads the second k-step of the stage
  // A DMAs whose 8 rows all lie past the tile's last record are not issued
  // (their LDS rows feed only outputs that are never stored)
  bool skip[D];
  const int live_rows = __builtin_amdgcn_readfirstlane(r1 - r0);
  int n_issue = full_d ? D : D - 1;  // DMAs this wave issues per stage
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int f = min(wave + NW * d, FA + FB - 1);  // the clamped slot is never issued
    skip[d] = f < FA && f * 8 >= live_rows;
    if (skip[d] && (d < D - 1 || full_d)) --n_issue;
    if (f < FA) {
      const int r = lane >> 3, c = (lane & 7) ^ r ^ (f & 1);  // this lane's row, chunk
      int row = r0 + f * 8 + r;
      if (row >= r1) row = r0;  // rows past the tile end are never stored
      const int8_t* rp;
      if constexpr (MODE == MODE_DENSE) rp = args.lin.act + (size_t)row * K;
      else if constexpr (MODE == MODE_GATE_UP) rp = args.a + (size_t)args.routes[row].token * K;
      else rp = args.a + (size_t)row * K;
      src[d] = rp + c * 16;
      dst_off[d] = f * 1024;
      is_a[d] = true;
      hi[d] = c >= 4;
    } else {
      const int g = f - FA;
      const int ks = g & 1, nsub = g >> 1;
      int wrow;
      bool ok;
      if constexpr (MODE == MODE_GATE_UP) {
        const int half = BN / 32;
        wrow = nsub < half ? n0 + nsub * 16 : args.inter + n0 + (nsub - half) * 16;
        ok = (n0 + (nsub % half) * 16) < args.inter;
      } else if constexpr (MODE == MODE_DENSE) {
        wrow = n0 + nsub * 16;
        ok = wrow < seg->n;
      } else {
        wrow = n0 + nsub * 16;
        ok = wrow < args.N;
      }
      if (!ok) wrow = 0;  // subtiles past N are never stored
      src[d] = wbase + ((size_t)(wrow >> 4) * K64 + ks) * 1024 + lane * 16;
      dst_off[d] = g * 1024;
      is_a[d] = false;
      hi[d] = ks == 1;
    }
  }

  if constexpr (PER_BLOCK) {
    const float* sc = MODE == MODE_DENSE ? args.lin.sa : args.a_scale;
    for (int i = tid; i < BM * nb; i += NT) {
      const int m = i / nb, b = i % nb;
      lds_sa[i] = r0 + m < r1 ? sc[(size_t)(r0 + m) * nb + b] * kInv127 : 0.0f;
    }
  }

  // The DMA is issued from inline asm so the compiler does not track it:
  // the only waits are the explicit vmcnt waits of the main loop (the
  // compiler would otherwise wait for every DMA before any LDS read).
  auto issue = [&](int8_t* abuf, int8_t* bbuf, int st) {
    const uint32_t a_lds = lds_addr(abuf), b_lds = lds_addr(bbuf);
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (d == D - 1 && !full_d) break;
      if (skip[d]) continue;
      // stage st starts at K byte 128*st (A) / fragment 2*st (B); in a
      // one-step tail stage the second-half reads fall back to the first half
      const int back = (odd && st == tail && hi[d]) ? (is_a[d] ? 64 : 1024) : 0;
      const int8_t* g = src[d] + (is_a[d] ? (size_t)st * 128 : (size_t)st * 2048) - back;
      const uint32_t l = __builtin_amdgcn_readfirstlane((is_a[d] ? a_lds : b_lds) + dst_off[d]);
      // M0 holds the LDS destination; one wait state separates its write from
      // the DMA (the M0 -> LDS-DMA hazard).  These kernels use M0 for nothing
      // else, so clobbering it is safe.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
      // weights are streamed once: non-temporal (measured 7.2 vs 6.0 TB/s
      // for HBM-sourced DMA streams); activations are re-read by other tiles
      if (is_a[d])
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                     :: "s"(l), "v"(g) : "memory", "m0");
      else
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt"
                     :: "s"(l), "v"(g) : "memory", "m0");
#pragma clang diagnostic pop
    }
  };

  // first 16-row weight strip (of the stage's BN/16) of this wave's tile ni;
  // a 32-wide tile spans strips bstrip and bstrip + 1
  int bstrip[NI];
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    if constexpr (MODE == MODE_GATE_UP) {
      const int half = BN / (2 * MF), hn = NI / 2;  // gate tiles [0, half), up [half, 2*half)
      bstrip[ni] = (ni < hn ? wn * hn + ni : half + wn * hn + (ni - hn)) * SPT;
    } else {
      bstrip[ni] = (wn * NI + ni) * SPT;
    }
  }
  // accumulator element v of tile (mi, .): row within the block tile; the
  // lane's column within tile ni is bstrip[ni] * 16 + (lane & (MF - 1))
  auto row_in = [&](int mi, int v) {
    if constexpr (MF == 16) return (wm * MI + mi) * 16 + 4 * (lane >> 4) + v;
    else return (wm * MI + mi) * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
  };
  const int lcol = lane & (MF - 1);

  // ---- epilogue operands, fetched now so their (dependent) loads are long
  // done at the epilogue: per output row an activation scale (x 1/127) or a
  // route weight -- thread t holds row t's, staged through LDS for the
  // epilogue -- and per output column the weight scale
  static_assert(NT >= BM, "one thread per tile row");
  float my_rs = 0.0f;
  if (tid < BM) {
    int row = r0 + tid;
    row = row < r1 ? row : r0;
    if constexpr (MODE == MODE_DENSE) my_rs = PER_BLOCK ? 0.0f : args.lin.sa[row] * kInv127;
    else if constexpr (MODE == MODE_GATE_UP) my_rs = args.a_scale[args.routes[row].token] * kInv127;
    else my_rs = args.routes[row].weight;
  }
  float ep_col[NI];
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    if constexpr (MODE == MODE_GATE_UP) {
      constexpr int hn = NI / 2;
      const int col = min(n0 + (wn * hn + (ni % hn)) * MF + lcol, args.inter - 1);
      ep_col[ni] = args.ws[(size_t)e * args.N + (ni < hn ? col : args.inter + col)];
    } else if constexpr (MODE == MODE_DENSE) {
      ep_col[ni] = seg->ws[min(n0 + bstrip[ni] * 16 + lcol, seg->n - 1)];
    } else {
      ep_col[ni] = args.ws[(size_t)e * args.N + min(n0 + bstrip[ni] * 16 + lcol, args.N - 1)];
    }
  }

  acc_t acc[MI][NI];
  float facc[MI][NI][EV];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      acc[mi][ni] = acc_t{};
#pragma unroll
      for (int v = 0; v < EV; ++v) facc[mi][ni][v] = 0.0f;
    }

  auto row_of = [&](int mi, int v) { return r0 + row_in(mi, v); };

  // LDS offset of this lane's A operand under the block swizzle: row
  // m = (wm*MI+mi)*MF + lane%MF, 16-byte chunk ks*4 + lane/16 (16x16x64) or
  // ks*4 + kh*2 + lane/32 (32x32x32, K half kh).  The swizzle term depends
  // on the lane only (m & 7 and (m >> 3) & 1 do not change with mi), so tile
  // mi adds the constant mi * MF * 128.
  int a_off[KS][KH];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int kh = 0; kh < KH; ++kh) {
      const int m = wm * MI * MF + (lane & (MF - 1));
      const int c = MF == 16 ? ks * 4 + (lane >> 4) : ks * 4 + kh * 2 + (lane >> 5);
      const int b = m >> 3, r = m & 7;
      a_off[ks][kh] = b * 1024 + r * 128 + ((c ^ r ^ (b & 1)) * 16);
    }
  // LDS offset (within the stage's B buffer, less ks * 1024) of this lane's B
  // operand of tile ni: 16x16x64 lane L = tile16x64 fragment lane L of strip
  // bstrip; 32x32x32 half kh: column L%32 (strip bstrip + (L/16)%2), K chunk
  // 2*kh + L/32 of the fragment
  int b_off[NI][KH];
#pragma unroll
  for (int ni = 0; ni < NI; ++ni)
#pragma unroll
    for (int kh = 0; kh < KH; ++kh) {
      if constexpr (MF == 16) {
        b_off[ni][kh] = bstrip[ni] * 2048 + lane * 16;
      } else {
        const int strip = bstrip[ni] + ((lane >> 4) & 1);
        b_off[ni][kh] = strip * 2048 + ((kh * 2 + (lane >> 5)) * 16 + (lane & 15)) * 16;
      }
    }

  // A wave whose MF*MI rows all lie past the tile's last record (a partial
  // m-tile of an expert with few records) still issues its DMAs and meets
  // every barrier, but skips its MFMAs: nothing it would compute is stored.
  // Within a busy wave, tiles mi whose rows all lie past it are skipped too.
  const int live = r1 - r0;
  const bool busy = wm * MI * MF < live;

  auto compute = [&](const int8_t* abuf, const int8_t* bbuf, int st) {
    if constexpr (MODE != MODE_DENSE) {
      if (!busy) return;
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks == 1 && odd && st == tail) break;
#pragma unroll
      for (int kh = 0; kh < KH; ++kh) {
        v4i a[MI], b[NI];
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
          a[mi] = *reinterpret_cast<const v4i*>(&abuf[a_off[ks][kh] + mi * MF * 128]);
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
          b[ni] = *reinterpret_cast<const v4i*>(&bbuf[b_off[ni][kh] + ks * 1024]);
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
          if (MI > 1 && (wm * MI + mi) * MF >= live) continue;  // wave-uniform
#pragma unroll
          for (int ni = 0; ni < NI; ++ni) {
            if constexpr (MF == 16) acc[mi][ni] = mfma16x16x64(a[mi], b[ni], acc[mi][ni]);
            else acc[mi][ni] = mfma32x32x32(a[mi], b[ni], acc[mi][ni]);
          }
        }
      }
      if constexpr (PER_BLOCK) {
        const int kt = st * KS + ks;
        if (((kt + 1) & (fpb - 1)) == 0) {
          const int b_idx = kt / fpb;
#pragma unroll
          for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
            for (int v = 0; v < EV; ++v) {
              const float adv = lds_sa[row_in(mi, v) * nb + b_idx];
#pragma unroll
              for (int ni = 0; ni < NI; ++ni)
                facc[mi][ni][v] = fmaf((float)acc[mi][ni][v], adv, facc[mi][ni][v]);
            }
#pragma unroll
            for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = acc_t{};
          }
        }
      }
    }
  };

  // ---- main loop: a ring of NBUF LDS stages, NBUF-1 in flight -------------
  // iteration s: wait for this wave's DMAs of stage s (those of the later
  // stages already issued may stay outstanding), barrier (all waves' stage-s
  // data has landed and every wave has finished reading stage s-1), refill
  // stage s-1's buffer with stage s+NBUF-1, multiply stage s.  The ring is
  // unrolled NBUF times so every buffer index is a compile-time constant.
  // K group kg runs stages [s_lo, s_lo + n_loc); both groups make the same
  // number of iterations (and barriers), a group with one stage fewer idles
  const int n_iter = (nstages + KSP - 1) / KSP;
  const int s_lo = kg * n_iter;
  const int n_loc = min(nstages - s_lo, n_iter);
  for (int p = 0; p < NBUF - 1 && p < n_loc; ++p) issue(abuf_[p], bbuf_[p], s_lo + p);
  for (int s0 = 0; s0 < n_iter; s0 += NBUF) {
#pragma unroll
    for (int i = 0; i < NBUF; ++i) {
      const int sl = s0 + i;
      if (sl >= n_iter) break;
      const int later = max(0, min(NBUF - 2, n_loc - 1 - sl));
      wait_dma_n<D, NBUF>(later, n_issue);
      lds_barrier();
      if (sl + NBUF - 1 < n_loc)
        issue(abuf_[(i + NBUF - 1) % NBUF], bbuf_[(i + NBUF - 1) % NBUF], s_lo + sl + NBUF - 1);
      if (sl < n_loc) compute(abuf_[i], bbuf_[i], s_lo + sl);
    }
  }
  // the row scales into the first B ring (free once every wave is done with
  // the last stage; the split-K partials use the second group's ring)
  float* s_rs = reinterpret_cast<float*>(&bbuf_all[0][0][0]);
  if constexpr (KSP == 1) {
    lds_barrier();
    if (tid < BM) s_rs[tid] = my_rs;
    lds_barrier();
  }
  if constexpr (KSP == 2) {
    // the second group's accumulators into its B ring, added by the first
    int* part = reinterpret_cast<int*>(&bbuf_all[1][0][0]);
    lds_barrier();
    if (tid < BM) s_rs[tid] = my_rs;
    if (kg == 1) {
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
          *reinterpret_cast<acc_t*>(&part[(((wave * MI + mi) * NI + ni) * 64 + lane) * EV]) = acc[mi][ni];
    }
    lds_barrier();
    if (kg == 1) return;
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        acc[mi][ni] += *reinterpret_cast<const acc_t*>(&part[(((wave * MI + mi) * NI + ni) * 64 + lane) * EV]);
  }

  // ---- epilogue ----------------------------------------------------------
  // fused block-quant (GATE_UP with bi8): the tile's bf16 bucket values go to
  // an LDS tile [BM][BN/2] over the A ring (free once every wave is done with
  // the last stage), then whole 64-column blocks are block-quantized from it
  [[maybe_unused]] uint16_t* qtile = reinterpret_cast<uint16_t*>(&abuf_all[0][0][0]);
  if constexpr (MODE == MODE_GATE_UP) {
    static_assert(BM * (BN / 2) * 2 <= NBUF * A_STAGE, "bucket tile fits the A ring");
  }
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
    for (int v = 0; v < EV; ++v) {
      const int row = row_of(mi, v);
      if (row >= r1) continue;
      if constexpr (MODE == MODE_DENSE) {
        const float ad = s_rs[row - r0];
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
          const int col = n0 + bstrip[ni] * 16 + lcol;
          if (col >= seg->n) continue;
          const float y = PER_BLOCK ? facc[mi][ni][v] * ep_col[ni]
                                    : (float)acc[mi][ni][v] * ad * ep_col[ni];
          seg->out[(size_t)row * seg->n + col] = f32_to_bf16(y);
          if (seg->out_f32) seg->out_f32[(size_t)row * seg->n + col] = y;
        }
      } else if constexpr (MODE == MODE_GATE_UP) {
        const float ad = s_rs[row - r0];
        constexpr int hn = NI / 2;
#pragma unroll
        for (int j = 0; j < hn; ++j) {
          const int col = n0 + (wn * hn + j) * MF + lcol;
          if (col >= args.inter) continue;
          const float g = (float)acc[mi][j][v] * ad * ep_col[j];
          const float u = (float)acc[mi][hn + j][v] * ad * ep_col[hn + j];
          const uint16_t hb = f32_to_bf16(gelu_tanh_f32(g) * u);
          if (args.bi8) qtile[(row - r0) * (BN / 2) + (col - n0)] = hb;
          else args.bucket[(size_t)row * args.inter + col] = hb;
        }
      } else {
        const float rw = s_rs[row - r0];
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
          const int col = n0 + bstrip[ni] * 16 + lcol;
          if (col >= args.N) continue;
          args.y[(size_t)row * args.N + col] = facc[mi][ni][v] * ep_col[ni] * rw;
        }
      }
    }
  }
  if constexpr (MODE == MODE_GATE_UP) {
    if (args.bi8) {
      // 8 lanes per (record, 64-column block), 8 values each, as bq_block_quant
      lds_barrier();
      const int live = r1 - r0, nblk = min(BN / 2, args.inter - n0) / 64;
      const int units = live * nblk, nb_all = args.inter / 64;
      for (int u0 = gwave * 8; u0 < units; u0 += NW * KSP * 8) {
        const int uu = u0 + (lane >> 3);
        const int u = min(uu, units - 1);  // groups past the end redo the last unit, unstored
        const int r = u / nblk, b = u - r * nblk, i = lane & 7;
        const v4i raw = *reinterpret_cast<const v4i*>(&qtile[r * (BN / 2) + b * 64 + i * 8]);
        float v[8];
        bf16x8_to_f32(raw, v);
        uint32_t w[2];
        const float m = block_quant_lanes<8>(v, true, args.fwht64, w);
        if (uu < units) {
          const size_t rec = (size_t)(r0 + r), col = (size_t)(n0 + b * 64 + i * 8);
          typedef uint32_t u2 __attribute__((ext_vector_type(2)));
          *reinterpret_cast<u2*>(args.bi8 + rec * args.inter + col) = u2{w[0], w[1]};
          if (i == 0) args.bsa[rec * nb_all + (n0 >> 6) + b] = m;
          if (args.bucket) *reinterpret_cast<v4i*>(args.bucket + rec * args.inter + col) = raw;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Down projection with the weights streamed through registers (K = inter, at
// most 64 * KMAX; per-block scales with block 64).  Persistent: one
// workgroup per CU walks a contiguous range of (m-tile, n-tile) items, m-tile
// major, so consecutive items mostly share their m-tile.
//
// Activations: the m-tile's whole block -- BM records x K bytes in the A
// layout of k_tiled, one 128-byte stage after another -- is DMA'd into LDS
// when the item's m-tile changes, with its per-block scales and route
// weights.  Weights: each of the 8 waves owns NI 16-column strips of the
// item's n-tile and holds all K of them in VGPRs; they are reloaded with the
// next item's during the item's last m-subtile pair, each k-step's registers
// as soon as that pair has multiplied them, so the bytes in flight per CU are
// bounded by the register file (8 waves x NI x K/64 KiB), not by LDS.
//
// m-subtile pairs are the outer loop: a pair runs its k-steps in order, then
// stores its records, so only two subtiles' accumulators are live (no
// spills).  Every k-step is one drain block: its int32 product (an MFMA from
// zero) is added to the f32 accumulator as fmaf(f32(dot), a_scale/127, acc),
// k-steps in ascending order -- the per-block order of k_tiled's DOWN mode.
// The product is taken transposed, D = W x A^T (the weight strip as the
// MFMA's A operand, 16 records as its B): lane L holds columns 4 (L/16) ..
// +3 of the strip for record L % 16, so a drain needs one activation scale
// per lane (a 4-byte LDS read, not 16) and a record's four y values are one
// 16-byte store.  The integer dot of each (record, column) is the same.
constexpr int kBregMaxExperts = 256;

template <int MI, int NI, int KMAX>
__global__ __launch_bounds__(512) void k_down_breg(TiledArgs args) {
  constexpr int NW = 8, BM = 16 * MI, BN = NW * NI * 16, FA = BM / 8;
  constexpr int SPT = (BM * KMAX + 64 * NW - 1) / (64 * NW);  // scales per thread
  static_assert(MI % 2 == 0 && BM <= 64 * NW, "m-subtile pairs; one route weight per thread");
  __shared__ __attribute__((aligned(16))) int8_t abuf[(KMAX + 1) / 2 * FA * 1024];
  __shared__ __attribute__((aligned(16))) float sa[KMAX * BM];  // [k-step][record] x 1/127
  __shared__ float s_rw[BM];                                     // route weights
  __shared__ int s_tp[kBregMaxExperts + 1];  // m-tiles before each expert (exclusive prefix)

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const v4i zero = {0, 0, 0, 0};
  const int E = args.E, K = args.K, K64 = K >> 6, nstages = (K64 + 1) / 2, N = args.N;
  const bool odd = K64 & 1;

  // ---- m-tile table: as find_mtile enumerates them ------------------------
  if (wave == 0) {
    int carry = 0;
    for (int base = 0; base < E; base += 64) {
      const int ex = base + lane;
      const int tiles = ex < E ? max(0, (args.eo[ex + 1] - args.eo[ex] + BM - 1) / BM) : 0;
      int inc = wave_incl_scan(tiles);
      if (ex < E) s_tp[ex] = carry + inc - tiles;
      carry += __shfl(inc, 63, kWave);
    }
    if (lane == 0) s_tp[E] = carry;
  }
  lds_barrier();
  const long items = (long)s_tp[E] * args.gn;
  const int first = (int)(items * blockIdx.x / gridDim.x);
  const int last = (int)(items * (blockIdx.x + 1) / gridDim.x);
  if (first >= last) return;

  // item -> expert (the last e with s_tp[e] <= mt), n-strip base
  auto expert_of = [&](int mt) {
    int lo = 0, hi = E;  // s_tp[lo] <= mt < s_tp[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_tp[mid] <= mt) lo = mid; else hi = mid;
    }
    return __builtin_amdgcn_readfirstlane(lo);
  };
  auto strips = [&](int item, const int8_t*& wb, int& ns0) {
    const int mt = item / args.gn, nt = item - mt * args.gn;
    wb = args.w + (size_t)expert_of(mt) * N * K;
    ns0 = nt * (BN / 16) + wave * NI;
  };
  // a uniform (scalar) strip base plus one 32-bit lane offset per load
  const uint32_t lane16 = (uint32_t)lane * 16u;
  auto load_strip = [&](const int8_t* wb, int ns0, int j, int ks) {
    const int ns = (ns0 + j) * 16 < N ? ns0 + j : 0;  // strips past N are never stored
    const uint64_t ob = (uint64_t)(wb - args.w) + ((uint64_t)ns * K64 + min(ks, K64 - 1)) * 1024u;
    const uint64_t ou = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(ob >> 32)) << 32) |
                        __builtin_amdgcn_readfirstlane((uint32_t)ob);
    // streamed once: non-temporal
    return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(args.w + ou + lane16));
  };

  // ---- the first item's weights ------------------------------------------
  v4i bw[KMAX][NI];
  {
    const int8_t* wb;
    int ns0;
    strips(first, wb, ns0);
#pragma unroll
    for (int ks = 0; ks < KMAX; ++ks)
#pragma unroll
      for (int j = 0; j < NI; ++j) bw[ks][j] = load_strip(wb, ns0, j, ks);
  }

  // per-column weight scales of an item's strips: lane L's columns
  // 4 (L/16) .. +3 of each strip (the transposed product's layout)
  float ep4[NI][4];
  auto load_ep4 = [&](int item) {
    const int mt = item / args.gn, nt = item - mt * args.gn;
    const int e = expert_of(mt), ns0 = nt * (BN / 16) + wave * NI;
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        ep4[j][v] = args.ws[(size_t)e * N + min((ns0 + j) * 16 + 4 * (lane >> 4) + v, N - 1)];
  };
  load_ep4(first);

  int cur_mt = -1, lds_mt = -1, r0 = 0, r1 = 0, nmi = 0;
  const uint32_t a_lds = lds_addr(abuf);
  for (int item = first; item < last; ++item) {
    const int mt = item / args.gn, nt = item - mt * args.gn;
    const int e = expert_of(mt);
    const int ns0 = nt * (BN / 16) + wave * NI;
    if (mt != cur_mt) {
      // ---- a new m-tile: its activations, scales and route weights -------
      cur_mt = mt;
      r0 = args.eo[e] + (mt - s_tp[e]) * BM;
      r1 = min(min(args.eo[e + 1], r0 + BM), args.max_routes);
      r0 = __builtin_amdgcn_readfirstlane(r0);
      r1 = __builtin_amdgcn_readfirstlane(r1);
      // An m-tile past max_routes (only an expert_offset beyond the route
      // count makes one) multiplies and stores nothing, but its items still
      // run the k-step loop: that is where the next item's weights load.
      nmi = r1 > r0 ? (r1 - r0 + 15) >> 4 : 0;
    }
    if (lds_mt != mt && nmi > 0) {  // wave-uniform
      lds_mt = mt;
      lds_barrier();  // every wave is done with the previous m-tile's LDS
      for (int q = wave; q < nstages * FA; q += NW) {
        const int st = q / FA, f = q % FA;
        const int r = lane >> 3, c = (lane & 7) ^ r ^ (f & 1);
        int row = r0 + f * 8 + r;
        if (row >= r1) row = r0;  // rows past the tile end are never stored
        // a one-step tail stage reads its second half from the first (never used)
        const int back = (odd && st == nstages - 1 && c >= 4) ? 64 : 0;
        const int8_t* g = args.a + (size_t)row * K + st * 128 + c * 16 - back;
        const uint32_t l = __builtin_amdgcn_readfirstlane(a_lds + (uint32_t)q * 1024u);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                     :: "s"(l), "v"(g) : "memory", "m0");
#pragma clang diagnostic pop
      }
      // scales and route weights, loaded unmasked (clamped indices) after
      // the DMAs: waiting for the first of them also retires this wave's
      // DMAs, which return in issue order before it
      const int nsc = BM * K64;
      float sv[SPT];
#pragma unroll
      for (int i = 0; i < SPT; ++i) {
        const int idx = min(tid + 64 * NW * i, nsc - 1);
        const int m = idx / K64, b = idx - m * K64;
        sv[i] = args.a_scale[(size_t)min(r0 + m, r1 - 1) * K64 + b];
      }
      const float rwv = args.routes[min(r0 + tid, r1 - 1)].weight;
#pragma unroll
      for (int i = 0; i < SPT; ++i) {
        const int idx = tid + 64 * NW * i;
        if (idx < nsc) {
          const int m = idx / K64, b = idx - m * K64;
          sa[b * BM + m] = r0 + m < r1 ? sv[i] * kInv127 : 0.0f;
        }
      }
      if (tid < BM) s_rw[tid] = rwv;
      // k-steps K/64 .. KMAX-1 (multiplied without a branch) scale by 0
      for (int i = nsc + tid; i < BM * KMAX; i += 64 * NW) sa[i] = 0.0f;
      asm volatile("" :: "v"(sv[0]));  // the first scale (and so every DMA) has landed
      lds_barrier();
    }
    // the next item's strips (the last item reloads its own: never used)
    const int8_t* wb_n;
    int ns0_n;
    strips(item + 1 < last ? item + 1 : item, wb_n, ns0_n);

    // ---- multiply: m-subtile pairs, each with its k-steps in order; the
    // last pair (or, for an m-tile with no record, a pair that multiplies
    // nothing) reloads each k-step's weight registers with the next item's
    // once it has multiplied them: straight-line, unconditional loads
    auto pair = [&](int mp, auto last_tag) {
      constexpr bool LAST = decltype(last_tag)::value;
      const bool active = mp < nmi;
      float facc[2][NI][4];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) facc[h][j][v] = 0.0f;
      // one branch per pair, none per k-step: k-steps past K/64 multiply
      // stale LDS rows by a zero scale, which leaves facc bit for bit
      // (facc is never -0)
      if (active) {  // wave-uniform
#pragma unroll
        for (int ks = 0; ks < KMAX; ++ks) {
          const int st = ks >> 1, c = (ks & 1) * 4 + (lane >> 4);
          v4i a[2];
          float adv[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int m = (mp + h) * 16 + (lane & 15), bb = m >> 3, r = m & 7;
            a[h] = *reinterpret_cast<const v4i*>(
                &abuf[(st * FA + bb) * 1024 + r * 128 + ((c ^ r ^ (bb & 1)) * 16)]);
            adv[h] = sa[ks * BM + m];
          }
          v4i t[2][NI];
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < NI; ++j) t[h][j] = mfma16x16x64(bw[ks][j], a[h], zero);
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < NI; ++j)
#pragma unroll
              for (int v = 0; v < 4; ++v)
                facc[h][j][v] = fmaf((float)t[h][j][v], adv[h], facc[h][j][v]);
          if constexpr (LAST) {
#pragma unroll
            for (int j = 0; j < NI; ++j) bw[ks][j] = load_strip(wb_n, ns0_n, j, ks);
          }
        }
      } else if constexpr (LAST) {
#pragma unroll
        for (int ks = 0; ks < KMAX; ++ks)
#pragma unroll
          for (int j = 0; j < NI; ++j) bw[ks][j] = load_strip(wb_n, ns0_n, j, ks);
      }
      // y[rec, n] = (facc * ws[n]) * route_w of the pair's records
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int row = r0 + (mp + h) * 16 + (lane & 15);
        if (mp + h < nmi && row < r1) {
          const float rw = s_rw[row - r0];
#pragma unroll
          for (int j = 0; j < NI; ++j) {
            const int col = (ns0 + j) * 16 + 4 * (lane >> 4);
            if (col < N)
              *reinterpret_cast<float4*>(&args.y[(size_t)row * N + col]) =
                  float4{facc[h][j][0] * ep4[j][0] * rw, facc[h][j][1] * ep4[j][1] * rw,
                         facc[h][j][2] * ep4[j][2] * rw, facc[h][j][3] * ep4[j][3] * rw};
          }
        }
      }
    };
    const int npair = (nmi + 1) >> 1;
    // (the column scales are waited for once here, before any pair's
    // stores: a wait inside the guarded stores would also wait for them)
    asm volatile("" :: "v"(ep4[0][0]), "v"(ep4[NI - 1][3]));
    for (int p = 0; p + 1 < npair; ++p) pair(2 * p, std::false_type{});
    pair(2 * max(npair - 1, 0), std::true_type{});
    if (item + 1 < last) load_ep4(item + 1);
  }
}

// ---------------------------------------------------------------------------
// Tile configuration: BM x BN output tile, NBUF-stage LDS ring.  Smaller
// rings leave room for several workgroups per CU (more waves to overlap the
// LDS-read -> MFMA -> barrier chain of each); the BQ_TILE_BN and BQ_RING
// switches (Tune) exist for tuning sweeps.
static inline int or_default(int v, int dflt) { return v ? v : dflt; }

constexpr size_t kLdsBytes = 160 * 1024;

template <int MODE, int BM, int BN, int WM, int WN, bool PB, int NBUF, int KSP = 1, int MF = 16>
static bool try_launch(dim3 g, size_t dyn, hipStream_t st, const TiledArgs& t) {
  constexpr size_t ring = (size_t)KSP * NBUF * (BM + BN) * 128;  // 128 bytes of K per stage
  if constexpr (ring > kLdsBytes) {
    return false;  // never instantiated: the ring alone exceeds LDS
  } else {
    if (ring + dyn > kLdsBytes) return false;
    hipLaunchKernelGGL((k_tiled<MODE, BM, BN, WM, WN, PB, NBUF, KSP, MF>), g,
                       dim3(64 * WM * WN * KSP), dyn, st, t);
    return true;
  }
}

// NBUF-stage ring: the largest of {6, 4, 3, 2} stages (at most `nbuf`) that
// fits in LDS next to the per-block scales.  The bytes in flight per CU
// ((NBUF-1) stages) must cover the L2/HBM latency at the MFMA's pace.
template <int MODE, int BM, int BN, int WM, int WN, bool PB, int MF>
static void launch_cfg(int nbuf, dim3 g, size_t dyn, hipStream_t st, const TiledArgs& t) {
  if (nbuf >= 6 && try_launch<MODE, BM, BN, WM, WN, PB, 6, 1, MF>(g, dyn, st, t)) return;
  if (nbuf >= 4 && try_launch<MODE, BM, BN, WM, WN, PB, 4, 1, MF>(g, dyn, st, t)) return;
  if (nbuf >= 3 && try_launch<MODE, BM, BN, WM, WN, PB, 3, 1, MF>(g, dyn, st, t)) return;
  try_launch<MODE, BM, BN, WM, WN, PB, 2, 1, MF>(g, dyn, st, t);
}

// 128/256-wide tiles: 16x16x64 tiles on 8 waves (2 x 4), each owning a
// (BM/2) x (BN/4) block -- two waves per SIMD keep MFMA and LDS reads
// overlapped; 32x32x32 tiles on 4 waves (2 x 2) of (BM/2) x (BN/2), whose
// larger blocks halve the LDS operand reads per product, with two or more
// workgroups per CU for the overlap.
template <int MODE, int BM, bool PB, int MF>
static void launch_bn(int bn, int nbuf, dim3 g, size_t dyn, hipStream_t st, const TiledArgs& t) {
  constexpr int WN = MF == 32 ? 2 : 4;
  if (bn >= 256) launch_cfg<MODE, BM, 256, 2, WN, PB, MF>(nbuf, g, dyn, st, t);
  else launch_cfg<MODE, BM, 128, 2, WN, PB, MF>(nbuf, g, dyn, st, t);
}

template <int MODE, bool PB, int MF>
static void launch_bm_mf(int bm, int bn, int nbuf, dim3 g, size_t dyn, hipStream_t st,
                         const TiledArgs& t) {
  // 256-record m-tiles (MoE): 4 x 2 waves of 64 x 64, one tile per expert for
  // up to 256 routes, so each expert's weights stream from HBM once
  if (bm >= 256) {
    // 256 x 256 (4 x 2 waves of 64 x 128) halves the operand traffic again;
    // the per-block drains' f32 accumulators would not fit next to it
    if constexpr (!PB) {
      if (bn >= 256) { launch_cfg<MODE, 256, 256, 4, 2, PB, MF>(nbuf, g, dyn, st, t); return; }
    }
    launch_cfg<MODE, 256, 128, 4, 2, PB, MF>(nbuf, g, dyn, st, t);
  }
  else if (bm >= 192) {
    // 192-record m-tiles: one tile per expert at ~128 routes per expert with
    // two thirds of the rows live, where 256-record tiles carry half of them
    // empty.  16x16x64: 4 x 2 waves of 48 x 64 (or 48 x 128); 32x32x32: 2 x 2
    // waves of 96 x 64 (or 96 x 128)
    constexpr int WM = MF == 32 ? 2 : 4;
    if constexpr (!PB) {
      if (bn >= 256) { launch_cfg<MODE, 192, 256, WM, 2, PB, MF>(nbuf, g, dyn, st, t); return; }
    }
    launch_cfg<MODE, 192, 128, WM, 2, PB, MF>(nbuf, g, dyn, st, t);
  }
  else if (bm >= 128) launch_bn<MODE, 128, PB, MF>(bn, nbuf, g, dyn, st, t);
  else if (bm >= 64) launch_bn<MODE, 64, PB, MF>(bn, nbuf, g, dyn, st, t);
  else launch_bn<MODE, 32, PB, 16>(bn, nbuf, g, dyn, st, t);  // 32 rows: 16x16 tiles
}

template <int MODE, bool PB>
static void launch_bm(int bm, int bn, int nbuf, dim3 g, size_t dyn, hipStream_t st,
                      const TiledArgs& t) {
  if (tune().mf == 32) launch_bm_mf<MODE, PB, 32>(bm, bn, nbuf, g, dyn, st, t);
  else launch_bm_mf<MODE, PB, 16>(bm, bn, nbuf, g, dyn, st, t);
}

static inline int tile_bn(int bn) { return bn >= 256 ? 256 : 128; }

hipError_t launch_linear_tiled(const LinArgs& a, int per_block, int bm, hipStream_t st) {
  const int bn = tile_bn(or_default(tune().tile_bn, 128));
  const int nbuf = or_default(tune().ring, 3);
  TiledArgs t{};
  t.lin = a;
  int gn = 0;
  for (int q = 0; q < a.nseg; ++q) gn += (a.seg[q].n + bn - 1) / bn;
  const int bmv = bm >= 128 ? 128 : bm >= 64 ? 64 : 32;
  t.gm = (a.M + bmv - 1) / bmv;
  t.gn = gn;
  dim3 g(t.gm * t.gn);
  const size_t dyn = per_block ? (size_t)bmv * (a.K / a.block) * sizeof(float) : 0;
  // per-row 64 x 128 tiles (chosen when larger tiles leave CUs idle) run with
  // two K groups per workgroup: 21.1 -> 19.4 us at M = 512, K = N = 4096
  if (!per_block && bmv == 64 && bn == 128 && or_default(tune().tile_ksp, 2) == 2) {
    if (tune().mf == 32) {  // 2 x (2 x 2) waves of 32 x 64
      if (nbuf >= 3 && try_launch<MODE_DENSE, 64, 128, 2, 2, false, 3, 2, 32>(g, 0, st, t))
        return hipGetLastError();
      try_launch<MODE_DENSE, 64, 128, 2, 2, false, 2, 2, 32>(g, 0, st, t);
      return hipGetLastError();
    }
    if (nbuf >= 3 && try_launch<MODE_DENSE, 64, 128, 2, 4, false, 3, 2>(g, 0, st, t))
      return hipGetLastError();
    try_launch<MODE_DENSE, 64, 128, 2, 4, false, 2, 2>(g, 0, st, t);
    return hipGetLastError();
  }
  // the grid is sized for bmv-row tiles, so the tile height is bmv (a larger
  // BQ_TILE_BM is clamped to it)
  if (per_block) launch_bm<MODE_DENSE, true>(bmv, bn, nbuf, g, dyn, st, t);
  else launch_bm<MODE_DENSE, false>(bmv, bn, nbuf, g, dyn, st, t);
  return hipGetLastError();
}

static unsigned moe_grid(const TiledArgs& t) {
  if (t.order == 2) return (unsigned)(8 * ((t.gm + 7) / 8) * t.gn);
  return (unsigned)((t.gm * t.gn + 7) / 8 * 8);
}

static inline int mtile_bound(int max_routes, int experts, int bm) {
  return (max_routes + bm - 1) / bm + experts;
}

hipError_t launch_moe_gate_up_tiled(const int8_t* x_i8, const float* x_sa, const int32_t* eo,
                                    const Route* routes, const int8_t* w_gu,
                                    const float* gu_scale, uint16_t* bucket, int8_t* bi8,
                                    float* bsa, int experts, int max_routes, int hidden,
                                    int inter, int bm, hipStream_t st) {
  TiledArgs t{};
  t.a = x_i8; t.a_scale = x_sa; t.eo = eo; t.routes = routes; t.w = w_gu; t.ws = gu_scale;
  t.bucket = bucket; t.bi8 = bi8; t.bsa = bsa; t.fwht64 = fwht_scale_host(64);
  t.E = experts; t.max_routes = max_routes; t.N = 2 * inter; t.K = hidden;
  t.inter = inter; t.block = hidden;
  const int bmv = bm >= 256 ? 256 : bm >= 192 ? 192 : bm >= 128 ? 128 : 64;
  t.gm = mtile_bound(max_routes, experts, bmv);
  t.order = tune().moe_order;
  // weight rows per tile: bn/2 gate + bn/2 up.  256-record tiles pair with
  // 256 weight rows; 192-record tiles (2048 tokens x top-8 over 128 experts)
  // with 128, whose 80 KB ring leaves room for two workgroups per CU
  // (measured 1.5% faster for that layer than 256 rows).
  const int bn = tile_bn(or_default(tune().tile_bn, bmv == 256 ? 256 : 128));
  const int nbuf = or_default(tune().ring, 2);
  t.gn = (inter + bn / 2 - 1) / (bn / 2);
  const dim3 g(moe_grid(t));
  launch_bm<MODE_GATE_UP, false>(bmv, bn, nbuf, g, 0, st, t);
  return hipGetLastError();
}

hipError_t launch_moe_down_tiled(const int8_t* b_i8, const float* b_sa, const int32_t* eo,
                                 const Route* routes, const int8_t* w_d, const float* d_scale,
                                 float* y, int experts, int max_routes, int hidden, int inter,
                                 int block, int bm, hipStream_t st) {
  TiledArgs t{};
  t.a = b_i8; t.a_scale = b_sa; t.eo = eo; t.routes = routes; t.w = w_d; t.ws = d_scale; t.y = y;
  t.E = experts; t.max_routes = max_routes; t.N = hidden; t.K = inter; t.inter = inter;
  t.block = block;
  // block-64 scales and K up to 704 (the model's inter): weights in registers,
  // 192-record m-tiles x 256 columns
  // (hidden % 16 == 0 and a 16-byte aligned y: its lanes store four
  // consecutive columns at once)
  if (block == 64 && inter % 64 == 0 && inter / 64 <= 11 && experts <= kBregMaxExperts &&
      hidden % 16 == 0 && !(reinterpret_cast<uintptr_t>(y) & 15u) && tune().down_breg) {
    constexpr int MI = 12, NI = 2;
    t.gn = (hidden + 8 * NI * 16 - 1) / (8 * NI * 16);
    hipLaunchKernelGGL((k_down_breg<MI, NI, 11>), dim3(tune().cus), dim3(512), 0, st, t);
    return hipGetLastError();
  }
  // the down projection's K (= inter) is short, and its per-block drains
  // keep f32 accumulators: 64-record tiles with a double-buffered stage run
  // fastest (more workgroups in flight per CU)
  const int bmv = bm >= 256 ? 256 : bm >= 192 ? 192 : bm >= 128 ? 128 : 64;
  const int bn = tile_bn(or_default(tune().tile_bn, 128));
  const int nbuf = or_default(tune().ring, 2);
  t.gn = (hidden + bn - 1) / bn;
  t.gm = mtile_bound(max_routes, experts, bmv);
  t.order = tune().moe_order;
  const dim3 g(moe_grid(t));
  const size_t dyn = (size_t)bmv * (inter / block) * sizeof(float);
  launch_bm<MODE_DOWN, true>(bmv, bn, nbuf, g, dyn, st, t);
  return hipGetLastError();
}

}  // namespace bq
