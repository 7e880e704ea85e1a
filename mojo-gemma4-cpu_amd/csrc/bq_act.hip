// bq_act.hip -- activation preparation kernels (HBM-bound byte work).
//
//   k_norm_quant  : dispatch_bq_norm_quant (butterquant_kernels/linear.mojo:25-82
//                   -> butterquant/runtime.mojo:11-37): RMS (reference
//                   accumulation order) -> x*inv_rms*g -> FWHT(B) in LDS/
//                   wave shuffles -> per-row int8, sa = amax.
//   k_block_quant : dispatch_bq_block_quant (linear.mojo:152-205 ->
//                   runtime.mojo:62-80): bf16 -> [FWHT(B)] -> per-block int8.
#include "bq_device.hpp"
#include "bq_kernels.hpp"

namespace bq {

// One workgroup (256 threads) per token row; the f32 row lives in LDS.
template <int R>
__global__ __launch_bounds__(256) void k_norm_quant(
    const uint16_t* __restrict__ src, const uint16_t* __restrict__ gamma,
    int8_t* __restrict__ xq, float* __restrict__ sa, int hidden, int block, int pu,
    float sqrt_n, float n_eps, float fwht_scale) {
  extern __shared__ float row[];
  __shared__ float accs[8 * 16];
  __shared__ float red[4];
  __shared__ float s_inv_rms;
  const int t = blockIdx.x, tid = threadIdx.x;
  const uint16_t* x = src + (size_t)t * hidden;

  // Sum of squares in the order of rms_reduce_row (rmsnorm.mojo:16-17 ->
  // dot_products.mojo:144-191): pu accumulators x 16 f32 lanes; lane j of
  // accumulator p takes bf16 pairs (2j, 2j+1) of every pu*32-wide stride
  // step at offset p*32, odd element first (one vdpbf16ps lane).
  const int chains = pu * 16;
  if (tid < chains) {
    const int p = tid >> 4, j = tid & 15, stride = pu * 32;
    float acc = 0.0f;
    for (int i = 0; i < hidden / stride; ++i) {
      uint32_t pair = *reinterpret_cast<const uint32_t*>(x + (size_t)i * stride + p * 32 + 2 * j);
      float e = __uint_as_float(pair << 16);
      float o = __uint_as_float(pair & 0xFFFF0000u);
      acc = fmaf(o, o, acc);
      acc = fmaf(e, e, acc);
    }
    accs[tid] = acc;
  }
  __syncthreads();
  if (tid == 0) {
    // s = sum_p acc[p] lane-wise (dot_products.mojo:127-140), then a 16-lane
    // halving-tree horizontal add.
    float s[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) s[j] = 0.0f;
    for (int p = 0; p < pu; ++p)
#pragma unroll
      for (int j = 0; j < 16; ++j) s[j] = s[j] + accs[p * 16 + j];
#pragma unroll
    for (int h = 8; h >= 1; h >>= 1)
#pragma unroll
      for (int j = 0; j < h; ++j) s[j] = s[j] + s[j + h];
    s_inv_rms = sqrt_n / __builtin_sqrtf(s[0] + n_eps);
  }
  __syncthreads();
  const float inv_rms = s_inv_rms;
  for (int k = tid; k < hidden; k += blockDim.x)
    row[k] = bf16_to_f32(x[k]) * inv_rms * bf16_to_f32(gamma[k]);
  __syncthreads();

  const int wave = tid >> 6, lane = lane_id(), nwaves = blockDim.x >> 6;
  const int S = R * kWave, nseg = hidden / S;
  float m = 0.0f;
  for (int sg = wave; sg < nseg; sg += nwaves) {
    float v[R];
#pragma unroll
    for (int i = 0; i < R; ++i) v[i] = row[sg * S + i * kWave + lane];
    fwht_wave<R>(v, block);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      v[i] = v[i] * fwht_scale;
      row[sg * S + i * kWave + lane] = v[i];
      m = fmaxf(m, fabsf(v[i]));
    }
  }
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  float amax = red[0];
  for (int i = 1; i < nwaves; ++i) amax = fmaxf(amax, red[i]);
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  int8_t* q = xq + (size_t)t * hidden;
  for (int k = tid; k < hidden; k += blockDim.x) q[k] = quantize_i8(row[k], inv);
  if (tid == 0) sa[t] = amax;
}

// Latency-optimised variant used whenever the row fits: the bf16 row is
// staged once into LDS with 16-byte loads; each wave then owns up to MAXSEG
// FWHT segments and transforms all of them together (independent shuffle
// chains), keeping the values in registers through quantization.
template <int R, int MAXSEG>
__global__ __launch_bounds__(1024) void k_norm_quant_reg(
    const uint16_t* __restrict__ src, const uint16_t* __restrict__ gamma,
    int8_t* __restrict__ xq, float* __restrict__ sa, int hidden, int block, int pu,
    float sqrt_n, float n_eps, float fwht_scale) {
  extern __shared__ uint32_t xs[];  // the bf16 row, two values per word
  __shared__ float accs[8 * 16];
  __shared__ float red[16];
  __shared__ float s_inv_rms;
  const int t = blockIdx.x, tid = threadIdx.x, nthr = blockDim.x;
  const int nw = nthr >> 6, wave = tid >> 6, lane = lane_id();
  const int S = R * kWave, nseg = hidden / S;
  // this thread's gamma values, fetched before anything waits on memory
  float gv[MAXSEG][R];
#pragma unroll
  for (int q = 0; q < MAXSEG; ++q)
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int sg = wave + q * nw;
      gv[q][i] = sg < nseg ? bf16_to_f32(gamma[sg * S + i * kWave + lane]) : 0.0f;
    }
  const int8_t* xrow = reinterpret_cast<const int8_t*>(src + (size_t)t * hidden);
  for (int c = tid; c < hidden / 8; c += nthr)
    reinterpret_cast<v4i*>(xs)[c] = ld16(xrow + (size_t)c * 16);
  __syncthreads();

  // rms_reduce_row order (see k_norm_quant): pu*16 chains, odd then even
  if (tid < pu * 16) {
    const int p = tid >> 4, j = tid & 15, stride = pu * 32;
    float acc = 0.0f;
    for (int i = 0; i < hidden / stride; ++i) {
      const uint32_t pair = xs[(i * stride + p * 32 + 2 * j) >> 1];
      const float e = __uint_as_float(pair << 16);
      const float o = __uint_as_float(pair & 0xFFFF0000u);
      acc = fmaf(o, o, acc);
      acc = fmaf(e, e, acc);
    }
    accs[tid] = acc;
  }
  __syncthreads();
  if (tid < 16) {
    float sum = 0.0f;
    for (int p = 0; p < pu; ++p) sum = sum + accs[p * 16 + tid];
    // 16-lane halving tree: lane j adds lane j+h for h = 8, 4, 2, 1
#pragma unroll
    for (int h = 8; h >= 1; h >>= 1) sum = sum + __shfl_down(sum, h, 16);
    if (tid == 0) s_inv_rms = sqrt_n / __builtin_sqrtf(sum + n_eps);
  }
  __syncthreads();
  const float inv_rms = s_inv_rms;

  float v[MAXSEG][R];
#pragma unroll
  for (int q = 0; q < MAXSEG; ++q) {
    const int sg = wave + q * nw;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      float val = 0.0f;
      if (sg < nseg) {
        const int k = sg * S + i * kWave + lane;
        const uint32_t w = xs[k >> 1];
        const float xv = __uint_as_float((k & 1) ? (w & 0xFFFF0000u) : (w << 16));
        val = xv * inv_rms * gv[q][i];
      }
      v[q][i] = val;
    }
  }
  for_each_xlane_stride(block, [&](auto st) {
    constexpr int ST = decltype(st)::value;
#pragma unroll
    for (int q = 0; q < MAXSEG; ++q) {
      if (wave + q * nw >= nseg) continue;
#pragma unroll
      for (int i = 0; i < R; ++i) v[q][i] = xlane_bfly<ST>(v[q][i]);
    }
  });
#pragma unroll
  for (int rs = 1; rs < R; rs <<= 1) {
    if (rs * kWave >= block) break;
#pragma unroll
    for (int q = 0; q < MAXSEG; ++q)
#pragma unroll
      for (int i = 0; i < R; ++i) {
        if (i & rs) continue;
        const float a = v[q][i], b = v[q][i + rs];
        v[q][i] = a + b;
        v[q][i + rs] = a - b;
      }
  }
  float m = 0.0f;
#pragma unroll
  for (int q = 0; q < MAXSEG; ++q)
#pragma unroll
    for (int i = 0; i < R; ++i) {
      v[q][i] = v[q][i] * fwht_scale;
      m = fmaxf(m, fabsf(v[q][i]));
    }
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  float amax = red[0];
  for (int i = 1; i < nw; ++i) amax = fmaxf(amax, red[i]);
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  int8_t* qrow = xq + (size_t)t * hidden;
#pragma unroll
  for (int q = 0; q < MAXSEG; ++q) {
    const int sg = wave + q * nw;
    if (sg >= nseg) continue;
#pragma unroll
    for (int i = 0; i < R; ++i) qrow[sg * S + i * kWave + lane] = quantize_i8(v[q][i], inv);
  }
  if (tid == 0) sa[t] = amax;
}

// Long sequences: one wave per token, four tokens per workgroup.  The row
// is staged in the wave's own LDS slice (the gain once per workgroup); the
// sum of squares keeps the rms_reduce_row order of k_norm_quant (chain c =
// p*16+j over pairs c + i*pu*16; lane-wise sum over p; 16-lane halving tree),
// and FWHT / quantization run on registers, value q*S + r*64 + lane of
// segment q.  Every one of the NSEG segments is processed without branches
// (segments past nseg read a clamped position and are zeroed): per-segment
// guards would split the shuffles into separate blocks and serialize them.
template <int R, int NSEG>
__global__ __launch_bounds__(256) void k_norm_quant_wave(
    const uint16_t* __restrict__ src, const uint16_t* __restrict__ gamma,
    int8_t* __restrict__ xq, float* __restrict__ sa, int T, int hidden, int block, int pu,
    float sqrt_n, float n_eps, float fwht_scale) {
  extern __shared__ uint32_t lds_rows[];  // [gain | row of wave 0..3], bf16 pairs
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int t = blockIdx.x * 4 + wave;
  constexpr int S = R * kWave;
  const int nseg = hidden / S, nchunk = hidden / 8;
  uint32_t* gs = lds_rows;
  // the row's loads go out before the gain's barrier so both latencies overlap
  const int8_t* xrow = reinterpret_cast<const int8_t*>(src + (size_t)min(t, T - 1) * hidden);
  constexpr int CH = (NSEG * R + 7) / 8;  // 16-byte chunks per lane (NSEG*R*64 values)
  v4i raw[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) raw[i] = ld16(xrow + (size_t)min(lane + 64 * i, nchunk - 1) * 16);
  for (int c = threadIdx.x; c < nchunk; c += blockDim.x)
    reinterpret_cast<v4i*>(gs)[c] = ld16(reinterpret_cast<const int8_t*>(gamma) + (size_t)c * 16);
  __syncthreads();
  if (t >= T) return;  // whole waves only; nothing below synchronizes the block
  uint32_t* xs = lds_rows + (size_t)(wave + 1) * (hidden / 2);
#pragma unroll
  for (int i = 0; i < CH; ++i)
    if (lane + 64 * i < nchunk) reinterpret_cast<v4i*>(xs)[lane + 64 * i] = raw[i];

  // chains c0 = lane and c1 = lane + 64 (pu*16 <= 128 chains), interleaved
  const int chains = pu * 16;  // also the pair stride of a chain
  const int iters = hidden / (pu * 32);
  const int c1 = min(lane + 64, chains - 1);
  float a0 = 0.0f, a1 = 0.0f;
#pragma unroll 4
  for (int i = 0; i < iters; ++i) {
    const uint32_t p0 = xs[i * chains + min(lane, chains - 1)], p1 = xs[i * chains + c1];
    a0 = fmaf(__uint_as_float(p0 & 0xFFFF0000u), __uint_as_float(p0 & 0xFFFF0000u), a0);
    a0 = fmaf(__uint_as_float(p0 << 16), __uint_as_float(p0 << 16), a0);
    a1 = fmaf(__uint_as_float(p1 & 0xFFFF0000u), __uint_as_float(p1 & 0xFFFF0000u), a1);
    a1 = fmaf(__uint_as_float(p1 << 16), __uint_as_float(p1 << 16), a1);
  }
  float sum = 0.0f;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int c = p * 16 + (lane & 15);
    const float v0 = __shfl(a0, c & 63, kWave);
    const float v1 = __shfl(a1, c & 63, kWave);
    if (p < pu) sum = sum + (c < 64 ? v0 : v1);
  }
#pragma unroll
  for (int h = 8; h >= 1; h >>= 1) sum = sum + __shfl_down(sum, h, 16);
  const float total = __shfl(sum, 0, kWave);
  const float inv_rms = sqrt_n / __builtin_sqrtf(total + n_eps);

  float v[NSEG][R];
#pragma unroll
  for (int q = 0; q < NSEG; ++q)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int k = min(q, nseg - 1) * S + r * kWave + lane;
      const uint32_t w = xs[k >> 1], gw = gs[k >> 1];
      const float xv = __uint_as_float((k & 1) ? (w & 0xFFFF0000u) : (w << 16));
      const float g = __uint_as_float((k & 1) ? (gw & 0xFFFF0000u) : (gw << 16));
      const float val = xv * inv_rms * g;
      v[q][r] = q < nseg ? val : 0.0f;
    }
  for_each_xlane_stride(block, [&](auto st) {
    constexpr int ST = decltype(st)::value;
#pragma unroll
    for (int q = 0; q < NSEG; ++q)
#pragma unroll
      for (int r = 0; r < R; ++r) v[q][r] = xlane_bfly<ST>(v[q][r]);
  });
#pragma unroll
  for (int rs = 1; rs < R; rs <<= 1) {
    if (rs * kWave >= block) continue;
#pragma unroll
    for (int q = 0; q < NSEG; ++q)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (r & rs) continue;
        const float a = v[q][r], b = v[q][r + rs];
        v[q][r] = a + b;
        v[q][r + rs] = a - b;
      }
  }
  float m = 0.0f;
#pragma unroll
  for (int q = 0; q < NSEG; ++q)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      v[q][r] = v[q][r] * fwht_scale;
      m = fmaxf(m, fabsf(v[q][r]));
    }
  const float amax = wave_max(m);
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  int8_t* qrow = xq + (size_t)t * hidden;
#pragma unroll
  for (int q = 0; q < NSEG; ++q)
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (q < nseg) qrow[q * S + r * kWave + lane] = quantize_i8(v[q][r], inv);
  if (lane == 0) sa[t] = amax;
}

template <int R, int NSEG>
static void launch_nq_wave(dim3 g, size_t lds, hipStream_t st, const uint16_t* src,
                           const uint16_t* gamma, int8_t* xq, float* sa, int T, int hidden,
                           int block, int pu, float sqrt_n, float n_eps, float sc) {
  hipLaunchKernelGGL((k_norm_quant_wave<R, NSEG>), g, dim3(256), lds, st, src, gamma, xq, sa, T,
                     hidden, block, pu, sqrt_n, n_eps, sc);
}

// Pair-layout norm-quant (nq_pair_* in bq_device.hpp).  A token takes
// WPT = ceil(nseg / SPW) waves: each loads the whole row and computes the sum
// of squares (it is cheap, and it keeps the chain order), then transforms and
// quantizes its own SPW segments; the row's amax is exchanged through LDS
// (one barrier) when WPT > 1.  WPT = 1 runs four tokens per workgroup without
// LDS or barriers.
template <int NSEG, int SPW>
__global__ __launch_bounds__(512) void k_norm_quant_pair(
    const uint16_t* __restrict__ src, const uint16_t* __restrict__ gamma,
    int8_t* __restrict__ xq, float* __restrict__ sa, int T, int hidden, int block,
    float sqrt_n, float n_eps, float fwht_scale) {
  __shared__ float s_max[8];
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int nseg = hidden >> 7;
  const int wpt = (nseg + SPW - 1) / SPW;  // waves per token
  const bool one = SPW >= NSEG;            // one wave per token
  const int t = one ? blockIdx.x * 4 + wave : blockIdx.x;
  const int q0 = one ? 0 : wave * SPW;     // this wave's first segment
  if (t >= T) return;                      // (one: whole waves, nothing synchronizes)
  const uint32_t* xr = reinterpret_cast<const uint32_t*>(src + (size_t)t * hidden) + lane;
  const uint32_t* gr = reinterpret_cast<const uint32_t*>(gamma) + lane;
  // A wave of a token's several loads its own segments again, into x:
  // cheaper than picking them out of xp by a run-time index.
  // (loads return in issue order: the row first, which the sum of squares
  // needs first)
  uint32_t xp[NSEG], x[SPW], gp[SPW];
#pragma unroll
  for (int q = 0; q < NSEG; ++q)
    if (q < nseg) xp[q] = xr[64 * q];
  // (segments past nseg are loaded nowhere and read nowhere)
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    if (q0 + i < nseg) {
      if constexpr (SPW < NSEG) x[i] = xr[64 * (q0 + i)];
      gp[i] = gr[64 * (q0 + i)];
    }
  }
  if constexpr (SPW >= NSEG) {  // one wave per token: q0 = 0, x is xp
#pragma unroll
    for (int i = 0; i < SPW; ++i) x[i] = xp[i];
  }
  const float total = nq_pair_sumsq<NSEG>(xp, nseg);
  const float inv_rms = sqrt_n / __builtin_sqrtf(total + n_eps);
  float v[SPW][2];
  const float m = nq_pair_transform<SPW>(x, gp, inv_rms, q0, nseg, block, fwht_scale, v);
  float amax = wave_max(m);
  if (!one) {
    if (lane == 0) s_max[wave] = amax;
    __syncthreads();
    amax = s_max[0];
    for (int w = 1; w < wpt; ++w) amax = fmaxf(amax, s_max[w]);
  }
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  uint16_t* qrow = reinterpret_cast<uint16_t*>(xq + (size_t)t * hidden) + lane;
#pragma unroll
  for (int i = 0; i < SPW; ++i)
    if (q0 + i < nseg) qrow[64 * (q0 + i)] = nq_pair_code(v[i], inv);
  if (lane == 0 && wave == (one ? wave : 0)) sa[t] = amax;
}

// Norm-quant with FWHT block 128, one wave per token (nq_v8_token): the
// transform on 8 consecutive values per lane, so a 128-value block is one
// row of 16 lanes and the FWHT's strides 1, 2, 4 run inside the lane and
// strides 8, 16, 32, 64 across lanes 1, 2, 4, 8 apart (one DPP row move
// each, two for lanes 4 apart) -- the reference's stages in its order, with
// no cross-row swaps.
template <int NSEG>
__global__ __launch_bounds__(256) void k_norm_quant_v8(
    const uint16_t* __restrict__ src, const uint16_t* __restrict__ gamma,
    int8_t* __restrict__ xq, float* __restrict__ sa, int T, int hidden, float sqrt_n,
    float n_eps, float fwht_scale) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // whole waves; nothing synchronizes
  nq_v8_token<NSEG>(src, gamma, xq, sa, t, hidden, sqrt_n, n_eps, fwht_scale);
}

// The same for a few tokens: one workgroup per token, wave w transforming
// round w (values 512 w .. + 511); every wave takes the whole row's sum of
// squares (the chain order forbids splitting it) and the row's amax meets
// in LDS (one barrier).
template <int NSEG>
__global__ __launch_bounds__(512) void k_norm_quant_v8_row(
    const uint16_t* __restrict__ src, const uint16_t* __restrict__ gamma,
    int8_t* __restrict__ xq, float* __restrict__ sa, int hidden, float sqrt_n, float n_eps,
    float fwht_scale) {
  __shared__ float s_max[8];
  // (the launch's waves, from hidden rather than blockDim: reading blockDim
  // would add the runtime's implicit arguments to the kernel's argument block)
  const int lane = lane_id(), wave = threadIdx.x >> 6, nw = (hidden + 511) >> 9;
  const int t = blockIdx.x, nseg = hidden >> 7;
  const uint16_t* row = src + (size_t)t * hidden;
  const uint32_t* xr = reinterpret_cast<const uint32_t*>(row) + lane;
  uint32_t xp[NSEG];
#pragma unroll
  for (int q = 0; q < NSEG; ++q)
    if (q < nseg) xp[q] = xr[64 * q];
  const int e0 = 512 * wave + 8 * lane;
  const int ec = min(e0, hidden - 8);  // runs past the row are read, never stored
  const v4i xv = *reinterpret_cast<const v4i*>(row + ec);
  const v4i gv = *reinterpret_cast<const v4i*>(gamma + ec);
  const float total = nq_pair_sumsq<NSEG>(xp, nseg);
  const float inv_rms = sqrt_n / __builtin_sqrtf(total + n_eps);
  float v[8];
  float m = nq_v8_transform(xv, gv, inv_rms, fwht_scale, v);
  if (e0 >= hidden) m = 0.0f;
  m = wave_max(m);
  if (lane == 0) s_max[wave] = m;
  __syncthreads();
  float amax = s_max[0];
  for (int w = 1; w < nw; ++w) amax = fmaxf(amax, s_max[w]);
  if (e0 < hidden) {
    uint32_t w[2];
    nq_v8_codes(v, amax > 0.0f ? 127.0f / amax : 0.0f, w);
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u2*>(xq + (size_t)t * hidden + e0) = u2{w[0], w[1]};
  }
  if (threadIdx.x == 0) sa[t] = amax;
}

// smallest instance holding nseg segments of R*64 values (hidden <= 4096)
static bool launch_norm_quant_wave(int R, int nseg, const uint16_t* src, const uint16_t* gamma,
                                   int8_t* xq, float* sa, int T, int hidden, int block, int pu,
                                   float sqrt_n, float n_eps, float sc, hipStream_t st) {
  const dim3 g((T + 3) / 4);
  const size_t lds = (size_t)5 * hidden * 2;  // gain + four rows
#define BQ_NQW(RR, NS) \
  if (R == RR && nseg <= NS) { launch_nq_wave<RR, NS>(g, lds, st, src, gamma, xq, sa, T, hidden, block, pu, sqrt_n, n_eps, sc); return true; }
  BQ_NQW(1, 16) BQ_NQW(1, 32) BQ_NQW(1, 44) BQ_NQW(1, 64)
  BQ_NQW(2, 8) BQ_NQW(2, 16) BQ_NQW(2, 22) BQ_NQW(2, 32)
  BQ_NQW(4, 4) BQ_NQW(4, 8) BQ_NQW(4, 11) BQ_NQW(4, 16)
  BQ_NQW(8, 2) BQ_NQW(8, 4) BQ_NQW(8, 6) BQ_NQW(8, 8)
#undef BQ_NQW
  return false;
}

// Flat over the whole [rows, cols] matrix: lane i owns the 8 consecutive
// values [8i, 8i+8); a block of B values spans LPB = B/8 aligned lanes and
// blocks never straddle rows (cols % B == 0), so block b's scale lands at
// sa[b] = sa[row * cols/B + col/B].  FWHT strides 1, 2, 4 run inside the lane,
// strides 8 ... B/2 across lanes, in the reference's ascending stage order.
template <int LPB>
__global__ __launch_bounds__(256) void k_block_quant(
    const uint16_t* __restrict__ src, int8_t* __restrict__ xq, float* __restrict__ sa,
    size_t nchunks, int apply_fwht, float fwht_scale) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;  // 256-thread blocks
  const size_t c = i < nchunks ? i : nchunks - 1;  // whole LPB groups are in or out
  const int lane = lane_id();
  float v[8];
  bf16x8_to_f32(*reinterpret_cast<const v4i*>(src + c * 8), v);
  uint32_t w[2];
  const float m = block_quant_lanes<LPB>(v, apply_fwht, fwht_scale, w);
  if (i < nchunks) {
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u2*>(xq + c * 8) = u2{w[0], w[1]};
    if ((lane & (LPB - 1)) == 0) sa[c / LPB] = m;
  }
}

// simd_math/matrixops.mojo:233-246 with the AVX-512 bf16 width 32
int pick_port_unroll(int cols) {
  const int w = 32;
  if (cols % (8 * w) == 0) return 8;
  if (cols % (4 * w) == 0) return 4;
  if (cols % (2 * w) == 0) return 2;
  return 1;
}

hipError_t launch_norm_quant(const uint16_t* src, const uint16_t* gamma, int8_t* xq, float* sa,
                             int seq_len, int hidden, int block, float sqrt_n, float n_eps,
                             hipStream_t st) {
  if (seq_len <= 0) return hipSuccess;
  const int pu = pick_port_unroll(hidden);
  const float sc = fwht_scale_host(block);
  const int R = block < 64 ? 1 : block / 64;
  const int nseg = hidden / (R * 64);
  constexpr int MAXSEG = 4;
  const int waves = (nseg + MAXSEG - 1) / MAXSEG;
  // pair-layout wave per token: hidden % 256 == 0 (128 sum-of-squares
  // chains), up to 4096 values, 2-byte aligned codes
  if (pu == 8 && hidden <= 4096 && tune().nq_pair && !(reinterpret_cast<uintptr_t>(xq) & 1u)) {
    const int ns = hidden >> 7;
    // many tokens: one wave each (4 per workgroup); few: a token over up to
    // 8 waves of SPW segments (a multiple of B/128 segments: whole blocks)
    // FWHT block 128: 8 values per lane for the transform (16-byte aligned
    // gain, 8-byte aligned codes); a workgroup per token below 256 tokens
    const bool v8 = block == 128 && tune().nq_v8 && !(reinterpret_cast<uintptr_t>(gamma) & 15u) &&
                    !(reinterpret_cast<uintptr_t>(xq) & 7u);
    if (v8 && seq_len < 256) {
      const dim3 g(seq_len), b(64 * ((hidden + 511) / 512));
#define BQ_NQ8R(N) if (ns <= N) { hipLaunchKernelGGL((k_norm_quant_v8_row<N>), g, b, 0, st, src, gamma, xq, sa, hidden, sqrt_n, n_eps, sc); return hipGetLastError(); }
      BQ_NQ8R(8) BQ_NQ8R(16) BQ_NQ8R(22) BQ_NQ8R(24) BQ_NQ8R(32)
#undef BQ_NQ8R
    }
    if (v8 && seq_len >= 256) {
      const dim3 g((seq_len + 3) / 4), b(256);
#define BQ_NQ8(N) if (ns <= N) { hipLaunchKernelGGL((k_norm_quant_v8<N>), g, b, 0, st, src, gamma, xq, sa, seq_len, hidden, sqrt_n, n_eps, sc); return hipGetLastError(); }
      BQ_NQ8(8) BQ_NQ8(16) BQ_NQ8(22) BQ_NQ8(24) BQ_NQ8(32)
#undef BQ_NQ8
    }
    if (seq_len >= 256) {
      const dim3 g((seq_len + 3) / 4), b(256);
#define BQ_NQP(N) if (ns <= N) { hipLaunchKernelGGL((k_norm_quant_pair<N, N>), g, b, 0, st, src, gamma, xq, sa, seq_len, hidden, block, sqrt_n, n_eps, sc); return hipGetLastError(); }
      BQ_NQP(4) BQ_NQP(8) BQ_NQP(12) BQ_NQP(16) BQ_NQP(22) BQ_NQP(24) BQ_NQP(32)
#undef BQ_NQP
    } else {
      const int unit = block > 128 ? block / 128 : 1;
      int spw = (ns + 7) / 8;
      spw = (spw + unit - 1) / unit * unit;
      const dim3 g(seq_len), b(64 * ((ns + spw - 1) / spw));
#define BQ_NQP(N, S) if (ns <= N && spw == S) { hipLaunchKernelGGL((k_norm_quant_pair<N, S>), g, b, 0, st, src, gamma, xq, sa, seq_len, hidden, block, sqrt_n, n_eps, sc); return hipGetLastError(); }
      BQ_NQP(8, 1) BQ_NQP(8, 2) BQ_NQP(8, 4) BQ_NQP(16, 2) BQ_NQP(16, 4)
      BQ_NQP(24, 3) BQ_NQP(24, 4) BQ_NQP(32, 4)
#undef BQ_NQP
    }
  }
  // one wave per token from 1792 tokens (hidden 2816: 13.6 vs 12.8 us at
  // 1536 tokens for the workgroup-per-row kernel, 14.3 vs 15.6 us at 2048)
  if (seq_len >= 1792 && hidden <= 4096 &&
      launch_norm_quant_wave(R, nseg, src, gamma, xq, sa, seq_len, hidden, block, pu, sqrt_n,
                             n_eps, sc, st))
    return hipGetLastError();
  if (waves <= 16) {
    const int threads = 64 * (waves < 4 ? 4 : waves);
    const size_t lds = (size_t)hidden * 2;
    dim3 g(seq_len), b(threads);
    switch (R) {
      case 1: hipLaunchKernelGGL((k_norm_quant_reg<1, MAXSEG>), g, b, lds, st, src, gamma, xq, sa, hidden, block, pu, sqrt_n, n_eps, sc); break;
      case 2: hipLaunchKernelGGL((k_norm_quant_reg<2, MAXSEG>), g, b, lds, st, src, gamma, xq, sa, hidden, block, pu, sqrt_n, n_eps, sc); break;
      case 4: hipLaunchKernelGGL((k_norm_quant_reg<4, MAXSEG>), g, b, lds, st, src, gamma, xq, sa, hidden, block, pu, sqrt_n, n_eps, sc); break;
      case 8: hipLaunchKernelGGL((k_norm_quant_reg<8, MAXSEG>), g, b, lds, st, src, gamma, xq, sa, hidden, block, pu, sqrt_n, n_eps, sc); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  const size_t lds = (size_t)hidden * sizeof(float);
  dim3 g(seq_len), b(256);
  switch (R) {
    case 1: hipLaunchKernelGGL(k_norm_quant<1>, g, b, lds, st, src, gamma, xq, sa, hidden, block, pu, sqrt_n, n_eps, sc); break;
    case 2: hipLaunchKernelGGL(k_norm_quant<2>, g, b, lds, st, src, gamma, xq, sa, hidden, block, pu, sqrt_n, n_eps, sc); break;
    case 4: hipLaunchKernelGGL(k_norm_quant<4>, g, b, lds, st, src, gamma, xq, sa, hidden, block, pu, sqrt_n, n_eps, sc); break;
    case 8: hipLaunchKernelGGL(k_norm_quant<8>, g, b, lds, st, src, gamma, xq, sa, hidden, block, pu, sqrt_n, n_eps, sc); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_block_quant(const uint16_t* src, int8_t* xq, float* sa, int rows, int cols,
                              int block, int apply_fwht, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  const float sc = fwht_scale_host(block);
  const size_t nchunks = (size_t)rows * cols / 8;
  dim3 g((unsigned)((nchunks + 255) / 256)), b(256);
  switch (block) {
    case 16: hipLaunchKernelGGL(k_block_quant<2>, g, b, 0, st, src, xq, sa, nchunks, apply_fwht, sc); break;
    case 32: hipLaunchKernelGGL(k_block_quant<4>, g, b, 0, st, src, xq, sa, nchunks, apply_fwht, sc); break;
    case 64: hipLaunchKernelGGL(k_block_quant<8>, g, b, 0, st, src, xq, sa, nchunks, apply_fwht, sc); break;
    case 128: hipLaunchKernelGGL(k_block_quant<16>, g, b, 0, st, src, xq, sa, nchunks, apply_fwht, sc); break;
    case 256: hipLaunchKernelGGL(k_block_quant<32>, g, b, 0, st, src, xq, sa, nchunks, apply_fwht, sc); break;
    case 512: hipLaunchKernelGGL(k_block_quant<64>, g, b, 0, st, src, xq, sa, nchunks, apply_fwht, sc); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bq
