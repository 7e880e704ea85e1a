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
  for (int st = 1; st < block && st < kWave; st <<= 1) {
#pragma unroll
    for (int q = 0; q < MAXSEG; ++q) {
      if (wave + q * nw >= nseg) continue;
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const float p = __shfl_xor(v[q][i], st, kWave);
        v[q][i] = (lane & st) ? (p - v[q][i]) : (v[q][i] + p);
      }
    }
  }
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

// Each wave owns segments of S = R*64 values (one block when B >= 64, or
// 64/B blocks when B < 64) of one row; grid-stride over all segments.
template <int R>
__global__ __launch_bounds__(256) void k_block_quant(
    const uint16_t* __restrict__ src, int8_t* __restrict__ xq, float* __restrict__ sa,
    int rows, int cols, int block, int apply_fwht, float fwht_scale) {
  const int lane = lane_id();
  const int S = R * kWave;
  const int segs_per_row = cols / S;
  const int nb = cols / block;
  const size_t total = (size_t)rows * segs_per_row;
  const size_t wave_id = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const size_t nwaves = ((size_t)gridDim.x * blockDim.x) >> 6;
  for (size_t g = wave_id; g < total; g += nwaves) {
    const int r = (int)(g / segs_per_row), sg = (int)(g % segs_per_row);
    const size_t base = (size_t)r * cols + (size_t)sg * S;
    float v[R];
#pragma unroll
    for (int i = 0; i < R; ++i) v[i] = bf16_to_f32(src[base + i * kWave + lane]);
    if (apply_fwht) {
      fwht_wave<R>(v, block);
#pragma unroll
      for (int i = 0; i < R; ++i) v[i] = v[i] * fwht_scale;
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < R; ++i) m = fmaxf(m, fabsf(v[i]));
    const float bm = block >= kWave ? wave_max(m) : group_max(m, block);
    const float inv = bm > 0.0f ? 127.0f / bm : 0.0f;
#pragma unroll
    for (int i = 0; i < R; ++i) xq[base + i * kWave + lane] = quantize_i8(v[i], inv);
    if (block >= kWave) {
      if (lane == 0) sa[(size_t)r * nb + (size_t)sg * S / block] = bm;
    } else if ((lane % block) == 0) {
      sa[(size_t)r * nb + ((size_t)sg * S + lane) / block] = bm;
    }
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
  const int R = block < 64 ? 1 : block / 64;
  const size_t segs = (size_t)rows * (cols / (R * 64));
  size_t blocks = (segs + 3) / 4;
  if (blocks > 8192) blocks = 8192;
  dim3 g((unsigned)blocks), b(256);
  switch (R) {
    case 1: hipLaunchKernelGGL(k_block_quant<1>, g, b, 0, st, src, xq, sa, rows, cols, block, apply_fwht, sc); break;
    case 2: hipLaunchKernelGGL(k_block_quant<2>, g, b, 0, st, src, xq, sa, rows, cols, block, apply_fwht, sc); break;
    case 4: hipLaunchKernelGGL(k_block_quant<4>, g, b, 0, st, src, xq, sa, rows, cols, block, apply_fwht, sc); break;
    case 8: hipLaunchKernelGGL(k_block_quant<8>, g, b, 0, st, src, xq, sa, rows, cols, block, apply_fwht, sc); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bq
