// bq_layout.hip -- weight preparation kernels: the one-time re-tile of packed
// int8 codes into the GPU tile16x64 layout, its inverse (for bit-exact tests),
// the reference's own VNNI pack + colsum (butterquant/vnni.mojo:31-114,
// butterquant/pack.mojo:19-99) and the offline weight encoder
// (butterquant/kernels.mojo:148-168 as driven by quant/quantizer.mojo:963-1051).
// All are integer/byte kernels bound by HBM; each thread moves 16 bytes.
#include "bq_device.hpp"
#include "bq_kernels.hpp"

namespace bq {

// dst (tile16x64) chunk c = fragment*64 + lane  <-  row-major src
__global__ void k_retile_rowmajor(const int8_t* __restrict__ src, int8_t* __restrict__ dst,
                                  int N, int K) {
  size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t chunks = (size_t)N * K / 16;
  if (c >= chunks) return;
  int k64 = K >> 6;
  size_t frag = c >> 6;
  int lane = (int)(c & 63);
  int n = (int)(frag / k64) * 16 + (lane & 15);
  int k0 = (int)(frag % k64) * 64 + (lane >> 4) * 16;
  st16(dst + c * 16, ld16(src + (size_t)n * K + k0));
}

// dst (tile16x64) chunk  <-  reference VNNI 32x64 layout: 4 dwords per chunk
__global__ void k_retile_vnni(const int8_t* __restrict__ src, int8_t* __restrict__ dst,
                              int N, int K) {
  size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t chunks = (size_t)N * K / 16;
  if (c >= chunks) return;
  int k64 = K >> 6;
  size_t frag = c >> 6;
  int lane = (int)(c & 63);
  int n = (int)(frag / k64) * 16 + (lane & 15);
  int k0 = (int)(frag % k64) * 64 + (lane >> 4) * 16;
  v4i v;
  v.x = *reinterpret_cast<const int*>(src + vnni_offset(n, k0 + 0, K));
  v.y = *reinterpret_cast<const int*>(src + vnni_offset(n, k0 + 4, K));
  v.z = *reinterpret_cast<const int*>(src + vnni_offset(n, k0 + 8, K));
  v.w = *reinterpret_cast<const int*>(src + vnni_offset(n, k0 + 12, K));
  st16(dst + c * 16, v);
}

// row-major dst chunk (n, k0..k0+15)  <-  tile16x64 src
__global__ void k_unpack_tiled(const int8_t* __restrict__ src, int8_t* __restrict__ dst,
                               int N, int K) {
  size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t chunks = (size_t)N * K / 16;
  if (c >= chunks) return;
  int kc = K >> 4;
  int n = (int)(c / kc);
  int k0 = (int)(c % kc) * 16;
  st16(dst + c * 16, ld16(src + tile_offset(n, k0, K)));
}

// Reference VNNI pack (vnni.mojo:146-163): one thread per dword (n, k..k+3).
__global__ void k_pack_vnni(const int8_t* __restrict__ src, int8_t* __restrict__ dst,
                            int N, int K) {
  size_t d = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t dwords = (size_t)N * K / 4;
  if (d >= dwords) return;
  int kd = K >> 2;
  int n = (int)(d / kd);
  int k = (int)(d % kd) * 4;
  *reinterpret_cast<int*>(dst + vnni_offset(n, k, K)) =
      *reinterpret_cast<const int*>(src + (size_t)n * K + k);
}

// colsum (vnni.mojo:128-144): exact integer sum of each row's codes over each
// block_cols segment, stored as f32; row-major [N, nb] or block-major [nb, N].
__global__ void k_colsum(const int8_t* __restrict__ src, float* __restrict__ colsum, int N,
                         int K, int block_cols, int row_major) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  int nb = K / block_cols;
  if (i >= (size_t)N * nb) return;
  int n = (int)(i / nb), b = (int)(i % nb);
  const int8_t* p = src + (size_t)n * K + (size_t)b * block_cols;
  int acc = 0;
  for (int k = 0; k < block_cols; k += 16) {
    v4i v = ld16(p + k);
    int w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc += (int)(int8_t)(w[j] & 0xFF) + (int)(int8_t)((w[j] >> 8) & 0xFF) +
             (int)(int8_t)((w[j] >> 16) & 0xFF) + (int)(int8_t)((w[j] >> 24) & 0xFF);
    }
  }
  float s = (float)acc;
  if (row_major) colsum[(size_t)n * nb + b] = s;
  else colsum[(size_t)b * N + n] = s;
}

// Offline weight encoder (rotate_and_quant, kernels.mojo:148-168): one
// workgroup per row.  bf16 row -> f32 (x gamma, quantizer.mojo:1011-1017)
// in LDS -> FWHT(B) per segment -> per-row (scale amax/127) or per-block
// int8.  Segments of S = max(B,64) values are handled one per wave.
template <int R>
__global__ __launch_bounds__(256) void k_quantize_weight(
    const uint16_t* __restrict__ w, const float* __restrict__ gamma, int8_t* __restrict__ q,
    float* __restrict__ scales, int cols, int block, float fwht_scale, int per_block) {
  extern __shared__ float row[];
  __shared__ float red[4];
  const int r = blockIdx.x;
  const uint16_t* src = w + (size_t)r * cols;
  for (int k = threadIdx.x; k < cols; k += blockDim.x) {
    float x = bf16_to_f32(src[k]);
    if (gamma) x = x * gamma[k];
    row[k] = x;
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int nwaves = blockDim.x >> 6;
  const int S = R * kWave;
  const int nseg = cols / S;
  float wmax = 0.0f;
  for (int sg = wave; sg < nseg; sg += nwaves) {
    float v[R];
#pragma unroll
    for (int i = 0; i < R; ++i) v[i] = row[sg * S + i * kWave + lane];
    fwht_wave<R>(v, block);
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      v[i] = v[i] * fwht_scale;
      row[sg * S + i * kWave + lane] = v[i];
      m = fmaxf(m, fabsf(v[i]));
    }
    if (per_block) {
      // per-block scales: blocks inside this segment
      float bm = (block >= kWave) ? wave_max(m) : group_max(m, block);
      int nb = cols / block;
      if (block >= kWave) {
        float inv = bm > 0.0f ? 127.0f / bm : 0.0f;
#pragma unroll
        for (int i = 0; i < R; ++i)
          q[(size_t)r * cols + sg * S + i * kWave + lane] = quantize_i8(v[i], inv);
        if (lane == 0) scales[(size_t)r * nb + (sg * S) / block] = bm / 127.0f;
      } else {
        float inv = bm > 0.0f ? 127.0f / bm : 0.0f;
        q[(size_t)r * cols + sg * S + lane] = quantize_i8(v[0], inv);
        if ((lane % block) == 0) scales[(size_t)r * nb + (sg * S + lane) / block] = bm / 127.0f;
      }
    }
    wmax = fmaxf(wmax, m);
  }
  if (per_block) return;
  wmax = wave_max(wmax);
  if (lane == 0) red[wave] = wmax;
  __syncthreads();
  float amax = red[0];
  for (int i = 1; i < nwaves; ++i) amax = fmaxf(amax, red[i]);
  float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  for (int k = threadIdx.x; k < cols; k += blockDim.x)
    q[(size_t)r * cols + k] = quantize_i8(row[k], inv);
  if (threadIdx.x == 0) scales[r] = amax / 127.0f;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
static inline unsigned blocks_for(size_t n, unsigned t) { return (unsigned)((n + t - 1) / t); }

hipError_t launch_retile(const int8_t* src, int layout, int8_t* dst, int N, int K,
                         hipStream_t st) {
  size_t chunks = (size_t)N * K / 16;
  if (chunks == 0) return hipSuccess;
  if (layout == 0)
    hipLaunchKernelGGL(k_retile_rowmajor, dim3(blocks_for(chunks, 256)), dim3(256), 0, st, src,
                       dst, N, K);
  else
    hipLaunchKernelGGL(k_retile_vnni, dim3(blocks_for(chunks, 256)), dim3(256), 0, st, src, dst,
                       N, K);
  return hipGetLastError();
}

hipError_t launch_unpack(const int8_t* src, int8_t* dst, int N, int K, hipStream_t st) {
  size_t chunks = (size_t)N * K / 16;
  if (chunks == 0) return hipSuccess;
  hipLaunchKernelGGL(k_unpack_tiled, dim3(blocks_for(chunks, 256)), dim3(256), 0, st, src, dst,
                     N, K);
  return hipGetLastError();
}

hipError_t launch_pack_colsum(const int8_t* src, int8_t* dst, float* colsum, int N, int K,
                              int block_cols, int row_major, hipStream_t st) {
  size_t dwords = (size_t)N * K / 4;
  if (dwords == 0) return hipSuccess;
  size_t ncs = (size_t)N * (K / block_cols);
  if (colsum)
    hipLaunchKernelGGL(k_colsum, dim3(blocks_for(ncs, 256)), dim3(256), 0, st, src, colsum, N,
                       K, block_cols, row_major);
  hipLaunchKernelGGL(k_pack_vnni, dim3(blocks_for(dwords, 256)), dim3(256), 0, st, src, dst, N,
                     K);
  return hipGetLastError();
}

hipError_t launch_quantize_weight(const uint16_t* w, const float* gamma, int8_t* q,
                                  float* scales, int rows, int cols, int block, int per_block,
                                  hipStream_t st) {
  if (rows == 0) return hipSuccess;
  float sc = fwht_scale_host(block);
  size_t lds = (size_t)cols * sizeof(float);
  dim3 g(rows), b(256);
  switch (block < 64 ? 1 : block / 64) {
    case 1: hipLaunchKernelGGL(k_quantize_weight<1>, g, b, lds, st, w, gamma, q, scales, cols, block, sc, per_block); break;
    case 2: hipLaunchKernelGGL(k_quantize_weight<2>, g, b, lds, st, w, gamma, q, scales, cols, block, sc, per_block); break;
    case 4: hipLaunchKernelGGL(k_quantize_weight<4>, g, b, lds, st, w, gamma, q, scales, cols, block, sc, per_block); break;
    case 8: hipLaunchKernelGGL(k_quantize_weight<8>, g, b, lds, st, w, gamma, q, scales, cols, block, sc, per_block); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bq
