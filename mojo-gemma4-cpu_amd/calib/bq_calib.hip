// bq_calib.hip -- measurement kernels for the benchmark's measured ceilings.
// They are not part of the butterquant API (libbq_calib.so, separate from
// libbq.so) and compute nothing a caller uses.
//
// bqc_stream_read: the decode GEMV's launch shape and read pattern with the
//   arithmetic taken out.  One workgroup per 16-row tile of a tile16x64
//   weight (tile t at byte t * K64 * 1024), W = 8 or 16 waves splitting the
//   K64 fragments of 1 KiB evenly, each lane loading its 16 bytes of every
//   fragment of its slice, the whole slice requested at once with
//   non-temporal loads (k_linear_skinny<16, false, 4> and <8, false, 8> do
//   exactly this for K <= 4096).  Each wave's bytes are XOR-folded into one 16-byte value per
//   lane, the waves' partial tiles reduced through LDS as the GEMV reduces its
//   int32 tiles, and 16 uint16 written per workgroup, the GEMV's 16 bf16
//   outputs.  Its per-launch time is the
//   ceiling of a kernel of this shape that reads these bytes.
// bqc_mfma_i8: back-to-back int8 MFMAs from registers (8 or 16 independent
//   v_mfma_i32_16x16x64_i8 chains, or 4 v_mfma_i32_32x32x32_i8 chains, per
//   wave), 4 waves per workgroup; one int per thread written at the end.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

namespace {

template <int kWaves, int kU>
__global__ __launch_bounds__(kWaves * 64) void k_stream_read(const int8_t* __restrict__ w,
                                                             int K64, uint16_t* __restrict__ out) {
  __shared__ int part[kWaves * 256];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int per = (K64 + kWaves - 1) / kWaves;
  const int kt0 = min(K64, wave * per), kt1 = min(K64, kt0 + per);
  const int8_t* wb = w + (size_t)blockIdx.x * K64 * 1024 + lane * 16;
  v4i acc = {0, 0, 0, 0};
  for (int kt = kt0; kt < kt1; kt += kU) {
    v4i b[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u)
      b[u] = __builtin_nontemporal_load(
          reinterpret_cast<const v4i*>(wb + (size_t)min(kt + u, kt1 - 1) * 1024));
#pragma unroll
    for (int u = 0; u < kU; ++u) acc ^= b[u];
  }
  // the GEMV's exact reduction of the waves' partial 16x16 tiles through LDS
  part[wave * 256 + 0 * 64 + lane] = acc.x;
  part[wave * 256 + 1 * 64 + lane] = acc.y;
  part[wave * 256 + 2 * 64 + lane] = acc.z;
  part[wave * 256 + 3 * 64 + lane] = acc.w;
  __syncthreads();
  if (threadIdx.x < 16) {
    int r = 0;
#pragma unroll
    for (int q = 0; q < kWaves; ++q) r ^= part[q * 256 + threadIdx.x];
    out[blockIdx.x * 16 + threadIdx.x] = (uint16_t)r;
  }
}

template <int SHAPE>
__global__ __launch_bounds__(256) void k_mfma_i8(int iters, int* __restrict__ out) {
  const int t = threadIdx.x + blockIdx.x;
  const v4i a = {t, t * 3, t * 5, t * 7}, b = {t ^ 1, t ^ 2, t ^ 3, t ^ 4};
  int s = 0;
  if constexpr (SHAPE == 16) {
    v4i c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = v4i{j, 0, 0, 0};
    for (int i = 0; i < iters; ++i) {
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c[j], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) s += c[j].x + c[j].y + c[j].z + c[j].w;
  } else if constexpr (SHAPE == 17) {  // 16x16x64 with 16 chains, 2 per 32x32x32's work
    v4i c[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) c[j] = v4i{j, 0, 0, 0};
    for (int i = 0; i < iters; i += 2) {
#pragma unroll
      for (int j = 0; j < 16; ++j) c[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c[j], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) s += c[j].x + c[j].y + c[j].z + c[j].w;
  } else {
    v16i c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int e = 0; e < 16; ++e) c[j][e] = j + e;
    }
    for (int i = 0; i < iters; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[j], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) s += c[j][e];
  }
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace

extern "C" {

// w: tiles * K64 * 1024 bytes (16-byte aligned); out: tiles * 16 uint16;
// waves 8 or 16 (the GEMV's workgroup).  K64 <= 64 keeps the launch the
// GEMV's one-shot shape; K64 = 0 launches the same grid reading nothing (the
// fixed cost of a launch).  Returns a hipError_t.
int bqc_stream_read(const int8_t* w, int tiles, int K64, int waves, uint16_t* out, void* stream) {
  if (!w || !out || tiles <= 0 || K64 < 0 || K64 > 64 || (waves != 8 && waves != 16))
    return (int)hipErrorInvalidValue;
  if (reinterpret_cast<uintptr_t>(w) & 15u) return (int)hipErrorInvalidValue;
  if (waves == 16)
    hipLaunchKernelGGL((k_stream_read<16, 4>), dim3(tiles), dim3(16 * 64), 0, (hipStream_t)stream,
                       w, K64, out);
  else
    hipLaunchKernelGGL((k_stream_read<8, 8>), dim3(tiles), dim3(8 * 64), 0, (hipStream_t)stream,
                       w, K64, out);
  return (int)hipGetLastError();
}

// shape 16 (v_mfma_i32_16x16x64_i8, 32768 ops each, 8 chains), 17 (the same
// instruction on 16 chains; iters even) or 32 (v_mfma_i32_32x32x32_i8, 65536
// ops each, 4 chains): 262144 ops per wave and iteration; blocks of 256
// threads; out: blocks * 256 ints.  Returns a hipError_t.
int bqc_mfma_i8(int shape, int blocks, int iters, int* out, void* stream) {
  if (!out || blocks <= 0 || iters <= 0 || (shape != 16 && shape != 17 && shape != 32) ||
      (shape == 17 && (iters & 1)))
    return (int)hipErrorInvalidValue;
  if (shape == 16)
    hipLaunchKernelGGL(k_mfma_i8<16>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, out);
  else if (shape == 17)
    hipLaunchKernelGGL(k_mfma_i8<17>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, out);
  else
    hipLaunchKernelGGL(k_mfma_i8<32>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, out);
  return (int)hipGetLastError();
}

// int8 ops that one call performs
double bqc_mfma_i8_ops(int shape, int blocks, int iters) {
  const double per = 262144.0;  // 8 x 32768 = 16 x 32768 / 2 = 4 x 65536
  return per * iters * (double)blocks * 4.0;  // 4 waves per block
}

}  // extern "C"
