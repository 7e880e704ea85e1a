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
// bqc_stream_sweep: the same 16 MiB read over a sweep of launch shapes
//   (workgroups, waves per workgroup, loads in flight per wave), each with
//   its empty launch, so the GEMV's launch shape can be compared with the
//   best shape that reads the same bytes.
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

// The launch-shape sweep of the same read: workgroup b takes SPW
// consecutive 16-row tiles and part b % ksplit of their K (K64 / ksplit
// fragments of each), W waves splitting that part into U fragments each, all
// of a wave's loads issued at once (non-temporal, as above).  Each (tile,
// part) writes its 16 uint16 to out[(tile * ksplit + part) * 16 ..].  With
// `empty` the same grid reads nothing: the fixed cost of that launch shape.
template <int W, int U, int SPW>
__global__ __launch_bounds__(W * 64) void k_stream_shape(const int8_t* __restrict__ w, int K64,
                                                         int ksplit, int empty,
                                                         uint16_t* __restrict__ out) {
  __shared__ int part[W * 256];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int p = blockIdx.x % ksplit, g = blockIdx.x / ksplit;
  const int F = K64 / ksplit;
  v4i acc[SPW];
#pragma unroll
  for (int s = 0; s < SPW; ++s) acc[s] = v4i{0, 0, 0, 0};
  if (!empty) {
    v4i b[SPW][U];
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const int8_t* wb = w + ((size_t)(g * SPW + s) * K64 + (size_t)p * F + wave * U) * 1024 +
                         lane * 16;
#pragma unroll
      for (int u = 0; u < U; ++u)
        b[s][u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wb + (size_t)u * 1024));
    }
#pragma unroll
    for (int s = 0; s < SPW; ++s)
#pragma unroll
      for (int u = 0; u < U; ++u) acc[s] ^= b[s][u];
  }
#pragma unroll
  for (int s = 0; s < SPW; ++s) {
    if (s) __syncthreads();
    part[wave * 256 + 0 * 64 + lane] = acc[s].x;
    part[wave * 256 + 1 * 64 + lane] = acc[s].y;
    part[wave * 256 + 2 * 64 + lane] = acc[s].z;
    part[wave * 256 + 3 * 64 + lane] = acc[s].w;
    __syncthreads();
    if (threadIdx.x < 16) {
      int r = 0;
#pragma unroll
      for (int q = 0; q < W; ++q) r ^= part[q * 256 + threadIdx.x];
      out[((size_t)(g * SPW + s) * ksplit + p) * 16 + threadIdx.x] = (uint16_t)r;
    }
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

// The launch shapes of the sweep: {waves, fragments per wave, tiles per
// workgroup, K parts}; a shape reads tiles x K64 fragments when waves x
// fragments x K parts = K64 (64 here: the decode GEMV's K = 4096).
struct StreamShape { int w, u, spw, ksplit; };
static const StreamShape kShapes[] = {
    {16, 4, 1, 1}, {8, 8, 1, 1}, {4, 16, 1, 1}, {2, 32, 1, 1},
    {16, 2, 1, 2}, {8, 4, 1, 2}, {4, 8, 1, 2}, {2, 16, 1, 2},
    {16, 1, 1, 4}, {8, 2, 1, 4}, {4, 4, 1, 4}, {2, 8, 1, 4}, {1, 16, 1, 4},
    {8, 1, 1, 8}, {4, 2, 1, 8}, {2, 4, 1, 8}, {1, 8, 1, 8},
    {16, 4, 2, 1}, {8, 8, 2, 1},
};
constexpr int kNumShapes = sizeof(kShapes) / sizeof(kShapes[0]);

int bqc_stream_shapes(void) { return kNumShapes; }

// shape i's {waves, fragments per wave, tiles per workgroup, K parts}
int bqc_stream_shape(int i, int* desc) {
  if (i < 0 || i >= kNumShapes || !desc) return (int)hipErrorInvalidValue;
  desc[0] = kShapes[i].w; desc[1] = kShapes[i].u; desc[2] = kShapes[i].spw;
  desc[3] = kShapes[i].ksplit;
  return 0;
}

// Sweep shape i over tiles 16-row tiles of K64 = 64 fragments each (w:
// tiles * 64 KiB, 16-byte aligned; out: tiles * ksplit * 16 uint16; tiles a
// multiple of the shape's tiles per workgroup); empty != 0 launches the same
// grid reading nothing.  Returns a hipError_t.
int bqc_stream_sweep(const int8_t* w, int tiles, int i, int empty, uint16_t* out, void* stream) {
  if (!w || !out || tiles <= 0 || i < 0 || i >= kNumShapes) return (int)hipErrorInvalidValue;
  if (reinterpret_cast<uintptr_t>(w) & 15u) return (int)hipErrorInvalidValue;
  const StreamShape sh = kShapes[i];
  constexpr int K64 = 64;
  if (sh.w * sh.u * sh.ksplit != K64 || tiles % sh.spw) return (int)hipErrorInvalidValue;
  const dim3 g(tiles / sh.spw * sh.ksplit), b(sh.w * 64);
  hipStream_t st = (hipStream_t)stream;
#define BQC_SHAPE(W, U, S)                                                                   \
  if (sh.w == W && sh.u == U && sh.spw == S) {                                              \
    hipLaunchKernelGGL((k_stream_shape<W, U, S>), g, b, 0, st, w, K64, sh.ksplit, empty, out); \
    return (int)hipGetLastError();                                                          \
  }
  BQC_SHAPE(16, 4, 1) BQC_SHAPE(8, 8, 1) BQC_SHAPE(4, 16, 1) BQC_SHAPE(2, 32, 1)
  BQC_SHAPE(16, 2, 1) BQC_SHAPE(8, 4, 1) BQC_SHAPE(4, 8, 1) BQC_SHAPE(2, 16, 1)
  BQC_SHAPE(16, 1, 1) BQC_SHAPE(8, 2, 1) BQC_SHAPE(4, 4, 1) BQC_SHAPE(2, 8, 1)
  BQC_SHAPE(1, 16, 1) BQC_SHAPE(8, 1, 1) BQC_SHAPE(4, 2, 1) BQC_SHAPE(2, 4, 1)
  BQC_SHAPE(1, 8, 1) BQC_SHAPE(16, 4, 2) BQC_SHAPE(8, 8, 2)
#undef BQC_SHAPE
  return (int)hipErrorInvalidValue;
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
