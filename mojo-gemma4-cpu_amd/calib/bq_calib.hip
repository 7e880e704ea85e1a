// bq_calib.hip -- measurement kernels for the benchmark's measured ceilings.
// They are not part of the butterquant API (libbq_calib.so, separate from
// libbq.so) and compute nothing a caller uses.
//
// bqc_stream_read: the decode GEMV's launch shape and read pattern with the
//   arithmetic taken out.  One workgroup per 16-row tile of a tile16x64
//   weight (tile t at byte t * K64 * 1024), W = 2, 4, 8 or 16 waves splitting
//   the K64 fragments of 1 KiB evenly, each lane loading its 16 bytes of every
//   fragment of its slice, the whole slice requested at once with
//   non-temporal loads (k_gemv_m1<2, 32> and <4, 16>, k_linear_skinny<16,
//   false, 4> and <8, false, 8> do exactly this for K <= 4096).  Each wave's bytes are XOR-folded into one 16-byte value per
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
// bqc_lds_read, bqc_dma_l2, bqc_vmem_l2, bqc_mfma_chain: the LDS, L2 -> LDS,
//   L2 -> VGPR and MFMA
//   latency figures behind the tiled kernels' design.  Each workgroup times
//   itself in shader clocks (s_memtime after a barrier at both ends) and
//   writes its cycle count, so the figures come out per clock.
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

// LDS read rate: W waves, each lane reading 16-byte words of a 64 KiB LDS
// buffer, 64 consecutive words per wave and instruction (conflict-free),
// 8 reads in flight per iteration; the words are XOR-folded so no read is
// dropped.  cyc[block] = the block's cycles; fold[block * W*64 + t] = folds.
template <int W>
__global__ __launch_bounds__(W * 64) void k_lds_read(int iters, long long* __restrict__ cyc,
                                                     int* __restrict__ fold) {
  // 96 KiB, of which the first 64 are read: one workgroup per CU
  __shared__ v4i buf[6144];
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  for (int i = t; i < 4096; i += W * 64) buf[i] = v4i{i, i * 3, i ^ 5, i + 7};
  __syncthreads();
  const long long c0 = clock64();
  int acc = 0;
  for (int i = 0; i < iters; ++i) {
    v4i b[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) b[u] = buf[((((i * 8 + u) * 7 + wave) & 63) << 6) + lane];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= (b[u].x ^ b[u].y) ^ (b[u].z ^ b[u].w);
  }
  __syncthreads();
  const long long c1 = clock64();
  if (t == 0) cyc[blockIdx.x] = c1 - c0;
  fold[blockIdx.x * W * 64 + t] = acc;
}

// L2-resident global -> LDS DMA (global_load_lds_dwordx4, 1 KiB per
// instruction): W waves, each issuing 8 DMAs per iteration into its own 8
// KiB of LDS and waiting for them.  The source is `rows` rows of `stride`
// bytes; shape 0 reads 8 rows x 128 bytes per DMA (whole 128-byte lines),
// shape 1 16 rows x 64 bytes (the raw 16x16x64 MFMA fragment), walking the
// source's row blocks, then its column blocks.  Every block reads the same
// small source, so after the first pass L2 serves it.
template <int W, int SHAPE>
__global__ __launch_bounds__(W * 64) void k_dma_l2(const int8_t* __restrict__ src, int stride,
                                                   int rows, int iters, long long* __restrict__ cyc) {
  // 96 KiB (one workgroup per CU), of which W * 8 KiB are written
  static_assert(W * 8 <= 96, "LDS");
  __shared__ __attribute__((aligned(16))) int8_t lds[96 * 1024];
  const int t = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
  // this lane's row and 16-byte chunk within a DMA's block of rows
  const int r = SHAPE == 0 ? lane >> 3 : lane & 15;
  const int c = SHAPE == 0 ? lane & 7 : lane >> 4;
  constexpr int RPD = SHAPE == 0 ? 8 : 16;    // rows per DMA
  constexpr int CPD = SHAPE == 0 ? 128 : 64;  // bytes of a row per DMA
  const int col_blocks = stride / CPD, row_blocks = rows / RPD;
  const uint32_t l0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) int8_t*)lds;
  __syncthreads();
  const long long c0 = clock64();
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      // DMA index; workgroups start 37 blocks apart, so the CUs sharing an
      // L2 read different lines at any moment
      const int q = (i * 8 + d) * W + wave + (int)blockIdx.x * 37;
      const int rb = q % row_blocks, cb = (q / row_blocks) % col_blocks;
      const int8_t* g = src + (size_t)(rb * RPD + r) * stride + cb * CPD + c * 16;
      const uint32_t l = __builtin_amdgcn_readfirstlane(l0 + (uint32_t)((wave * 8 + d) * 1024));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                   :: "s"(l), "v"(g) : "memory", "m0");
#pragma clang diagnostic pop
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  __syncthreads();
  const long long c1 = clock64();
  if (t == 0) cyc[blockIdx.x] = c1 - c0;
}

// The same reads as k_dma_l2's shape 0 (8 rows x 128 bytes per wave
// instruction, workgroups staggered) into VGPRs instead of LDS: each wave
// issues 8 global_load_dwordx4 per iteration and folds them (XOR) before the
// next, so 8 KiB per wave are in flight.
template <int W>
__global__ __launch_bounds__(W * 64) void k_vmem_l2(const int8_t* __restrict__ src, int stride,
                                                    int rows, int iters, long long* __restrict__ cyc,
                                                    int* __restrict__ fold) {
  // 96 KiB of LDS, unused: one workgroup per CU, as the DMA probe
  __shared__ int pad[96 * 256];
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int r = lane >> 3, c = lane & 7;
  const int col_blocks = stride / 128, row_blocks = rows / 8;
  if (iters < 0) pad[t] = 0;  // never: keeps the allocation
  __syncthreads();
  const long long c0 = clock64();
  v4i acc = {0, 0, 0, 0};
  for (int i = 0; i < iters; ++i) {
    v4i b[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const int q = (i * 8 + d) * W + wave + (int)blockIdx.x * 37;
      const int rb = q % row_blocks, cb = (q / row_blocks) % col_blocks;
      b[d] = *reinterpret_cast<const v4i*>(src + (size_t)(rb * 8 + r) * stride + cb * 128 + c * 16);
    }
#pragma unroll
    for (int d = 0; d < 8; ++d) acc ^= b[d];
  }
  __syncthreads();
  const long long c1 = clock64();
  if (t == 0) cyc[blockIdx.x] = c1 - c0;
  fold[blockIdx.x * W * 64 + t] = acc.x ^ acc.y ^ acc.z ^ acc.w ^ (iters < 0 ? pad[t] : 0);
}

// One wave's dependent v_mfma_i32_16x16x64_i8 chain (each MFMA takes the
// previous one's result as its accumulator): cycles per link.
__global__ __launch_bounds__(64) void k_mfma_chain(int n, long long* __restrict__ cyc,
                                                   int* __restrict__ out) {
  const int t = threadIdx.x;
  const v4i a = {t, t * 3, t * 5, t * 7}, b = {t ^ 1, t ^ 2, t ^ 3, t ^ 4};
  v4i c = {t, 0, 0, 0};
  const long long c0 = clock64();
  for (int i = 0; i < n; ++i) c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  // the last link's result is read before the clock stops
  int s = c.x + c.y + c.z + c.w;
  s = __builtin_amdgcn_readfirstlane(s);
  const long long c1 = clock64();
  if (t == 0) cyc[blockIdx.x] = c1 - c0;
  out[blockIdx.x * 64 + t] = s + t;
}

}  // namespace

extern "C" {

// w: tiles * K64 * 1024 bytes (16-byte aligned); out: tiles * 16 uint16;
// waves 8 or 16 (the GEMV's workgroup).  K64 <= 64 keeps the launch the
// GEMV's one-shot shape; K64 = 0 launches the same grid reading nothing (the
// fixed cost of a launch).  Returns a hipError_t.
int bqc_stream_read(const int8_t* w, int tiles, int K64, int waves, uint16_t* out, void* stream) {
  if (!w || !out || tiles <= 0 || K64 < 0 || K64 > 64 ||
      (waves != 2 && waves != 4 && waves != 8 && waves != 16))
    return (int)hipErrorInvalidValue;
  if (reinterpret_cast<uintptr_t>(w) & 15u) return (int)hipErrorInvalidValue;
  const hipStream_t st = (hipStream_t)stream;
  if (waves == 16)
    hipLaunchKernelGGL((k_stream_read<16, 4>), dim3(tiles), dim3(16 * 64), 0, st, w, K64, out);
  else if (waves == 8)
    hipLaunchKernelGGL((k_stream_read<8, 8>), dim3(tiles), dim3(8 * 64), 0, st, w, K64, out);
  else if (waves == 4)
    hipLaunchKernelGGL((k_stream_read<4, 16>), dim3(tiles), dim3(4 * 64), 0, st, w, K64, out);
  else
    hipLaunchKernelGGL((k_stream_read<2, 32>), dim3(tiles), dim3(2 * 64), 0, st, w, K64, out);
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

// LDS read rate: blocks of `waves` (4, 8 or 16) waves, iters x 8 reads of 16
// bytes per lane; cyc: blocks long longs (cycles per block), fold: blocks *
// waves * 64 ints.  Bytes read per block: waves * 64 * 16 * 8 * iters.
int bqc_lds_read(int waves, int blocks, int iters, long long* cyc, int* fold, void* stream) {
  if (!cyc || !fold || blocks <= 0 || iters <= 0) return (int)hipErrorInvalidValue;
  hipStream_t st = (hipStream_t)stream;
  if (waves == 4) hipLaunchKernelGGL(k_lds_read<4>, dim3(blocks), dim3(256), 0, st, iters, cyc, fold);
  else if (waves == 8) hipLaunchKernelGGL(k_lds_read<8>, dim3(blocks), dim3(512), 0, st, iters, cyc, fold);
  else if (waves == 16) hipLaunchKernelGGL(k_lds_read<16>, dim3(blocks), dim3(1024), 0, st, iters, cyc, fold);
  else return (int)hipErrorInvalidValue;
  return (int)hipGetLastError();
}

// L2-resident LDS DMA: blocks of `waves` (4 or 8) waves, iters x 8 DMAs of 1
// KiB per wave; shape 0 = 8 rows x 128 bytes, 1 = 16 rows x 64 bytes per
// DMA.  src: rows x stride bytes, 16-byte aligned (stride a multiple of 128,
// rows a multiple of 16).  cyc: blocks long longs.  Bytes per block: waves *
// 8 * 1024 * iters.
int bqc_dma_l2(int shape, int waves, const int8_t* src, int stride, int rows, int blocks,
               int iters, long long* cyc, void* stream) {
  if (!src || !cyc || blocks <= 0 || iters <= 0 || stride <= 0 || stride % 128 || rows <= 0 ||
      rows % 16 || (shape != 0 && shape != 1) || (reinterpret_cast<uintptr_t>(src) & 15u))
    return (int)hipErrorInvalidValue;
  hipStream_t st = (hipStream_t)stream;
#define BQC_DMA(W, S)                                                                        \
  if (waves == W && shape == S) {                                                            \
    hipLaunchKernelGGL((k_dma_l2<W, S>), dim3(blocks), dim3(W * 64), 0, st, src, stride, rows, \
                       iters, cyc);                                                          \
    return (int)hipGetLastError();                                                           \
  }
  BQC_DMA(4, 0) BQC_DMA(4, 1) BQC_DMA(8, 0) BQC_DMA(8, 1)
#undef BQC_DMA
  return (int)hipErrorInvalidValue;
}

// k_dma_l2's shape-0 reads into VGPRs: blocks of `waves` (4, 8 or 16) waves,
// iters x 8 loads of 1 KiB per wave (src as for bqc_dma_l2); cyc: blocks
// long longs, fold: blocks * waves * 64 ints.
int bqc_vmem_l2(int waves, const int8_t* src, int stride, int rows, int blocks, int iters,
                long long* cyc, int* fold, void* stream) {
  if (!src || !cyc || !fold || blocks <= 0 || iters <= 0 || stride <= 0 || stride % 128 ||
      rows <= 0 || rows % 16 || (reinterpret_cast<uintptr_t>(src) & 15u))
    return (int)hipErrorInvalidValue;
  hipStream_t st = (hipStream_t)stream;
  if (waves == 4)
    hipLaunchKernelGGL(k_vmem_l2<4>, dim3(blocks), dim3(256), 0, st, src, stride, rows, iters, cyc, fold);
  else if (waves == 8)
    hipLaunchKernelGGL(k_vmem_l2<8>, dim3(blocks), dim3(512), 0, st, src, stride, rows, iters, cyc, fold);
  else if (waves == 16)
    hipLaunchKernelGGL(k_vmem_l2<16>, dim3(blocks), dim3(1024), 0, st, src, stride, rows, iters, cyc, fold);
  else
    return (int)hipErrorInvalidValue;
  return (int)hipGetLastError();
}

// A dependent chain of n v_mfma_i32_16x16x64_i8 in one wave per block; cyc:
// blocks long longs, out: blocks * 64 ints.
int bqc_mfma_chain(int n, int blocks, long long* cyc, int* out, void* stream) {
  if (!cyc || !out || n <= 0 || blocks <= 0) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(k_mfma_chain, dim3(blocks), dim3(64), 0, (hipStream_t)stream, n, cyc, out);
  return (int)hipGetLastError();
}

}  // extern "C"
