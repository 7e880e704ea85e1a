// bq_head.hip -- the butterquant vocabulary head and embedding
// (butterquant_kernels/head.mojo, butterquant_kernels/embedding.mojo).
//
// Head prep (BqHeadPrepKernel, head.mojo:25-78 -> runtime.mojo:11-47): the
//   norm-quant of the final hidden rows with per-block activation scales.
// Flash sample (BqFlashSampleKernel, head.mojo:81-167, finalize_outcomes in
//   kernels/flash_sample.mojo:221-265), in two kernels:
//   1. k_head_logits streams the [V, H] int8 head once (tile16x64 strips of
//      16 vocabulary rows, every strip a contiguous H KiB run) and computes,
//      for every (row, vocabulary index), head_logit_row's per-block f32
//      chain, the softcap, the bf16 rounding, the Gumbel score; it stores
//      the bf16 logit and folds the score argmax and the log-sum-exp into
//      per-workgroup partials.
//   2. k_head_select, one workgroup per row, merges the partials and picks
//      the top 256 logits (value descending, lower index first: the order
//      SampleAccum.topn_insert keeps) by a two-level byte histogram of the
//      bf16 keys, then applies the min_p / top_k rule and writes the
//      SampleOutcome.
//   The argmax and the top-256 list are independent of how the vocabulary
//   is partitioned, so they match the reference exactly; the log-sum-exp is
//   a sum whose f32 rounding follows the partition (the reference's too).
// Embedding (BqEmbedLookupKernel, embedding.mojo:21-62): per token, the
//   owning shard's int8 row is dequantized per block, FWHT-rotated and
//   scaled to bf16.
#include "bq_device.hpp"
#include "bq_kernels.hpp"

namespace bq {

constexpr float kNegInf = -1.0e30f;  // kernels/flash_sample.mojo:17 NEG_INF

// ---------------------------------------------------------------------------
// head prep: per-block norm-quant, one workgroup (4 waves) per row; block =
// R*64, wave w takes blocks w, w+4, ...
// ---------------------------------------------------------------------------
template <int R>
__global__ __launch_bounds__(256) void k_head_prep(
    const uint16_t* __restrict__ src, const uint16_t* __restrict__ gamma,
    int8_t* __restrict__ xq, float* __restrict__ sa, int hidden, int pu, float sqrt_n,
    float n_eps, float fwht_scale) {
  const int t = blockIdx.x, wave = threadIdx.x >> 6, lane = lane_id();
  const uint16_t* x = src + (size_t)t * hidden;
  __shared__ float s_inv;
  if (wave == 0) {
    const float ssq = wave_row_ssq(reinterpret_cast<const uint32_t*>(x), hidden, pu);
    if (lane == 0) s_inv = sqrt_n / __builtin_sqrtf(ssq + n_eps);
  }
  __syncthreads();
  const float inv_rms = s_inv;
  constexpr int B = R * kWave;
  const int nb = hidden / B;
  for (int b = wave; b < nb; b += 4) {
    float v[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int k = b * B + i * kWave + lane;
      v[i] = bf16_to_f32(x[k]) * inv_rms * bf16_to_f32(gamma[k]);
    }
    fwht_wave<R>(v, B);
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      v[i] = v[i] * fwht_scale;
      m = fmaxf(m, fabsf(v[i]));
    }
    const float amax = wave_max(m);
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
#pragma unroll
    for (int i = 0; i < R; ++i) xq[(size_t)t * hidden + b * B + i * kWave + lane] = quantize_i8(v[i], inv);
    if (lane == 0) sa[(size_t)t * nb + b] = amax;
  }
}

// Head prep with FWHT block 128 (hidden % 256 == 0, hidden <= 128 * NSEG <=
// 4096, 16-byte aligned gain, 8-byte aligned codes): a workgroup of
// ceil(hidden / 512) waves per row, wave w holding values 512w .. 512w + 511
// as 8 consecutive values per lane, so a 128-value block is one row of 16
// lanes and its scale is the max over those lanes.  The same norm and
// transform as the per-row norm-quant (nq_pair_sumsq's chains, x * inv_rms *
// gain, nq_v8_transform), quantized per block (runtime.mojo:11-37 with a
// per-block scale).
template <int NSEG>
__global__ __launch_bounds__(512) void k_head_prep_v8(
    const uint16_t* __restrict__ src, const uint16_t* __restrict__ gamma,
    int8_t* __restrict__ xq, float* __restrict__ sa, int hidden, float sqrt_n, float n_eps,
    float fwht_scale) {
  const int lane = lane_id(), wave = threadIdx.x >> 6;
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
  m = fmaxf(m, xlane_partner<8>(m));  // the block's 16 lanes
  m = fmaxf(m, xlane_partner<4>(m));
  m = fmaxf(m, xlane_partner<2>(m));
  m = fmaxf(m, xlane_partner<1>(m));
  if (e0 < hidden) {  // a whole 16-lane block is in or out (hidden % 128 == 0)
    uint32_t w[2];
    nq_v8_codes(v, m > 0.0f ? 127.0f / m : 0.0f, w);
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u2*>(xq + (size_t)t * hidden + e0) = u2{w[0], w[1]};
    if ((lane & 15) == 0) sa[(size_t)t * nseg + (e0 >> 7)] = m;
  }
}

// ---------------------------------------------------------------------------
// embedding lookup: one workgroup (4 waves) per token; wave w rotates blocks
// w, w+4, ... of the row read from the tile16x64 layout.
// ---------------------------------------------------------------------------
template <int R>
__global__ __launch_bounds__(256) void k_embed(
    const int32_t* __restrict__ tokens, const int8_t* __restrict__ w,
    const float* __restrict__ ws, uint16_t* __restrict__ dst, int hidden, int shard_rows,
    int rank, float scale, float fwht_scale) {
  const int t = blockIdx.x, wave = threadIdx.x >> 6, lane = lane_id();
  constexpr int B = R * kWave;
  const int nb = hidden / B;
  const int tid = tokens[t];
  // the owner is Mojo's floor division tid // shard_rows (embedding.mojo:42):
  // a negative id belongs to no rank and gives a zero row
  const int owner = tid / shard_rows - ((tid % shard_rows != 0 && tid < 0) ? 1 : 0);
  uint16_t* d = dst + (size_t)t * hidden;
  if (owner != rank) {  // embedding.mojo:53: zero_row for another shard's token
    for (int k = threadIdx.x; k < hidden; k += blockDim.x) d[k] = 0;
    return;
  }
  const int n = tid - owner * shard_rows;
  for (int b = wave; b < nb; b += 4) {
    const float s = ws[(size_t)n * nb + b];
    float v[R];
#pragma unroll
    for (int i = 0; i < R; ++i) v[i] = (float)w[tile_offset(n, b * B + i * kWave + lane, hidden)] * s;
    fwht_wave<R>(v, B);
#pragma unroll
    for (int i = 0; i < R; ++i) d[b * B + i * kWave + lane] = f32_to_bf16(v[i] * fwht_scale * scale);
  }
}

// ---------------------------------------------------------------------------
// flash sample, pass 1
// ---------------------------------------------------------------------------
struct HeadArgs {
  const int8_t* x;         // [R, H] int8 activation
  const float* xsa;        // [R, H/block]
  const int8_t* w;         // [V, H] tile16x64
  const float* ws;         // [V, H/block]
  const SamplingParams* params;
  uint16_t* y;             // [R, V] bf16 logits (workspace)
  float* part;             // [grid, 4, RP] partials (workspace)
  uint32_t* tot1;          // [R, 256] the selection's row histogram, cleared here
  int R, V, H, block, nstrips;
  float cap;
  int64_t vbase;
};

constexpr int kHeadWaves = 8;

// LSE accumulator merge (SampleAccum.merge, flash_sample.mojo:92-104)
__device__ inline void lse_merge(float& mx, float& sum, float omx, float osum) {
  if (osum > 0.0f) {
    if (sum <= 0.0f) {
      mx = omx;
      sum = osum;
    } else if (omx > mx) {
      sum = sum * exp_f32(mx - omx) + osum;
      mx = omx;
    } else {
      sum = sum + osum * exp_f32(omx - mx);
    }
  }
}

// score argmax, ties to the lower vocabulary index
__device__ inline void samp_merge(float& s, int& i, float os, int oi) {
  if (os > s || (os == s && oi < i)) {
    s = os;
    i = oi;
  }
}

template <int MI, int CH>
__global__ __launch_bounds__(64 * kHeadWaves) void k_head_logits(HeadArgs a) {
  constexpr int RP = 16 * MI;  // padded rows
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int H = a.H, K64 = H >> 6, nb = H / a.block, fpb = a.block >> 6;
  const int xstride = H + 16;  // padded LDS row stride (bank spread)
  extern __shared__ __attribute__((aligned(16))) int8_t smem[];
  int8_t* s_x = smem;                                                   // [RP][H+16]
  if (blockIdx.x == 0)  // the selection's first pass adds into it after this launch
    for (int i = threadIdx.x; i < a.R * 256; i += blockDim.x) a.tot1[i] = 0u;
  float* s_sa = reinterpret_cast<float*>(smem + (size_t)RP * xstride);  // [nb][RP] sa/127
  __shared__ float s_invt[RP];
  __shared__ uint64_t s_seed[RP];
  __shared__ int s_greedy[RP];
  __shared__ float s_red[kHeadWaves][4][RP];

  // The wave's strips s0, s0 + stride, ... as a sequence of chunks of CH
  // fragments (a strip's last chunk may be partial: its clamped loads are
  // never multiplied), two register slots deep: chunk i + 1's fragments and
  // block scales are in flight while chunk i multiplies.  Every block (fpb
  // fragments; the launch picks CH with fpb dividing CH, and K64 is a
  // multiple of fpb) lies inside one chunk; its int32 MFMA chain starts
  // from zero and is drained into the f32 sum once.
  const int stride = gridDim.x * kHeadWaves;
  const int s0 = blockIdx.x * kHeadWaves + wave;
  const int nch = (K64 + CH - 1) / CH;
  const int nmine = s0 < a.nstrips ? (a.nstrips - 1 - s0) / stride + 1 : 0;
  const int nsteps = nmine * nch;
  const int bpc = CH / fpb;  // blocks per chunk
  v4i wf[2][CH];
  float wsc[2][CH];
  auto load = [&](int slot, int step) {
    const int si = step / nch, ch = step - si * nch;
    const int s = s0 + si * stride;
    const int8_t* wstrip = a.w + (size_t)s * K64 * 1024 + lane * 16;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      wf[slot][j] = *reinterpret_cast<const v4i*>(wstrip + (size_t)min(ch * CH + j, K64 - 1) * 1024);
    }
    const float* wsr = a.ws + (size_t)(s * 16 + (lane & 15)) * nb;
#pragma unroll
    for (int q = 0; q < CH; ++q)
      if (q < bpc) wsc[slot][q] = wsr[min(ch * bpc + q, nb - 1)];
  };
  // the first chunk's loads go out before the activation tile is staged,
  // so their latency overlaps the staging's
  if (nsteps > 0) load(0, 0);

  for (int i = threadIdx.x; i < RP * (H / 16); i += blockDim.x) {
    const int r = i / (H / 16), c = i % (H / 16);
    v4i v = {0, 0, 0, 0};
    if (r < a.R) v = *reinterpret_cast<const v4i*>(a.x + (size_t)r * H + c * 16);
    *reinterpret_cast<v4i*>(s_x + (size_t)r * xstride + c * 16) = v;
  }
  for (int i = threadIdx.x; i < RP * nb; i += blockDim.x) {
    const int b = i / RP, r = i % RP;
    // head_logit_row divides: sa[b] / 127 (dot_products.mojo:87)
    s_sa[i] = r < a.R ? a.xsa[(size_t)r * nb + b] / 127.0f : 0.0f;
  }
  if (threadIdx.x < RP) {
    const int r = threadIdx.x;
    const SamplingParams p = a.params[r < a.R ? r : 0];
    s_invt[r] = 1.0f / p.temperature;
    s_seed[r] = p.seed;
    s_greedy[r] = p.greedy != 0;
  }
  // (not __syncthreads: its fence would wait for the chunk loads in flight)
  lds_barrier();

  // running partials per (mi, v) row slot: rows 16*mi + 4*(lane>>4) + v
  float best[MI][4], lmx[MI][4], lsum[MI][4];
  int bidx[MI][4];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      best[mi][v] = kNegInf;
      bidx[mi][v] = 0x7FFFFFFF;
      lmx[mi][v] = kNegInf;
      lsum[mi][v] = 0.0f;
    }

  float raw[MI][4];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int v = 0; v < 4; ++v) raw[mi][v] = 0.0f;
  auto compute = [&](int slot, int step) {
    const int si = step / nch, ch = step - si * nch;
#pragma unroll
    for (int j0 = 0; j0 < CH; ++j0) {
      const int f = ch * CH + j0;
      if (f >= K64 || (j0 % fpb) != 0) continue;
      const int b = f / fpb;
      const float wsb = wsc[slot][j0 / fpb];
      v4i acc[MI];
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) acc[mi] = {0, 0, 0, 0};
#pragma unroll
      for (int q = 0; q < CH; ++q) {
        if (q >= fpb) break;
        const int ff = f + q;
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
          const v4i xa = *reinterpret_cast<const v4i*>(
              s_x + (size_t)(16 * mi + (lane & 15)) * xstride + ff * 64 + (lane >> 4) * 16);
          acc[mi] = mfma16x16x64(xa, wf[slot][(j0 + q) % CH], acc[mi]);
        }
      }
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
        const float4 sv = *reinterpret_cast<const float4*>(s_sa + b * RP + 16 * mi + 4 * (lane >> 4));
        raw[mi][0] = raw[mi][0] + (float)acc[mi][0] * sv.x * wsb;
        raw[mi][1] = raw[mi][1] + (float)acc[mi][1] * sv.y * wsb;
        raw[mi][2] = raw[mi][2] + (float)acc[mi][2] * sv.z * wsb;
        raw[mi][3] = raw[mi][3] + (float)acc[mi][3] * sv.w * wsb;
      }
    }
    if (ch != nch - 1) return;  // uniform
    // the strip's epilogue: y = bf16(softcap(raw)), score = y/T + gumbel
    const int col = (s0 + si * stride) * 16 + (lane & 15);  // this lane's vocabulary row
    const int64_t gidx = a.vbase + col;
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = 16 * mi + 4 * (lane >> 4) + v;
        const float rv = raw[mi][v];
        raw[mi][v] = 0.0f;
        if (r >= a.R) continue;
        const uint16_t yb = f32_to_bf16(tanh_f32(rv / a.cap) * a.cap);
        a.y[(size_t)r * a.V + col] = yb;
        const float yt = bf16_to_f32(yb) * s_invt[r];
        const float g = s_greedy[r] ? 0.0f : gumbel_noise(s_seed[r], r, gidx);
        samp_merge(best[mi][v], bidx[mi][v], yt + g, (int)gidx);
        // lse_push (flash_sample.mojo:77-85)
        lse_merge(lmx[mi][v], lsum[mi][v], yt, 1.0f);
      }
  };
  for (int st = 0; st < nsteps; st += 2) {
    if (st + 1 < nsteps) load(1, st + 1);
    compute(0, st);
    if (st + 1 >= nsteps) break;
    if (st + 2 < nsteps) load(0, st + 2);
    compute(1, st + 1);
  }

  // fold the 16 lanes sharing each row (lane & 15 = vocabulary column) and
  // then the waves, in a fixed order
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const float os = __shfl_xor(best[mi][v], o, 16);
        const int oi = __shfl_xor(bidx[mi][v], o, 16);
        const float om = __shfl_xor(lmx[mi][v], o, 16);
        const float ou = __shfl_xor(lsum[mi][v], o, 16);
        // the lower lane keeps the merge order (lower lane first)
        if (lane & o) {
          float m2 = om, s2 = ou;
          lse_merge(m2, s2, lmx[mi][v], lsum[mi][v]);
          lmx[mi][v] = m2;
          lsum[mi][v] = s2;
        } else {
          lse_merge(lmx[mi][v], lsum[mi][v], om, ou);
        }
        samp_merge(best[mi][v], bidx[mi][v], os, oi);
      }
      if ((lane & 15) == 0) {
        const int r = 16 * mi + 4 * (lane >> 4) + v;
        s_red[wave][0][r] = best[mi][v];
        s_red[wave][1][r] = __int_as_float(bidx[mi][v]);
        s_red[wave][2][r] = lmx[mi][v];
        s_red[wave][3][r] = lsum[mi][v];
      }
    }
  __syncthreads();
  if (threadIdx.x < RP) {
    const int r = threadIdx.x;
    float bs = kNegInf, mx = kNegInf, sm = 0.0f;
    int bi = 0x7FFFFFFF;
    for (int wv = 0; wv < kHeadWaves; ++wv) {
      samp_merge(bs, bi, s_red[wv][0][r], __float_as_int(s_red[wv][1][r]));
      lse_merge(mx, sm, s_red[wv][2][r], s_red[wv][3][r]);
    }
    float* part = a.part + (size_t)blockIdx.x * 4 * RP;
    part[0 * RP + r] = bs;
    part[1 * RP + r] = __int_as_float(bi);
    part[2 * RP + r] = mx;
    part[3 * RP + r] = sm;
  }
}

// ---------------------------------------------------------------------------
// flash sample, pass 2: exact top-256 selection over the bf16 logits of each
// row, spread over chunks of 4096 logits (one workgroup each), then one
// workgroup per row to sort and finalize.
//   hist_hi   : per chunk, a histogram of the keys' high byte
//   thr_hi    : per row, the high byte hb of the 256th largest key
//   hist_lo   : per chunk, a histogram of the low byte among keys in hb
//   thr_lo    : per row, the threshold key t, the count of keys above it,
//               how many ties (keys equal to t) are needed, and each chunk's
//               count of earlier ties
//   collect   : per chunk, appends the keys above t and the needed ties
//               (lowest indices first) to the row's candidate list
//   finalize  : per row, sorts the 256 candidates, applies min_p / top_k,
//               writes the SampleOutcome
// ---------------------------------------------------------------------------
constexpr int kChunk = 4096, kChunkThreads = 256;  // 16 logits per thread
constexpr int kSelThreads = 256, kSelWaves = kSelThreads / 64;

// bf16 bits -> unsigned order (-0 taken as +0: the reference compares floats)
__device__ inline uint32_t bf16_key(uint16_t b) {
  if (b == 0x8000u) b = 0;
  return (b & 0x8000u) ? (uint32_t)(~b & 0xFFFFu) : (uint32_t)(b | 0x8000u);
}
__device__ inline uint16_t key_bf16(uint32_t k) {
  return (k & 0x8000u) ? (uint16_t)(k & 0x7FFFu) : (uint16_t)(~k & 0xFFFFu);
}

struct SelArgs {
  const uint16_t* y;   // [R, V]
  uint32_t* tot1;      // [R, 256] high-byte histogram of the row (all chunks)
  uint32_t* tot2;      // [R, 256] low-byte histogram of the row's keys in bin hb
  uint32_t* hist2;     // [R, nc, 256]
  int* thr;            // [R, 4]: hb, keys above hb, threshold key, ties needed
  int* eqpre;          // [R, nc] ties in earlier chunks
  int* cnt;            // [R] candidates appended
  uint64_t* cand;      // [R, 256] (key << 32) | (0x7FFFFFFF - index)
  int V, nc;
  int fused;           // 1: each chunk workgroup derives its row's thresholds itself
};

// this thread's 16 keys of chunk c (V % 16 == 0: all valid or none)
__device__ inline bool chunk_keys(const SelArgs& a, int r, int c, uint32_t (&k)[16]) {
  const int i0 = c * kChunk + threadIdx.x * 16;
  if (i0 >= a.V) return false;
  const v4i* src = reinterpret_cast<const v4i*>(a.y + (size_t)r * a.V + i0);
  const v4i u0 = src[0], u1 = src[1];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    k[2 * q] = bf16_key((uint16_t)((uint32_t)u0[q] & 0xFFFFu));
    k[2 * q + 1] = bf16_key((uint16_t)((uint32_t)u0[q] >> 16));
    k[8 + 2 * q] = bf16_key((uint16_t)((uint32_t)u1[q] & 0xFFFFu));
    k[8 + 2 * q + 1] = bf16_key((uint16_t)((uint32_t)u1[q] >> 16));
  }
  return true;
}

// LDS histogram increment (no return value: the hardware serializes only
// the lanes of one instruction that hit the same bin)
__device__ inline void hist_add(uint32_t* hist, uint32_t bin, bool active) {
  if (active) atomicAdd(&hist[bin], 1u);
}

__global__ __launch_bounds__(kChunkThreads) void k_sel_hist_hi(SelArgs a) {
  const int c = blockIdx.x, r = blockIdx.y, tid = threadIdx.x;
  __shared__ uint32_t hist[256];
  hist[tid] = 0;
  if (c == 0 && tid == 0) a.cnt[r] = 0;
  __syncthreads();
  uint32_t k[16];
  const bool ok = chunk_keys(a, r, c, k);
#pragma unroll
  for (int q = 0; q < 16; ++q) hist_add(hist, ok ? k[q] >> 8 : 0u, ok);
  __syncthreads();
  // the row's histogram: one atomic per non-empty bin; chunk 0 also clears
  // the low-byte one the next pass adds into
  if (hist[tid]) atomicAdd(&a.tot1[r * 256 + tid], hist[tid]);
  if (c == 0) a.tot2[r * 256 + tid] = 0u;
}

// Block-wide inclusive suffix sum over 256 bins (bin 255 first), 256 threads.
__device__ inline int suffix_sum256(int v, int* tmp) {
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  // scan in descending bin order: reversed position j = 255 - tid
  int s = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_down(s, o, 64);  // lanes above hold higher bins
    if (lane + o < 64) s += u;
  }
  if (lane == 0) tmp[wave] = s;
  __syncthreads();
  int above = 0;
  for (int w = wave + 1; w < 4; ++w) above += tmp[w];
  __syncthreads();
  return s + above;
}

// Find bin b with suffix(b) >= need > suffix(b + 1); writes (b, suffix(b+1)).
__device__ inline void pick_bin(int suffix, int total, int need, int base, int* out_bin,
                                int* out_above) {
  const int tid = threadIdx.x;
  const int s_incl = base + suffix, s_excl = base + suffix - total;
  if (s_incl >= need && s_excl < need) {
    *out_bin = tid;
    *out_above = s_excl;
  }
}

// Row r's high byte hb of the 256th largest key and the count of keys in
// higher bins, from the row's high-byte histogram (all kChunkThreads
// threads call it; every thread gets the results).
__device__ inline void row_thr_hi(const SelArgs& a, int r, int& hb, int& above_hb) {
  const int tid = threadIdx.x;
  __shared__ int tmp[4];
  __shared__ int s_bin, s_above;
  const int total = (int)a.tot1[r * 256 + tid];
  const int need = a.V < kSampleNmax ? a.V : kSampleNmax;
  if (tid == 0) { s_bin = 0; s_above = 0; }
  __syncthreads();
  const int suf = suffix_sum256(total, tmp);
  pick_bin(suf, total, need, 0, &s_bin, &s_above);
  __syncthreads();
  hb = s_bin;
  above_hb = s_above;
}

__global__ __launch_bounds__(kChunkThreads) void k_sel_thr_hi(SelArgs a) {
  int hb, above;
  row_thr_hi(a, blockIdx.x, hb, above);
  if (threadIdx.x == 0) {
    a.thr[blockIdx.x * 4 + 0] = hb;
    a.thr[blockIdx.x * 4 + 1] = above;
  }
}

__global__ __launch_bounds__(kChunkThreads) void k_sel_hist_lo(SelArgs a) {
  const int c = blockIdx.x, r = blockIdx.y, tid = threadIdx.x;
  __shared__ uint32_t hist[256];
  hist[tid] = 0;
  uint32_t hb;
  if (a.fused) {  // uniform
    int b, above;
    row_thr_hi(a, r, b, above);  // (its barriers also cover the zeroing above)
    hb = (uint32_t)b;
    if (c == 0 && tid == 0) {
      a.thr[r * 4 + 0] = b;
      a.thr[r * 4 + 1] = above;
    }
  } else {
    __syncthreads();
    hb = (uint32_t)a.thr[r * 4 + 0];
  }
  uint32_t k[16];
  const bool ok = chunk_keys(a, r, c, k);
#pragma unroll
  for (int q = 0; q < 16; ++q) hist_add(hist, ok ? k[q] & 255u : 0u, ok && (k[q] >> 8) == hb);
  __syncthreads();
  a.hist2[((size_t)r * a.nc + c) * 256 + tid] = hist[tid];  // for the ties before each chunk
  if (hist[tid]) atomicAdd(&a.tot2[r * 256 + tid], hist[tid]);
}

// Row r's threshold key t (its 256th largest), the ties (keys == t) the
// selection needs, and the ties in the chunks before chunk `want` (every
// chunk's with want < 0, written to eqpre), from the row's low-byte
// histogram of the keys in bin hb and, for the ties, every chunk's count of
// the threshold key.  All kChunkThreads threads call it.
__device__ inline void row_thr_lo(const SelArgs& a, int r, int want, uint32_t& t_out,
                                  int& ties_out, int& eqb_out) {
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  __shared__ int tmp[4];
  __shared__ int s_bin, s_above, s_eqb;
  const int total = (int)a.tot2[r * 256 + tid];
  const int need = a.V < kSampleNmax ? a.V : kSampleNmax;
  const int hb = a.thr[r * 4 + 0], above_hb = a.thr[r * 4 + 1];
  if (tid == 0) { s_bin = 0; s_above = above_hb; }
  __syncthreads();
  const int suf = suffix_sum256(total, tmp);
  pick_bin(suf, total, need, above_hb, &s_bin, &s_above);
  __syncthreads();
  const int lb = s_bin;
  // ties (key == threshold) in the chunks before each chunk: exclusive scan
  // over chunks (nc <= 256: thread c holds chunk c)
  const int e = tid < a.nc ? (int)a.hist2[((size_t)r * a.nc + tid) * 256 + lb] : 0;
  int incl = wave_incl_scan(e);
  if (lane == 63) tmp[wave] = incl;
  __syncthreads();
  int before = 0;
  for (int w = 0; w < wave; ++w) before += tmp[w];
  if (want < 0 && tid < a.nc) a.eqpre[(size_t)r * a.nc + tid] = before + incl - e;
  if (tid == want) s_eqb = before + incl - e;
  __syncthreads();
  t_out = (uint32_t)((hb << 8) | lb);
  ties_out = need - s_above;
  eqb_out = want >= 0 ? s_eqb : 0;
}

__global__ __launch_bounds__(kChunkThreads) void k_sel_thr_lo(SelArgs a) {
  uint32_t t;
  int ties, eqb;
  row_thr_lo(a, blockIdx.x, -1, t, ties, eqb);
  if (threadIdx.x == 0) {
    a.thr[blockIdx.x * 4 + 2] = (int)t;
    a.thr[blockIdx.x * 4 + 3] = ties;  // ties needed
  }
}

__global__ __launch_bounds__(kChunkThreads) void k_sel_collect(SelArgs a) {
  const int c = blockIdx.x, r = blockIdx.y, tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  __shared__ int tmp_e[4], tmp_s[4];
  __shared__ int s_base;
  uint32_t t;
  int ties_needed, eq_before;
  if (a.fused) {  // uniform
    row_thr_lo(a, r, c, t, ties_needed, eq_before);
  } else {
    t = (uint32_t)a.thr[r * 4 + 2];
    ties_needed = a.thr[r * 4 + 3];
    eq_before = a.eqpre[(size_t)r * a.nc + c];
  }
  uint32_t k[16];
  const bool ok = chunk_keys(a, r, c, k);
  // ties before this thread's keys, in index order
  int n_eq = 0;
#pragma unroll
  for (int q = 0; q < 16; ++q) n_eq += (ok && k[q] == t) ? 1 : 0;
  int inc_e = wave_incl_scan(n_eq);
  if (lane == 63) tmp_e[wave] = inc_e;
  __syncthreads();
  int be = 0;
  for (int w = 0; w < wave; ++w) be += tmp_e[w];
  int rank = eq_before + be + inc_e - n_eq;
  // which of this thread's keys are selected
  uint32_t sel = 0;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const bool eq = ok && k[q] == t;
    if ((ok && k[q] > t) || (eq && rank < ties_needed)) sel |= 1u << q;
    rank += eq ? 1 : 0;
  }
  // one global atomic per workgroup reserves the chunk's slots
  const int n_sel = __popc(sel);
  int inc_s = wave_incl_scan(n_sel);
  if (lane == 63) tmp_s[wave] = inc_s;
  __syncthreads();
  if (tid == 0) {
    const int total = tmp_s[0] + tmp_s[1] + tmp_s[2] + tmp_s[3];
    s_base = total ? atomicAdd(&a.cnt[r], total) : 0;
  }
  __syncthreads();
  int pos = s_base + inc_s - n_sel;
  for (int w = 0; w < wave; ++w) pos += tmp_s[w];
  const int i0 = c * kChunk + tid * 16;
#pragma unroll
  for (int q = 0; q < 16; ++q)
    if (sel & (1u << q)) a.cand[(size_t)r * kSampleNmax + pos++] = ((uint64_t)k[q] << 32) | (uint32_t)(0x7FFFFFFF - (i0 + q));
}

__global__ __launch_bounds__(kSelThreads) void k_head_select(
    const uint64_t* __restrict__ cand_g, const float* __restrict__ part, int nparts, int RP,
    const SamplingParams* __restrict__ params, SampleOutcome* __restrict__ out, int V,
    int64_t vbase) {
  const int r = blockIdx.x, tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  __shared__ uint64_t cand[kSampleNmax];
  __shared__ int s_nout;
  __shared__ float s_score0;
  __shared__ float r_bs[kSelWaves], r_mx[kSelWaves], r_sm[kSelWaves], r_ps[kSelWaves];
  __shared__ int r_bi[kSelWaves], r_pk[kSelWaves];
  const SamplingParams p = params[r];
  // lane ^ stride's value (stride < 64) by the DPP / permlane moves of
  // xlane_partner: bit moves, no LDS
  auto partner = [](uint32_t x, int stride) -> uint32_t {
    const float f = __uint_as_float(x);
    switch (stride) {
      case 1: return __float_as_uint(xlane_partner<1>(f));
      case 2: return __float_as_uint(xlane_partner<2>(f));
      case 4: return __float_as_uint(xlane_partner<4>(f));
      case 8: return __float_as_uint(xlane_partner<8>(f));
      case 16: return __float_as_uint(xlane_partner<16>(f));
      default: return __float_as_uint(xlane_partner<32>(f));
    }
  };

  // 1. merge the per-workgroup partials in order
  float bs = kNegInf, mx = kNegInf, sm = 0.0f;
  int bi = 0x7FFFFFFF;
  {
    // thread i folds partials i, i + 256, ... in order; then the threads
    // fold in order through the waves
    for (int i = tid; i < nparts; i += kSelThreads) {
      const float* pp = part + (size_t)i * 4 * RP;
      samp_merge(bs, bi, pp[r], __float_as_int(pp[RP + r]));
      lse_merge(mx, sm, pp[2 * RP + r], pp[3 * RP + r]);
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float os = __uint_as_float(partner(__float_as_uint(bs), o));
      const int oi = (int)partner((uint32_t)bi, o);
      const float om = __uint_as_float(partner(__float_as_uint(mx), o));
      const float ou = __uint_as_float(partner(__float_as_uint(sm), o));
      if (lane & o) {
        float m2 = om, s2 = ou;
        lse_merge(m2, s2, mx, sm);
        mx = m2;
        sm = s2;
      } else {
        lse_merge(mx, sm, om, ou);
      }
      samp_merge(bs, bi, os, oi);
    }
    if (lane == 0) {
      r_bs[wave] = bs;
      r_bi[wave] = bi;
      r_mx[wave] = mx;
      r_sm[wave] = sm;
    }
  }

  // 2. the selected candidates, padded and sorted descending by
  // (key, -index): bitonic over 256 entries, one per thread, in registers.
  // A stride below 64 pairs lanes of one wave (partner on both halves of the
  // key, no barrier); strides
  // 64 and 128 (three of the 36 stages) pair waves through LDS, alternating
  // two buffers so one barrier per stage suffices.
  static_assert(kSampleNmax == kSelThreads, "one candidate per thread");
  const int need = V < kSampleNmax ? V : kSampleNmax;
  uint64_t key = tid < need ? cand_g[(size_t)r * kSampleNmax + tid] : 0ull;
  __shared__ uint64_t xch[2][kSampleNmax];
  int xb = 0;
#pragma unroll
  for (int size = 2; size <= kSampleNmax; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      uint64_t other;
      if (stride < 64) {
        const uint32_t lo = partner((uint32_t)key, stride);
        const uint32_t hi = partner((uint32_t)(key >> 32), stride);
        other = ((uint64_t)hi << 32) | lo;
      } else {
        xch[xb][tid] = key;
        __syncthreads();
        other = xch[xb][tid ^ stride];
        xb ^= 1;
      }
      // the lower entry of a pair takes the larger key in a descending run
      const bool take_max = ((tid & stride) == 0) == ((tid & size) == 0);
      key = take_max ? (other > key ? other : key) : (other < key ? other : key);
    }
  }
  cand[tid] = key;
  __syncthreads();

  // 3. finalize (flash_sample.mojo:232-265).  The min_p / top_k pick scans
  // the top list keeping the first strictly larger score among entries
  // 1..limit-1 that pass the min_p threshold, starting from entry 0: that is
  // entry 0 unless the best passing score M beats it, else the first entry
  // scoring M -- a max / min-index reduction over the 256 entries.
  const float inv_t = 1.0f / p.temperature;
  const bool use_min_p = p.min_p > 0.0f, use_top_k = p.top_k > 0;
  int limit = need;
  if (use_top_k && p.top_k < limit) limit = (int)p.top_k;
  const float v0 = bf16_to_f32(key_bf16((uint32_t)(cand[0] >> 32)));
  const float thr = use_min_p ? v0 + p.temperature * log_f32(p.min_p) : kNegInf;
  float sc = kNegInf;
  int kk = 0x7FFFFFFF;
  if (tid < need) {
    const float yv = bf16_to_f32(key_bf16((uint32_t)(cand[tid] >> 32)));
    const int64_t gi = vbase + (0x7FFFFFFF - (int)(uint32_t)cand[tid]);
    const float g = p.greedy ? 0.0f : gumbel_noise(p.seed, r, gi);
    const float score = yv * inv_t + g;
    if (tid == 0) s_score0 = score;
    if (tid >= 1 && tid < limit && yv >= thr) {
      sc = score;
      kk = tid;
    }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float os = __uint_as_float(partner(__float_as_uint(sc), o));
    const int ok = (int)partner((uint32_t)kk, o);
    if (os > sc || (os == sc && ok < kk)) {
      sc = os;
      kk = ok;
    }
  }
  if (lane == 0) {
    r_ps[wave] = sc;
    r_pk[wave] = kk;
  }
  __syncthreads();
  if (tid == 0) {
    float fbs = kNegInf, fmx = kNegInf, fsm = 0.0f;
    int fbi = 0x7FFFFFFF;
    for (int wv = 0; wv < kSelWaves; ++wv) {
      samp_merge(fbs, fbi, r_bs[wv], r_bi[wv]);
      lse_merge(fmx, fsm, r_mx[wv], r_sm[wv]);
    }
    const int n = need;
    const int n_out = (int64_t)n < p.n_keep ? n : (int)p.n_keep;
    int token = fbi == 0x7FFFFFFF ? -1 : fbi;
    if ((use_min_p || use_top_k) && n > 0) {
      float best = kNegInf;
      int bk = 0x7FFFFFFF;
      for (int wv = 0; wv < kSelWaves; ++wv)
        if (r_ps[wv] > best || (r_ps[wv] == best && r_pk[wv] < bk)) {
          best = r_ps[wv];
          bk = r_pk[wv];
        }
      const int pick = (bk != 0x7FFFFFFF && best > s_score0) ? bk : 0;
      token = (int)(vbase + (0x7FFFFFFF - (int)(uint32_t)cand[pick]));
    }
    out[r].token_id = token;
    out[r].logz = fmx + log_f32(fsm);
    out[r].n = n_out;
    s_nout = n_out;
  }
  __syncthreads();
  const int n_out = s_nout;
  if (tid < kSampleNmax) {
    const bool keep = tid < n_out;
    out[r].topn_val[tid] = keep ? bf16_to_f32(key_bf16((uint32_t)(cand[tid] >> 32))) : kNegInf;
    out[r].topn_idx[tid] = keep ? (int)(vbase + (0x7FFFFFFF - (int)(uint32_t)cand[tid])) : -1;
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
static int pick_pu_bf16(int cols) {
  if (cols % 256 == 0) return 8;
  if (cols % 128 == 0) return 4;
  if (cols % 64 == 0) return 2;
  return 1;
}

hipError_t launch_head_prep(const uint16_t* src, const uint16_t* gamma, int8_t* xq, float* sa,
                            int rows, int hidden, int block, float sqrt_n, float n_eps,
                            hipStream_t st) {
  const float sc = fwht_scale_host(block);
  const int pu = pick_pu_bf16(hidden);
  if (rows > 0 && hidden > 0 && block == 128 && pu == 8 && hidden <= 4096 && tune().nq_v8 &&
      !(reinterpret_cast<uintptr_t>(gamma) & 15u) && !(reinterpret_cast<uintptr_t>(xq) & 7u)) {
    // hidden 2816, one row: 7.4 us (k_head_prep<2>, min) -> 4.1 us
    const int ns = hidden >> 7;
    const dim3 g(rows), b(64 * ((hidden + 511) / 512));
#define BQ_HP8(N) if (ns <= N) { hipLaunchKernelGGL((k_head_prep_v8<N>), g, b, 0, st, src, gamma, xq, sa, hidden, sqrt_n, n_eps, sc); return hipGetLastError(); }
    BQ_HP8(8) BQ_HP8(16) BQ_HP8(22) BQ_HP8(24) BQ_HP8(32)
#undef BQ_HP8
  }
  const dim3 g(rows), b(256);
  switch (block) {
    case 64: hipLaunchKernelGGL(k_head_prep<1>, g, b, 0, st, src, gamma, xq, sa, hidden, pu, sqrt_n, n_eps, sc); break;
    case 128: hipLaunchKernelGGL(k_head_prep<2>, g, b, 0, st, src, gamma, xq, sa, hidden, pu, sqrt_n, n_eps, sc); break;
    case 256: hipLaunchKernelGGL(k_head_prep<4>, g, b, 0, st, src, gamma, xq, sa, hidden, pu, sqrt_n, n_eps, sc); break;
    case 512: hipLaunchKernelGGL(k_head_prep<8>, g, b, 0, st, src, gamma, xq, sa, hidden, pu, sqrt_n, n_eps, sc); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_embed(const int32_t* tokens, const int8_t* w, const float* ws, uint16_t* dst,
                        int T, int hidden, int block, int shard_rows, int rank, float scale,
                        hipStream_t st) {
  const float sc = fwht_scale_host(block);
  const dim3 g(T), b(256);
  switch (block) {
    case 64: hipLaunchKernelGGL(k_embed<1>, g, b, 0, st, tokens, w, ws, dst, hidden, shard_rows, rank, scale, sc); break;
    case 128: hipLaunchKernelGGL(k_embed<2>, g, b, 0, st, tokens, w, ws, dst, hidden, shard_rows, rank, scale, sc); break;
    case 256: hipLaunchKernelGGL(k_embed<4>, g, b, 0, st, tokens, w, ws, dst, hidden, shard_rows, rank, scale, sc); break;
    case 512: hipLaunchKernelGGL(k_embed<8>, g, b, 0, st, tokens, w, ws, dst, hidden, shard_rows, rank, scale, sc); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// One workgroup of 8 waves per CU, each wave walking its strips: the
// 262144 x 2816 head (761 MB) 1 row 190.5 -> 182.2 us, 16 rows 237.1 ->
// 230.2 us against 1024 workgroups (two per CU in two rounds; 512: 188.2 /
// 235.3 us).  BQ_HEAD_GRID overrides it.
int head_grid(int vocab) {
  const int strips = vocab / 16;
  const int g = (strips + kHeadWaves - 1) / kHeadWaves;
  const int cap = tune().head_grid ? tune().head_grid : tune().cus;
  return g < cap ? g : cap;
}

struct HeadWs {
  size_t y, part, tot, hist2, thr, eqpre, cnt, cand, total;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static HeadWs head_ws_layout(int rows, int vocab) {
  const int RP = rows <= 16 ? 16 : 32;
  const int nc = (vocab + kChunk - 1) / kChunk;
  HeadWs w{};
  size_t o = 0;
  w.y = o; o = align256(o + (size_t)rows * vocab * 2);
  w.part = o; o = align256(o + (size_t)head_grid(vocab) * 4 * RP * sizeof(float));
  w.tot = o; o = align256(o + (size_t)rows * 2 * 256 * 4);
  w.hist2 = o; o = align256(o + (size_t)rows * nc * 256 * 4);
  w.thr = o; o = align256(o + (size_t)rows * 4 * 4);
  w.eqpre = o; o = align256(o + (size_t)rows * nc * 4);
  w.cnt = o; o = align256(o + (size_t)rows * 4);
  w.cand = o; o = align256(o + (size_t)rows * kSampleNmax * 8);
  w.total = o;
  return w;
}

size_t head_workspace_bytes(int rows, int vocab) { return head_ws_layout(rows, vocab).total; }

hipError_t launch_flash_sample(const int8_t* x, const float* xsa, const int8_t* w, const float* ws,
                               const SamplingParams* params, SampleOutcome* out, int R, int V,
                               int H, int block, float cap, int64_t vbase, void* workspace,
                               hipStream_t st) {
  const HeadWs L = head_ws_layout(R, V);
  char* base = reinterpret_cast<char*>(workspace);
  HeadArgs a{};
  a.x = x; a.xsa = xsa; a.w = w; a.ws = ws; a.params = params;
  a.y = reinterpret_cast<uint16_t*>(base + L.y);
  a.part = reinterpret_cast<float*>(base + L.part);
  a.tot1 = reinterpret_cast<uint32_t*>(base + L.tot);
  a.R = R; a.V = V; a.H = H; a.block = block; a.nstrips = V / 16; a.cap = cap; a.vbase = vbase;
  const int grid = head_grid(V);
  const int RP = R <= 16 ? 16 : 32;
  const size_t lds = (size_t)RP * (H + 16) + (size_t)(H / block) * RP * sizeof(float);
  // chunks of 4 fragments up to block 256 (104 VGPRs, two slots of 4 KiB
  // per wave), else 8 (a block never spans two chunks)
  const bool ch4 = block <= 256;
  if (R <= 16 && ch4)
    hipLaunchKernelGGL((k_head_logits<1, 4>), dim3(grid), dim3(64 * kHeadWaves), lds, st, a);
  else if (R <= 16)
    hipLaunchKernelGGL((k_head_logits<1, 8>), dim3(grid), dim3(64 * kHeadWaves), lds, st, a);
  else if (ch4)
    hipLaunchKernelGGL((k_head_logits<2, 4>), dim3(grid), dim3(64 * kHeadWaves), lds, st, a);
  else
    hipLaunchKernelGGL((k_head_logits<2, 8>), dim3(grid), dim3(64 * kHeadWaves), lds, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;

  SelArgs s{};
  s.y = a.y;
  s.tot1 = a.tot1;
  s.tot2 = a.tot1 + (size_t)R * 256;
  s.hist2 = reinterpret_cast<uint32_t*>(base + L.hist2);
  s.thr = reinterpret_cast<int*>(base + L.thr);
  s.eqpre = reinterpret_cast<int*>(base + L.eqpre);
  s.cnt = reinterpret_cast<int*>(base + L.cnt);
  s.cand = reinterpret_cast<uint64_t*>(base + L.cand);
  s.V = V;
  s.nc = (V + kChunk - 1) / kChunk;
  const dim3 cg(s.nc, R), cb(kChunkThreads);
  // each chunk workgroup of hist_lo and collect derives its row's thresholds
  // from the row's histograms itself (the chunks add theirs into them) (the two one-workgroup-per-row threshold
  // launches go; BQ_SEL_FUSED=0 keeps them)
  s.fused = tune().sel_fused;
  hipLaunchKernelGGL(k_sel_hist_hi, cg, cb, 0, st, s);
  if (!s.fused) hipLaunchKernelGGL(k_sel_thr_hi, dim3(R), cb, 0, st, s);
  hipLaunchKernelGGL(k_sel_hist_lo, cg, cb, 0, st, s);
  if (!s.fused) hipLaunchKernelGGL(k_sel_thr_lo, dim3(R), cb, 0, st, s);
  hipLaunchKernelGGL(k_sel_collect, cg, cb, 0, st, s);
  hipLaunchKernelGGL(k_head_select, dim3(R), dim3(kSelThreads), 0, st, s.cand, a.part, grid, RP,
                     params, out, V, vbase);
  return hipGetLastError();
}

}  // namespace bq
