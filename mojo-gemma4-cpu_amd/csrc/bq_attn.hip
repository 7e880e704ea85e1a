// int8-KV attention on gfx950: the attention prep (per-head RMS norm, RoPE,
// FWHT, absmax int8 with the code sum) that fills the paged int8 KV cache,
// and flash attention over that cache.
//
// Reference: butterquant/head_prep.mojo:9-92 (per-head prep),
// butterquant_kernels/attention.mojo:32-80 (bq_process_kv_tile), :83-146
// (decode kernel), :149-247 (sliding prefill), :250-327 (full prefill),
// :474-534 (BqAttnPrepKernel), kernels/attention_ops.mojo:45-51 (PagedKV),
// :166-182 (online_softmax_tile), kernels/logsum_merge.mojo:29-122 (merge).
//
// Layout.  KV cache rows are slots: k_cache[slot][kv_head][head_dim] int8 with
// k_scale[slot][kv_head] f32 (amax), the same for V.  A token's position p
// maps to slot base_rows[run.rows_off + ((p >> shift) & page_mask)] +
// (p & row_mask).  Q codes are [token][q_head][head_dim] int8 with
// qi_bias = 128 * sum(codes) and f_q = amax per (token, q_head).
//
// Flash attention: one wave per (token, kv head, split).  The split is a
// contiguous range of the token's KV positions (worker_range of the range
// into S = min(s_max, ceil(L / kAttnMinSplit)) parts).  A wave walks its
// range in tiles of 16 positions exactly as the reference does: the 16 x G
// scores of a tile come from head_dim/64 int8 MFMAs (A = the G query heads
// of this kv head, B = 16 K rows); per head the tile max, corr and weights
// use the reference's fast exp and its 16-lane tree sum; then acc *= corr and
// acc += (w * vs / 127) * v position by position, each lane owning head_dim/64
// consecutive output columns of every head.  A token whose range is one split
// of a sliding layer is finalized in the wave (acc * (1/l), the sliding
// prefill kernel), and so is every token of a one-split plan (full layers:
// the merge of one split); every other token's splits are written as
// (m, l, acc) partials and merged by k_attn_merge / k_attn_merge_lds in split
// order with the reference's merge (corrections masked by l > 0, a 16-lane
// tree per batch of 16 splits, the first contributing split multiplied, the
// rest fma-accumulated).  One-split plans with head_dim <= 256 run
// k_flash_attn_mt instead: 16/G tokens per wave on a shared tile grid.
#include "bq_kernels.hpp"
#include "bq_device.hpp"

namespace bq {

namespace {

// The run holding buffer row tok: the reference advances r while
// tok >= runs[r + 1].buf_start (attention.mojo:489-492), i.e. r + 1 is the
// first j >= 1 with tok < runs[j].buf_start, else num_runs - 1.
__device__ inline int run_of(const KvRun* __restrict__ runs, int n, int tok) {
  const int lane = lane_id();
  for (int base = 1; base < n; base += kWave) {
    const int j = base + lane;
    const bool stop = j < n && tok < runs[j].buf_start;
    const unsigned long long m = __ballot(stop);
    if (m) return base + (__ffsll((long long)m) - 1) - 1;
  }
  return n - 1;
}

__device__ inline int64_t paged_slot(const int32_t* __restrict__ rows, int shift, int row_mask,
                                     int page_mask, int64_t p) {
  return (int64_t)rows[(p >> shift) & page_mask] + (p & row_mask);
}

// sum over the 16 lanes of each aligned 16-lane group in the order of a
// SIMD[f32, 16].reduce_add (halving tree: j + 8, j + 4, j + 2, j + 1); the
// result is broadcast to the group.  Lane j of each row adds lane j + H of
// the same row by a DPP row shift (the lanes whose partner falls outside the
// row compute values no one reads), so lane 0 of each row ends with the
// tree's sum; readlane brings the four row sums back.
__device__ inline float tree16(float v) {
  v = v + row_shl<8>(v);
  v = v + row_shl<4>(v);
  v = v + row_shl<2>(v);
  v = v + row_shl<1>(v);
  const int x = __float_as_int(v);
  const int s0 = __builtin_amdgcn_readlane(x, 0), s1 = __builtin_amdgcn_readlane(x, 16);
  const int s2 = __builtin_amdgcn_readlane(x, 32), s3 = __builtin_amdgcn_readlane(x, 48);
  const int row = lane_id() >> 4;
  return __int_as_float(row == 0 ? s0 : row == 1 ? s1 : row == 2 ? s2 : s3);
}

__device__ inline float max87(float x) { return x > -87.0f ? x : -87.0f; }

__device__ inline float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// token metadata shared by the attention and merge kernels
struct TokRange {
  const int32_t* rows;
  int64_t lo;
  int L;
};

__device__ inline TokRange token_range(const AttnArgs& a, int tok) {
  const int r = run_of(a.runs, a.num_runs, tok);
  const KvRun run = a.runs[r];
  const int64_t pos = (int64_t)run.base_pos + (tok - run.buf_start);
  TokRange t;
  t.rows = a.base_rows + run.rows_off;
  if (a.window > 0) {  // attention.mojo:196-199: [max(0, pos - window + 1), pos]
    t.lo = pos - a.window + 1 > 0 ? pos - a.window + 1 : 0;
    t.L = (int)(pos + 1 - t.lo);
  } else {             // attention_ops.mojo:146-152 at one rank: rows [0, pos]
    t.lo = 0;
    t.L = pos < 0 ? 0 : (int)(pos + 1);
  }
  return t;
}

__device__ inline int num_splits(int L, int s_max) {
  if (L <= 0) return 1;
  const int s = (L + kAttnMinSplit - 1) / kAttnMinSplit;
  return s < s_max ? s : s_max;
}

}  // namespace

// ---------------------------------------------------------------------------
// attention prep: one wave per (token, head) over q heads, then k heads, then
// v heads.  Element e of the head is value r = e / 64 of lane e % 64.
// ---------------------------------------------------------------------------
template <int R>
__global__ __launch_bounds__(256) void k_attn_prep(PrepArgs a) {
  constexpr int HD = R * kWave;
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int nh = a.num_q + 2 * a.num_kv;
  const int item = blockIdx.x * 4 + wave;
  if (item >= a.T * nh) return;
  const int tok = item / nh, j = item % nh;
  const int r = run_of(a.runs, a.num_runs, tok);
  const KvRun run = a.runs[r];
  const int64_t pos = (int64_t)run.base_pos + (tok - run.buf_start);
  const bool is_q = j < a.num_q, is_v = j >= a.num_q + a.num_kv;
  const int h = is_q ? j : is_v ? j - a.num_q - a.num_kv : j - a.num_q;
  // attention.mojo:515: K/V rows only for positions this cache rank owns
  if (!is_q && pos % a.cache_degree != a.rank) return;
  const int64_t kvs = (int64_t)a.num_kv * HD;
  const uint16_t* src = is_q ? a.q_src + (int64_t)tok * a.num_q * HD + (int64_t)h * HD
                      : (is_v ? a.v_src : a.k_src) + (int64_t)tok * kvs + (int64_t)h * HD;
  float v[R];
#pragma unroll
  for (int i = 0; i < R; ++i) v[i] = bf16_to_f32(src[i * kWave + lane]);

  // head_inv_rms (head_prep.mojo:9-16): chain k of 16 takes x[16i + k] in i
  // order (product first, then fma), then the 16-lane tree.  x[16i + k] is
  // value i / 4 of lane 16 * (i % 4) + k: the row moves of row_to_row0 bring
  // it to lane k of row 0, which runs the chains (the other rows' sums are
  // not used), and lane 0 ends the tree.
  float ssq = v[0] * v[0];
#pragma unroll
  for (int i4 = 0; i4 < R; ++i4) {
    if (i4 > 0) ssq = fmaf(v[i4], v[i4], ssq);
    const float x1 = row_to_row0<1>(v[i4]), x2 = row_to_row0<2>(v[i4]);
    const float x3 = row_to_row0<3>(v[i4]);
    ssq = fmaf(x1, x1, ssq);
    ssq = fmaf(x2, x2, ssq);
    ssq = fmaf(x3, x3, ssq);
  }
  ssq = ssq + row_shl<8>(ssq);
  ssq = ssq + row_shl<4>(ssq);
  ssq = ssq + row_shl<2>(ssq);
  ssq = ssq + row_shl<1>(ssq);
  ssq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ssq), 0));
  const float inv = a.sqrt_n / __builtin_sqrtf(ssq + a.n_eps);

  const uint16_t* gamma = is_q ? a.q_norm : a.k_norm;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    v[i] = v[i] * inv;
    if (!is_v) v[i] = v[i] * bf16_to_f32(gamma[i * kWave + lane]);
  }
  if (!is_v) {
    // RoPE on (e, pair_stride + e) for e < rope_half (head_prep.mojo:58-65);
    // rope_half and pair_stride are multiples of 64, so both elements of a
    // pair are values of the same lane
    const int ps = a.pair_stride / kWave, rh = a.rope_half / kWave;
    const float* cs = a.cos_table + pos * a.rope_half;
    const float* sn = a.sin_table + pos * a.rope_half;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (i >= rh) continue;
      const float c = cs[i * kWave + lane], s = sn[i * kWave + lane];
#pragma unroll
      for (int i2 = 0; i2 < R; ++i2) {
        if (i2 != i + ps) continue;
        const float lo = v[i], hi = v[i2];
        v[i] = lo * c - hi * s;
        v[i2] = hi * c + lo * s;
      }
    }
  }
  fwht_wave<R>(v, HD);
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    v[i] = v[i] * a.fwht_scale;
    m = fmaxf(m, fabsf(v[i]));
  }
  float amax = wave_max(m);
  if (amax < 1e-10f) amax = 1e-10f;
  const float qinv = 127.0f / amax;
  int8_t* dst;
  if (is_q) {
    dst = a.q_i8 + (int64_t)tok * a.num_q * HD + (int64_t)h * HD;
  } else {
    const int64_t slot = paged_slot(a.base_rows + run.rows_off, a.page_shift, a.row_mask,
                                    a.page_mask, pos / a.cache_degree);
    dst = (is_v ? a.v_cache : a.k_cache) + slot * kvs + (int64_t)h * HD;
    if (lane == 0) (is_v ? a.v_scale : a.k_scale)[slot * a.num_kv + h] = amax;
  }
  int qs = 0;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int8_t c = quantize_i8(v[i], qinv);
    dst[i * kWave + lane] = c;
    qs += c;
  }
  if (is_q) {
    qs = __builtin_amdgcn_readlane(wave_incl_scan(qs), 63);  // integer sum: exact
    if (lane == 0) {
      a.qi_bias[(int64_t)tok * a.num_q + h] = (float)qs * 128.0f;
      a.f_q[(int64_t)tok * a.num_q + h] = amax;
    }
  }
}

// ---------------------------------------------------------------------------
// flash attention: one wave per (token, kv head, split); G query heads share
// the kv head (G <= 16).
// ---------------------------------------------------------------------------
template <int HD, int G>
__global__ __launch_bounds__(256) void k_flash_attn(AttnArgs a) {
  constexpr int C = HD / 64;  // 64-byte K chunks per row = V bytes per lane
  const int wave = threadIdx.x >> 6, lane = lane_id();
  __shared__ __attribute__((aligned(16))) float s_w[4][16 * G];  // per wave: weights [p][head]
  float* wsh = s_w[wave];
  const int per_tok = a.num_kv * a.s_max;
  const int item = blockIdx.x * 4 + wave;
  if (item >= a.T * per_tok) return;
  // later buffer rows first: in a prefill chunk they have the longest KV
  // ranges, so the long waves start early and the short ones fill the tail
  const int tok = a.T - 1 - item / per_tok, rem = item % per_tok;
  const int kvh = rem / a.s_max, s = rem % a.s_max;
  const TokRange tr = token_range(a, tok);
  const int S = num_splits(tr.L, a.s_max);
  if (s >= S) return;
  int start, end;
  {
    const int per = (tr.L + S - 1) / S;
    start = s * per;
    end = start + per < tr.L ? start + per : tr.L;
    if (start >= tr.L) start = end = tr.L;
  }
  const int64_t kvs = (int64_t)a.num_kv * HD;
  const int p16 = lane & 15, grp = lane >> 4;
  const int qh0 = kvh * G;  // first query head of this kv head

  // A operand: lane (h + 16 g) holds head h's bytes [c*64 + g*16, +16)
  v4i qa[C];
  const v4i zero4 = {0, 0, 0, 0};
  {
    const int hq = lane & 15;
    const int8_t* qrow = a.q_i8 + ((int64_t)tok * a.num_q + qh0 + hq) * HD + grp * 16;
#pragma unroll
    for (int c = 0; c < C; ++c) qa[c] = hq < G ? ld16(qrow + c * 64) : zero4;
  }
  // score layout: lane (p + 16 g), value i <-> head 4 g + i, position p.
  // The u8-shifted dot of the reference is dot + 128 * sum(q).
  float qb[4], fq[4];
  int qsum128[4];
  {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * grp + i;
      qb[i] = 0.0f; fq[i] = 0.0f; qsum128[i] = 0;
      if (h < G) {
        qb[i] = a.qi_bias[(int64_t)tok * a.num_q + qh0 + h];
        fq[i] = a.f_q[(int64_t)tok * a.num_q + qh0 + h];
      }
    }
    // sum of the query codes of head hq, lane-parallel over the 16-byte pieces
    int part = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int w4[4] = {qa[c].x, qa[c].y, qa[c].z, qa[c].w};
#pragma unroll
      for (int q = 0; q < 4; ++q)
        part += (int)(int8_t)w4[q] + (int)(int8_t)(w4[q] >> 8) + (int)(int8_t)(w4[q] >> 16) +
                (w4[q] >> 24);
    }
    part += __shfl_xor(part, 16, kWave);
    part += __shfl_xor(part, 32, kWave);  // lane hq (and hq + 16 g): sum of head hq
#pragma unroll
    for (int i = 0; i < 4; ++i) qsum128[i] = 128 * __shfl(part, 4 * grp + i, kWave);
  }

  const float inv127 = 1.0f / 127.0f;
  const float inv127sq = inv127 * inv127;
  float m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) { m[i] = -1e30f; l[i] = 0.0f; }
  float acc[G][C];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[h][c] = 0.0f;

  const int8_t* kbase = a.k_cache + (int64_t)kvh * HD;
  const int8_t* vbase = a.v_cache + (int64_t)kvh * HD + lane * C;
  // Slots of 64 consecutive positions [sb, sb + 64) of the split, one per
  // lane (lanes past the end repeat the last position); slots fit in 32 bits.
  auto slot_batch = [&](int sb) -> int {
    const int pj = sb + lane < end ? sb + lane : end - 1;
    return (int)paged_slot(tr.rows, a.page_shift, a.row_mask, a.page_mask, tr.lo + pj);
  };
  // One tile's operands: lane (p + 16 g) holds K row p's bytes [c*64 + g*16,
  // +16) for every chunk c, its ks and vs; every lane holds its C bytes of
  // each V row.  Idle positions repeat the tile's first row.
  struct Tile {
    v4i kb[C];
    uint32_t vraw[16][(C + 3) / 4];
    float ks, vs;
  };
  auto load_tile = [&](Tile& t, int p0, int slots, int sb) {
    const int tl = end - p0 < 16 ? end - p0 : 16;
    const int off = p0 - sb;
    const int my = __shfl(slots, off + (p16 < tl ? p16 : 0), kWave);
    const int8_t* krow = kbase + (int64_t)my * kvs + grp * 16;
#pragma unroll
    for (int c = 0; c < C; ++c) t.kb[c] = ld16(krow + c * 64);
    t.ks = a.k_scale[(int64_t)my * a.num_kv + kvh];
    t.vs = a.v_scale[(int64_t)my * a.num_kv + kvh];
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      {
        const int sp = __builtin_amdgcn_readlane(slots, off + (p < tl ? p : 0));
        const int8_t* vr = vbase + (int64_t)sp * kvs;
        if constexpr (C >= 8) {
          const uint2 w = *reinterpret_cast<const uint2*>(vr);
          t.vraw[p][0] = w.x; t.vraw[p][1] = w.y;
        } else if constexpr (C == 4) {
          t.vraw[p][0] = *reinterpret_cast<const uint32_t*>(vr);
        } else if constexpr (C == 2) {
          t.vraw[p][0] = *reinterpret_cast<const uint16_t*>(vr);
        } else {
          t.vraw[p][0] = (uint8_t)*vr;
        }
      }
    }
  };

  // (loading the next tile before this tile's arithmetic measured no faster:
  // the kernel is bound by VALU issue once several waves share a SIMD)
  Tile cur;
  int sb = start, slots = 0;
  if (start < end) slots = slot_batch(sb);
  for (int p0 = start; p0 < end; p0 += 16) {
    const int tl = end - p0 < 16 ? end - p0 : 16;
    if (p0 - sb >= 64) {
      sb = p0;
      slots = slot_batch(sb);
    }
    load_tile(cur, p0, slots, sb);
    v4i d = zero4;
#pragma unroll
    for (int c = 0; c < C; ++c) d = mfma16x16x64(qa[c], cur.kb[c], d);
    const int dv[4] = {d.x, d.y, d.z, d.w};
    // per head of this lane's group (heads 4 g + i, only i < G exist)
    constexpr int NI = G < 4 ? G : 4;
    float sc[4], corr[4];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float sco = -1e30f;
      if (4 * grp + i < G && p16 < tl)
        sco = (((float)(dv[i] + qsum128[i]) - qb[i]) * fq[i]) * cur.ks * inv127sq;
      const float tmax = group_max(sco, 16);
      const float m_new = tmax > m[i] ? tmax : m[i];
      corr[i] = fast_exp_softmax_biased(max87(m[i] - m_new));
      const float w = fast_exp_softmax_biased(max87(sco - m_new));
      l[i] = l[i] * corr[i] + tree16(w);
      m[i] = m_new;
      sc[i] = p16 < tl ? w * cur.vs * inv127 : 0.0f;
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float ch = readlane_f(corr[h % 4], 16 * (h / 4));
#pragma unroll
      for (int c = 0; c < C; ++c) acc[h][c] = acc[h][c] * ch;
    }
    // positions past the tile's end carry weight 0: acc + v*0 leaves acc
    // unchanged bit for bit (acc is never -0: it starts at +0 and only an
    // exact -0 product added to -0 gives -0), so the loop needs no branch.
    // The weights go through LDS as [p][head] and are read broadcast.
    if constexpr (G >= 4) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
        if (4 * grp + i < G) wsh[p16 * G + 4 * grp + i] = sc[i];
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i)
        if (grp == 0) wsh[p16 * G + i] = sc[i];
    }
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      float vf[C];
#pragma unroll
      for (int c = 0; c < C; ++c)
        vf[c] = (float)(int8_t)(cur.vraw[p][c / 4] >> (8 * (c % 4)));
      float w[G];
      if constexpr (G >= 4) {
#pragma unroll
        for (int h4 = 0; h4 < G / 4; ++h4) {
          const float4 w4 = *reinterpret_cast<const float4*>(&wsh[p * G + 4 * h4]);
          w[4 * h4] = w4.x; w[4 * h4 + 1] = w4.y; w[4 * h4 + 2] = w4.z; w[4 * h4 + 3] = w4.w;
        }
      } else {
#pragma unroll
        for (int h = 0; h < G; ++h) w[h] = wsh[p * G + h];
      }
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int c = 0; c < C; ++c) acc[h][c] = fmaf(vf[c], w[h], acc[h][c]);
    }
  }

  // finished here: a sliding token with one split (acc * (1/l)), and every
  // token when the plan has one split (full layers: the merge of one split,
  // (acc * c) * (1/(l * c)) with c = fast_exp(0))
  const bool direct = S == 1 && (a.window > 0 || a.s_max == 1);
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float mh = readlane_f(m[h % 4], 16 * (h / 4));
    const float lh = readlane_f(l[h % 4], 16 * (h / 4));
    const int64_t qrow = (int64_t)tok * a.num_q + qh0 + h;
    if (direct) {
      uint16_t o[C];
      if (a.window > 0) {
        const float inv_l = lh > 0.0f ? 1.0f / lh : 0.0f;
#pragma unroll
        for (int c = 0; c < C; ++c) o[c] = lh > 0.0f ? f32_to_bf16(acc[h][c] * inv_l) : 0;
      } else {
        const float cm = lh > 0.0f ? fast_exp_softmax_biased(0.0f) : 0.0f;
        const float gl = 0.0f + lh * cm;
        const float inv_l = gl > 0.0f ? 1.0f / gl : 0.0f;
#pragma unroll
        for (int c = 0; c < C; ++c) o[c] = gl > 0.0f ? f32_to_bf16((acc[h][c] * cm) * inv_l) : 0;
      }
      uint16_t* dst = a.out + qrow * HD + lane * C;
#pragma unroll
      for (int c = 0; c < C; ++c) dst[c] = o[c];
    } else {
      float* pa = a.ws_acc + (qrow * a.s_max + s) * HD + lane * C;
#pragma unroll
      for (int c = 0; c < C; ++c) pa[c] = acc[h][c];
      if (lane == 0) {
        a.ws_ml[(qrow * a.s_max + s) * 2 + 0] = mh;
        a.ws_ml[(qrow * a.s_max + s) * 2 + 1] = lh;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Single-split tokens (s_max == 1, prefill chunks): TPW = 16 / G query tokens
// per wave share every K/V tile.  The wave takes the tokens tok0 + 16 k
// (k < TPW) of one run: their ranges start at positions that are equal mod 16
// (sliding: lo = pos - window + 1 once pos >= window - 1, else 0; full: 0),
// so all their 16-position tiles sit on one grid and a tile of the grid is,
// for each token, either one of its own tiles or outside its range.  Rows of
// the MFMA are (token k, head h) = 16 rows; each row keeps its own m, l, acc
// and runs the reference's tile recursion; the V conversion and the K/V loads
// are shared by the 16 rows.  Tokens that do not share a grid (a group that
// straddles pos = window - 1, or spans two runs) are processed one per pass.
// Results are those of the one-split path: acc * (1/l) for sliding layers,
// the one-split merge ((acc * c) * (1/(l * c)), c = fast_exp(0)) for full.
// ---------------------------------------------------------------------------
template <int HD, int G>
__global__ __launch_bounds__(256) void k_flash_attn_mt(AttnArgs a) {
  constexpr int C = HD / 64, TPW = 16 / G;
  const int wave = threadIdx.x >> 6, lane = lane_id();
  __shared__ __attribute__((aligned(16))) float s_w[4][16 * 16];  // per wave: weights [p][row]
  const int nblk = (a.T + 16 * TPW - 1) / (16 * TPW);
  const int item = blockIdx.x * 4 + wave;
  if (item >= nblk * a.num_kv * 16) return;
  // later token blocks first (the longest KV ranges of a prefill chunk)
  const int cls = item % 16, kvh = (item / 16) % a.num_kv;
  const int blk = nblk - 1 - item / (16 * a.num_kv);
  const int tok0 = blk * 16 * TPW + cls;
  const int64_t kvs = (int64_t)a.num_kv * HD;
  const int p16 = lane & 15, grp = lane >> 4;

  // per-token range (wave-uniform): run, [lo, hi) of positions
  int run_k[TPW];
  int lo_k[TPW], hi_k[TPW];  // positions fit in 32 bits
  bool shared = true;
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    const int tok = tok0 + 16 * k;
    run_k[k] = -1; lo_k[k] = 0; hi_k[k] = 0;
    if (tok >= a.T) continue;
    const TokRange tr = token_range(a, tok);
    run_k[k] = run_of(a.runs, a.num_runs, tok);
    lo_k[k] = (int)tr.lo;
    hi_k[k] = (int)tr.lo + tr.L;
    if (run_k[k] != run_k[0] || ((lo_k[k] - lo_k[0]) & 15) != 0) shared = false;
  }

  // A operand: row r = k * G + h (token k, head h); lane (r + 16 g) holds
  // row r's bytes [c*64 + g*16, +16)
  const v4i zero4 = {0, 0, 0, 0};
  v4i qa[C];
  {
    const int r = lane & 15, k = r / G, h = r % G;
    const int tok = tok0 + 16 * k;
    const int8_t* qrow = a.q_i8 + ((int64_t)(tok < a.T ? tok : 0) * a.num_q + kvh * G + h) * HD +
                         grp * 16;
#pragma unroll
    for (int c = 0; c < C; ++c) qa[c] = tok < a.T ? ld16(qrow + c * 64) : zero4;
  }
  // score layout: lane (p + 16 g), value i <-> row 4 g + i
  float qb[4], fq[4];
  int qsum128[4];
  {
    int part = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int w4[4] = {qa[c].x, qa[c].y, qa[c].z, qa[c].w};
#pragma unroll
      for (int q = 0; q < 4; ++q)
        part += (int)(int8_t)w4[q] + (int)(int8_t)(w4[q] >> 8) + (int)(int8_t)(w4[q] >> 16) +
                (w4[q] >> 24);
    }
    part += __shfl_xor(part, 16, kWave);
    part += __shfl_xor(part, 32, kWave);  // lane r (and r + 16 g): sum of row r's codes
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * grp + i, k = r / G, h = r % G, tok = tok0 + 16 * k;
      qsum128[i] = 128 * __shfl(part, r, kWave);
      qb[i] = 0.0f; fq[i] = 0.0f;
      if (tok < a.T) {
        qb[i] = a.qi_bias[(int64_t)tok * a.num_q + kvh * G + h];
        fq[i] = a.f_q[(int64_t)tok * a.num_q + kvh * G + h];
      }
    }
  }

  const float inv127 = 1.0f / 127.0f;
  const float inv127sq = inv127 * inv127;
  float m[4], l[4];
  float acc[16][C];
#pragma unroll
  for (int i = 0; i < 4; ++i) { m[i] = -1e30f; l[i] = 0.0f; }
#pragma unroll
  for (int r = 0; r < 16; ++r)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[r][c] = 0.0f;
  const int8_t* kbase = a.k_cache + (int64_t)kvh * HD;
  const int8_t* vbase = a.v_cache + (int64_t)kvh * HD + lane * C;

  // one pass over all tokens (shared grid) or one pass per token
  const int npass = shared ? 1 : TPW;
  for (int pass = 0; pass < npass; ++pass) {
    // active tokens of this pass and the position range they cover
    unsigned amask = 0;
    int pbeg = 0, pend = 0;
    int run = -1;
#pragma unroll
    for (int k = 0; k < TPW; ++k) {
      const bool on = run_k[k] >= 0 && (shared || k == pass) && hi_k[k] > lo_k[k];
      if (!on) continue;
      if (amask == 0) { pbeg = lo_k[k]; pend = hi_k[k]; run = run_k[k]; }
      pbeg = lo_k[k] < pbeg ? lo_k[k] : pbeg;
      pend = hi_k[k] > pend ? hi_k[k] : pend;
      amask |= 1u << k;
    }
    if (amask == 0) continue;
    const int32_t* rows = a.base_rows + a.runs[run].rows_off;
    for (int P = pbeg; P < pend; P += 16) {
      // rows taking part in this tile, and their tile lengths
      unsigned rmask = 0;
      int tl_k[TPW];
#pragma unroll
      for (int k = 0; k < TPW; ++k) {
        tl_k[k] = 0;
        if (!((amask >> k) & 1u) || P < lo_k[k] || P >= hi_k[k]) continue;
        tl_k[k] = hi_k[k] - P < 16 ? hi_k[k] - P : 16;
        rmask |= ((1u << G) - 1u) << (k * G);
      }
      const int tlen = pend - P < 16 ? pend - P : 16;
      const int pp = p16 < tlen ? p16 : 0;
      const int slot = (int)paged_slot(rows, a.page_shift, a.row_mask, a.page_mask, P + pp);
      v4i kb[C];
      const int8_t* krow = kbase + (int64_t)slot * kvs + grp * 16;
#pragma unroll
      for (int c = 0; c < C; ++c) kb[c] = ld16(krow + c * 64);
      const float ks = a.k_scale[(int64_t)slot * a.num_kv + kvh];
      const float vs = a.v_scale[(int64_t)slot * a.num_kv + kvh];
      uint32_t vraw[16][(C + 3) / 4];
#pragma unroll
      for (int p = 0; p < 16; ++p) {
        const int sp = __builtin_amdgcn_readlane(slot, p < tlen ? p : 0);
        const int8_t* vr = vbase + (int64_t)sp * kvs;
        if constexpr (C >= 8) {
          const uint2 w = *reinterpret_cast<const uint2*>(vr);
          vraw[p][0] = w.x; vraw[p][1] = w.y;
        } else if constexpr (C == 4) {
          vraw[p][0] = *reinterpret_cast<const uint32_t*>(vr);
        } else if constexpr (C == 2) {
          vraw[p][0] = *reinterpret_cast<const uint16_t*>(vr);
        } else {
          vraw[p][0] = (uint8_t)*vr;
        }
      }
      v4i d = zero4;
#pragma unroll
      for (int c = 0; c < C; ++c) d = mfma16x16x64(qa[c], kb[c], d);
      const int dv[4] = {d.x, d.y, d.z, d.w};
      float sc[4], corr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * grp + i;
        const bool on = (rmask >> r) & 1u;
        // this row's tile length (lane-varying through the token index)
        int tl = 0;
#pragma unroll
        for (int k = 0; k < TPW; ++k) tl = r / G == k ? tl_k[k] : tl;
        float sco = -1e30f;
        if (on && p16 < tl)
          sco = (((float)(dv[i] + qsum128[i]) - qb[i]) * fq[i]) * ks * inv127sq;
        const float tmax = group_max(sco, 16);
        const float m_new = tmax > m[i] ? tmax : m[i];
        const float cr = fast_exp_softmax_biased(max87(m[i] - m_new));
        const float w = fast_exp_softmax_biased(max87(sco - m_new));
        const float wsum = tree16(w);
        corr[i] = on ? cr : 1.0f;
        if (on) {
          l[i] = l[i] * cr + wsum;
          m[i] = m_new;
        }
        sc[i] = on && p16 < tl ? w * vs * inv127 : 0.0f;
      }
      // every row takes part in the update: a row outside this tile has
      // corr 1 and weights 0, which leave its acc bit for bit (acc * 1 = acc,
      // acc + v*0 = acc since acc is never -0), so the loops need no branches.
      // The weights go through LDS as [p][row]; every lane reads them
      // broadcast, four rows per read.
      float* wsh = s_w[wave];
#pragma unroll
      for (int i = 0; i < 4; ++i) wsh[p16 * 16 + 4 * grp + i] = sc[i];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float ch = readlane_f(corr[r % 4], 16 * (r / 4));
#pragma unroll
        for (int c = 0; c < C; ++c) acc[r][c] = acc[r][c] * ch;
      }
#pragma unroll
      for (int p = 0; p < 16; ++p) {
        float vf[C];
#pragma unroll
        for (int c = 0; c < C; ++c) vf[c] = (float)(int8_t)(vraw[p][c / 4] >> (8 * (c % 4)));
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const float4 w4 = *reinterpret_cast<const float4*>(&wsh[p * 16 + 4 * r4]);
          const float wr[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int c = 0; c < C; ++c)
              acc[4 * r4 + q][c] = fmaf(vf[c], wr[q], acc[4 * r4 + q][c]);
        }
      }
    }
  }

  // finalize every row of a real token
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int k = r / G, h = r % G, tok = tok0 + 16 * k;
    if (tok >= a.T) continue;
    const float lr = readlane_f(l[r % 4], 16 * (r / 4));
    uint16_t o[C];
    if (a.window > 0) {  // sliding prefill: acc * (1/l), or zeros
      const float inv_l = lr > 0.0f ? 1.0f / lr : 0.0f;
#pragma unroll
      for (int c = 0; c < C; ++c) o[c] = lr > 0.0f ? f32_to_bf16(acc[r][c] * inv_l) : 0;
    } else {             // the merge of one split
      const float cm = lr > 0.0f ? fast_exp_softmax_biased(0.0f) : 0.0f;
      const float gl = 0.0f + lr * cm;
      const float inv_l = gl > 0.0f ? 1.0f / gl : 0.0f;
#pragma unroll
      for (int c = 0; c < C; ++c) o[c] = gl > 0.0f ? f32_to_bf16((acc[r][c] * cm) * inv_l) : 0;
    }
    uint16_t* dst = a.out + ((int64_t)tok * a.num_q + kvh * G + h) * HD + lane * C;
#pragma unroll
    for (int c = 0; c < C; ++c) dst[c] = o[c];
  }
}

// ---------------------------------------------------------------------------
// merge of the split partials: one wave per (token, query head)
// ---------------------------------------------------------------------------
template <int HD>
__global__ __launch_bounds__(256) void k_attn_merge(AttnArgs a) {
  // one wave per (token, query head, 128-column slice); lane owns CL columns
  constexpr int CW = HD < 128 ? HD : 128, CL = CW / 64, NW = HD / CW;
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int witem = blockIdx.x * 4 + wave;
  if (witem >= a.T * a.num_q * NW) return;
  const int item = witem / NW, col0 = (witem % NW) * CW + lane * CL;
  const int tok = item / a.num_q;
  const TokRange tr = token_range(a, tok);
  const int S = num_splits(tr.L, a.s_max);
  if (a.window > 0 && S == 1) return;  // finalized by the attention wave
  const int64_t base = (int64_t)item * a.s_max;
  const float* ml = a.ws_ml + base * 2;
  float gm = -1e30f;
  for (int s0 = 0; s0 < S; s0 += kWave) {
    const float v = s0 + lane < S ? ml[(s0 + lane) * 2] : -1e30f;
    gm = fmaxf(gm, wave_max(v));
  }
  float gl = 0.0f, out[CL];
  bool first = true;
  for (int s0 = 0; s0 < S; s0 += kWave) {
    // the corrections of 64 splits, lane-parallel; masked by l > 0
    const int sidx = s0 + lane;
    float d = -1e30f, ls = 0.0f;
    if (sidx < S) { d = ml[sidx * 2] - gm; ls = ml[sidx * 2 + 1]; }
    float c = fast_exp_softmax_biased(max87(d));
    if (!(ls > 0.0f)) c = 0.0f;
    // global l: batches of 16 splits, each a 16-lane tree of l * c
    const float bsum = tree16(ls * c);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (s0 + 16 * q < S) gl = gl + readlane_f(bsum, 16 * q);
    // acc: splits in order, 8 rows in flight
    const int n = S - s0 < kWave ? S - s0 : kWave;
    const float* src0 = a.ws_acc + (base + s0) * HD + col0;
    for (int b0 = 0; b0 < n; b0 += 8) {
      float rows[8][CL];
#pragma unroll
      for (int b = 0; b < 8; ++b)
        if (b0 + b < n) {
#pragma unroll
          for (int cc = 0; cc < CL; ++cc) rows[b][cc] = src0[(int64_t)(b0 + b) * HD + cc];
        }
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        if (b0 + b >= n) break;
        const float cb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c), b0 + b));
        if (cb <= 0.0f) continue;
#pragma unroll
        for (int cc = 0; cc < CL; ++cc)
          out[cc] = first ? rows[b][cc] * cb : fmaf(rows[b][cc], cb, out[cc]);
        first = false;
      }
    }
  }
  uint16_t* dst = a.out + (int64_t)item * HD + col0;
  if (!(gl > 0.0f)) {
#pragma unroll
    for (int cc = 0; cc < CL; ++cc) dst[cc] = 0;
    return;
  }
  const float inv_l = 1.0f / gl;
#pragma unroll
  for (int cc = 0; cc < CL; ++cc) dst[cc] = f32_to_bf16(out[cc] * inv_l);
}

// Merge for many splits: one workgroup per (token, query head, 64-column
// slice).  The four waves stage up to 240 splits (their (m, l) and the slice
// of their acc rows) in LDS with all loads in flight at once; wave 0 then runs
// the ordered chain from LDS, eight rows per batch.
constexpr int kMergeStage = 240;  // 240 x 66 floats: under 64 KiB of LDS

template <int HD>
__global__ __launch_bounds__(256) void k_attn_merge_lds(AttnArgs a) {
  constexpr int NW = HD / 64;
  extern __shared__ float stage[];  // [n][64] acc slice, then [n] m, [n] l
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int item = blockIdx.x / NW, col = (blockIdx.x % NW) * 64 + lane;
  const int tok = item / a.num_q;
  const TokRange tr = token_range(a, tok);
  const int S = num_splits(tr.L, a.s_max);
  if (a.window > 0 && S == 1) return;  // finalized by the attention wave
  const int64_t base = (int64_t)item * a.s_max;
  const float* ml = a.ws_ml + base * 2;
  const int cap = a.s_max < kMergeStage ? a.s_max : kMergeStage;
  float* sm = stage + cap * 64;
  float* sl = sm + cap;
  // global max over all splits (every wave, lane-parallel)
  float gm = -1e30f;
  for (int s0 = 0; s0 < S; s0 += kWave) {
    const float v = s0 + lane < S ? ml[(s0 + lane) * 2] : -1e30f;
    gm = fmaxf(gm, wave_max(v));
  }
  float gl = 0.0f, out = 0.0f;
  bool first = true;
  for (int c0 = 0; c0 < S; c0 += kMergeStage) {
    const int n = S - c0 < kMergeStage ? S - c0 : kMergeStage;
    __syncthreads();
    for (int r = wave; r < n; r += 4) stage[r * 64 + lane] = a.ws_acc[(base + c0 + r) * HD + col];
    for (int r = threadIdx.x; r < n; r += 256) {
      sm[r] = ml[(c0 + r) * 2];
      sl[r] = ml[(c0 + r) * 2 + 1];
    }
    __syncthreads();
    if (wave != 0) continue;
    for (int s0 = 0; s0 < n; s0 += kWave) {
      const int m = n - s0 < kWave ? n - s0 : kWave;
      float d = -1e30f, ls = 0.0f;
      if (lane < m) { d = sm[s0 + lane] - gm; ls = sl[s0 + lane]; }
      float c = fast_exp_softmax_biased(max87(d));
      if (!(ls > 0.0f)) c = 0.0f;
      // global l: batches of 16 splits, each a 16-lane tree of l * c
      const float bsum = tree16(ls * c);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (16 * q < m) gl = gl + readlane_f(bsum, 16 * q);
      const unsigned long long live = __ballot(lane < m && c > 0.0f);
      const unsigned long long all = m == 64 ? ~0ull : ((1ull << m) - 1);
      int b = 0;
      if (first && (live & 1ull)) {  // the first contributing split is multiplied
        out = stage[s0 * 64 + lane] * readlane_f(c, 0);
        first = false;
        b = 1;
      }
      if (!first && live == all) {
        // every split contributes: branch-free chain, eight LDS rows per batch
        for (; b + 8 <= m; b += 8) {
          float v[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) v[u] = stage[(s0 + b + u) * 64 + lane];
#pragma unroll
          for (int u = 0; u < 8; ++u) out = fmaf(v[u], readlane_f(c, b + u), out);
        }
      }
      for (; b < m; ++b) {
        const float cb = readlane_f(c, b);
        if (cb <= 0.0f) continue;
        const float v = stage[(s0 + b) * 64 + lane];
        out = first ? v * cb : fmaf(v, cb, out);
        first = false;
      }
    }
  }
  if (wave != 0) return;
  uint16_t* dst = a.out + (int64_t)item * HD + col;
  *dst = gl > 0.0f ? f32_to_bf16(out * (1.0f / gl)) : (uint16_t)0;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
hipError_t launch_attn_prep(const PrepArgs& args, int head_dim, hipStream_t st) {
  PrepArgs a = args;
  a.fwht_scale = fwht_scale_host(head_dim);
  const int items = a.T * (a.num_q + 2 * a.num_kv);
  if (items <= 0) return hipSuccess;
  const dim3 g((items + 3) / 4), b(256);
  switch (head_dim) {
    case 64: hipLaunchKernelGGL(k_attn_prep<1>, g, b, 0, st, a); break;
    case 128: hipLaunchKernelGGL(k_attn_prep<2>, g, b, 0, st, a); break;
    case 256: hipLaunchKernelGGL(k_attn_prep<4>, g, b, 0, st, a); break;
    case 512: hipLaunchKernelGGL(k_attn_prep<8>, g, b, 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int HD>
static hipError_t launch_attn_hd(const AttnArgs& a, int gqa, hipStream_t st) {
  const dim3 b(256);
  if (a.s_max == 1 && gqa <= 8 && HD <= 256) {
    // one split per token: 16/G tokens per wave, finalized in the wave
    const int tpw = 16 / gqa;
    const int items = (a.T + 16 * tpw - 1) / (16 * tpw) * a.num_kv * 16;
    const dim3 g((items + 3) / 4);
    switch (gqa) {
      case 1: hipLaunchKernelGGL((k_flash_attn_mt<HD, 1>), g, b, 0, st, a); break;
      case 2: hipLaunchKernelGGL((k_flash_attn_mt<HD, 2>), g, b, 0, st, a); break;
      case 4: hipLaunchKernelGGL((k_flash_attn_mt<HD, 4>), g, b, 0, st, a); break;
      case 8: hipLaunchKernelGGL((k_flash_attn_mt<HD, 8>), g, b, 0, st, a); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  const int items = a.T * a.num_kv * a.s_max;
  const dim3 g((items + 3) / 4);
  switch (gqa) {
    case 1: hipLaunchKernelGGL((k_flash_attn<HD, 1>), g, b, 0, st, a); break;
    case 2: hipLaunchKernelGGL((k_flash_attn<HD, 2>), g, b, 0, st, a); break;
    case 4: hipLaunchKernelGGL((k_flash_attn<HD, 4>), g, b, 0, st, a); break;
    case 8: hipLaunchKernelGGL((k_flash_attn<HD, 8>), g, b, 0, st, a); break;
    case 16: hipLaunchKernelGGL((k_flash_attn<HD, 16>), g, b, 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  if (a.s_max == 1) return hipGetLastError();  // every token finished in the wave
  if (a.s_max > 8) {
    const size_t lds = (size_t)(a.s_max < kMergeStage ? a.s_max : kMergeStage) * 66 * sizeof(float);
    hipLaunchKernelGGL(k_attn_merge_lds<HD>, dim3(a.T * a.num_q * (HD / 64)), b, lds, st, a);
  } else {
    constexpr int NW = HD < 128 ? 1 : HD / 128;
    const dim3 gm((a.T * a.num_q * NW + 3) / 4);
    hipLaunchKernelGGL(k_attn_merge<HD>, gm, b, 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_flash_attn(const AttnArgs& a, int head_dim, hipStream_t st) {
  if (a.T <= 0) return hipSuccess;
  const int gqa = a.num_q / a.num_kv;
  switch (head_dim) {
    case 64: return launch_attn_hd<64>(a, gqa, st);
    case 128: return launch_attn_hd<128>(a, gqa, st);
    case 256: return launch_attn_hd<256>(a, gqa, st);
    case 512: return launch_attn_hd<512>(a, gqa, st);
    default: return hipErrorInvalidValue;
  }
}

int attn_splits(int seq_len, int num_kv, int max_kv_len) {
  // enough splits for ~2048 waves (BQ_ATTN_WAVES), each at least
  // kAttnMinSplit positions
  if (seq_len <= 0 || num_kv <= 0) return 1;
  const int64_t items = (int64_t)seq_len * num_kv;
  const int64_t target = tune().attn_waves ? tune().attn_waves : 2048;
  int s = (int)((target + items - 1) / items);
  const int cap = max_kv_len > 0 ? (max_kv_len + kAttnMinSplit - 1) / kAttnMinSplit : 1;
  if (s > cap) s = cap;
  return s < 1 ? 1 : s;
}

}  // namespace bq
