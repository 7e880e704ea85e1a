/*
 * bq_oracle.c -- CPU restatement of the butterquant hot path (test
 * infrastructure only: the parity checker and the CPU baseline).  See
 * bq_oracle.h for the function list; each body cites the reference lines it
 * follows.  Build: gcc -O2 -fPIC -ffp-contract=off -fno-fast-math (oracle/Makefile).
 */
#include "bq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* bf16                                                                      */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* convert.mojo:14-17 -- software RNE: (bits + ((bits>>16)&1) + 0x7FFF) >> 16 */
uint16_t bqo_f32_to_bf16(float v) {
    uint32_t bits = f2u(v);
    uint32_t rne = bits + ((bits >> 16) & 1u) + 0x7FFFu;
    return (uint16_t)(rne >> 16);
}

float bqo_bf16_to_f32(uint16_t b) { return u2f(((uint32_t)b) << 16); }

/* ------------------------------------------------------------------------ */
/* FWHT                                                                      */
/* ------------------------------------------------------------------------ */

static int is_fwht_block(int block) {
    /* kernels.mojo:123-145 dispatch_fwht_block: 16,32,64,128,256,512 */
    return block == 16 || block == 32 || block == 64 || block == 128 ||
           block == 256 || block == 512;
}

/* fwht.mojo:55 -- Scalar[T](1.0 / Float64(sqrt[T,1](Scalar[T](block)))) */
float bqo_fwht_scale(int block) {
    float s = sqrtf((float)block);
    return (float)(1.0 / (double)s);
}

/* fwht.mojo:20-57.  Stage s (stride 1<<s, ascending) maps every pair
 * (i, i+stride) with bit s of i clear to (a+b, a-b).  The in-register stages
 * (fwht.mojo:33-42) compute r*sign + partner with sign = -1 on lanes whose bit
 * s is set, i.e. partner - self = a - b on the upper lane: the same values.
 * Then every element is multiplied by the scale (fwht.mojo:55-57). */
int bqo_fwht_block(float* buf, int block) {
    if (!is_fwht_block(block)) return -1;
    for (int stride = 1; stride < block; stride <<= 1) {
        for (int i = 0; i < block; ++i) {
            if (i & stride) continue;
            float a = buf[i], b = buf[i + stride];
            buf[i] = a + b;
            buf[i + stride] = a - b;
        }
    }
    float sc = bqo_fwht_scale(block);
    for (int i = 0; i < block; ++i) buf[i] = buf[i] * sc;
    return 0;
}

/* fwht.mojo:73-76 (cols % block must be 0: kernels.mojo:81-83 aborts) */
int bqo_fwht_row(float* buf, int cols, int block) {
    if (!is_fwht_block(block) || cols % block != 0) return -1;
    for (int b = 0; b < cols / block; ++b) bqo_fwht_block(buf + (size_t)b * block, block);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* quantization                                                              */
/* ------------------------------------------------------------------------ */

/* kernels.mojo:48-55 */
float bqo_row_absmax(const float* x, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; ++i) {
        float a = fabsf(x[i]);
        if (a > m) m = a;
    }
    return m;
}

/* simd_math/ops.mojo:26-31 quantize_i8: min(max(roundeven(v*inv), -128), 127) */
static inline int8_t quantize_i8(float v, float inv) {
    float r = nearbyintf(v * inv); /* default rounding mode: to nearest even */
    if (r < -128.0f) r = -128.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)r;
}

/* kernels.mojo:68-78: scale = amax/127 (weights) or amax (activations);
 * inv = 127/amax if amax > 0 else 0. */
void bqo_quant_segment(const float* work, int8_t* qi, float* scale_slot, int n,
                       int store_divided) {
    float amax = bqo_row_absmax(work, n);
    *scale_slot = store_divided ? amax / 127.0f : amax;
    float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    for (int i = 0; i < n; ++i) qi[i] = quantize_i8(work[i], inv);
}

/* kernels.mojo:148-168 (single-sided; two-sided M-axis rotation is not on the
 * hot path's recipes, gemma_4_moe_bq.mojo:91-121) */
int bqo_rotate_and_quant(int block, float* work, int8_t* qi, float* scales,
                         int rows, int cols, int per_block) {
    if (!is_fwht_block(block) || cols % block != 0) return -1;
    for (int r = 0; r < rows; ++r) bqo_fwht_row(work + (size_t)r * cols, cols, block);
    if (per_block) { /* kernels.mojo:110-120 */
        int nb = cols / block;
        for (int r = 0; r < rows; ++r)
            for (int b = 0; b < nb; ++b)
                bqo_quant_segment(work + (size_t)r * cols + (size_t)b * block,
                                  qi + (size_t)r * cols + (size_t)b * block,
                                  scales + (size_t)r * nb + b, block, 1);
    } else { /* kernels.mojo:105-107 */
        for (int r = 0; r < rows; ++r)
            bqo_quant_segment(work + (size_t)r * cols, qi + (size_t)r * cols,
                              scales + r, cols, 1);
    }
    return 0;
}

/* kernels.mojo:36-45: g -> sign(g) * sqrt(max(|g|, eps)), stored bf16 */
void bqo_bake_split_gain(uint16_t* gamma, int cols, float eps) {
    for (int k = 0; k < cols; ++k) {
        float g = bqo_bf16_to_f32(gamma[k]);
        float a = fabsf(g);
        float s = sqrtf(a > eps ? a : eps);
        gamma[k] = bqo_f32_to_bf16(g < 0.0f ? -s : s);
    }
}

/* ------------------------------------------------------------------------ */
/* activation prep                                                           */
/* ------------------------------------------------------------------------ */

/* simd_math/matrixops.mojo:233-246 with width = BW = 32 (AVX-512 bf16 lanes) */
static int pick_port_unroll(int width, int cols) {
    if (cols % (8 * width) == 0) return 8;
    if (cols % (4 * width) == 0) return 4;
    if (cols % (2 * width) == 0) return 2;
    return 1;
}

/* rms_reduce_row = dot_to_scalar[hidden](src, src) (rmsnorm.mojo:16-17,
 * dot_products.mojo:144-191).  PU accumulators of W=16 f32 lanes; per 32
 * bf16: vdpbf16ps adds the odd product then the even product to lane j, each
 * a single-rounded fma (exact bf16 products).  Then s = sum_p acc[p] lane-wise
 * (dot_products.mojo:127-140) and a 16-lane halving-tree reduce_add. */
float bqo_rms_reduce_row(const uint16_t* src, int hidden) {
    enum { W = 16, BW = 32 };
    int pu = pick_port_unroll(BW, hidden);
    int stride = pu * BW;
    float acc[8][W];
    memset(acc, 0, sizeof(acc));
    for (int i = 0; i < hidden / stride; ++i) {
        for (int p = 0; p < pu; ++p) {
            const uint16_t* x = src + (size_t)i * stride + (size_t)p * BW;
            for (int j = 0; j < W; ++j) {
                float o = bqo_bf16_to_f32(x[2 * j + 1]);
                float e = bqo_bf16_to_f32(x[2 * j]);
                acc[p][j] = fmaf(o, o, acc[p][j]);
                acc[p][j] = fmaf(e, e, acc[p][j]);
            }
        }
    }
    float s[W];
    for (int j = 0; j < W; ++j) s[j] = 0.0f;
    for (int p = 0; p < pu; ++p)
        for (int j = 0; j < W; ++j) s[j] = s[j] + acc[p][j];
    for (int half = W / 2; half >= 1; half /= 2)
        for (int j = 0; j < half; ++j) s[j] = s[j] + s[j + half];
    return s[0];
}

/* runtime.mojo:11-37: inv_rms = sqrt_n / sqrt(ssq + n_eps); w = x*inv_rms*g;
 * FWHT(block) over the row; per-row (sa = amax) or per-block quant. */
int bqo_prepare_norm_activation(const uint16_t* src, const uint16_t* gamma,
                                int8_t* x_i8, float* sa, int hidden, int block,
                                float sqrt_n, float n_eps, int per_block) {
    if (!is_fwht_block(block) || hidden % block != 0) return -1;
    float* ws = (float*)malloc(sizeof(float) * (size_t)hidden);
    float ssq = bqo_rms_reduce_row(src, hidden);
    float inv_rms = sqrt_n / sqrtf(ssq + n_eps);
    for (int k = 0; k < hidden; ++k) {
        float x = bqo_bf16_to_f32(src[k]);
        float g = bqo_bf16_to_f32(gamma[k]);
        ws[k] = x * inv_rms * g;
    }
    bqo_fwht_row(ws, hidden, block);
    if (per_block) {
        for (int b = 0; b < hidden / block; ++b)
            bqo_quant_segment(ws + b * block, x_i8 + b * block, sa + b, block, 0);
    } else {
        bqo_quant_segment(ws, x_i8, sa, hidden, 0);
    }
    free(ws);
    return 0;
}

/* runtime.mojo:62-80 + quantize.mojo:12-23 */
int bqo_prepare_block_activation(const uint16_t* src, int8_t* x_i8, float* sa,
                                 int cols, int block, int apply_fwht) {
    if (cols % block != 0 || block % 16 != 0) return -1;
    if (apply_fwht && !is_fwht_block(block)) return -1;
    float* ws = (float*)malloc(sizeof(float) * (size_t)cols);
    for (int k = 0; k < cols; ++k) ws[k] = bqo_bf16_to_f32(src[k]);
    if (apply_fwht) bqo_fwht_row(ws, cols, block);
    for (int b = 0; b < cols / block; ++b)
        bqo_quant_segment(ws + b * block, x_i8 + b * block, sa + b, block, 0);
    free(ws);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* VNNI pack                                                                 */
/* ------------------------------------------------------------------------ */

/* vnni.mojo:146-163: 32 rows x 64 K per 2 KiB tile; within a tile two 16-row
 * halves of 1 KiB, each the 16x16 dword transpose of the row-major bytes. */
size_t bqo_vnni_offset(int n, int k, int cols) {
    return (size_t)(n / 32) * 32 * (size_t)cols + (size_t)(k / 64) * 2048 +
           (size_t)((n % 32) / 16) * 1024 + (size_t)((k % 64) / 4) * 64 +
           (size_t)(n % 16) * 4 + (size_t)(k % 4);
}

/* vnni.mojo:31-114.  colsum = per-row sum of codes over each block_cols
 * segment; row-major [rows, nb] or block-major [nb, rows] (vnni.mojo:61-64). */
int bqo_pack_and_colsum_vnni(const int8_t* src, int8_t* dst, int rows, int cols,
                             int block_cols, float* colsum, int colsum_row_major) {
    if (cols % 64 != 0 || rows % 32 != 0 || block_cols <= 0 ||
        cols % block_cols != 0 || block_cols % 16 != 0)
        return -1; /* vnni.mojo:91-99 contracts */
    int nb = cols / block_cols;
    int8_t* tmp = (int8_t*)malloc((size_t)rows * cols);
    for (int n = 0; n < rows; ++n) {
        for (int b = 0; b < nb; ++b) {
            int32_t acc = 0;
            for (int k = b * block_cols; k < (b + 1) * block_cols; ++k)
                acc += src[(size_t)n * cols + k];
            float s = (float)acc;
            if (colsum_row_major) colsum[(size_t)n * nb + b] = s;
            else colsum[(size_t)b * rows + n] = s;
        }
        for (int k = 0; k < cols; ++k)
            tmp[bqo_vnni_offset(n, k, cols)] = src[(size_t)n * cols + k];
    }
    memcpy(dst, tmp, (size_t)rows * cols); /* in-place capable, as pack.mojo:38-44 */
    free(tmp);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* GEMM                                                                      */
/* ------------------------------------------------------------------------ */

/* dot_products.mojo:7-37 restated: sum over k of (x^0x80 as u8) * w as i32,
 * reading W through the packed layout (gemm.mojo:36-75). */
static int32_t vnni_u8_dot(const int8_t* x, const int8_t* wp, int n, int K,
                           int k_lo, int k_hi) {
    int32_t acc = 0;
    for (int k = k_lo; k < k_hi; ++k) {
        uint8_t a = (uint8_t)x[k] ^ 0x80u;
        acc += (int32_t)a * (int32_t)wp[bqo_vnni_offset(n, k, K)];
    }
    return acc;
}

static int32_t signed_dot(const int8_t* x, const int8_t* wp, int n, int K,
                          int k_lo, int k_hi) {
    int32_t acc = 0;
    for (int k = k_lo; k < k_hi; ++k)
        acc += (int32_t)x[k] * (int32_t)wp[bqo_vnni_offset(n, k, K)];
    return acc;
}

void bqo_int_acc(const int8_t* act, int m, const int8_t* wpacked, int N, int K,
                 int k_lo, int k_hi, int64_t* acc) {
    for (int r = 0; r < m; ++r)
        for (int n = 0; n < N; ++n) {
            int64_t s = 0;
            for (int k = k_lo; k < k_hi; ++k)
                s += (int64_t)act[(size_t)r * K + k] *
                     (int64_t)wpacked[bqo_vnni_offset(n, k, K)];
            acc[(size_t)r * N + n] = s;
        }
}

/* gemm.mojo:114-142 epilogue: ((f32(iacc) - 128*cs) * (sa*(1/127))) * sw */
void bqo_gemm_i8_per_row(const int8_t* act, const float* act_scale, int m,
                         const int8_t* wpacked, const float* wsc,
                         const float* colsum, int n_rows, int K,
                         uint16_t* out_bf16, float* out_f32) {
    const float inv127 = 1.0f / 127.0f;
    for (int r = 0; r < m; ++r) {
        float ad = act_scale[r] * inv127;
        for (int n = 0; n < n_rows; ++n) {
            int32_t iacc = vnni_u8_dot(act + (size_t)r * K, wpacked, n, K, 0, K);
            float corrected = (float)iacc - 128.0f * colsum[n];
            float res = corrected * ad * wsc[n];
            if (out_f32) out_f32[(size_t)r * n_rows + n] = res;
            if (out_bf16) out_bf16[(size_t)r * n_rows + n] = bqo_f32_to_bf16(res);
        }
    }
}

/* gemm.mojo:173-215: facc = fma(f32(iacc_b) - 128*cs[b,n], sa[m,b]/127, facc)
 * over blocks in order, then y = facc * sw. */
void bqo_gemm_i8_per_block(const int8_t* act, const float* act_scale, int m,
                           const int8_t* wpacked, const float* wsc,
                           const float* colsum, int N, int k_dim, int block,
                           uint16_t* out_bf16, float* out_f32) {
    const float inv127 = 1.0f / 127.0f;
    int nb = k_dim / block;
    for (int r = 0; r < m; ++r)
        for (int n = 0; n < N; ++n) {
            float facc = 0.0f;
            for (int b = 0; b < nb; ++b) {
                int32_t iacc = vnni_u8_dot(act + (size_t)r * k_dim, wpacked, n,
                                           k_dim, b * block, (b + 1) * block);
                float adv = act_scale[(size_t)r * nb + b] * inv127;
                float corrected = (float)iacc - 128.0f * colsum[(size_t)b * N + n];
                facc = fmaf(corrected, adv, facc);
            }
            float res = facc * wsc[n];
            if (out_f32) out_f32[(size_t)r * N + n] = res;
            if (out_bf16) out_bf16[(size_t)r * N + n] = bqo_f32_to_bf16(res);
        }
}

/* amx_gemm.mojo:28-44 (dequant_fused): f32(acc) * (sa*INV127) * ws */
void bqo_gemm_signed_per_row(const int8_t* act, const float* act_scale, int m,
                             const int8_t* wpacked, const float* wsc, int n_rows,
                             int K, uint16_t* out_bf16, float* out_f32) {
    const float inv127 = 1.0f / 127.0f;
    for (int r = 0; r < m; ++r) {
        float ad = act_scale[r] * inv127;
        for (int n = 0; n < n_rows; ++n) {
            int32_t acc = signed_dot(act + (size_t)r * K, wpacked, n, K, 0, K);
            float res = (float)acc * ad * wsc[n];
            if (out_f32) out_f32[(size_t)r * n_rows + n] = res;
            if (out_bf16) out_bf16[(size_t)r * n_rows + n] = bqo_f32_to_bf16(res);
        }
    }
}

/* Per-block signed form with the VNNI path's explicit fma (gemm.mojo:208-209)
 * applied to the signed accumulator (the AMX block_accumulate at
 * amx_gemm.mojo:47-63 writes the same sum as slot + cv*adv). */
void bqo_gemm_signed_per_block(const int8_t* act, const float* act_scale, int m,
                               const int8_t* wpacked, const float* wsc, int N,
                               int k_dim, int block, uint16_t* out_bf16,
                               float* out_f32) {
    const float inv127 = 1.0f / 127.0f;
    int nb = k_dim / block;
    for (int r = 0; r < m; ++r)
        for (int n = 0; n < N; ++n) {
            float facc = 0.0f;
            for (int b = 0; b < nb; ++b) {
                int32_t acc = signed_dot(act + (size_t)r * k_dim, wpacked, n, k_dim,
                                         b * block, (b + 1) * block);
                float adv = act_scale[(size_t)r * nb + b] * inv127;
                facc = fmaf((float)acc, adv, facc);
            }
            float res = facc * wsc[n];
            if (out_f32) out_f32[(size_t)r * N + n] = res;
            if (out_bf16) out_bf16[(size_t)r * N + n] = bqo_f32_to_bf16(res);
        }
}

/* ------------------------------------------------------------------------ */
/* MoE                                                                       */
/* ------------------------------------------------------------------------ */

static inline float roundeven_f(float x) { return nearbyintf(x); }

/* simd_math/ops.mojo:73-96 */
float bqo_exp_f32_fast(float x) {
    const float LN2 = 0.6931471805599453f;
    const float INV_LN2 = 1.4426950408889634f;
    float xc = x > -87.0f ? x : -87.0f;             /* max(x, -87) */
    float xn = xc * INV_LN2;
    int32_t n = (int32_t)roundeven_f(xn);
    float r = xc - (float)n * LN2;
    float p = 1.0f + r * (0.9999f + r * (0.4985f + r * (0.1681f)));
    int32_t nc = n > -126 ? n : -126;
    float pow2n = u2f(((uint32_t)(nc + 127)) << 23);
    return p * pow2n;
}

/* simd_math/ops.mojo:128-141 */
float bqo_tanh_f32(float x) {
    uint32_t sign_bits = f2u(x) & 0x80000000u;
    float ax = u2f(f2u(x) & 0x7FFFFFFFu);
    float e = bqo_exp_f32_fast(-2.0f * ax);
    float t = (1.0f - e) / (1.0f + e);
    return u2f(f2u(t) ^ sign_bits);
}

/* simd_math/ops.mojo:145-156 */
float bqo_gelu_tanh_f32(float x) {
    const float sqrt_2_over_pi = 0.7978845608028654f;
    const float gelu_a = 0.044715f;
    float x3 = x * x * x;
    float inner = sqrt_2_over_pi * (x + gelu_a * x3);
    float t = bqo_tanh_f32(inner);
    return 0.5f * x * (1.0f + t);
}

/* simd_math/exponential.mojo:178-194 */
float bqo_fast_exp_softmax_biased(float x) {
    const float A_MAGIC = 12102203.16156148f;
    const float BIAS_F = 1059208216.0f;
    const float INV_TWO23 = 1.0f / (float)(1 << 23);
    const float QC_A = 1.6501418352127075f;
    const float QC_B = -0.37554836273193359f;
    const float QC_C = 0.38696467876434326f;
    float v = A_MAGIC * x + BIAS_F;
    /* the f32 -> i32 truncation of the x86 build the reference runs on
     * (cvttps2dq): NaN and values outside [-2^31, 2^31) give INT32_MIN, so
     * a sentinel candidate's x near -1e30 yields -0.0 */
    int32_t i = (v >= -2147483648.0f && v < 2147483648.0f) ? (int32_t)v : INT32_MIN;
    uint32_t u = (uint32_t)i;
    float k = u2f(u);
    float f = (float)(u & 0x7FFFFFu) * INV_TWO23;
    return k * (QC_A + f * (QC_B + f * QC_C));
}

/* dot_to_scalar[cols](x f32, w bf16) (dot_products.mojo:195-205): PU =
 * pick_port_unroll(W=16, cols) accumulators of 16 f32 lanes; accumulator p
 * lane j is an fma chain over elements i*PU*16 + p*16 + j, i ascending
 * (dot_f32_bf16_into_accs, :162-178); then tree_merge_accs (pairwise:
 * acc[i] += acc[i+stride] for stride 1, 2, 4; simd_math/matrixops.mojo:265-
 * 283) and a 16-lane halving-tree reduce_add. */
static float dot_f32_bf16(const float* x, const uint16_t* w, int cols) {
    enum { W = 16 };
    int pu = pick_port_unroll(W, cols);
    float acc[8][W];
    memset(acc, 0, sizeof(acc));
    for (int i = 0; i < cols / (pu * W); ++i)
        for (int p = 0; p < pu; ++p)
            for (int j = 0; j < W; ++j) {
                size_t off = (size_t)i * pu * W + (size_t)p * W + j;
                acc[p][j] = fmaf(x[off], bqo_bf16_to_f32(w[off]), acc[p][j]);
            }
    for (int stride = 1; stride < pu; stride *= 2)
        for (int i = 0; i < pu; i += 2 * stride)
            for (int j = 0; j < W; ++j) acc[i][j] = acc[i][j] + acc[i + stride][j];
    for (int half = W / 2; half >= 1; half /= 2)
        for (int j = 0; j < half; ++j) acc[0][j] = acc[0][j] + acc[0][j + half];
    return acc[0][0];
}

/* RouterExpertKernel.execute (kernels/moe_router.mojo:164-187) up to the
 * candidate insert: inv_rms = sqrt_n / sqrt(rms_reduce_row(x) + n_eps);
 * scaled[j] = (x[j] * router_scale[j]) * inv_rms; logit[e] =
 * dot_to_scalar(scaled, router_proj[e]).  logits [T, E] f32. */
void bqo_router_logits(const uint16_t* x, const uint16_t* router_proj,
                       const uint16_t* router_scale, int T, int H, int E, float sqrt_n,
                       float n_eps, float* logits) {
    float* scaled = (float*)malloc(sizeof(float) * H);
    for (int t = 0; t < T; ++t) {
        const uint16_t* xr = x + (size_t)t * H;
        float inv_rms = sqrt_n / sqrtf(bqo_rms_reduce_row(xr, H) + n_eps);
        for (int j = 0; j < H; ++j)
            scaled[j] = bqo_bf16_to_f32(xr[j]) * bqo_bf16_to_f32(router_scale[j]) * inv_rms;
        for (int e = 0; e < E; ++e)
            logits[(size_t)t * E + e] = dot_f32_bf16(scaled, router_proj + (size_t)e * H, H);
    }
    free(scaled);
}

/* kernels/moe_router.mojo:43-57 insert_candidate (candidates start as the
 * sentinel {expert 0, logit -1e30}; a logit enters at the first slot it beats,
 * ties going to the lower expert) + :276-293 the merge's softmax over the k:
 * ev = fast_exp_softmax_biased(logit - max), sum in slot order, w = ev *
 * (1/sum) * f32(per_expert_scale[expert]) (scale 1 when NULL). */
void bqo_route_topk_softmax(const float* logits, int T, int E, int top_k,
                            const uint16_t* per_expert_scale, int32_t* route_idx,
                            float* route_w) {
    int32_t* ce = (int32_t*)malloc(sizeof(int32_t) * top_k);
    float* cl = (float*)malloc(sizeof(float) * top_k);
    float* ev = (float*)malloc(sizeof(float) * top_k);
    for (int t = 0; t < T; ++t) {
        for (int k = 0; k < top_k; ++k) { ce[k] = 0; cl[k] = -1.0e30f; }
        const float* row = logits + (size_t)t * E;
        for (int e = 0; e < E; ++e) {
            float lg = row[e];
            for (int k = 0; k < top_k; ++k) {
                if (lg > cl[k] || (lg == cl[k] && e < ce[k])) {
                    for (int j = top_k - 1; j > k; --j) { ce[j] = ce[j - 1]; cl[j] = cl[j - 1]; }
                    ce[k] = e; cl[k] = lg;
                    break;
                }
            }
        }
        float mx = cl[0], sum = 0.0f;
        for (int k = 0; k < top_k; ++k) { ev[k] = bqo_fast_exp_softmax_biased(cl[k] - mx); sum += ev[k]; }
        float inv_sum = 1.0f / sum;
        for (int k = 0; k < top_k; ++k) {
            const float sc = per_expert_scale ? bqo_bf16_to_f32(per_expert_scale[ce[k]]) : 1.0f;
            route_idx[(size_t)t * top_k + k] = ce[k];
            route_w[(size_t)t * top_k + k] = ev[k] * inv_sum * sc;
        }
    }
    free(ce); free(cl); free(ev);
}

/* moe_router.mojo:60-106 */
void bqo_build_schedule(const int32_t* route_idx, const float* route_w, int T,
                        int top_k, int E, int32_t* expert_offset,
                        bqo_route* routes) {
    int32_t* counts = (int32_t*)calloc((size_t)E, sizeof(int32_t));
    int32_t* wr = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    for (int t = 0; t < T; ++t)
        for (int k = 0; k < top_k; ++k) {
            int e = route_idx[(size_t)t * top_k + k];
            if (e >= 0 && e < E) counts[e] += 1;
        }
    int32_t running = 0;
    for (int e = 0; e < E; ++e) { expert_offset[e] = running; wr[e] = running; running += counts[e]; }
    expert_offset[E] = running;
    for (int t = 0; t < T; ++t)
        for (int k = 0; k < top_k; ++k) {
            size_t slot = (size_t)t * top_k + k;
            int e = route_idx[slot];
            if (e >= 0 && e < E) {
                routes[wr[e]].token = t;
                routes[wr[e]].weight = route_w[slot];
                wr[e] += 1;
            }
        }
    free(counts); free(wr);
}

/* moe.mojo:25-129: bucket[rec, it*32+j] = bf16(gelu(g) * u) with
 * g = ((f32(iacc)-128cs)*(sa/127))*sw for gate row it*32+j and up row
 * inter + it*32+j of the expert (gate tile it, up tile n_inter_tiles+it). */
void bqo_moe_phase1(const int8_t* x_i8, const float* x_sa, int hidden,
                    const int32_t* expert_offset, const bqo_route* routes, int E,
                    const int8_t* w_gu_packed, const float* gu_scale,
                    const float* gu_colsum, int inter, uint16_t* bucket) {
    const float inv127 = 1.0f / 127.0f;
    int gate_up = 2 * inter;
    for (int e = 0; e < E; ++e) {
        const int8_t* w = w_gu_packed + (size_t)e * gate_up * hidden;
        const float* wsc = gu_scale + (size_t)e * gate_up;
        const float* cs = gu_colsum + (size_t)e * gate_up;
        for (int rec = expert_offset[e]; rec < expert_offset[e + 1]; ++rec) {
            int tok = routes[rec].token;
            const int8_t* x = x_i8 + (size_t)tok * hidden;
            float ad = x_sa[tok] * inv127;
            for (int i = 0; i < inter; ++i) {
                int ng = i, nu = inter + i;
                int32_t ga = vnni_u8_dot(x, w, ng, hidden, 0, hidden);
                int32_t ua = vnni_u8_dot(x, w, nu, hidden, 0, hidden);
                float gv = ((float)ga - 128.0f * cs[ng]) * ad * wsc[ng];
                float uv = ((float)ua - 128.0f * cs[nu]) * ad * wsc[nu];
                float res = bqo_gelu_tanh_f32(gv) * uv;
                bucket[(size_t)rec * inter + i] = bqo_f32_to_bf16(res);
            }
        }
    }
}

/* moe.mojo:167-295: accum zeroed; experts ascending, records ascending;
 * facc = fma over blocks; accum[tok] += (facc*sw)*route_w; out = bf16(accum). */
void bqo_moe_phase2(const int8_t* bucket_i8, const float* bucket_sa, int inter,
                    int block, const int32_t* expert_offset,
                    const bqo_route* routes, int E, int T,
                    const int8_t* w_d_packed, const float* d_scale,
                    const float* d_colsum, int hidden, float* accum,
                    uint16_t* out) {
    const float inv127 = 1.0f / 127.0f;
    int nb = inter / block;
    size_t data_n = (size_t)E * hidden;
    memset(accum, 0, sizeof(float) * (size_t)T * hidden);
    for (int e = 0; e < E; ++e) {
        const int8_t* w = w_d_packed + (size_t)e * hidden * inter;
        const float* wsc = d_scale + (size_t)e * hidden;
        size_t e_row_base = (size_t)e * hidden;
        for (int rec = expert_offset[e]; rec < expert_offset[e + 1]; ++rec) {
            const int8_t* x = bucket_i8 + (size_t)rec * inter;
            float* dst = accum + (size_t)routes[rec].token * hidden;
            float rw = routes[rec].weight;
            for (int n = 0; n < hidden; ++n) {
                float facc = 0.0f;
                for (int b = 0; b < nb; ++b) {
                    int32_t iacc = vnni_u8_dot(x, w, n, inter, b * block, (b + 1) * block);
                    float adv = bucket_sa[(size_t)rec * nb + b] * inv127;
                    float ccs = d_colsum[(size_t)b * data_n + e_row_base + n];
                    float corrected = (float)iacc - 128.0f * ccs;
                    facc = fmaf(corrected, adv, facc);
                }
                float res = facc * wsc[n] * rw;
                dst[n] = dst[n] + res;
            }
        }
    }
    for (size_t i = 0; i < (size_t)T * hidden; ++i) out[i] = bqo_f32_to_bf16(accum[i]);
}

/* ------------------------------------------------------------------------ */
/* synthetic inputs                                                          */
/* ------------------------------------------------------------------------ */

uint64_t bqo_splitmix64(uint64_t* state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* uniform in (0,1]: (top 53 bits + 1) * 2^-53 */
static double u01(uint64_t* st) {
    return ((double)(bqo_splitmix64(st) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

void bqo_synth_normal_f32(uint64_t seed, double sigma, float* out, size_t n) {
    uint64_t st = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = u01(&st), u2 = u01(&st);
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(sigma * r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(sigma * r * sin(two_pi * u2));
    }
}

void bqo_synth_normal_bf16(uint64_t seed, double sigma, uint16_t* out, size_t n) {
    const size_t chunk = 1 << 16;
    float* tmp = (float*)malloc(sizeof(float) * chunk);
    /* one generator stream across chunks: regenerate with a running state */
    uint64_t st = seed;
    const double two_pi = 6.283185307179586476925286766559;
    size_t i = 0;
    while (i < n) {
        size_t m = n - i < chunk ? n - i : chunk;
        for (size_t j = 0; j < m; j += 2) {
            double u1 = u01(&st), u2 = u01(&st);
            double r = sqrt(-2.0 * log(u1));
            tmp[j] = (float)(sigma * r * cos(two_pi * u2));
            if (j + 1 < m) tmp[j + 1] = (float)(sigma * r * sin(two_pi * u2));
        }
        for (size_t j = 0; j < m; ++j) out[i + j] = bqo_f32_to_bf16(tmp[j]);
        i += m;
    }
    free(tmp);
}

/* ========================================================================
 * bq head and embedding (butterquant_kernels/head.mojo, embedding.mojo)
 * ======================================================================== */

/* simd_math/ops.mojo:35-69 exp_f32: clamp to [-87, 88] through bit masks,
 * n = trunc(xn + 0.5 - sign(xn)), two-constant Cody-Waite reduction, degree-6
 * polynomial, times 2^n. */
float bqo_exp_f32(float x) {
    const float LN2_HI = 0.693145751953125f, LN2_LO = 1.4286068203094172e-06f;
    const float INV_LN2 = 1.4426950408889634f, EXP_LO = -87.0f, EXP_HI = 88.0f;
    float lo = (float)((f2u(x - EXP_LO) >> 31) & 1u);
    float xc = x * (1.0f - lo) + EXP_LO * lo;
    float hi = (float)((f2u(EXP_HI - xc) >> 31) & 1u);
    xc = xc * (1.0f - hi) + EXP_HI * hi;
    float xn = xc * INV_LN2;
    float sign = (float)(f2u(xn) >> 31);
    int32_t n = (int32_t)(xn + 0.5f - sign);
    float nf = (float)n;
    float r = (xc - nf * LN2_HI) - nf * LN2_LO;
    float p = 1.0f + r * (0.9999999995f + r * (0.5000000004f + r * (0.1666666456f +
              r * (0.04166685110f + r * (0.008333621758f + r * 0.001389404636f)))));
    return p * u2f(((uint32_t)(n + 127)) << 23);
}

/* simd_math/ops.mojo:100-124 log_f32: exponent/mantissa split, mantissa
 * folded into [sqrt2/2, sqrt2), atanh series in z = (m-1)/(m+1). */
float bqo_log_f32(float x) {
    const float LN2 = 0.6931471805599453f, SQRT2 = 1.4142135623730951f;
    uint32_t bits = f2u(x);
    int32_t e = (int32_t)(bits >> 23) - 127;
    float m = u2f((bits & 0x007FFFFFu) | 0x3F800000u);
    uint32_t big = f2u(SQRT2 - m) >> 31;
    float big_f = (float)big;
    m = m * (1.0f - 0.5f * big_f);
    e = e + (int32_t)big;
    float z = (m - 1.0f) / (m + 1.0f);
    float z2 = z * z;
    float t = (float)(1.0 / 11.0);
    t = (float)(1.0 / 9.0) + z2 * t;
    t = (float)(1.0 / 7.0) + z2 * t;
    t = (float)(1.0 / 5.0) + z2 * t;
    t = (float)(1.0 / 3.0) + z2 * t;
    t = 1.0f + z2 * t;
    return 2.0f * z * t + (float)e * LN2;
}

/* simd_math/sampling_rng.mojo:10-43: the SplitMix64 finalizer keyed on
 * (row << 32) ^ idx; u = (f32(h >> 40) + 1) / (2^24 + 1 rounded to f32);
 * gumbel = -log(-log(u)). */
uint64_t bqo_mix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

float bqo_gumbel_noise(uint64_t seed, int64_t row, int64_t idx) {
    uint64_t counter = ((uint64_t)row << 32) ^ (uint64_t)idx;
    uint64_t h = bqo_mix64(seed ^ bqo_mix64(counter));
    const float top24 = 16777216.0f;
    float u = ((float)(int64_t)(h >> 40) + 1.0f) / (top24 + 1.0f);
    return -bqo_log_f32(-bqo_log_f32(u));
}

/* simd_math/ops.mojo:160-167 softcap_value[cap] = tanh_f32(x / cap) * cap */
float bqo_softcap(float x, float cap) { return bqo_tanh_f32(x / cap) * cap; }

/* butterquant/dot_products.mojo:76-88 head_logit_row: per block the exact
 * int32 dot, then acc += f32(r) * (sa[b] / 127) * scales[b] in block order. */
float bqo_head_logit_row(const int8_t* x_i8, const float* sa, const int8_t* w,
                         const float* wscales, int cols, int block) {
    float acc = 0.0f;
    for (int b = 0; b < cols / block; ++b) {
        int32_t r = 0;
        for (int k = b * block; k < (b + 1) * block; ++k) r += (int32_t)x_i8[k] * (int32_t)w[k];
        acc += (float)r * (sa[b] / 127.0f) * wscales[b];
    }
    return acc;
}

/* kernels/flash_sample.mojo:33-117 SampleAccum (one accumulator). */
typedef struct {
    int n;
    float* val;
    float* g;
    int32_t* idx;
    float lse_max, lse_sum, samp_score;
    int32_t samp_idx;
} accum_t;

static void topn_insert(accum_t* a, float y, float g, int32_t idx, int cap) {
    if (a->n == cap && y <= a->val[cap - 1]) return;
    int p;
    if (a->n < cap) { p = a->n; a->n += 1; } else { p = cap - 1; }
    while (p > 0 && a->val[p - 1] < y) {
        a->val[p] = a->val[p - 1]; a->g[p] = a->g[p - 1]; a->idx[p] = a->idx[p - 1];
        p -= 1;
    }
    a->val[p] = y; a->g[p] = g; a->idx[p] = idx;
}

static void lse_push(accum_t* a, float yt) {
    if (a->lse_sum <= 0.0f) {
        a->lse_max = yt; a->lse_sum = 1.0f;
    } else if (yt > a->lse_max) {
        a->lse_sum = a->lse_sum * bqo_exp_f32(a->lse_max - yt) + 1.0f;
        a->lse_max = yt;
    } else {
        a->lse_sum = a->lse_sum + bqo_exp_f32(yt - a->lse_max);
    }
}

/* BqFlashSampleKernel.execute (butterquant_kernels/head.mojo:85-117) over the
 * whole vocabulary as one worker, then finalize_outcomes
 * (kernels/flash_sample.mojo:221-265).  weight int8 [V, cols] row-major,
 * wscales [V, cols/block]; params / outcomes as bqo_sampling_params /
 * bqo_sample_outcome. */
void bqo_flash_sample(const int8_t* x_i8, const float* x_sa, const int8_t* weight,
                      const float* wscales, int rows, int vocab, int cols, int block,
                      float cap, int64_t vocab_base, const bqo_sampling_params* params,
                      bqo_sample_outcome* out) {
    const int nmax = BQO_SAMPLE_NMAX, nb = cols / block;
    accum_t* acc = (accum_t*)calloc((size_t)rows, sizeof(accum_t));
    for (int r = 0; r < rows; ++r) {
        acc[r].val = (float*)malloc(sizeof(float) * nmax);
        acc[r].g = (float*)malloc(sizeof(float) * nmax);
        acc[r].idx = (int32_t*)malloc(sizeof(int32_t) * nmax);
        for (int k = 0; k < nmax; ++k) { acc[r].val[k] = -1.0e30f; acc[r].g[k] = -1.0e30f; acc[r].idx[k] = -1; }
        acc[r].n = 0; acc[r].lse_max = -1.0e30f; acc[r].lse_sum = 0.0f;
        acc[r].samp_score = -1.0e30f; acc[r].samp_idx = -1;
    }
    for (int v = 0; v < vocab; ++v) {
        const int64_t gidx = vocab_base + v;
        for (int r = 0; r < rows; ++r) {
            const bqo_sampling_params* p = &params[r];
            float raw = bqo_head_logit_row(x_i8 + (size_t)r * cols, x_sa + (size_t)r * nb,
                                           weight + (size_t)v * cols, wscales + (size_t)v * nb,
                                           cols, block);
            float inv_t = 1.0f / p->temperature;
            float y = bqo_bf16_to_f32(bqo_f32_to_bf16(bqo_softcap(raw, cap)));
            float g = p->greedy ? 0.0f : bqo_gumbel_noise(p->seed, r, gidx);
            float yt = y * inv_t;
            lse_push(&acc[r], yt);
            float score = yt + g;
            if (score > acc[r].samp_score) { acc[r].samp_score = score; acc[r].samp_idx = (int32_t)gidx; }
            topn_insert(&acc[r], y, score, (int32_t)gidx, nmax);
        }
    }
    for (int r = 0; r < rows; ++r) {
        accum_t* f = &acc[r];
        const bqo_sampling_params* p = &params[r];
        int n_out = f->n < p->n_keep ? f->n : (int)p->n_keep;
        int32_t token = f->samp_idx;
        int use_min_p = p->min_p > 0.0f, use_top_k = p->top_k > 0;
        if ((use_min_p || use_top_k) && f->n > 0) {
            int limit = f->n;
            if (use_top_k && p->top_k < limit) limit = (int)p->top_k;
            float thr = -1.0e30f;
            if (use_min_p) thr = f->val[0] + p->temperature * bqo_log_f32(p->min_p);
            int32_t best_idx = f->idx[0];
            float best_g = f->g[0];
            for (int k = 1; k < limit; ++k)
                if (f->val[k] >= thr && f->g[k] > best_g) { best_g = f->g[k]; best_idx = f->idx[k]; }
            token = best_idx;
        }
        bqo_sample_outcome* o = &out[r];
        o->token_id = token;
        o->logz = f->lse_max + bqo_log_f32(f->lse_sum);
        o->n = n_out;
        for (int k = 0; k < nmax; ++k) { o->topn_val[k] = -1.0e30f; o->topn_idx[k] = -1; }
        for (int k = 0; k < n_out; ++k) { o->topn_val[k] = f->val[k]; o->topn_idx[k] = f->idx[k]; }
        free(f->val); free(f->g); free(f->idx);
    }
    free(acc);
}

/* BqEmbedLookupKernel.execute (butterquant_kernels/embedding.mojo:36-53):
 * per token, the owning shard's row is dequantized per block (q * scale,
 * butterquant/dequantize.mojo:6-21), FWHT(block)-rotated and written as
 * bf16(x * scale) (dequantize.mojo:25-32); a token owned by another shard
 * gives a zero row.  The owner is Mojo's floor division tid // shard_rows
 * (embedding.mojo:42), so a negative id belongs to no rank >= 0.
 * weight int8 [shard_rows, hidden] row-major. */
void bqo_embed_lookup(const int32_t* token_ids, int T, const int8_t* weight,
                      const float* wscales, int hidden, int block, int shard_rows,
                      int rank, float scale, uint16_t* dst) {
    const int nb = hidden / block;
    float* ws = (float*)malloc(sizeof(float) * hidden);
    for (int t = 0; t < T; ++t) {
        int tid = token_ids[t], owner = tid / shard_rows;
        if (tid % shard_rows != 0 && tid < 0) owner -= 1;  /* floor division */
        uint16_t* d = dst + (size_t)t * hidden;
        if (owner != rank) { for (int k = 0; k < hidden; ++k) d[k] = 0; continue; }
        int local = tid - owner * shard_rows;
        const int8_t* q = weight + (size_t)local * hidden;
        for (int b = 0; b < nb; ++b)
            for (int k = b * block; k < (b + 1) * block; ++k)
                ws[k] = (float)q[k] * wscales[(size_t)local * nb + b];
        bqo_fwht_row(ws, hidden, block);
        for (int k = 0; k < hidden; ++k) d[k] = bqo_f32_to_bf16(ws[k] * scale);
    }
    free(ws);
}

/* ------------------------------------------------------------------------ */
/* int8-KV attention: prep and flash attention                               */
/* ------------------------------------------------------------------------ */

/* 16-lane halving-tree reduce_add of one SIMD[f32, 16] */
static float tree16(float* s) {
    for (int half = 8; half >= 1; half /= 2)
        for (int j = 0; j < half; ++j) s[j] = s[j] + s[j + half];
    return s[0];
}

/* attention_ops.mojo:45-51 PagedKV.slot(0, p) */
static int64_t paged_slot(const int32_t* rows, int shift, int row_mask, int page_mask, int64_t p) {
    return (int64_t)rows[(p >> shift) & page_mask] + (p & row_mask);
}

/* attention.mojo:489-492: the run holding buffer row tok (runs advance while
 * tok >= runs[r+1].buf_start) */
static int run_of(const bqo_kv_run* runs, int num_runs, int tok) {
    int r = 0;
    while (r + 1 < num_runs && tok >= runs[r + 1].buf_start) ++r;
    return r;
}

/* head_prep.mojo:9-92.  head_inv_rms (:9-16): 16 f32 lanes, lane k is
 * x[k]*x[k] then an fma chain over x[16i + k], then a 16-lane tree;
 * inv = sqrt_n / sqrt(ssq + n_eps).  q/k (prep_head_qk_i8 :39-71): x*inv*g,
 * RoPE on pairs (i, pair_stride + i) for i < rope_half, FWHT(head_dim),
 * absmax quantize (:19-36: amax floored at 1e-10, codes, their i32 sum).
 * v (prep_head_v_i8 :74-92): x*inv, FWHT, quantize.  gamma == NULL selects
 * the v form. */
static void prep_head(const uint16_t* src, const uint16_t* gamma, const float* cs,
                      const float* sn, int hd, int rope_half, int pair_stride, float sqrt_n,
                      float n_eps, int8_t* out, float* amax_out, int32_t* qsum_out) {
    float r[1024];
    for (int i = 0; i < hd; ++i) r[i] = bqo_bf16_to_f32(src[i]);
    float ssq[16];
    for (int k = 0; k < 16; ++k) {
        ssq[k] = r[k] * r[k];
        for (int i = 1; i < hd / 16; ++i) ssq[k] = fmaf(r[16 * i + k], r[16 * i + k], ssq[k]);
    }
    float inv = sqrt_n / sqrtf(tree16(ssq) + n_eps);
    for (int i = 0; i < hd; ++i) {
        r[i] = r[i] * inv;
        if (gamma) r[i] = r[i] * bqo_bf16_to_f32(gamma[i]);
    }
    if (gamma) {
        for (int i = 0; i < rope_half; ++i) {
            float lo = r[i], hi = r[pair_stride + i];
            r[i] = lo * cs[i] - hi * sn[i];
            r[pair_stride + i] = hi * cs[i] + lo * sn[i];
        }
    }
    bqo_fwht_block(r, hd);
    float amax = 0.0f;
    for (int i = 0; i < hd; ++i) amax = fmaxf(amax, fabsf(r[i]));
    if (amax < 1e-10f) amax = 1e-10f;
    float qinv = 127.0f / amax;
    int32_t qsum = 0;
    for (int i = 0; i < hd; ++i) {
        out[i] = quantize_i8(r[i], qinv);
        qsum += out[i];
    }
    *amax_out = amax;
    if (qsum_out) *qsum_out = qsum;
}

/* attention.mojo:474-534 BqAttnPrepKernel.execute */
void bqo_attn_prep(const uint16_t* q_src, const uint16_t* k_src, const uint16_t* v_src,
                   const uint16_t* q_norm, const uint16_t* k_norm, int8_t* q_i8,
                   float* qi_bias, float* f_q, int8_t* k_cache, float* k_scale,
                   int8_t* v_cache, float* v_scale, const float* cos_table,
                   const float* sin_table, const bqo_kv_run* runs, int num_runs,
                   const int32_t* base_rows, int seq_len, int num_q, int num_kv,
                   int head_dim, int rope_half, int pair_stride, float sqrt_n, float n_eps,
                   int cache_degree, int rank, int page_shift, int row_mask, int page_mask) {
    const int64_t qs = (int64_t)num_q * head_dim, kvs = (int64_t)num_kv * head_dim;
    for (int tok = 0; tok < seq_len; ++tok) {
        int r = run_of(runs, num_runs, tok);
        int64_t pos = runs[r].base_pos + (tok - runs[r].buf_start);
        const float* cs = cos_table + pos * rope_half;
        const float* sn = sin_table + pos * rope_half;
        for (int h = 0; h < num_q; ++h) {
            float amax;
            int32_t qsum;
            prep_head(q_src + tok * qs + h * head_dim, q_norm, cs, sn, head_dim, rope_half,
                      pair_stride, sqrt_n, n_eps, q_i8 + tok * qs + h * head_dim, &amax, &qsum);
            qi_bias[(int64_t)tok * num_q + h] = (float)qsum * 128.0f;
            f_q[(int64_t)tok * num_q + h] = amax;
        }
        if (pos % cache_degree != rank) continue;
        int64_t slot = paged_slot(base_rows + runs[r].rows_off, page_shift, row_mask, page_mask,
                                  pos / cache_degree);
        for (int h = 0; h < num_kv; ++h) {
            prep_head(k_src + tok * kvs + h * head_dim, k_norm, cs, sn, head_dim, rope_half,
                      pair_stride, sqrt_n, n_eps, k_cache + slot * kvs + h * head_dim,
                      k_scale + slot * num_kv + h, NULL);
            prep_head(v_src + tok * kvs + h * head_dim, NULL, NULL, NULL, head_dim, 0, 0, sqrt_n,
                      n_eps, v_cache + slot * kvs + h * head_dim, v_scale + slot * num_kv + h,
                      NULL);
        }
    }
}

/* Splits of one query token's KV range of length L: S = min(s_max,
 * max(1, ceil(L / min_split))) ranges, range s = worker_range(L, S, s)
 * (kernels/helpers.mojo:182-190).  This is the GPU's partition (the
 * reference's decode splits by its worker pool); it fixes the f32 merge
 * order, so the oracle takes it as an input. */
int bqo_attn_num_splits(int L, int s_max, int min_split) {
    if (L <= 0) return 1;
    int s = (L + min_split - 1) / min_split;
    return s < s_max ? s : s_max;
}

static void worker_range(int total, int n, int id, int* s, int* e) {
    int per = (total + n - 1) / n;
    *s = id * per;
    *e = *s + per < total ? *s + per : total;
    if (*s >= total) *s = *e = total;
}

static inline float max87(float x) { return x > -87.0f ? x : -87.0f; }

typedef struct { float m, l; } ml_t;

/* attention.mojo:32-80 bq_process_kv_tile for one q head over positions
 * [lo + pos, lo + pos + tile_len), plus the tile loop of attention.mojo:127-
 * 136.  score = (f32(sum (k^0x80) * q) - qi_bias) * f_q * ks / 127^2 (the
 * u8-shifted VNNI dot, butterquant/dot_products.mojo:41-60, of K against Q);
 * online_softmax_tile (attention_ops.mojo:166-182); acc *= corr;
 * l = l*corr + reduce_add(w); acc += (w*vs/127) * v (fma per element,
 * helpers.mojo:48-66). */
static void attn_range(const int8_t* q, float qb, float fq, const int8_t* k_cache,
                       const float* k_scale, const int8_t* v_cache, const float* v_scale,
                       const int32_t* rows, int shift, int row_mask, int page_mask,
                       int64_t kvs, int num_kv, int kv_h, int hd, int64_t lo, int start,
                       int end, ml_t* ml, float* acc) {
    const float inv127 = 1.0f / 127.0f;
    const float inv127sq = inv127 * inv127;
    ml->m = -1e30f;
    ml->l = 0.0f;
    for (int j = 0; j < hd; ++j) acc[j] = 0.0f;
    for (int pos = start; pos < end; pos += 16) {
        int tl = end - pos < 16 ? end - pos : 16;
        int64_t slots[16];
        float sc[16], w[16];
        for (int t = 0; t < 16; ++t) sc[t] = -1e30f;
        for (int t = 0; t < tl; ++t) {
            slots[t] = paged_slot(rows, shift, row_mask, page_mask, lo + pos + t);
            const int8_t* kh = k_cache + slots[t] * kvs + (int64_t)kv_h * hd;
            int32_t rr = 0;
            for (int j = 0; j < hd; ++j) rr += (int32_t)((uint8_t)kh[j] ^ 0x80u) * q[j];
            float ks = k_scale[slots[t] * num_kv + kv_h];
            sc[t] = (((float)rr - qb) * fq) * ks * inv127sq;
        }
        float tmax = sc[0];
        for (int t = 1; t < 16; ++t) tmax = sc[t] > tmax ? sc[t] : tmax;
        float m_new = tmax > ml->m ? tmax : ml->m;
        float corr = bqo_fast_exp_softmax_biased(max87(ml->m - m_new));
        for (int t = 0; t < 16; ++t) w[t] = bqo_fast_exp_softmax_biased(max87(sc[t] - m_new));
        for (int j = 0; j < hd; ++j) acc[j] = acc[j] * corr;
        float wl[16];
        memcpy(wl, w, sizeof(wl));
        ml->l = ml->l * corr + tree16(wl);
        ml->m = m_new;
        for (int t = 0; t < tl; ++t) {
            const int8_t* vh = v_cache + slots[t] * kvs + (int64_t)kv_h * hd;
            float s = w[t] * v_scale[slots[t] * num_kv + kv_h] * inv127;
            for (int j = 0; j < hd; ++j) acc[j] = fmaf((float)vh[j], s, acc[j]);
        }
    }
}

/* logsum_merge.mojo:29-122 merge_segments + write_finalized_head over the n
 * split partials of one head, in split order */
static void merge_write(const ml_t* ml, const float* acc, int n, int hd, uint16_t* dst,
                        float* dst32) {
    float gm = -1e30f;
    for (int s = 0; s < n; ++s) if (ml[s].m > gm) gm = ml[s].m;
    float gl = 0.0f, out[1024];
    int first = 1;
    for (int b0 = 0; b0 < n; b0 += 16) {
        int bl = n - b0 < 16 ? n - b0 : 16;
        float d[16], ls[16], c[16], prod[16];
        for (int b = 0; b < 16; ++b) { d[b] = -1e30f; ls[b] = 0.0f; }
        for (int b = 0; b < bl; ++b) { d[b] = ml[b0 + b].m - gm; ls[b] = ml[b0 + b].l; }
        for (int b = 0; b < 16; ++b) {
            c[b] = bqo_fast_exp_softmax_biased(max87(d[b]));
            if (!(ls[b] > 0.0f)) c[b] = 0.0f;
            prod[b] = ls[b] * c[b];
        }
        gl += tree16(prod);
        for (int b = 0; b < bl; ++b) {
            if (c[b] <= 0.0f) continue;
            const float* src = acc + (size_t)(b0 + b) * hd;
            if (first) { for (int j = 0; j < hd; ++j) out[j] = src[j] * c[b]; first = 0; }
            else for (int j = 0; j < hd; ++j) out[j] = fmaf(src[j], c[b], out[j]);
        }
    }
    if (gl <= 0.0f) {
        for (int j = 0; j < hd; ++j) { dst[j] = 0; if (dst32) dst32[j] = 0.0f; }
        return;
    }
    float inv_l = 1.0f / gl;
    for (int j = 0; j < hd; ++j) {
        float y = out[j] * inv_l;
        dst[j] = bqo_f32_to_bf16(y);
        if (dst32) dst32[j] = y;
    }
}

/* attention.mojo:83-146 (decode, split + merge), :149-247 (sliding prefill:
 * window [pos - window + 1, pos], out = acc * (1/l) or zeros) and :250-327
 * (full prefill: rank-local rows [0, full_local_kv_count), attention_ops.mojo:
 * 146-152, then the merge).  window > 0 selects the sliding form: a token
 * whose range is one split is finalized directly as the sliding prefill
 * kernel does; every other token goes through the merge.  out_f32 (may be
 * NULL) receives the values before the bf16 cast. */
void bqo_flash_attention(const int8_t* q_i8, const float* qi_bias, const float* f_q,
                         const int8_t* k_cache, const float* k_scale, const int8_t* v_cache,
                         const float* v_scale, const bqo_kv_run* runs, int num_runs,
                         const int32_t* base_rows, int seq_len, int num_q, int num_kv,
                         int head_dim, int window, int degree, int rank, int page_shift,
                         int row_mask, int page_mask, int s_max, int min_split,
                         uint16_t* out, float* out_f32) {
    const int gqa = num_q / num_kv;
    const int64_t kvs = (int64_t)num_kv * head_dim, qs = (int64_t)num_q * head_dim;
    ml_t* ml = (ml_t*)malloc(sizeof(ml_t) * (size_t)s_max);
    float* acc = (float*)malloc(sizeof(float) * (size_t)s_max * head_dim);
    for (int tok = 0; tok < seq_len; ++tok) {
        int r = run_of(runs, num_runs, tok);
        int64_t pos = runs[r].base_pos + (tok - runs[r].buf_start);
        const int32_t* rows = base_rows + runs[r].rows_off;
        int64_t lo;
        int L;
        if (window > 0) {
            lo = pos - window + 1 > 0 ? pos - window + 1 : 0;
            L = (int)(pos + 1 - lo);
        } else {
            lo = 0;
            L = pos < 0 ? 0 : (rank <= pos % degree ? (int)(pos / degree + 1) : (int)(pos / degree));
        }
        int S = bqo_attn_num_splits(L, s_max, min_split);
        for (int h = 0; h < num_q; ++h) {
            const int8_t* q = q_i8 + tok * qs + (int64_t)h * head_dim;
            float qb = qi_bias[(int64_t)tok * num_q + h], fq = f_q[(int64_t)tok * num_q + h];
            for (int s = 0; s < S; ++s) {
                int a, e;
                worker_range(L, S, s, &a, &e);
                attn_range(q, qb, fq, k_cache, k_scale, v_cache, v_scale, rows, page_shift,
                           row_mask, page_mask, kvs, num_kv, h / gqa, head_dim, lo, a, e, &ml[s],
                           acc + (size_t)s * head_dim);
            }
            uint16_t* dst = out + tok * qs + (int64_t)h * head_dim;
            float* d32 = out_f32 ? out_f32 + tok * qs + (int64_t)h * head_dim : NULL;
            if (window > 0 && S == 1) {
                float inv_l = ml[0].l > 0.0f ? 1.0f / ml[0].l : 0.0f;
                for (int j = 0; j < head_dim; ++j) {
                    float y = ml[0].l > 0.0f ? acc[j] * inv_l : 0.0f;
                    dst[j] = ml[0].l > 0.0f ? bqo_f32_to_bf16(y) : 0;
                    if (d32) d32[j] = y;
                }
            } else {
                merge_write(ml, acc, S, head_dim, dst, d32);
            }
        }
    }
    free(ml);
    free(acc);
}
