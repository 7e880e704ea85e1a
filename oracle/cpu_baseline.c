/*
 * cpu_baseline.c -- the reference's CPU hot path ported to C with AVX-512 VNNI
 * intrinsics and OpenMP, for the CPU baseline that bench.py reports beside the
 * GPU numbers (test infrastructure: never linked into the HIP library).
 *
 * It follows the reference's VNNI branch (the one non-AMX hosts take,
 * butterquant_kernels/linear.mojo:100-111):
 *   - packed 32x64 tiles, 4 activation bytes XOR 0x80 broadcast, vpdpbusd
 *     (butterquant/gemm.mojo:36-75, dot_products.mojo:7-37);
 *   - M panels of PR = 4 rows (gemm.mojo:20-33 reg_capped_panel at width 16);
 *   - the colsum epilogues (gemm.mojo:133-142, 200-215);
 *   - 32-row N tiles split over workers by worker_range
 *     (kernels/helpers.mojo:181-190); MoE phase 1 over 22 intermediate tiles,
 *     phase 2 over 88 hidden tiles (moe.mojo:132-164, 298-335).
 * When the host lacks AVX-512 VNNI the scalar oracle runs instead and
 * bqcpu_isa() reports "scalar".
 */
#define _GNU_SOURCE
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>

#include "bq_oracle.h"

#define VNNI_FN __attribute__((target("avx512f,avx512bw,avx512vnni")))

static int have_vnni(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw");
}

const char* bqcpu_isa(void) { return have_vnni() ? "avx512vnni" : "scalar"; }

/* kernels/helpers.mojo:181-190 */
static void worker_range(int total, int workers, int w, int* s, int* e) {
    int per = (total + workers - 1) / workers;
    *s = w * per;
    *e = *s + per < total ? *s + per : total;
    if (*s >= total) { *s = total; *e = total; }
}

static inline uint16_t f2bf(float v) { return bqo_f32_to_bf16(v); }

/* Worker-count policies of the reference's dispatchers, `capacity` being the
 * pool size (the thread count the caller gives):
 *   recommended_workers (kernels/helpers.mojo:204-218) with the constants of
 *   kernels/dispatch_heuristics.mojo:9-14 -- the default policy (norm-quant,
 *   block-quant), matmul_workers (helpers.mojo:289-292: linears),
 *   saturate_workers (:284-286: MoE phases) and merge_workers
 *   (kernels/logsum_merge.mojo:199-202: the router merge);
 *   fanout_dispatch runs inline (one worker) when data_bytes <= its
 *   inline threshold (helpers.mojo:309-315). */
static int recommended_workers(long bw_product, long amortized, long data_bytes, int capacity) {
    if (capacity <= 1) return capacity;
    if (data_bytes >= amortized) return capacity;
    long target = data_bytes / bw_product;
    int n = 1;
    while ((long)(n + 1) * (n + 1) <= target && n < capacity) ++n;
    return n;
}
static int default_workers(long data_bytes, int capacity) {
    return recommended_workers(2280, 1L << 20, data_bytes, capacity);
}
static int matmul_workers(long data_bytes, int capacity) {
    return recommended_workers(22528, 1L << 30, data_bytes, capacity);
}
static int merge_workers(long data_bytes, int capacity) {
    if (data_bytes >= (1L << 20)) return capacity;
    return capacity < 8 ? capacity : 8;
}
static int min_i(int a, int b) { return a < b ? a : b; }

/* Pin the OpenMP team of n threads (the calling thread is thread 0), thread
 * i to CPU cpus[i] -- the reference pins one worker per core of its NUMA
 * rank (threading/topological_dispatch.mojo).  libgomp keeps the team's
 * threads for later parallel regions of at most n threads.  0 on success. */
int bqcpu_pin(const int* cpus, int n) {
    int bad = 0;
#pragma omp parallel num_threads(n) reduction(+ : bad)
    {
        cpu_set_t set;
        CPU_ZERO(&set);
        CPU_SET(cpus[omp_get_thread_num()], &set);
        bad += pthread_setaffinity_np(pthread_self(), sizeof(set), &set) != 0;
        bad += omp_get_num_threads() != n;
    }
    return bad ? -1 : 0;
}

/* One 32-row tile x PR rows: accumulate_tiles (gemm.mojo:36-75) over K range
 * [k_base, k_base+k_len) starting at packed byte offset packed_base. */
VNNI_FN static void acc_tile(const int8_t* const* rows, int pr, const int8_t* wp,
                             size_t packed_base, int k_base, int k_len,
                             __m512i acc[][2]) {
    size_t off = packed_base;
    for (int ks = 0; ks < k_len; ks += 64) {
        for (int dc = 0; dc < 16; ++dc) {
            int kpos = k_base + ks + dc * 4;
            __m512i w0 = _mm512_loadu_si512((const void*)(wp + off + (size_t)dc * 64));
            __m512i w1 = _mm512_loadu_si512((const void*)(wp + off + 1024 + (size_t)dc * 64));
            for (int r = 0; r < pr; ++r) {
                uint32_t b4;
                memcpy(&b4, rows[r] + kpos, 4);
                __m512i ab = _mm512_set1_epi32((int)(b4 ^ 0x80808080u));
                acc[r][0] = _mm512_dpbusd_epi32(acc[r][0], ab, w0);
                acc[r][1] = _mm512_dpbusd_epi32(acc[r][1], ab, w1);
            }
        }
        off += 2048;
    }
}

/* gemm.mojo:114-170 over tiles [t0,t1) */
VNNI_FN static void per_row_tiles(const int8_t* act, const float* sa, int m,
                                  const int8_t* wp, const float* wsc, const float* cs,
                                  int N, int K, uint16_t* out, int t0, int t1) {
    const float inv127 = 1.0f / 127.0f;
    for (int mp = 0; mp < m; mp += 4) {
        int pr = m - mp < 4 ? m - mp : 4;
        const int8_t* rows[4];
        for (int r = 0; r < pr; ++r) rows[r] = act + (size_t)(mp + r) * K;
        for (int t = t0; t < t1; ++t) {
            __m512i acc[4][2];
            for (int r = 0; r < 4; ++r) { acc[r][0] = _mm512_setzero_si512(); acc[r][1] = _mm512_setzero_si512(); }
            acc_tile(rows, pr, wp, (size_t)t * 32 * K, 0, K, acc);
            for (int r = 0; r < pr; ++r) {
                __m512 ad = _mm512_set1_ps(sa[mp + r] * inv127);
                for (int a = 0; a < 2; ++a) {
                    int nb = t * 32 + a * 16;
                    __m512 corr = _mm512_sub_ps(_mm512_cvtepi32_ps(acc[r][a]),
                                                _mm512_mul_ps(_mm512_set1_ps(128.0f), _mm512_loadu_ps(cs + nb)));
                    __m512 res = _mm512_mul_ps(_mm512_mul_ps(corr, ad), _mm512_loadu_ps(wsc + nb));
                    float tmp[16];
                    _mm512_storeu_ps(tmp, res);
                    for (int j = 0; j < 16; ++j) out[(size_t)(mp + r) * N + nb + j] = f2bf(tmp[j]);
                }
            }
        }
    }
}

/* gemm.mojo:173-243 over tiles [t0,t1) */
VNNI_FN static void per_block_tiles(const int8_t* act, const float* sa, int m,
                                    const int8_t* wp, const float* wsc, const float* cs,
                                    int N, int K, int block, uint16_t* out, int t0, int t1) {
    const float inv127 = 1.0f / 127.0f;
    int nb = K / block;
    for (int mp = 0; mp < m; mp += 4) {
        int pr = m - mp < 4 ? m - mp : 4;
        const int8_t* rows[4];
        for (int r = 0; r < pr; ++r) rows[r] = act + (size_t)(mp + r) * K;
        for (int t = t0; t < t1; ++t) {
            __m512 facc[4][2];
            for (int r = 0; r < 4; ++r) { facc[r][0] = _mm512_setzero_ps(); facc[r][1] = _mm512_setzero_ps(); }
            for (int b = 0; b < nb; ++b) {
                __m512i acc[4][2];
                for (int r = 0; r < 4; ++r) { acc[r][0] = _mm512_setzero_si512(); acc[r][1] = _mm512_setzero_si512(); }
                acc_tile(rows, pr, wp, (size_t)t * 32 * K + (size_t)b * block * 32, b * block, block, acc);
                for (int r = 0; r < pr; ++r) {
                    __m512 adv = _mm512_set1_ps(sa[(size_t)(mp + r) * nb + b] * inv127);
                    for (int a = 0; a < 2; ++a) {
                        int n0 = t * 32 + a * 16;
                        __m512 corr = _mm512_sub_ps(_mm512_cvtepi32_ps(acc[r][a]),
                                                    _mm512_mul_ps(_mm512_set1_ps(128.0f), _mm512_loadu_ps(cs + (size_t)b * N + n0)));
                        facc[r][a] = _mm512_fmadd_ps(corr, adv, facc[r][a]);
                    }
                }
            }
            for (int r = 0; r < pr; ++r)
                for (int a = 0; a < 2; ++a) {
                    int n0 = t * 32 + a * 16;
                    __m512 res = _mm512_mul_ps(facc[r][a], _mm512_loadu_ps(wsc + n0));
                    float tmp[16];
                    _mm512_storeu_ps(tmp, res);
                    for (int j = 0; j < 16; ++j) out[(size_t)(mp + r) * N + n0 + j] = f2bf(tmp[j]);
                }
        }
    }
}

/* dispatch_bq_linear (linear.mojo:119-149) */
void bqcpu_linear(const int8_t* act, const float* sa, int m, const int8_t* wp,
                  const float* wsc, const float* cs, int N, int K, uint16_t* out,
                  int nthreads) {
    if (m <= 0) return;
    if (!have_vnni()) { bqo_gemm_i8_per_row(act, sa, m, wp, wsc, cs, N, K, out, NULL); return; }
    int tiles = N / 32;
    int workers = min_i(matmul_workers((long)N * K * m, nthreads), tiles);
#pragma omp parallel num_threads(workers)
    {
        int s, e;
        worker_range(tiles, workers, omp_get_thread_num(), &s, &e);
        per_row_tiles(act, sa, m, wp, wsc, cs, N, K, out, s, e);
    }
}

/* dispatch_bq_block_linear (linear.mojo:240-270) */
void bqcpu_block_linear(const int8_t* act, const float* sa, int m, const int8_t* wp,
                        const float* wsc, const float* cs, int N, int K, int block,
                        uint16_t* out, int nthreads) {
    if (m <= 0) return;
    if (!have_vnni()) { bqo_gemm_i8_per_block(act, sa, m, wp, wsc, cs, N, K, block, out, NULL); return; }
    int tiles = N / 32;
    int workers = min_i(matmul_workers((long)N * K * m, nthreads), tiles);
#pragma omp parallel num_threads(workers)
    {
        int s, e;
        worker_range(tiles, workers, omp_get_thread_num(), &s, &e);
        per_block_tiles(act, sa, m, wp, wsc, cs, N, K, block, out, s, e);
    }
}

/* dispatch_bq_norm_quant (linear.mojo:58-82): tokens over workers, inline
 * up to NORM_INLINE_TOKENS = 16 tokens */
void bqcpu_norm_quant(const uint16_t* src, const uint16_t* gamma, int8_t* x_i8,
                      float* sa, int m, int hidden, int block, float sqrt_n,
                      float n_eps, int nthreads) {
    long bytes = (long)m * hidden * 6;
    int workers = bytes <= 16L * hidden * 6 ? 1 : min_i(default_workers(bytes, nthreads), m);
#pragma omp parallel for num_threads(workers) schedule(static)
    for (int t = 0; t < m; ++t)
        bqo_prepare_norm_activation(src + (size_t)t * hidden, gamma, x_i8 + (size_t)t * hidden,
                                    sa + t, hidden, block, sqrt_n, n_eps, 0);
}

/* dispatch_bq_block_quant (linear.mojo:182-205) */
void bqcpu_block_quant(const uint16_t* src, int8_t* x_i8, float* sa, int rows,
                       int cols, int block, int apply_fwht, int nthreads) {
    int nb = cols / block;
    long bytes = (long)rows * cols * 6;
    int workers = bytes <= 16L * cols * 6 ? 1 : min_i(default_workers(bytes, nthreads), rows);
#pragma omp parallel for num_threads(workers) schedule(static)
    for (int t = 0; t < rows; ++t)
        bqo_prepare_block_activation(src + (size_t)t * cols, x_i8 + (size_t)t * cols,
                                     sa + (size_t)t * nb, cols, block, apply_fwht);
}

static inline float gelu(float x) { return bqo_gelu_tanh_f32(x); }

/* moe.mojo:77-129: workers own intermediate tiles; loop experts, 4-route panels */
VNNI_FN static void phase1_tiles(const int8_t* x_i8, const float* x_sa, int hidden,
                                 const int32_t* eo, const bqo_route* routes, int E,
                                 const int8_t* wgu, const float* gsc, const float* gcs,
                                 int inter, uint16_t* bucket, int it0, int it1) {
    const float inv127 = 1.0f / 127.0f;
    int gate_up = 2 * inter, ntiles = inter / 32;
    for (int e = 0; e < E; ++e) {
        int lo = eo[e], hi = eo[e + 1];
        if (hi <= lo) continue;
        const int8_t* w = wgu + (size_t)e * gate_up * hidden;
        const float* wsc = gsc + (size_t)e * gate_up;
        const float* cs = gcs + (size_t)e * gate_up;
        for (int it = it0; it < it1; ++it) {
            for (int rb = lo; rb < hi; rb += 4) {
                int pr = hi - rb < 4 ? hi - rb : 4;
                const int8_t* rows[4];
                float sc[4];
                for (int r = 0; r < pr; ++r) {
                    int tok = routes[rb + r].token;
                    rows[r] = x_i8 + (size_t)tok * hidden;
                    sc[r] = x_sa[tok];
                }
                __m512i g[4][2], u[4][2];
                for (int r = 0; r < 4; ++r) {
                    g[r][0] = g[r][1] = u[r][0] = u[r][1] = _mm512_setzero_si512();
                }
                acc_tile(rows, pr, w, (size_t)it * 32 * hidden, 0, hidden, g);
                acc_tile(rows, pr, w, (size_t)(ntiles + it) * 32 * hidden, 0, hidden, u);
                for (int r = 0; r < pr; ++r) {
                    float ad = sc[r] * inv127;
                    for (int a = 0; a < 2; ++a) {
                        int32_t gi[16], ui[16];
                        _mm512_storeu_si512(gi, g[r][a]);
                        _mm512_storeu_si512(ui, u[r][a]);
                        for (int j = 0; j < 16; ++j) {
                            int ng = it * 32 + a * 16 + j, nu = inter + ng;
                            float gv = ((float)gi[j] - 128.0f * cs[ng]) * ad * wsc[ng];
                            float uv = ((float)ui[j] - 128.0f * cs[nu]) * ad * wsc[nu];
                            bucket[(size_t)(rb + r) * inter + it * 32 + a * 16 + j] = f2bf(gelu(gv) * uv);
                        }
                    }
                }
            }
        }
    }
}

void bqcpu_moe_phase1(const int8_t* x_i8, const float* x_sa, int hidden,
                      const int32_t* eo, const bqo_route* routes, int E,
                      const int8_t* wgu, const float* gsc, const float* gcs,
                      int inter, uint16_t* bucket, int nthreads) {
    if (!have_vnni()) { bqo_moe_phase1(x_i8, x_sa, hidden, eo, routes, E, wgu, gsc, gcs, inter, bucket); return; }
    int tiles = inter / 32;
    int workers = nthreads < tiles ? nthreads : tiles;
#pragma omp parallel num_threads(workers)
    {
        int s, e;
        worker_range(tiles, workers, omp_get_thread_num(), &s, &e);
        phase1_tiles(x_i8, x_sa, hidden, eo, routes, E, wgu, gsc, gcs, inter, bucket, s, e);
    }
}

/* moe.mojo:167-295: workers own hidden tiles of accum/out */
VNNI_FN static void phase2_tiles(const int8_t* bi8, const float* bsa, int inter, int block,
                                 const int32_t* eo, const bqo_route* routes, int E, int T,
                                 const int8_t* wd, const float* dsc, const float* dcs,
                                 int hidden, float* accum, uint16_t* out, int t0, int t1) {
    const float inv127 = 1.0f / 127.0f;
    int nb = inter / block;
    size_t data_n = (size_t)E * hidden;
    for (int tok = 0; tok < T; ++tok)
        memset(accum + (size_t)tok * hidden + t0 * 32, 0, sizeof(float) * (size_t)(t1 - t0) * 32);
    for (int e = 0; e < E; ++e) {
        int lo = eo[e], hi = eo[e + 1];
        if (hi <= lo) continue;
        const int8_t* w = wd + (size_t)e * hidden * inter;
        const float* wsc = dsc + (size_t)e * hidden;
        size_t erb = (size_t)e * hidden;
        for (int rb = lo; rb < hi; rb += 4) {
            int pr = hi - rb < 4 ? hi - rb : 4;
            const int8_t* rows[4];
            for (int r = 0; r < pr; ++r) rows[r] = bi8 + (size_t)(rb + r) * inter;
            for (int t = t0; t < t1; ++t) {
                __m512 facc[4][2];
                for (int r = 0; r < 4; ++r) facc[r][0] = facc[r][1] = _mm512_setzero_ps();
                for (int b = 0; b < nb; ++b) {
                    __m512i acc[4][2];
                    for (int r = 0; r < 4; ++r) acc[r][0] = acc[r][1] = _mm512_setzero_si512();
                    acc_tile(rows, pr, w, (size_t)t * 32 * inter + (size_t)b * block * 32, b * block, block, acc);
                    for (int r = 0; r < pr; ++r) {
                        __m512 adv = _mm512_set1_ps(bsa[(size_t)(rb + r) * nb + b] * inv127);
                        for (int a = 0; a < 2; ++a) {
                            int n0 = t * 32 + a * 16;
                            __m512 ccs = _mm512_loadu_ps(dcs + (size_t)b * data_n + erb + n0);
                            __m512 corr = _mm512_sub_ps(_mm512_cvtepi32_ps(acc[r][a]),
                                                        _mm512_mul_ps(_mm512_set1_ps(128.0f), ccs));
                            facc[r][a] = _mm512_fmadd_ps(corr, adv, facc[r][a]);
                        }
                    }
                }
                for (int r = 0; r < pr; ++r) {
                    float* dst = accum + (size_t)routes[rb + r].token * hidden;
                    __m512 rw = _mm512_set1_ps(routes[rb + r].weight);
                    for (int a = 0; a < 2; ++a) {
                        int n0 = t * 32 + a * 16;
                        __m512 res = _mm512_mul_ps(_mm512_mul_ps(facc[r][a], _mm512_loadu_ps(wsc + n0)), rw);
                        _mm512_storeu_ps(dst + n0, _mm512_add_ps(_mm512_loadu_ps(dst + n0), res));
                    }
                }
            }
        }
    }
    for (int tok = 0; tok < T; ++tok)
        for (int c = t0 * 32; c < t1 * 32; ++c)
            out[(size_t)tok * hidden + c] = f2bf(accum[(size_t)tok * hidden + c]);
}

void bqcpu_moe_phase2(const int8_t* bi8, const float* bsa, int inter, int block,
                      const int32_t* eo, const bqo_route* routes, int E, int T,
                      const int8_t* wd, const float* dsc, const float* dcs, int hidden,
                      float* accum, uint16_t* out, int nthreads) {
    if (T <= 0) return;
    if (!have_vnni()) {
        bqo_moe_phase2(bi8, bsa, inter, block, eo, routes, E, T, wd, dsc, dcs, hidden, accum, out);
        return;
    }
    int tiles = hidden / 32;
    int workers = nthreads < tiles ? nthreads : tiles;
#pragma omp parallel num_threads(workers)
    {
        int s, e;
        worker_range(tiles, workers, omp_get_thread_num(), &s, &e);
        phase2_tiles(bi8, bsa, inter, block, eo, routes, E, T, wd, dsc, dcs, hidden, accum, out, s, e);
    }
}

/* The router merge's top-k + softmax (kernels/moe_router.mojo:248-293) from
 * logits, tokens over merge_workers. */
void bqcpu_route_topk(const float* logits, int T, int E, int top_k, const uint16_t* pes,
                      int32_t* route_idx, float* route_w, int nthreads) {
    int workers = min_i(merge_workers((long)T * E * 4, nthreads), T);
#pragma omp parallel num_threads(workers)
    {
        int s, e;
        worker_range(T, workers, omp_get_thread_num(), &s, &e);
        if (e > s)
            bqo_route_topk_softmax(logits + (size_t)s * E, e - s, E, top_k, pes,
                                   route_idx + (size_t)s * top_k, route_w + (size_t)s * top_k);
    }
}

/* One MoE expert layer from router logits, in the model's order
 * (modeling/gemma_4_moe_bq.mojo:666-704): route top-k + softmax, expert
 * schedule (one worker, kernels/moe_router.mojo:108-145), norm-quant,
 * phase 1, FWHT64 block-quant of the bucket, phase 2.  Caller-owned
 * buffers: route_idx/route_w [T*top_k], eo [E+1], routes [T*top_k], xq
 * [T,hidden], xsa [T], bucket [T*top_k, inter], bi8 [T*top_k, inter], bsa
 * [T*top_k, inter/64], accum/out [T, hidden]. */
void bqcpu_moe_layer(const float* logits, const uint16_t* pes, const uint16_t* x,
                     const uint16_t* gamma, int T, int E, int top_k, int hidden, int inter,
                     float sqrt_n, float n_eps, const int8_t* wgu, const float* gsc,
                     const float* gcs, const int8_t* wd, const float* dsc, const float* dcs,
                     int32_t* route_idx, float* route_w, int32_t* eo, bqo_route* routes,
                     int8_t* xq, float* xsa, uint16_t* bucket, int8_t* bi8, float* bsa,
                     float* accum, uint16_t* out, int nthreads) {
    if (T <= 0) return;
    bqcpu_route_topk(logits, T, E, top_k, pes, route_idx, route_w, nthreads);
    bqo_build_schedule(route_idx, route_w, T, top_k, E, eo, routes);
    bqcpu_norm_quant(x, gamma, xq, xsa, T, hidden, 128, sqrt_n, n_eps, nthreads);
    bqcpu_moe_phase1(xq, xsa, hidden, eo, routes, E, wgu, gsc, gcs, inter, bucket, nthreads);
    bqcpu_block_quant(bucket, bi8, bsa, eo[E], inter, 64, 1, nthreads);
    bqcpu_moe_phase2(bi8, bsa, inter, 64, eo, routes, E, T, wd, dsc, dcs, hidden, accum, out,
                     nthreads);
}
