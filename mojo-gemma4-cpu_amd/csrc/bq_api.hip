// bq_api.hip -- the extern "C" boundary (include/bq_api.h): argument and
// shape validation (the reference's compile-time asserts / debug_asserts
// become status codes), then kernel launches on the caller's stream.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <atomic>
#include <mutex>

#include "../../include/bq_api.h"
#include "bq_kernels.hpp"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(BQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return BQ_OK;
}

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }
inline bool fwht_block_ok(int b) {
  return b == 16 || b == 32 || b == 64 || b == 128 || b == 256 || b == 512;
}
constexpr int kMaxRowLds = 16128;  // f32 row kept in 64 KiB of LDS

// int8 operands are moved 16 bytes per lane
inline bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

namespace bq {
// the shared last-error slot, for entry points defined in other files
int api_failv(int code, const char* fmt, va_list ap) {
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  return code;
}

namespace {
// The tuning settings in force: each tune_init publishes a new immutable
// Tune through this pointer (release / acquire), so a launch on another
// thread reads either the old settings or the new ones, never a torn copy.
// Replaced settings are never freed (a launch may still be reading them);
// each is a few dozen bytes, once per bq_init.
std::atomic<const Tune*> g_tune{nullptr};
std::mutex g_tune_mu;

// The allocation-free phase 2 (bq_moe_phase2_down_noalloc) keeps its
// workspace -- the per-route f32 rows of the down projection -- in this
// file-scope device array: every GPU the library runs on holds one copy, at
// its own address, until the process ends.  Host code uses only the address
// hipGetSymbolAddress returns for the current device (kept per device in
// g_scratch), never the array's name.
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];
void* g_scratch[kMaxDevices] = {};
std::mutex g_scratch_mu;

// the scratch address on `device` (the current device), looked up once
hipError_t scratch_ptr(int device, void** out) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch[device] = p;
  }
  *out = g_scratch[device];
  return hipSuccess;
}

int env_int(const char* name) {
  const char* s = getenv(name);
  return s ? atoi(s) : 0;
}
}  // namespace

hipError_t scratch_address(int device, void** out) { return scratch_ptr(device, out); }

void tune_init(int device) {
  std::lock_guard<std::mutex> lock(g_tune_mu);
  Tune t{};
  t.gemv_waves = env_int("BQ_GEMV_WAVES");
  t.gemv_m1_waves = env_int("BQ_GEMV_M1_WAVES");
  t.skinny2 = getenv("BQ_SKINNY2") ? env_int("BQ_SKINNY2") : 1;
  t.tile_bm = env_int("BQ_TILE_BM");
  t.tile_bn = env_int("BQ_TILE_BN");
  t.ring = env_int("BQ_RING");
  t.tile_ksp = env_int("BQ_TILE_KSP");
  t.moe_bm = env_int("BQ_MOE_BM");
  t.moe_bm_down = env_int("BQ_MOE_BM_DOWN");
  // n-tile fastest over the whole grid: the 2048-token layer 310.9 -> 308.0
  // us against an m-tile's n-tiles on one XCD (order 2, faster when the
  // gate/up and down kernels took 142 / 128 us)
  t.moe_order = getenv("BQ_MOE_ORDER") ? env_int("BQ_MOE_ORDER") : 0;
  t.down_breg = getenv("BQ_DOWN_BREG") ? env_int("BQ_DOWN_BREG") : 1;
  t.nq_pair = getenv("BQ_NQ_PAIR") ? env_int("BQ_NQ_PAIR") : 1;
  t.moe_prep = getenv("BQ_MOE_PREP") ? env_int("BQ_MOE_PREP") : 1;
  t.nq_v8 = getenv("BQ_NQ_V8") ? env_int("BQ_NQ_V8") : 1;
  t.down_skinny = getenv("BQ_DOWN_SKINNY") ? env_int("BQ_DOWN_SKINNY") : 32;
  t.gu_skinny = getenv("BQ_GU_SKINNY") ? env_int("BQ_GU_SKINNY") : 4;
  t.head_grid = env_int("BQ_HEAD_GRID");
  t.attn_waves = env_int("BQ_ATTN_WAVES");
  t.sel_fused = getenv("BQ_SEL_FUSED") ? env_int("BQ_SEL_FUSED") : 1;
  t.prep_one = getenv("BQ_PREP_ONE") ? env_int("BQ_PREP_ONE") : 1;
  // 16x16x64 by default: these LDS-ring kernels wait on their operand
  // stream, not on the MFMA rate (gate/up at 2048 tokens: 142 us with
  // 16x16x64 on 8-wave workgroups, 158 us with 32x32x32 on 4-wave ones)
  t.mf = env_int("BQ_MF") == 32 ? 32 : 16;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      cus <= 0)
    cus = 256;
  t.cus = cus;
  g_tune.store(new Tune(t), std::memory_order_release);
}

const Tune& tune() {
  const Tune* t = g_tune.load(std::memory_order_acquire);
  if (!t) {  // a process that never called bq_init: read the switches once
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    {
      std::lock_guard<std::mutex> lock(g_tune_mu);
      t = g_tune.load(std::memory_order_acquire);
    }
    if (!t) tune_init(dev);
    t = g_tune.load(std::memory_order_acquire);
  }
  return *t;
}
}  // namespace bq

extern "C" {

const char* bq_version(void) { return "bq-mi355x 0.1 (gfx950)"; }

const char* bq_last_error(void) { return g_err; }

int bq_init(int device) {
  int r = check_hip(hipSetDevice(device), "hipSetDevice");
  if (r) return r;
  r = check_hip(hipFree(nullptr), "hip runtime init");
  if (r) return r;
  bq::tune_init(device);
  void* sp = nullptr;
  return check_hip(bq::scratch_address(device, &sp), "scratch symbol address");
}

int bq_stream_synchronize(void* stream) {
  return check_hip(hipStreamSynchronize(S(stream)), "hipStreamSynchronize");
}

int bq_weight_retile(const int8_t* src, int src_layout, int8_t* dst, int n_rows, int k,
                     void* stream) {
  if (!src || !dst) return fail(BQ_ERR_INVALID, "bq_weight_retile: null pointer");
  if (src_layout != BQ_LAYOUT_ROWMAJOR && src_layout != BQ_LAYOUT_VNNI)
    return fail(BQ_ERR_INVALID, "bq_weight_retile: unknown layout %d", src_layout);
  if (n_rows < 0 || k < 0 || n_rows % 16 || k % 64)
    return fail(BQ_ERR_SHAPE, "bq_weight_retile: need n_rows %% 16 == 0 and k %% 64 == 0 (got %d x %d)",
                n_rows, k);
  if (!a16(src) || !a16(dst)) return fail(BQ_ERR_INVALID, "bq_weight_retile: pointers must be 16-byte aligned");
  if (src_layout == BQ_LAYOUT_VNNI && n_rows % 32)
    return fail(BQ_ERR_SHAPE, "bq_weight_retile: VNNI source needs n_rows %% 32 == 0 (got %d)", n_rows);
  return check_hip(bq::launch_retile(src, src_layout, dst, n_rows, k, S(stream)), "retile");
}

int bq_weight_unpack(const int8_t* tiled, int8_t* dst, int n_rows, int k, void* stream) {
  if (!tiled || !dst) return fail(BQ_ERR_INVALID, "bq_weight_unpack: null pointer");
  if (n_rows < 0 || k < 0 || n_rows % 16 || k % 64)
    return fail(BQ_ERR_SHAPE, "bq_weight_unpack: need n_rows %% 16 == 0 and k %% 64 == 0");
  if (!a16(tiled) || !a16(dst)) return fail(BQ_ERR_INVALID, "bq_weight_unpack: pointers must be 16-byte aligned");
  return check_hip(bq::launch_unpack(tiled, dst, n_rows, k, S(stream)), "unpack");
}

int bq_pack_colsum_vnni(const int8_t* src, int8_t* dst, float* colsum, int rows, int cols,
                        int block_cols, int colsum_row_major, void* stream) {
  if (!src || !dst) return fail(BQ_ERR_INVALID, "bq_pack_colsum_vnni: null pointer");
  if (src == dst) return fail(BQ_ERR_INVALID, "bq_pack_colsum_vnni: src and dst must differ on the GPU");
  // butterquant/vnni.mojo:91-99
  if (rows < 0 || cols <= 0 || cols % 64 || rows % 32 || block_cols <= 0 || cols % block_cols ||
      block_cols % 16)
    return fail(BQ_ERR_SHAPE,
                "bq_pack_colsum_vnni: need cols %% 64 == 0, rows %% 32 == 0, block_cols | cols, "
                "block_cols %% 16 == 0 (got %d x %d, block %d)", rows, cols, block_cols);
  if (!a16(src) || (reinterpret_cast<uintptr_t>(dst) & 3u))
    return fail(BQ_ERR_INVALID, "bq_pack_colsum_vnni: src must be 16-byte and dst 4-byte aligned");
  return check_hip(bq::launch_pack_colsum(src, dst, colsum, rows, cols, block_cols,
                                          colsum_row_major, S(stream)), "pack_colsum");
}

int bq_quantize_weight(const uint16_t* w, const float* gamma, int8_t* codes, float* scales,
                       int rows, int cols, int fwht_block, int per_block, void* stream) {
  if (!w || !codes || !scales) return fail(BQ_ERR_INVALID, "bq_quantize_weight: null pointer");
  if (!fwht_block_ok(fwht_block))  // kernels.mojo:167-168 aborts
    return fail(BQ_ERR_SHAPE, "bq_quantize_weight: unsupported FWHT block %d", fwht_block);
  if (rows < 0 || cols <= 0 || cols % 64 || cols % fwht_block)
    return fail(BQ_ERR_SHAPE, "bq_quantize_weight: cols %d not a multiple of 64 and the FWHT block", cols);
  if (cols > kMaxRowLds) return fail(BQ_ERR_UNSUPPORTED, "bq_quantize_weight: cols %d > %d", cols, kMaxRowLds);
  return check_hip(bq::launch_quantize_weight(w, gamma, codes, scales, rows, cols, fwht_block,
                                              per_block, S(stream)), "quantize_weight");
}

int bq_norm_quant(const uint16_t* src, const uint16_t* gamma, int8_t* x_i8, float* x_sa,
                  int seq_len, int hidden, int block, float sqrt_n, float n_eps, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!src || !gamma || !x_i8 || !x_sa) return fail(BQ_ERR_INVALID, "bq_norm_quant: null pointer");
  if (!fwht_block_ok(block)) return fail(BQ_ERR_SHAPE, "bq_norm_quant: unsupported FWHT block %d", block);
  // runtime.mojo:18-21
  if (hidden <= 0 || hidden % 64 || hidden % block)
    return fail(BQ_ERR_SHAPE, "bq_norm_quant: hidden %d must be a multiple of 64 and of block %d", hidden, block);
  if (hidden > kMaxRowLds) return fail(BQ_ERR_UNSUPPORTED, "bq_norm_quant: hidden %d > %d", hidden, kMaxRowLds);
  if (!a16(src)) return fail(BQ_ERR_INVALID, "bq_norm_quant: src must be 16-byte aligned");
  return check_hip(bq::launch_norm_quant(src, gamma, x_i8, x_sa, seq_len, hidden, block, sqrt_n,
                                         n_eps, S(stream)), "norm_quant");
}

int bq_block_quant(const uint16_t* src, int8_t* x_i8, float* x_sa, int cols, int seq_len,
                   int block, int apply_fwht, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!src || !x_i8 || !x_sa) return fail(BQ_ERR_INVALID, "bq_block_quant: null pointer");
  if (apply_fwht ? !fwht_block_ok(block) : !(pow2(block) && block >= 16 && block <= 512))
    return fail(BQ_ERR_SHAPE, "bq_block_quant: unsupported block %d", block);
  if (cols <= 0 || cols % 64 || cols % block)  // runtime.mojo:68-70
    return fail(BQ_ERR_SHAPE, "bq_block_quant: cols %d must be a multiple of 64 and of block %d", cols, block);
  if (!a16(src) || !a16(x_i8))
    return fail(BQ_ERR_INVALID, "bq_block_quant: src and x_i8 must be 16-byte aligned");
  return check_hip(bq::launch_block_quant(src, x_i8, x_sa, seq_len, cols, block, apply_fwht,
                                          S(stream)), "block_quant");
}

int bq_linear(const int8_t* x_i8, const float* x_sa, const int8_t* w, const float* w_scale,
              uint16_t* out, float* out_f32, int n_rows, int seq_len, int hidden, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!x_i8 || !x_sa || !w || !w_scale || !out) return fail(BQ_ERR_INVALID, "bq_linear: null pointer");
  if (n_rows <= 0 || n_rows % 16 || hidden <= 0 || hidden % 64)
    return fail(BQ_ERR_SHAPE, "bq_linear: need n_rows %% 16 == 0 and hidden %% 64 == 0 (got %d, %d)",
                n_rows, hidden);
  bq::LinArgs a{};
  if (!a16(x_i8) || !a16(w)) return fail(BQ_ERR_INVALID, "bq_linear: int8 operands must be 16-byte aligned");
  a.seg[0] = {w, w_scale, out, out_f32, n_rows, 0};
  a.nseg = 1;
  a.act = x_i8; a.sa = x_sa; a.M = seq_len; a.K = hidden; a.block = hidden;
  return check_hip(bq::launch_linear(a, 0, S(stream)), "linear");
}

int bq_block_linear(const int8_t* x_i8, const float* x_sa, const int8_t* w, const float* w_scale,
                    uint16_t* out, float* out_f32, int n_rows, int k_dim, int seq_len, int block,
                    void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!x_i8 || !x_sa || !w || !w_scale || !out) return fail(BQ_ERR_INVALID, "bq_block_linear: null pointer");
  if (!pow2(block) || block < 64)  // amx_gemm.mojo:222 (block % 64 == 0)
    return fail(BQ_ERR_SHAPE, "bq_block_linear: block %d must be a power of two >= 64", block);
  if (n_rows <= 0 || n_rows % 16 || k_dim <= 0 || k_dim % block)
    return fail(BQ_ERR_SHAPE, "bq_block_linear: need n_rows %% 16 == 0 and k_dim %% block == 0 (got %d, %d, %d)",
                n_rows, k_dim, block);
  if (k_dim / block > 64)
    return fail(BQ_ERR_UNSUPPORTED, "bq_block_linear: k_dim/block = %d > 64", k_dim / block);
  bq::LinArgs a{};
  if (!a16(x_i8) || !a16(w)) return fail(BQ_ERR_INVALID, "bq_block_linear: int8 operands must be 16-byte aligned");
  a.seg[0] = {w, w_scale, out, out_f32, n_rows, 0};
  a.nseg = 1;
  a.act = x_i8; a.sa = x_sa; a.M = seq_len; a.K = k_dim; a.block = block;
  return check_hip(bq::launch_linear(a, 1, S(stream)), "block_linear");
}

int bq_qkv(const int8_t* x_i8, const float* x_sa, const int8_t* q_w, const float* q_scale,
           const int8_t* k_w, const float* k_scale, const int8_t* v_w, const float* v_scale,
           uint16_t* q_out, uint16_t* k_out, uint16_t* v_out, int qn, int kvn, int seq_len,
           int hidden, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!x_i8 || !x_sa || !q_w || !q_scale || !k_w || !k_scale || !v_w || !v_scale || !q_out ||
      !k_out || !v_out)
    return fail(BQ_ERR_INVALID, "bq_qkv: null pointer");
  if (qn <= 0 || kvn <= 0 || qn % 16 || kvn % 16 || hidden <= 0 || hidden % 64)
    return fail(BQ_ERR_SHAPE, "bq_qkv: need qn, kvn %% 16 == 0 and hidden %% 64 == 0");
  if (!a16(x_i8) || !a16(q_w) || !a16(k_w) || !a16(v_w))
    return fail(BQ_ERR_INVALID, "bq_qkv: int8 operands must be 16-byte aligned");
  bq::LinArgs a{};
  a.seg[0] = {q_w, q_scale, q_out, nullptr, qn, 0};
  a.seg[1] = {k_w, k_scale, k_out, nullptr, kvn, qn / 16};
  a.seg[2] = {v_w, v_scale, v_out, nullptr, kvn, qn / 16 + kvn / 16};
  a.nseg = 3;
  a.act = x_i8; a.sa = x_sa; a.M = seq_len; a.K = hidden; a.block = hidden;
  return check_hip(bq::launch_linear(a, 0, S(stream)), "qkv");
}

int bq_linear_pair(const int8_t* x_i8, const float* x_sa, const int8_t* w0, const float* w0_scale,
                   const int8_t* w1, const float* w1_scale, uint16_t* out0, uint16_t* out1,
                   int n0, int n1, int seq_len, int hidden, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!x_i8 || !x_sa || !w0 || !w0_scale || !w1 || !w1_scale || !out0 || !out1)
    return fail(BQ_ERR_INVALID, "bq_linear_pair: null pointer");
  if (n0 <= 0 || n1 <= 0 || n0 % 16 || n1 % 16 || hidden <= 0 || hidden % 64)
    return fail(BQ_ERR_SHAPE, "bq_linear_pair: need n0, n1 %% 16 == 0 and hidden %% 64 == 0");
  if (!a16(x_i8) || !a16(w0) || !a16(w1))
    return fail(BQ_ERR_INVALID, "bq_linear_pair: int8 operands must be 16-byte aligned");
  bq::LinArgs a{};
  a.seg[0] = {w0, w0_scale, out0, nullptr, n0, 0};
  a.seg[1] = {w1, w1_scale, out1, nullptr, n1, n0 / 16};
  a.nseg = 2;
  a.act = x_i8; a.sa = x_sa; a.M = seq_len; a.K = hidden; a.block = hidden;
  return check_hip(bq::launch_linear(a, 0, S(stream)), "linear_pair");
}

// shared checks of the fused norm-quant + linear entries (those of
// bq_norm_quant and of the linear on its output)
static int norm_linear_args(const char* who, const uint16_t* src, const uint16_t* gamma,
                            int8_t* x_i8, float* x_sa, int hidden, int block, float sqrt_n,
                            float n_eps, bq::NormArgs& nq) {
  if (!src || !gamma || !x_i8 || !x_sa) return fail(BQ_ERR_INVALID, "%s: null pointer", who);
  if (!fwht_block_ok(block)) return fail(BQ_ERR_SHAPE, "%s: unsupported FWHT block %d", who, block);
  if (hidden <= 0 || hidden % 64 || hidden % block)
    return fail(BQ_ERR_SHAPE, "%s: hidden %d must be a multiple of 64 and of block %d", who, hidden, block);
  if (hidden > kMaxRowLds) return fail(BQ_ERR_UNSUPPORTED, "%s: hidden %d > %d", who, hidden, kMaxRowLds);
  if (!a16(src) || !a16(x_i8)) return fail(BQ_ERR_INVALID, "%s: src and x_i8 must be 16-byte aligned", who);
  nq = bq::NormArgs{src, gamma, x_i8, x_sa, block, sqrt_n, n_eps, 0.0f};
  return BQ_OK;
}

int bq_norm_linear(const uint16_t* src, const uint16_t* gamma, int8_t* x_i8, float* x_sa,
                   const int8_t* w, const float* w_scale, uint16_t* out, float* out_f32,
                   int n_rows, int seq_len, int hidden, int block, float sqrt_n, float n_eps,
                   void* stream) {
  if (seq_len <= 0) return BQ_OK;
  bq::NormArgs nq{};
  const int r = norm_linear_args("bq_norm_linear", src, gamma, x_i8, x_sa, hidden, block, sqrt_n,
                                 n_eps, nq);
  if (r != BQ_OK) return r;
  if (!w || !w_scale || !out) return fail(BQ_ERR_INVALID, "bq_norm_linear: null pointer");
  if (n_rows <= 0 || n_rows % 16)
    return fail(BQ_ERR_SHAPE, "bq_norm_linear: need n_rows %% 16 == 0 (got %d)", n_rows);
  if (!a16(w)) return fail(BQ_ERR_INVALID, "bq_norm_linear: int8 operands must be 16-byte aligned");
  bq::LinArgs a{};
  a.seg[0] = {w, w_scale, out, out_f32, n_rows, 0};
  a.nseg = 1;
  a.act = x_i8; a.sa = x_sa; a.M = seq_len; a.K = hidden; a.block = hidden;
  return check_hip(bq::launch_norm_linear(a, nq, S(stream)), "norm_linear");
}

int bq_norm_qkv(const uint16_t* src, const uint16_t* gamma, int8_t* x_i8, float* x_sa,
                const int8_t* q_w, const float* q_scale, const int8_t* k_w, const float* k_scale,
                const int8_t* v_w, const float* v_scale, uint16_t* q_out, uint16_t* k_out,
                uint16_t* v_out, int qn, int kvn, int seq_len, int hidden, int block,
                float sqrt_n, float n_eps, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  bq::NormArgs nq{};
  const int r = norm_linear_args("bq_norm_qkv", src, gamma, x_i8, x_sa, hidden, block, sqrt_n,
                                 n_eps, nq);
  if (r != BQ_OK) return r;
  if (!q_w || !q_scale || !k_w || !k_scale || !v_w || !v_scale || !q_out || !k_out || !v_out)
    return fail(BQ_ERR_INVALID, "bq_norm_qkv: null pointer");
  if (qn <= 0 || kvn <= 0 || qn % 16 || kvn % 16)
    return fail(BQ_ERR_SHAPE, "bq_norm_qkv: need qn, kvn %% 16 == 0");
  if (!a16(q_w) || !a16(k_w) || !a16(v_w))
    return fail(BQ_ERR_INVALID, "bq_norm_qkv: int8 operands must be 16-byte aligned");
  bq::LinArgs a{};
  a.seg[0] = {q_w, q_scale, q_out, nullptr, qn, 0};
  a.seg[1] = {k_w, k_scale, k_out, nullptr, kvn, qn / 16};
  a.seg[2] = {v_w, v_scale, v_out, nullptr, kvn, qn / 16 + kvn / 16};
  a.nseg = 3;
  a.act = x_i8; a.sa = x_sa; a.M = seq_len; a.K = hidden; a.block = hidden;
  return check_hip(bq::launch_norm_linear(a, nq, S(stream)), "norm_qkv");
}

int bq_norm_linear_pair(const uint16_t* src, const uint16_t* gamma, int8_t* x_i8, float* x_sa,
                        const int8_t* w0, const float* w0_scale, const int8_t* w1,
                        const float* w1_scale, uint16_t* out0, uint16_t* out1, int n0, int n1,
                        int seq_len, int hidden, int block, float sqrt_n, float n_eps,
                        void* stream) {
  if (seq_len <= 0) return BQ_OK;
  bq::NormArgs nq{};
  const int r = norm_linear_args("bq_norm_linear_pair", src, gamma, x_i8, x_sa, hidden, block,
                                 sqrt_n, n_eps, nq);
  if (r != BQ_OK) return r;
  if (!w0 || !w0_scale || !w1 || !w1_scale || !out0 || !out1)
    return fail(BQ_ERR_INVALID, "bq_norm_linear_pair: null pointer");
  if (n0 <= 0 || n1 <= 0 || n0 % 16 || n1 % 16)
    return fail(BQ_ERR_SHAPE, "bq_norm_linear_pair: need n0, n1 %% 16 == 0");
  if (!a16(w0) || !a16(w1))
    return fail(BQ_ERR_INVALID, "bq_norm_linear_pair: int8 operands must be 16-byte aligned");
  bq::LinArgs a{};
  a.seg[0] = {w0, w0_scale, out0, nullptr, n0, 0};
  a.seg[1] = {w1, w1_scale, out1, nullptr, n1, n0 / 16};
  a.nseg = 2;
  a.act = x_i8; a.sa = x_sa; a.M = seq_len; a.K = hidden; a.block = hidden;
  return check_hip(bq::launch_norm_linear(a, nq, S(stream)), "norm_linear_pair");
}

int bq_moe_router_logits(const uint16_t* x, const uint16_t* router_proj,
                         const uint16_t* router_scale, float* logits, int seq_len, int hidden,
                         int experts, float sqrt_n, float n_eps, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!x || !router_proj || !router_scale || !logits)
    return fail(BQ_ERR_INVALID, "bq_moe_router_logits: null pointer");
  if (hidden <= 0 || hidden % 64 || experts <= 0)
    return fail(BQ_ERR_SHAPE, "bq_moe_router_logits: need hidden %% 64 == 0 and experts > 0");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(router_proj) |
       reinterpret_cast<uintptr_t>(router_scale)) & 3u)
    return fail(BQ_ERR_INVALID, "bq_moe_router_logits: bf16 operands must be 4-byte aligned");
  return check_hip(bq::launch_router_logits(x, router_proj, router_scale, logits, seq_len, hidden,
                                            experts, sqrt_n, n_eps, S(stream)),
                   "router_logits");
}

int bq_moe_route_topk(const float* logits, const uint16_t* per_expert_scale, int seq_len,
                      int experts, int top_k, int32_t* route_idx, float* route_w, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!logits || !route_idx || !route_w) return fail(BQ_ERR_INVALID, "bq_moe_route_topk: null pointer");
  if (experts <= 0 || top_k <= 0) return fail(BQ_ERR_SHAPE, "bq_moe_route_topk: bad top_k/experts");
  if (experts > 1024 || top_k > 16)
    return fail(BQ_ERR_UNSUPPORTED, "bq_moe_route_topk: experts %d > 1024 or top_k %d > 16", experts,
                top_k);
  return check_hip(bq::launch_route_topk(logits, per_expert_scale, seq_len, experts, top_k,
                                         route_idx, route_w, S(stream)),
                   "route_topk");
}

int bq_moe_route_schedule(const float* logits, const uint16_t* per_expert_scale, int seq_len,
                          int experts, int top_k, int32_t* route_idx, float* route_w,
                          int32_t* expert_offset, bq_route* routes, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!logits || !route_idx || !route_w || !expert_offset || !routes)
    return fail(BQ_ERR_INVALID, "bq_moe_route_schedule: null pointer");
  if (experts <= 0 || top_k <= 0) return fail(BQ_ERR_SHAPE, "bq_moe_route_schedule: bad top_k/experts");
  if (experts > 256 || top_k > 16)
    return fail(BQ_ERR_UNSUPPORTED, "bq_moe_route_schedule: experts %d > 256 or top_k %d > 16",
                experts, top_k);
  return check_hip(bq::launch_route_schedule(logits, per_expert_scale, seq_len, experts, top_k,
                                             route_idx, route_w, expert_offset,
                                             reinterpret_cast<bq::Route*>(routes), S(stream)),
                   "route_schedule");
}

int bq_moe_prep(const float* logits, const uint16_t* per_expert_scale, const uint16_t* x,
                const uint16_t* gamma, int seq_len, int experts, int top_k, int hidden, int block,
                float sqrt_n, float n_eps, int32_t* route_idx, float* route_w,
                int32_t* expert_offset, bq_route* routes, int8_t* x_i8, float* x_sa,
                void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!logits || !x || !gamma || !route_idx || !route_w || !expert_offset || !routes || !x_i8 ||
      !x_sa)
    return fail(BQ_ERR_INVALID, "bq_moe_prep: null pointer");
  if (experts <= 0 || top_k <= 0) return fail(BQ_ERR_SHAPE, "bq_moe_prep: bad top_k/experts");
  if (experts > 256 || top_k > 16)
    return fail(BQ_ERR_UNSUPPORTED, "bq_moe_prep: experts %d > 256 or top_k %d > 16", experts,
                top_k);
  // the norm-quant's contract (bq_norm_quant)
  if (!fwht_block_ok(block)) return fail(BQ_ERR_SHAPE, "bq_moe_prep: unsupported FWHT block %d", block);
  if (hidden <= 0 || hidden % 64 || hidden % block)
    return fail(BQ_ERR_SHAPE, "bq_moe_prep: hidden %d must be a multiple of 64 and of block %d", hidden, block);
  if (hidden > kMaxRowLds) return fail(BQ_ERR_UNSUPPORTED, "bq_moe_prep: hidden %d > %d", hidden, kMaxRowLds);
  if (!a16(x)) return fail(BQ_ERR_INVALID, "bq_moe_prep: x must be 16-byte aligned");
  return check_hip(bq::launch_moe_prep(logits, per_expert_scale, x, gamma, seq_len, experts,
                                       top_k, hidden, block, sqrt_n, n_eps, route_idx, route_w,
                                       expert_offset, reinterpret_cast<bq::Route*>(routes), x_i8,
                                       x_sa, S(stream)),
                   "moe_prep");
}

int bq_ffn_prep(const float* logits, const uint16_t* per_expert_scale, const uint16_t* x,
                const uint16_t* gamma, const uint16_t* dense_gamma, int seq_len, int experts,
                int top_k, int hidden, int block, float sqrt_n, float n_eps, int32_t* route_idx,
                float* route_w, int32_t* expert_offset, bq_route* routes, int8_t* x_i8,
                float* x_sa, int8_t* dense_i8, float* dense_sa, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!logits || !x || !gamma || !dense_gamma || !route_idx || !route_w || !expert_offset ||
      !routes || !x_i8 || !x_sa || !dense_i8 || !dense_sa)
    return fail(BQ_ERR_INVALID, "bq_ffn_prep: null pointer");
  if (experts <= 0 || top_k <= 0) return fail(BQ_ERR_SHAPE, "bq_ffn_prep: bad top_k/experts");
  if (experts > 256 || top_k > 16)
    return fail(BQ_ERR_UNSUPPORTED, "bq_ffn_prep: experts %d > 256 or top_k %d > 16", experts,
                top_k);
  if (!fwht_block_ok(block)) return fail(BQ_ERR_SHAPE, "bq_ffn_prep: unsupported FWHT block %d", block);
  if (hidden <= 0 || hidden % 64 || hidden % block)
    return fail(BQ_ERR_SHAPE, "bq_ffn_prep: hidden %d must be a multiple of 64 and of block %d", hidden, block);
  if (hidden > kMaxRowLds) return fail(BQ_ERR_UNSUPPORTED, "bq_ffn_prep: hidden %d > %d", hidden, kMaxRowLds);
  if (!a16(x)) return fail(BQ_ERR_INVALID, "bq_ffn_prep: x must be 16-byte aligned");
  return check_hip(bq::launch_moe_prep(logits, per_expert_scale, x, gamma, seq_len, experts,
                                       top_k, hidden, block, sqrt_n, n_eps, route_idx, route_w,
                                       expert_offset, reinterpret_cast<bq::Route*>(routes), x_i8,
                                       x_sa, S(stream), dense_gamma, dense_i8, dense_sa),
                   "ffn_prep");
}

int bq_moe_build_schedule(const int32_t* route_idx, const float* route_w, int seq_len, int top_k,
                          int expert_base, int experts, int32_t* expert_offset, bq_route* routes,
                          void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!route_idx || !route_w || !expert_offset || !routes)
    return fail(BQ_ERR_INVALID, "bq_moe_build_schedule: null pointer");
  if (top_k <= 0 || experts <= 0) return fail(BQ_ERR_SHAPE, "bq_moe_build_schedule: bad top_k/experts");
  if (experts > 256) return fail(BQ_ERR_UNSUPPORTED, "bq_moe_build_schedule: experts %d > 256", experts);
  return check_hip(bq::launch_build_schedule(route_idx, route_w, seq_len, top_k, expert_base,
                                             experts, expert_offset,
                                             reinterpret_cast<bq::Route*>(routes), S(stream)),
                   "build_schedule");
}

int bq_moe_phase1_gate_up(const int8_t* x_i8, const float* x_sa, const int32_t* expert_offset,
                          const bq_route* routes, const int8_t* w_gate_up,
                          const float* gate_up_scale, uint16_t* bucket, int experts_per_rank,
                          int seq_len, int top_k, int hidden, int inter, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!x_i8 || !x_sa || !expert_offset || !routes || !w_gate_up || !gate_up_scale || !bucket)
    return fail(BQ_ERR_INVALID, "bq_moe_phase1_gate_up: null pointer");
  if (experts_per_rank <= 0 || top_k <= 0 || hidden <= 0 || hidden % 64 || inter <= 0 || inter % 16)
    return fail(BQ_ERR_SHAPE, "bq_moe_phase1_gate_up: need hidden %% 64 == 0, inter %% 16 == 0");
  if (!a16(x_i8) || !a16(w_gate_up))
    return fail(BQ_ERR_INVALID, "bq_moe_phase1_gate_up: int8 operands must be 16-byte aligned");
  return check_hip(bq::launch_moe_phase1(x_i8, x_sa, expert_offset,
                                         reinterpret_cast<const bq::Route*>(routes), w_gate_up,
                                         gate_up_scale, bucket, nullptr, nullptr,
                                         experts_per_rank, seq_len * top_k, hidden, inter,
                                         S(stream)), "moe_phase1");
}

int bq_moe_phase1_gate_up_quant(const int8_t* x_i8, const float* x_sa,
                                const int32_t* expert_offset, const bq_route* routes,
                                const int8_t* w_gate_up, const float* gate_up_scale,
                                uint16_t* bucket, int8_t* bucket_i8, float* bucket_sa,
                                int experts_per_rank, int seq_len, int top_k, int hidden,
                                int inter, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!x_i8 || !x_sa || !expert_offset || !routes || !w_gate_up || !gate_up_scale ||
      !bucket_i8 || !bucket_sa)
    return fail(BQ_ERR_INVALID, "bq_moe_phase1_gate_up_quant: null pointer");
  if (experts_per_rank <= 0 || top_k <= 0 || hidden <= 0 || hidden % 64 || inter <= 0 ||
      inter % 64)
    return fail(BQ_ERR_SHAPE, "bq_moe_phase1_gate_up_quant: need hidden %% 64 == 0 and "
                              "inter %% 64 == 0 (the 64-column block-quant)");
  if (!a16(x_i8) || !a16(w_gate_up) || (reinterpret_cast<uintptr_t>(bucket_i8) & 7u) ||
      (reinterpret_cast<uintptr_t>(bucket_sa) & 3u) || (bucket && !a16(bucket)))
    return fail(BQ_ERR_INVALID, "bq_moe_phase1_gate_up_quant: x_i8, w_gate_up (and bucket) must "
                                "be 16-byte, bucket_i8 8-byte, bucket_sa 4-byte aligned");
  return check_hip(bq::launch_moe_phase1(x_i8, x_sa, expert_offset,
                                         reinterpret_cast<const bq::Route*>(routes), w_gate_up,
                                         gate_up_scale, bucket, bucket_i8, bucket_sa,
                                         experts_per_rank, seq_len * top_k, hidden, inter,
                                         S(stream)),
                   "moe_phase1_quant");
}

size_t bq_moe_phase2_workspace_size(int seq_len, int top_k, int hidden) {
  if (seq_len <= 0 || top_k <= 0 || hidden <= 0) return 0;
  return bq::moe_phase2_workspace(seq_len * top_k, seq_len, hidden);
}

// The checks both phase-2 entry points share (all but the workspace), in one
// order, so the two return the same status for the same arguments.
static int phase2_args(const char* who, const int8_t* bucket_i8, const float* bucket_sa,
                       const int32_t* expert_offset, const bq_route* routes,
                       const int8_t* w_down, const float* down_scale, float* moe_accum,
                       uint16_t* moe_out, int top_k, int hidden, int inter, int block) {
  if (!bucket_i8 || !bucket_sa || !expert_offset || !routes || !w_down || !down_scale ||
      !moe_accum || !moe_out)
    return fail(BQ_ERR_INVALID, "%s: null pointer", who);
  if (top_k <= 0 || top_k > 16) return fail(BQ_ERR_UNSUPPORTED, "%s: top_k %d not in [1,16]", who, top_k);
  if (!pow2(block) || block < 64 || inter % block || inter % 64 || hidden % 16 || hidden <= 0)
    return fail(BQ_ERR_SHAPE, "%s: need block a power of two >= 64 dividing inter, hidden %% 16 == 0", who);
  if (inter / block > 64) return fail(BQ_ERR_UNSUPPORTED, "%s: inter/block = %d > 64", who, inter / block);
  if (!a16(bucket_i8) || !a16(w_down) || !a16(moe_accum) || !a16(moe_out))
    return fail(BQ_ERR_INVALID, "%s: int8 operands, moe_accum and moe_out must be 16-byte aligned", who);
  return BQ_OK;
}

int bq_moe_phase2_down(const int8_t* bucket_i8, const float* bucket_sa,
                       const int32_t* expert_offset, const bq_route* routes, const int8_t* w_down,
                       const float* down_scale, float* moe_accum, uint16_t* moe_out,
                       int experts_per_rank, int seq_len, int top_k, int hidden, int inter,
                       int block, void* workspace, size_t workspace_bytes, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  const int r = phase2_args("bq_moe_phase2_down", bucket_i8, bucket_sa, expert_offset, routes,
                            w_down, down_scale, moe_accum, moe_out, top_k, hidden, inter, block);
  if (r != BQ_OK) return r;
  if (!workspace) return fail(BQ_ERR_INVALID, "bq_moe_phase2_down: null pointer");
  if (reinterpret_cast<uintptr_t>(workspace) % 256)
    return fail(BQ_ERR_INVALID, "bq_moe_phase2_down: workspace must be 256-byte aligned");
  const size_t need = bq::moe_phase2_workspace(seq_len * top_k, seq_len, hidden);
  if (workspace_bytes < need)
    return fail(BQ_ERR_SHAPE, "bq_moe_phase2_down: workspace %zu < %zu bytes", workspace_bytes, need);
  return check_hip(bq::launch_moe_phase2(bucket_i8, bucket_sa, expert_offset,
                                         reinterpret_cast<const bq::Route*>(routes), w_down,
                                         down_scale, moe_accum, moe_out, experts_per_rank, seq_len,
                                         seq_len * top_k, hidden, inter, block, workspace,
                                         S(stream)), "moe_phase2");
}

int bq_ffn_gate_up(const int8_t* x_i8, const float* x_sa, const int32_t* expert_offset,
                   const bq_route* routes, const int8_t* w_gate_up, const float* gate_up_scale,
                   int8_t* bucket_i8, float* bucket_sa, int experts_per_rank, int seq_len,
                   int top_k, int hidden, int inter, const int8_t* dense_x_i8,
                   const float* dense_x_sa, const int8_t* dense_gate,
                   const float* dense_gate_scale, const int8_t* dense_up,
                   const float* dense_up_scale, int dense_inter, int8_t* dense_i8,
                   float* dense_sa, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!x_i8 || !x_sa || !expert_offset || !routes || !w_gate_up || !gate_up_scale ||
      !bucket_i8 || !bucket_sa || !dense_x_i8 || !dense_x_sa || !dense_gate ||
      !dense_gate_scale || !dense_up || !dense_up_scale || !dense_i8 || !dense_sa)
    return fail(BQ_ERR_INVALID, "bq_ffn_gate_up: null pointer");
  if (experts_per_rank <= 0 || top_k <= 0 || hidden <= 0 || hidden % 64 || inter <= 0 ||
      inter % 64 || dense_inter <= 0 || dense_inter % 64)
    return fail(BQ_ERR_SHAPE, "bq_ffn_gate_up: need hidden, inter and dense_inter multiples of 64");
  if (!a16(x_i8) || !a16(w_gate_up) || (reinterpret_cast<uintptr_t>(bucket_i8) & 7u) ||
      (reinterpret_cast<uintptr_t>(bucket_sa) & 3u) || !a16(dense_x_i8) || !a16(dense_gate) ||
      !a16(dense_up) || (reinterpret_cast<uintptr_t>(dense_i8) & 7u) ||
      (reinterpret_cast<uintptr_t>(dense_sa) & 3u))
    return fail(BQ_ERR_INVALID, "bq_ffn_gate_up: x_i8, w_gate_up, dense_x_i8, dense_gate, dense_up "
                                "must be 16-byte, bucket_i8 and dense_i8 8-byte, the scales "
                                "4-byte aligned");
  bq::DenseGateUp dn{};
  dn.wg = dense_gate;
  dn.wu = dense_up;
  dn.sg = dense_gate_scale;
  dn.su = dense_up_scale;
  dn.x_i8 = dense_x_i8;
  dn.x_sa = dense_x_sa;
  dn.out_i8 = dense_i8;
  dn.out_sa = dense_sa;
  dn.T = seq_len;
  dn.inter = dense_inter;
  return check_hip(bq::launch_moe_phase1(x_i8, x_sa, expert_offset,
                                         reinterpret_cast<const bq::Route*>(routes), w_gate_up,
                                         gate_up_scale, nullptr, bucket_i8, bucket_sa,
                                         experts_per_rank, seq_len * top_k, hidden, inter,
                                         S(stream), &dn),
                   "ffn_gate_up");
}

int bq_ffn_down(const int8_t* bucket_i8, const float* bucket_sa, const int32_t* expert_offset,
                const bq_route* routes, const int8_t* w_down, const float* down_scale,
                float* moe_accum, uint16_t* moe_out, int experts_per_rank, int seq_len, int top_k,
                int hidden, int inter, int block, const int8_t* dense_i8, const float* dense_sa,
                const int8_t* dense_down, const float* dense_down_scale, int dense_inter,
                uint16_t* dense_out, void* workspace, size_t workspace_bytes, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  const int r = phase2_args("bq_ffn_down", bucket_i8, bucket_sa, expert_offset, routes, w_down,
                            down_scale, moe_accum, moe_out, top_k, hidden, inter, block);
  if (r != BQ_OK) return r;
  if (!workspace || !dense_i8 || !dense_sa || !dense_down || !dense_down_scale || !dense_out)
    return fail(BQ_ERR_INVALID, "bq_ffn_down: null pointer");
  if (dense_inter <= 0 || dense_inter % 64 || dense_inter % block)
    return fail(BQ_ERR_SHAPE, "bq_ffn_down: dense_inter %d must be a multiple of 64 and of block %d",
                dense_inter, block);
  if (dense_inter / block > 64)
    return fail(BQ_ERR_UNSUPPORTED, "bq_ffn_down: dense_inter/block = %d > 64", dense_inter / block);
  if (!a16(dense_i8) || !a16(dense_down) || (reinterpret_cast<uintptr_t>(dense_out) & 7u))
    return fail(BQ_ERR_INVALID, "bq_ffn_down: dense_i8 and dense_down must be 16-byte, dense_out "
                                "8-byte aligned");
  if (reinterpret_cast<uintptr_t>(workspace) % 256)
    return fail(BQ_ERR_INVALID, "bq_ffn_down: workspace must be 256-byte aligned");
  const size_t need = bq::moe_phase2_workspace(seq_len * top_k, seq_len, hidden);
  if (workspace_bytes < need)
    return fail(BQ_ERR_SHAPE, "bq_ffn_down: workspace %zu < %zu bytes", workspace_bytes, need);
  bq::DenseDown dn{};
  dn.w = dense_down;
  dn.ws = dense_down_scale;
  dn.x_i8 = dense_i8;
  dn.x_sa = dense_sa;
  dn.out = dense_out;
  dn.T = seq_len;
  dn.inter = dense_inter;
  return check_hip(bq::launch_moe_phase2(bucket_i8, bucket_sa, expert_offset,
                                         reinterpret_cast<const bq::Route*>(routes), w_down,
                                         down_scale, moe_accum, moe_out, experts_per_rank, seq_len,
                                         seq_len * top_k, hidden, inter, block, workspace,
                                         S(stream), &dn),
                   "ffn_down");
}

int bq_moe_phase2_down_noalloc(const int8_t* bucket_i8, const float* bucket_sa,
                               const int32_t* expert_offset, const bq_route* routes,
                               const int8_t* w_down, const float* down_scale, float* moe_accum,
                               uint16_t* moe_out, int experts_per_rank, int seq_len, int top_k,
                               int hidden, int inter, int block, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  int r = phase2_args("bq_moe_phase2_down_noalloc", bucket_i8, bucket_sa, expert_offset, routes,
                      w_down, down_scale, moe_accum, moe_out, top_k, hidden, inter, block);
  if (r != BQ_OK) return r;
  // the workspace is seq_len*top_k f32 rows of hidden (bq_moe_phase2_workspace_size)
  const size_t need = bq::moe_phase2_workspace(seq_len * top_k, seq_len, hidden);
  if (need > bq::kNoallocScratchBytes)
    return fail(BQ_ERR_UNSUPPORTED,
                "bq_moe_phase2_down_noalloc: seq_len*top_k*hidden*4 = %zu bytes exceeds the "
                "%zu-byte static scratch (use bq_moe_phase2_down with a workspace)",
                need, bq::kNoallocScratchBytes);
  int device = 0;
  r = check_hip(hipGetDevice(&device), "hipGetDevice");
  if (r) return r;
  void* ws = nullptr;
  r = check_hip(bq::scratch_address(device, &ws), "scratch symbol address");
  if (r) return r;
  return check_hip(bq::launch_moe_phase2(bucket_i8, bucket_sa, expert_offset,
                                         reinterpret_cast<const bq::Route*>(routes), w_down,
                                         down_scale, moe_accum, moe_out, experts_per_rank, seq_len,
                                         seq_len * top_k, hidden, inter, block, ws, S(stream)),
                   "moe_phase2_noalloc");
}

}  // extern "C"

// ---- vocabulary head and embedding -----------------------------------------
static_assert(sizeof(bq_sampling_params) == 40 && sizeof(bq::SamplingParams) == 40,
              "SamplingParams layout");
static_assert(sizeof(bq_sample_outcome) == 2064 && sizeof(bq::SampleOutcome) == 2064,
              "SampleOutcome layout");
static_assert(BQ_SAMPLE_NMAX == bq::kSampleNmax, "n_max");

static bool head_block_ok(int block) {
  return block == 64 || block == 128 || block == 256 || block == 512;
}

int bq_head_prep(const uint16_t* src, const uint16_t* gamma, int8_t* x_i8, float* x_sa,
                 int num_rows, int hidden, int block, float sqrt_n, float n_eps, void* stream) {
  if (num_rows <= 0) return BQ_OK;
  if (!src || !gamma || !x_i8 || !x_sa) return fail(BQ_ERR_INVALID, "bq_head_prep: null pointer");
  if (!head_block_ok(block) || hidden <= 0 || hidden % block)
    return fail(BQ_ERR_SHAPE, "bq_head_prep: need block in {64,128,256,512} dividing hidden %d", hidden);
  if (reinterpret_cast<uintptr_t>(src) & 3u)
    return fail(BQ_ERR_INVALID, "bq_head_prep: src must be 4-byte aligned");
  return check_hip(bq::launch_head_prep(src, gamma, x_i8, x_sa, num_rows, hidden, block, sqrt_n,
                                        n_eps, S(stream)),
                   "head_prep");
}

size_t bq_flash_sample_workspace_size(int num_rows, int vocab) {
  if (num_rows <= 0 || vocab <= 0) return 0;
  return bq::head_workspace_bytes(num_rows, vocab);
}

int bq_flash_sample(const int8_t* x_i8, const float* x_sa, const int8_t* weight,
                    const float* wscales, const bq_sampling_params* params,
                    bq_sample_outcome* outcome, int num_rows, int vocab, int hidden, int block,
                    float cap, int64_t vocab_base, void* workspace, size_t workspace_bytes,
                    void* stream) {
  if (num_rows <= 0) return BQ_OK;
  if (!x_i8 || !x_sa || !weight || !wscales || !params || !outcome || !workspace)
    return fail(BQ_ERR_INVALID, "bq_flash_sample: null pointer");
  if (num_rows > 32 || vocab > (1 << 20))
    return fail(BQ_ERR_UNSUPPORTED, "bq_flash_sample: num_rows %d > 32 or vocab %d > 2^20", num_rows,
                vocab);
  if (vocab <= 0 || vocab % 16 || !head_block_ok(block) || hidden <= 0 || hidden % block ||
      hidden / block > 64)
    return fail(BQ_ERR_SHAPE, "bq_flash_sample: need vocab %% 16 == 0, block in {64..512} "
                              "dividing hidden, hidden/block <= 64");
  if (!(cap > 0.0f)) return fail(BQ_ERR_SHAPE, "bq_flash_sample: cap must be positive");
  if (!a16(x_i8) || !a16(weight) || (reinterpret_cast<uintptr_t>(workspace) & 255u))
    return fail(BQ_ERR_INVALID, "bq_flash_sample: x_i8/weight 16-byte, workspace 256-byte aligned");
  if (workspace_bytes < bq::head_workspace_bytes(num_rows, vocab))
    return fail(BQ_ERR_SHAPE, "bq_flash_sample: workspace %zu < %zu bytes", workspace_bytes,
                bq::head_workspace_bytes(num_rows, vocab));
  return check_hip(bq::launch_flash_sample(x_i8, x_sa, weight, wscales,
                                           reinterpret_cast<const bq::SamplingParams*>(params),
                                           reinterpret_cast<bq::SampleOutcome*>(outcome),
                                           num_rows, vocab, hidden, block, cap, vocab_base,
                                           workspace, S(stream)),
                   "flash_sample");
}

int bq_embed_lookup(const int32_t* token_ids, const int8_t* weight, const float* wscales,
                    uint16_t* dst, int seq_len, int hidden, int block, int shard_rows, int rank,
                    float scale, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!token_ids || !weight || !wscales || !dst) return fail(BQ_ERR_INVALID, "bq_embed_lookup: null pointer");
  if (!head_block_ok(block) || hidden <= 0 || hidden % block || shard_rows <= 0 || rank < 0)
    return fail(BQ_ERR_SHAPE, "bq_embed_lookup: need block in {64,128,256,512} dividing hidden, "
                              "shard_rows > 0");
  return check_hip(bq::launch_embed(token_ids, weight, wscales, dst, seq_len, hidden, block,
                                    shard_rows, rank, scale, S(stream)),
                   "embed_lookup");
}

static_assert(sizeof(bq_kv_run) == sizeof(bq::KvRun), "bq_kv_run layout");

namespace {
inline bool attn_hd_ok(int hd) { return hd == 64 || hd == 128 || hd == 256 || hd == 512; }

int attn_common(const char* who, const int8_t* q_i8, const float* qi_bias, const float* f_q,
                const int8_t* k_cache, const float* k_scale, const int8_t* v_cache,
                const float* v_scale, uint16_t* output, void* workspace,
                size_t workspace_bytes, const bq_kv_run* runs, int num_runs,
                const int32_t* base_rows, int num_q, int num_kv, int head_dim, int window,
                int page_shift, int row_mask, int page_mask, int s_max, int seq_len,
                void* stream) {
  if (!q_i8 || !qi_bias || !f_q || !k_cache || !k_scale || !v_cache || !v_scale || !output ||
      !runs || !base_rows || !workspace)
    return fail(BQ_ERR_INVALID, "%s: null pointer", who);
  if (num_runs <= 0 || num_q <= 0 || num_kv <= 0 || num_q % num_kv || s_max <= 0 ||
      page_shift < 0 || page_shift > 30)
    return fail(BQ_ERR_SHAPE, "%s: need num_runs > 0, num_q %% num_kv == 0, s_max > 0", who);
  const int gqa = num_q / num_kv;
  if (!attn_hd_ok(head_dim) || !(gqa == 1 || gqa == 2 || gqa == 4 || gqa == 8 || gqa == 16))
    return fail(BQ_ERR_SHAPE, "%s: need head_dim in {64,128,256,512} and num_q/num_kv in "
                              "{1,2,4,8,16}", who);
  if (!a16(q_i8) || !a16(k_cache) || !a16(v_cache) || !a16(workspace) || !a16(output))
    return fail(BQ_ERR_INVALID, "%s: q_i8, caches, output and workspace must be 16-byte aligned",
                who);
  const size_t need = bq_attention_workspace_size(seq_len, num_q, head_dim, s_max);
  if (workspace_bytes < need)
    return fail(BQ_ERR_SHAPE, "%s: workspace of %zu bytes, need %zu", who, workspace_bytes, need);
  bq::AttnArgs a{};
  a.q_i8 = q_i8; a.qi_bias = qi_bias; a.f_q = f_q; a.k_cache = k_cache; a.k_scale = k_scale;
  a.v_cache = v_cache; a.v_scale = v_scale;
  a.runs = reinterpret_cast<const bq::KvRun*>(runs); a.base_rows = base_rows; a.out = output;
  a.ws_acc = static_cast<float*>(workspace);
  a.ws_ml = a.ws_acc + (size_t)seq_len * num_q * s_max * head_dim;
  a.num_runs = num_runs; a.T = seq_len; a.num_q = num_q; a.num_kv = num_kv; a.window = window;
  a.page_shift = page_shift; a.row_mask = row_mask; a.page_mask = page_mask; a.s_max = s_max;
  return check_hip(bq::launch_flash_attn(a, head_dim, S(stream)), who);
}
}  // namespace

extern "C" {

int bq_attn_prep(const uint16_t* q_src, const uint16_t* k_src, const uint16_t* v_src,
                 const uint16_t* q_norm, const uint16_t* k_norm, int8_t* q_i8, float* qi_bias,
                 float* f_q, int8_t* k_cache, float* k_scale, int8_t* v_cache, float* v_scale,
                 const float* cos_table, const float* sin_table, const bq_kv_run* runs,
                 int num_runs, const int32_t* base_rows, int num_q, int num_kv, int head_dim,
                 int rope_half, int pair_stride, float sqrt_n, float n_eps, int cache_degree,
                 int rank, int page_shift, int row_mask, int page_mask, int seq_len,
                 void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (!q_src || !k_src || !v_src || !q_norm || !k_norm || !q_i8 || !qi_bias || !f_q ||
      !k_cache || !k_scale || !v_cache || !v_scale || !runs || !base_rows ||
      (rope_half > 0 && (!cos_table || !sin_table)))
    return fail(BQ_ERR_INVALID, "bq_attn_prep: null pointer");
  if (!attn_hd_ok(head_dim) || num_runs <= 0 || num_q <= 0 || num_kv <= 0 ||
      cache_degree <= 0 || rank < 0 || rank >= cache_degree || page_shift < 0 || page_shift > 30)
    return fail(BQ_ERR_SHAPE, "bq_attn_prep: need head_dim in {64,128,256,512}, num_runs, "
                              "num_q, num_kv > 0, 0 <= rank < cache_degree");
  if (rope_half < 0 || rope_half % 64 || pair_stride % 64 || rope_half > pair_stride ||
      pair_stride + rope_half > head_dim || (rope_half > 0 && pair_stride <= 0))
    return fail(BQ_ERR_SHAPE, "bq_attn_prep: rope_half and pair_stride must be multiples of 64 "
                              "with rope_half <= pair_stride and pair_stride + rope_half <= "
                              "head_dim");
  bq::PrepArgs a{};
  a.q_src = q_src; a.k_src = k_src; a.v_src = v_src; a.q_norm = q_norm; a.k_norm = k_norm;
  a.q_i8 = q_i8; a.qi_bias = qi_bias; a.f_q = f_q; a.k_cache = k_cache; a.k_scale = k_scale;
  a.v_cache = v_cache; a.v_scale = v_scale; a.cos_table = cos_table; a.sin_table = sin_table;
  a.runs = reinterpret_cast<const bq::KvRun*>(runs); a.base_rows = base_rows;
  a.num_runs = num_runs; a.T = seq_len; a.num_q = num_q; a.num_kv = num_kv;
  a.rope_half = rope_half; a.pair_stride = pair_stride; a.sqrt_n = sqrt_n; a.n_eps = n_eps;
  a.cache_degree = cache_degree; a.rank = rank;
  a.page_shift = page_shift; a.row_mask = row_mask; a.page_mask = page_mask;
  return check_hip(bq::launch_attn_prep(a, head_dim, S(stream)), "attn_prep");
}

int bq_attention_splits(int seq_len, int num_kv, int max_kv_len) {
  return bq::attn_splits(seq_len, num_kv, max_kv_len);
}

size_t bq_attention_workspace_size(int seq_len, int num_q, int head_dim, int s_max) {
  if (seq_len <= 0 || num_q <= 0 || head_dim <= 0 || s_max <= 0) return 0;
  return (size_t)seq_len * num_q * s_max * ((size_t)head_dim + 2) * sizeof(float);
}

int bq_sliding_attention(const int8_t* q_i8, const float* qi_bias, const float* f_q,
                         const int8_t* k_cache, const float* k_scale, const int8_t* v_cache,
                         const float* v_scale, uint16_t* output, void* workspace,
                         size_t workspace_bytes, const bq_kv_run* runs, int num_runs,
                         const int32_t* base_rows, int num_q, int num_kv, int head_dim,
                         int window, int page_shift, int row_mask, int page_mask, int s_max,
                         int seq_len, void* stream) {
  if (seq_len <= 0) return BQ_OK;
  if (window <= 0) return fail(BQ_ERR_SHAPE, "bq_sliding_attention: window must be > 0");
  return attn_common("bq_sliding_attention", q_i8, qi_bias, f_q, k_cache, k_scale, v_cache,
                     v_scale, output, workspace, workspace_bytes, runs, num_runs, base_rows,
                     num_q, num_kv, head_dim, window, page_shift, row_mask, page_mask, s_max,
                     seq_len, stream);
}

int bq_full_attention(const int8_t* q_i8, const float* qi_bias, const float* f_q,
                      const int8_t* k_cache, const float* k_scale, const int8_t* v_cache,
                      const float* v_scale, uint16_t* output, void* workspace,
                      size_t workspace_bytes, const bq_kv_run* runs, int num_runs,
                      const int32_t* base_rows, int num_q, int num_kv, int head_dim,
                      int page_shift, int row_mask, int page_mask, int s_max, int seq_len,
                      void* stream) {
  if (seq_len <= 0) return BQ_OK;
  return attn_common("bq_full_attention", q_i8, qi_bias, f_q, k_cache, k_scale, v_cache,
                     v_scale, output, workspace, workspace_bytes, runs, num_runs, base_rows,
                     num_q, num_kv, head_dim, 0, page_shift, row_mask, page_mask, s_max,
                     seq_len, stream);
}

}  // extern "C"
