// capi.cpp — C ABI: contexts, device memory, weight packing/upload and the
// tensor-level GEMM entry points (the internal/tensor mirror).
//
// Host-side quantization restates the reference exactly (it runs once at
// load, as PackB8/PackB8VNNI do); the device kernels then consume the packed
// bytes. Every entry point validates its arguments and returns an RH_*
// status with a thread-local message instead of aborting.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "context.h"

namespace rh {

static thread_local char g_err[512];

void set_error(const char* msg) noexcept { snprintf(g_err, sizeof g_err, "%s", msg ? msg : ""); }

int fail(int code, const char* msg) noexcept {
  set_error(msg);
  return code;
}

int fail_exception(int code, const char* what) noexcept {
  snprintf(g_err, sizeof g_err, "internal error: %s", what ? what : "exception");
  return code;
}

int hip_fail(hipError_t e, const char* what, const char* file, int line) noexcept {
  snprintf(g_err, sizeof g_err, "%s failed: %s (%s:%d)", what, hipGetErrorString(e), file,
           line);
  return e == hipErrorOutOfMemory ? RH_ERR_OOM : RH_ERR_HIP;
}

}  // namespace rh

// ---- profiling ---------------------------------------------------------------
namespace rh {
LaunchTiming& launch_timing() {
  thread_local LaunchTiming t;
  return t;
}
}  // namespace rh

hipError_t rh_context::prof_begin(int kind, double ops, double bytes, int* slot) {
  *slot = -1;
  if (!profiling) return hipSuccess;
  ProfRec r{};
  hipError_t e = hipEventCreate(&r.a);
  if (e != hipSuccess) return e;
  e = hipEventCreate(&r.b);
  if (e != hipSuccess) return e;
  r.kind = kind;
  r.ops = ops;
  r.bytes = bytes;
  recs.push_back(r);
  *slot = (int)recs.size() - 1;
  // the next timed launch attaches the pair to its own dispatch packet
  rh::launch_timing() = rh::LaunchTiming{r.a, r.b};
  return hipSuccess;
}

// Grows only; the old buffer may still be read by queued kernels, so the
// stream drains before it is freed.
hipError_t rh_context::ensure_ws(size_t bytes) {
  if (bytes <= ws_bytes) return hipSuccess;
  if (ws) {
    hipError_t e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return e;
    (void)hipFree(ws);
    ws = nullptr;
    ws_bytes = 0;
  }
  const size_t want = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
  hipError_t e = hipMalloc(&ws, want);
  if (e == hipSuccess) ws_bytes = want;
  else ws = nullptr;
  return e;
}

hipError_t rh_context::prof_end(int slot) {
  if (slot < 0) return hipSuccess;
  rh::LaunchTiming& t = rh::launch_timing();
  if (t.start == recs[slot].a) {  // nothing was launched (empty problem)
    t = rh::LaunchTiming{};
    recs[slot].kind = -1;
  }
  return hipSuccess;
}

void rh_context::prof_clear() {
  for (auto& r : recs) {
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  recs.clear();
}

namespace rh {

// ---- host quantizers (restated from the reference) ----------------------------

// PackB8, internal/tensor/pack8.go:25-76.
int quantize_b8(const float* bT, int k, int n, std::vector<int8_t>& q,
                std::vector<float>& scales) {
  q.assign((size_t)n * k, 0);
  scales.assign(n, 0.0f);
  for (int j = 0; j < n; j++) {
    const float* row = bT + (size_t)j * k;
    float maxAbs = 0.0f;
    for (int p = 0; p < k; p++) {
      const float v = row[p];
      if (std::isnan(v) || std::isinf(v)) {
        char buf[160];
        snprintf(buf, sizeof buf, "PackB8 channel %d has a non-finite weight", j);
        return fail(RH_ERR_NONFINITE, buf);
      }
      const float a = std::fabs(v);
      if (a > maxAbs) maxAbs = a;
    }
    float scale = maxAbs / 127.0f;
    if (scale == 0.0f) scale = 1.0f;
    scales[j] = scale;
    for (int p = 0; p < k; p++) {
      double qd = std::rint((double)row[p] / (double)scale);
      if (qd > 127.0) qd = 127.0;
      if (qd < -127.0) qd = -127.0;
      q[(size_t)j * k + p] = (int8_t)qd;
    }
  }
  return RH_OK;
}

// PackB8VNNI, internal/tensor/pack_vnni.go:28-77.
int quantize_b8_vnni(const float* bT, int k, int n, std::vector<int8_t>& q,
                     std::vector<float>& scales, std::vector<int32_t>& colsum) {
  q.assign((size_t)n * k, 0);
  scales.assign(n, 0.0f);
  colsum.assign(n, 0);
  for (int c = 0; c < n; c++) {
    const float* row = bT + (size_t)c * k;
    double maxAbs = 0.0;
    for (int p = 0; p < k; p++) {
      const double v = (double)row[p];
      if (std::isnan(v) || std::isinf(v)) {
        char buf[160];
        snprintf(buf, sizeof buf, "PackB8VNNI weight [%d,%d] is not finite", c, p);
        return fail(RH_ERR_NONFINITE, buf);
      }
      const double a = std::fabs(v);
      if (a > maxAbs) maxAbs = a;
    }
    double scale = maxAbs / 127.0;
    if (scale == 0.0) scale = 1.0;
    scales[c] = (float)scale;
    uint32_t sum = 0;
    for (int p = 0; p < k; p++) {
      const int8_t qv = (int8_t)std::rint((double)row[p] / scale);
      sum += (uint32_t)(int32_t)qv;
      q[(size_t)c * k + p] = qv;
    }
    colsum[c] = (int32_t)sum;
  }
  return RH_OK;
}

static int check_pack_shape(const char* who, int k, int n) {
  char buf[160];
  if (n < 16 || n % 16 != 0) {
    snprintf(buf, sizeof buf, "%s needs n%%16==0 and n>=16, got n=%d", who, n);
    return fail(RH_ERR_SHAPE, buf);
  }
  if (k < 1) {
    snprintf(buf, sizeof buf, "%s needs k>=1, got k=%d", who, k);
    return fail(RH_ERR_SHAPE, buf);
  }
  return RH_OK;
}

// bf16 with round-to-nearest-even (the device conversion rounds the same
// way); NaN stays NaN.
static uint16_t bf16_rne(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float bf16_value(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// The bf16 planes of a padded [np][kp] weight image for the bf16-MFMA GEMMs:
// weight-only int8 gets its integers (exact in bf16), fp32 the split
// hi = bf16(w), lo = bf16(w - hi). Zero padding stays zero.
static hipError_t upload_planes(rh_weight* w, const std::vector<uint8_t>& img) {
  const size_t count = (size_t)w->np * w->kp;
  std::vector<uint16_t> hi(count), lo;
  if (w->mode == RH_MODE_W8) {
    const int8_t* q = reinterpret_cast<const int8_t*>(img.data());
    for (size_t i = 0; i < count; i++) hi[i] = bf16_rne((float)q[i]);
  } else {
    const float* f = reinterpret_cast<const float*>(img.data());
    lo.resize(count);
    for (size_t i = 0; i < count; i++) {
      hi[i] = bf16_rne(f[i]);
      lo[i] = bf16_rne(f[i] - bf16_value(hi[i]));
    }
  }
  hipError_t e = hipMalloc(&w->d_bf, count * 2);
  if (e == hipSuccess) e = hipMemcpy(w->d_bf, hi.data(), count * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess && !lo.empty()) {
    e = hipMalloc(&w->d_bf_lo, count * 2);
    if (e == hipSuccess) e = hipMemcpy(w->d_bf_lo, lo.data(), count * 2, hipMemcpyHostToDevice);
  }
  return e;
}

// The s8 image [np][kp] rearranged into B-fragment order (rh_weight::d_frag).
static hipError_t upload_frag(rh_weight* w, const std::vector<uint8_t>& img) {
  const int ks_n = w->kp / 32;
  std::vector<uint8_t> frag(img.size());
  for (int nb = 0; nb < w->np / 32; nb++)
    for (int ks = 0; ks < ks_n; ks++)
      for (int l = 0; l < 64; l++)
        memcpy(&frag[(((size_t)nb * ks_n + ks) * 64 + l) * 16],
               &img[(size_t)(nb * 32 + l % 32) * w->kp + ks * 32 + (l / 32) * 16], 16);
  hipError_t e = hipMalloc(&w->d_frag, frag.size());
  if (e == hipSuccess) e = hipMemcpy(w->d_frag, frag.data(), frag.size(), hipMemcpyHostToDevice);
  return e;
}

// The unpacked fp32 fallback (MatMulFunc's raw weights, tensor.go:16-70)
// takes any shape the device epilogue can store: k >= 1 and n a positive
// multiple of 4 (4-column vector stores).
static int check_raw_shape(int k, int n) {
  char buf[160];
  if (n < 4 || n % 4 != 0 || k < 1) {
    snprintf(buf, sizeof buf, "unpacked fp32 weight needs k>=1 and n%%4==0, got k=%d n=%d", k, n);
    return fail(RH_ERR_SHAPE, buf);
  }
  return RH_OK;
}

int pack_check(int mode, const float* bT, int k, int n, bool raw_ok) {
  static const char* names[] = {"PackB", "PackB8", "PackB8VNNI"};
  int st = raw_ok && mode == RH_MODE_F32 ? check_raw_shape(k, n)
                                         : check_pack_shape(names[mode], k, n);
  if (st != RH_OK || mode == RH_MODE_F32) return st;
  const size_t count = (size_t)n * k;
  for (size_t i = 0; i < count; i++)
    if (!std::isfinite(bT[i])) {
      char buf[160];
      snprintf(buf, sizeof buf, "%s: weight [%zu,%zu] is not finite", names[mode], i / k, i % k);
      return fail(RH_ERR_NONFINITE, buf);
    }
  return RH_OK;
}

int pack_weight(Context* ctx, int mode, const float* bT, const float* bias, int k,
                int n, rh_weight** out, bool raw_ok) {
  static const char* names[] = {"PackB", "PackB8", "PackB8VNNI"};
  int st = raw_ok && mode == RH_MODE_F32 ? check_raw_shape(k, n)
                                         : check_pack_shape(names[mode], k, n);
  if (st != RH_OK) return st;
  // owned here until the upload succeeds (a throw or a failed upload frees it)
  std::unique_ptr<rh_weight, void (*)(rh_weight*)> w(new rh_weight(), destroy_weight);
  w->ctx = ctx;
  w->mode = mode;
  w->k = k;
  w->n = n;
  w->kp = (int)round_up(k, kWeightKPad);
  w->np = (int)round_up(n, kWeightRowPad);
  std::vector<int8_t> q;
  std::vector<float> scales;
  std::vector<int32_t> colsum;
  size_t elem = mode == RH_MODE_F32 ? 4 : 1;
  if (mode == RH_MODE_W8) st = quantize_b8(bT, k, n, q, scales);
  else if (mode == RH_MODE_A8W8) st = quantize_b8_vnni(bT, k, n, q, scales, colsum);
  if (st != RH_OK) return st;
  // Padded [np][kp] image, zero outside [n][k].
  std::vector<uint8_t> img((size_t)w->np * w->kp * elem, 0);
  for (int j = 0; j < n; j++) {
    uint8_t* dst = img.data() + (size_t)j * w->kp * elem;
    if (mode == RH_MODE_F32) memcpy(dst, bT + (size_t)j * k, (size_t)k * 4);
    else memcpy(dst, q.data() + (size_t)j * k, (size_t)k);
  }
  hipError_t e = hipMalloc(&w->d_data, img.size());
  if (e == hipSuccess) e = hipMemcpy(w->d_data, img.data(), img.size(), hipMemcpyHostToDevice);
  if (e == hipSuccess && mode != RH_MODE_A8W8) e = upload_planes(w.get(), img);
  if (e == hipSuccess && mode == RH_MODE_A8W8) e = upload_frag(w.get(), img);
  if (e == hipSuccess && !scales.empty()) {
    e = hipMalloc(&w->d_scales, n * sizeof(float));
    if (e == hipSuccess)
      e = hipMemcpy(w->d_scales, scales.data(), n * sizeof(float), hipMemcpyHostToDevice);
  }
  if (e == hipSuccess && !colsum.empty()) {
    e = hipMalloc(&w->d_colsum, n * sizeof(int32_t));
    if (e == hipSuccess)
      e = hipMemcpy(w->d_colsum, colsum.data(), n * sizeof(int32_t), hipMemcpyHostToDevice);
  }
  if (e == hipSuccess && bias) {
    e = hipMalloc(&w->d_bias, n * sizeof(float));
    if (e == hipSuccess)
      e = hipMemcpy(w->d_bias, bias, n * sizeof(float), hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) return hip_fail(e, "weight upload", __FILE__, __LINE__);
  ctx_retain(ctx);
  *out = w.release();
  return RH_OK;
}

// Frees the device copy; the caller holds the context's mutex (or is the
// last owner) and then drops the weight's context reference.
void destroy_weight(rh_weight* w) {
  if (!w) return;
  if (w->d_data) (void)hipFree(w->d_data);
  if (w->d_scales) (void)hipFree(w->d_scales);
  if (w->d_colsum) (void)hipFree(w->d_colsum);
  if (w->d_bias) (void)hipFree(w->d_bias);
  if (w->d_bf) (void)hipFree(w->d_bf);
  if (w->d_bf_lo) (void)hipFree(w->d_bf_lo);
  if (w->d_frag) (void)hipFree(w->d_frag);
  delete w;
}

void ctx_retain(Context* ctx) { ctx->refs.fetch_add(1); }

void ctx_release(Context* ctx) {
  if (ctx->refs.fetch_sub(1) != 1) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  ctx->prof_clear();
  if (ctx->ws) (void)hipFree(ctx->ws);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

// The int8 GEMM over already-quantized rows with an explicit epilogue.
// Profiled as kind 0; `ops` is the algorithmic work credited to the launch
// (a recompute pass credits 0 so the pair counts 2·M·K·N once).
int pack_weight_gated(Context* ctx, int mode, const float* gate, const float* up, int k,
                      int i, rh_weight** out, bool raw_ok) {
  // gate and up are each a PackB*-shaped matrix in the reference (two
  // newDense calls), so each must pass the packers' shape rule on its own
  // (the unpacked fp32 fallback: whole groups of kGluGroup rows)
  int st0 = raw_ok && mode == RH_MODE_F32 ? check_raw_shape(k, i)
                                          : check_pack_shape("gated PackB", k, i);
  if (st0 != RH_OK) return st0;
  std::vector<float> inter((size_t)2 * i * k);
  for (int t = 0; t < i / kGluGroup; t++)
    for (int r = 0; r < kGluGroup; r++) {
      memcpy(&inter[((size_t)2 * kGluGroup * t + r) * k], gate + ((size_t)kGluGroup * t + r) * k,
             sizeof(float) * k);
      memcpy(&inter[((size_t)2 * kGluGroup * t + kGluGroup + r) * k],
             up + ((size_t)kGluGroup * t + r) * k, sizeof(float) * k);
    }
  int st = pack_weight(ctx, mode, inter.data(), nullptr, k, 2 * i, out, raw_ok);
  if (st == RH_OK) (*out)->glu = true;
  return st;
}

int run_gemm_i8(Context* ctx, const rh_weight* w, const uint8_t* qa, int ldq,
                const float* rs, int m, int epi, void* out, int ldo, int act,
                const float* bias, float* row_absmax, float* rs_out, double ops,
                void* out_lo, unsigned* sync, unsigned* slots, int slot_ld,
                unsigned* sync_err) {
  if (m <= 0) return RH_OK;
  if (epi == EPI_PLANES && !out_lo) return fail(RH_ERR_INVALID, "planes epilogue needs a lo plane");
  if (epi == EPI_QSYNC && (!sync || !slots || !sync_err))
    return fail(RH_ERR_INVALID, "single-pass quantizing epilogue needs its counters");
  GemmI8Args g{};
  g.A = qa;
  g.lda = ldq;
  g.B = static_cast<const int8_t*>(w->d_data);
  g.ldb = w->kp;
  g.Bf = static_cast<const int8_t*>(w->d_frag);
  g.M = m;
  g.N = w->n;
  g.K = w->k;
  g.row_scales = rs;
  g.col_scales = w->d_scales;
  g.colsum = w->d_colsum;
  g.bias = bias;
  g.out = out;
  g.out_lo = out_lo;
  g.ldo = ldo;
  g.act = act;
  g.epi = epi;
  g.row_absmax = row_absmax;
  g.rs_out = rs_out;
  g.tile_group = ctx->tile_group;
  g.sync = sync;
  g.slots = slots;
  g.slot_ld = slot_ld;
  g.sync_err = sync_err;
  const double M = m, K = w->k, N = w->n;
  static const double out_bytes[] = {4, 2, 0, 1, 4, 4, 1};  // per output element
  const double bytes = M * K + K * N + M * N * out_bytes[epi] + 4 * M + 8 * N +
                       (bias ? 4 * N : 0) +
                       (epi == EPI_QUANT || epi == EPI_QSYNC ? 4 * M : 0);
  int slot = -1;
  hipError_t e = ctx->prof_begin(epi == EPI_QSYNC ? 5 : 0, ops, bytes, &slot);
  if (e == hipSuccess) e = launch_gemm_i8(g, ctx->i8_tile, ctx->stream);
  if (e == hipSuccess) e = ctx->prof_end(slot);
  if (e != hipSuccess) return hip_fail(e, "int8 gemm launch", __FILE__, __LINE__);
  return RH_OK;
}

// The full-int8 linear with the residual + LayerNorm finish (launch_gemm_i8_ln).
int run_gemm_i8_ln(Context* ctx, const rh_weight* w, const uint8_t* qa, int ldq,
                   const float* rs, int m, const I8LnArgs& f, double ops) {
  if (m <= 0) return RH_OK;
  if (w->mode != RH_MODE_A8W8 || !w->d_frag || w->glu)
    return fail(RH_ERR_INVALID, "fused LayerNorm linear needs a full-int8 weight");
  GemmI8Args g{};
  g.A = qa;
  g.lda = ldq;
  g.B = static_cast<const int8_t*>(w->d_data);
  g.ldb = w->kp;
  g.Bf = static_cast<const int8_t*>(w->d_frag);
  g.M = m;
  g.N = w->n;
  g.K = w->k;
  g.row_scales = rs;
  g.col_scales = w->d_scales;
  g.colsum = w->d_colsum;
  g.bias = w->d_bias;
  g.act = ACT_NONE;
  g.epi = EPI_F32;
  g.tile_group = ctx->tile_group;
  const double M = m, K = w->k, N = w->n;
  // A, B, the residual read and written, the u8 rows, scales
  const double bytes = M * K + K * N + 8 * M * N + (f.qa ? M * N + 4 * M : 0) + 4 * M + 16 * N;
  int slot = -1;
  hipError_t e = ctx->prof_begin(0, ops, bytes, &slot);
  if (e == hipSuccess) e = launch_gemm_i8_ln(g, f, ctx->stream);
  if (e == hipSuccess) e = ctx->prof_end(slot);
  if (e != hipSuccess) return hip_fail(e, "int8 gemm + layernorm launch", __FILE__, __LINE__);
  return RH_OK;
}

// Weight-only int8 / fp32 linear on bf16 planes: split the activations once
// into the context workspace, then the planes GEMM. Rows go in chunks that
// keep the kernel's 32-bit element offsets in range.
bool linear_on_planes(const Context* ctx, const rh_weight* w) {
  return w->mode != RH_MODE_A8W8 && ctx->bf_algo == 0 &&
         !(w->mode == RH_MODE_F32 && ctx->f32_algo == F32_NATIVE);
}

int linear_a_terms(const Context* ctx, const rh_weight* w) {
  return w->mode == RH_MODE_W8 ? ctx->w8_terms : 2;
}

// Weight-only int8 / fp32 linear on bf16 planes. The activations come as
// producer-written planes (pin) or are split once here into the context
// workspace; the output goes to fp32 dst or to planes (pout). Rows go in
// chunks that keep the kernel's 32-bit element offsets in range.
int run_linear_qk(Context* ctx, const rh_weight* w, const Planes& pin, int m,
                  const QkEpilogue& q, __bf16* out, int ldo, bool* applied) {
  *applied = false;
  if (!linear_on_planes(ctx, w) || w->mode != RH_MODE_W8 || linear_a_terms(ctx, w) != 1 ||
      w->glu || ctx->bf_tile != 0 || !pin.hi || m <= 0)
    return RH_OK;
  if (w->n % 256 != 0 || !(q.dh == 64 || q.dh == 128 || q.dh == 256) || ldo % 4 != 0)
    return RH_OK;
  // the fused tile only where the 256x256 grid keeps the CUs busy, and
  // without row chunking (32-bit element offsets)
  if ((long long)ceil_div(m, 256) * (w->n / 256) < 128) return RH_OK;
  if ((long long)m * std::max(pin.ld, ldo) >= (1LL << 30)) return RH_OK;
  GemmPlArgs g{};
  g.Ah = pin.hi;
  g.Al = nullptr;
  g.lda = pin.ld;
  g.Bh = static_cast<const __bf16*>(w->d_bf);
  g.Bl = nullptr;
  g.ldb = w->kp;
  g.M = m;
  g.N = w->n;
  g.K = w->k;
  g.col_scales = w->d_scales;
  g.bias = w->d_bias;
  g.ldc = ldo;
  g.act = ACT_NONE;
  g.tile_group = ctx->tile_group;
  g.qk_qg = q.q_g;
  g.qk_kg = q.k_g;
  g.qk_cos = q.cos_t;
  g.qk_sin = q.sin_t;
  g.qk_pos = q.pos;
  g.qk_out = out;
  g.qk_nq = q.nq;
  g.qk_nkv = q.nkv;
  g.qk_dh = q.dh;
  g.qk_eps = q.eps;
  const double M = m, K = w->k, N = w->n;
  const double bytes = M * K * 2.0 + K * N + 4 * N + M * N * 2.0;
  int slot = -1;
  hipError_t e = ctx->prof_begin(1, 2.0 * M * K * N, bytes, &slot);
  if (e == hipSuccess) e = launch_gemm_planes_qk(g, ctx->stream);
  if (e == hipSuccess) e = ctx->prof_end(slot);
  if (e != hipSuccess) return hip_fail(e, "planes gemm (qk epilogue) launch", __FILE__, __LINE__);
  *applied = true;
  return RH_OK;
}

static int run_linear_planes(Context* ctx, const rh_weight* w, const float* a, int lda, int m,
                             float* dst, int ldc, int act, const float* bias,
                             const Planes* pin, const Planes* pout) {
  hipStream_t s = ctx->stream;
  const int a_terms = linear_a_terms(ctx, w);
  const int b_terms = w->mode == RH_MODE_W8 ? 1 : 2;
  const int ldk = pin ? pin->ld : (int)round_up(w->k, 64);
  const int ldo = pout ? pout->ld : ldc;
  const long long big = std::max((long long)ldk, (long long)ldo);
  const int chunk = std::min(m, (int)((1u << 30) / (unsigned long long)big));
  const size_t plane = (size_t)chunk * ldk * 2;
  __bf16* hi = nullptr;
  __bf16* lo = nullptr;
  if (!pin) {
    hipError_t e = ctx->ensure_ws(plane * a_terms);
    if (e != hipSuccess) return hip_fail(e, "gemm workspace", __FILE__, __LINE__);
    hi = static_cast<__bf16*>(ctx->ws);
    lo = a_terms == 2 ? reinterpret_cast<__bf16*>(static_cast<uint8_t*>(ctx->ws) + plane)
                      : nullptr;
  }
  hipError_t e = hipSuccess;
  for (int r0 = 0; r0 < m; r0 += chunk) {
    const int mc = std::min(chunk, m - r0);
    const double M = mc, K = w->k, N = w->n;
    int slot = -1;
    if (!pin) {
      e = ctx->prof_begin(4, 0.0, M * K * 4 + M * ldk * 2.0 * a_terms, &slot);
      if (e == hipSuccess)
        e = launch_split_bf16(a + (size_t)r0 * lda, lda, mc, w->k, hi, lo, ldk, s);
      if (e == hipSuccess) e = ctx->prof_end(slot);
      if (e != hipSuccess) return hip_fail(e, "split_bf16", __FILE__, __LINE__);
    }
    GemmPlArgs g{};
    g.Ah = pin ? pin->hi + (size_t)r0 * ldk : hi;
    g.Al = pin ? (a_terms == 2 ? pin->lo + (size_t)r0 * ldk : nullptr) : lo;
    g.lda = ldk;
    g.Bh = static_cast<const __bf16*>(w->d_bf);
    g.Bl = static_cast<const __bf16*>(w->d_bf_lo);
    g.ldb = w->kp;
    g.M = mc;
    g.N = w->n;
    g.K = w->k;
    g.col_scales = w->mode == RH_MODE_W8 ? w->d_scales : nullptr;
    g.bias = bias;
    if (pout) {
      g.Ch = pout->hi + (size_t)r0 * ldo;
      g.Cl = pout->lo ? pout->lo + (size_t)r0 * ldo : nullptr;
    } else {
      g.C = dst + (size_t)r0 * ldc;
    }
    g.ldc = ldo;
    g.act = act;
    g.tile_group = ctx->tile_group;
    // algorithmic bytes: the activations (fp32, or the planes a producer
    // wrote), the weights as stored for the mode (int8 / fp32), the output
    // (fp32 or planes)
    const double wbytes = w->mode == RH_MODE_W8 ? K * N + 4 * N : 4 * K * N;
    const double abytes = pin ? M * K * 2.0 * a_terms : M * K * 4;
    const double obytes = pout ? (pout->lo ? 4.0 : 2.0) : 4.0;
    const double bytes = abytes + wbytes + M * (w->glu ? N / 2 : N) * obytes + (bias ? 4 * N : 0);
    e = ctx->prof_begin(w->mode == RH_MODE_W8 ? 1 : 2, 2.0 * M * K * N, bytes, &slot);
    if (e == hipSuccess) e = launch_gemm_planes(g, a_terms, b_terms, ctx->bf_tile, s);
    if (e == hipSuccess) e = ctx->prof_end(slot);
    if (e != hipSuccess) return hip_fail(e, "planes gemm launch", __FILE__, __LINE__);
  }
  return RH_OK;
}

// One linear with fp32 output: the GEMM family dispatch of applyDense
// (bert.go:282-301) with bias/activation fused. For A8W8 the input must
// already be quantized into qa/rs (row stride ldq) unless quantize_first,
// in which case `a` is quantized here first.
int run_linear(Context* ctx, const rh_weight* w, const float* a, int lda, int m,
               float* dst, int ldc, int act, const float* bias, uint8_t* qa,
               int ldq, float* rs, bool quantize_first, const Planes* pin,
               const Planes* pout) {
  if (m <= 0) return RH_OK;
  hipStream_t s = ctx->stream;
  const double M = m, K = w->k, N = w->n;
  const double ops = 2.0 * M * K * N;
  if (w->mode == RH_MODE_A8W8) {
    if (quantize_first) {
      hipError_t e = launch_quantize_rows_u8(a, lda, m, w->k, qa, ldq, rs, s);
      if (e != hipSuccess) return hip_fail(e, "quantize_rows_u8", __FILE__, __LINE__);
    }
    return run_gemm_i8(ctx, w, qa, ldq, rs, m, EPI_F32, dst, ldc, act, bias, nullptr,
                       nullptr, ops);
  }
  if (linear_on_planes(ctx, w))
    return run_linear_planes(ctx, w, a, lda, m, dst, ldc, act, bias, pin, pout);
  if (pin || pout) return fail(RH_ERR_INVALID, "planes given to a linear that does not use them");
  int slot = -1;
  hipError_t e = hipSuccess;
  GemmBfArgs g{};
  g.A = a;
  g.lda = lda;
  g.B = w->d_data;
  g.ldb = w->kp;
  g.M = m;
  g.N = w->n;
  g.K = w->k;
  g.col_scales = w->mode == RH_MODE_W8 ? w->d_scales : nullptr;
  g.bias = bias;
  g.C = dst;
  g.ldc = ldc;
  g.act = act;
  if (w->mode == RH_MODE_W8) {
    const double bytes = M * K * 4 + K * N + M * N * 4 + 4 * N + (bias ? 4 * N : 0);
    e = ctx->prof_begin(1, ops, bytes, &slot);
    if (e == hipSuccess) e = launch_gemm_w8(g, ctx->w8_terms, s);
  } else {
    const double bytes = M * K * 4 + K * N * 4 + M * N * 4 + (bias ? 4 * N : 0);
    e = ctx->prof_begin(2, ops, bytes, &slot);
    if (e == hipSuccess) e = launch_gemm_f32(g, ctx->f32_algo, s);
  }
  if (e == hipSuccess) e = ctx->prof_end(slot);
  if (e != hipSuccess) return hip_fail(e, "gemm launch", __FILE__, __LINE__);
  return RH_OK;
}

}  // namespace rh

// ---- scratch of the allocation-free linear -------------------------------------
// rh_linear_noalloc stages its activations (u8 rows and row scales, or bf16
// planes) in this file-scope device array instead of a workspace it would
// have to allocate. Every GPU the library runs on holds its own copy for the
// life of the process. In host code the array's name is not a device
// address: each device's address is looked up once, with that device
// current, when the first context on it is created, and only that address
// is handed to kernels.
static __device__ __align__(256) uint8_t scratch[RH_NOALLOC_SCRATCH_BYTES];

namespace rh {
constexpr int kMaxScratchDevices = 64;
static void* g_scratch_addr[kMaxScratchDevices] = {};
static std::mutex g_scratch_mu;

// Resolve this device's copy of `scratch` (the device is current).
static int resolve_scratch(int device) {
  if (device >= kMaxScratchDevices)
    return fail(RH_ERR_INVALID, "device index beyond the scratch address table");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_addr[device]) return RH_OK;
  void* addr = nullptr;
  RH_HIP(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)));
  if (!addr) return fail(RH_ERR_HIP, "hipGetSymbolAddress returned a null scratch address");
  g_scratch_addr[device] = addr;
  return RH_OK;
}

static void* scratch_addr(int device) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  return device >= 0 && device < kMaxScratchDevices ? g_scratch_addr[device] : nullptr;
}
}  // namespace rh

using namespace rh;

// ---- C ABI ---------------------------------------------------------------------

#define CTX_GUARD(ctx)                                               \
  if (!(ctx)) return fail(RH_ERR_INVALID, "null context");           \
  std::lock_guard<std::mutex> lk_((ctx)->mu);                         \
  RH_HIP(hipSetDevice((ctx)->device))

extern "C" {

const char* rh_last_error(void) { return g_err; }

int rh_version(void) { return 300; }

int rh_device_count(int* count) {
  if (!count) return fail(RH_ERR_INVALID, "null count");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) {
    *count = 0;
    return fail(RH_ERR_NO_DEVICE, "no HIP device available");
  }
  *count = n;
  return RH_OK;
}

int rh_context_create(int device, rh_context** out) {
  return api_call([&]() -> int {
    if (!out) return fail(RH_ERR_INVALID, "null out");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
      return fail(RH_ERR_NO_DEVICE, "no HIP device available");
    if (device < 0 || device >= n) return fail(RH_ERR_INVALID, "device index out of range");
    RH_HIP(hipSetDevice(device));
    if (int st = resolve_scratch(device)) return st;
    auto* c = new rh_context();
    c->device = device;
    hipError_t e = hipStreamCreate(&c->stream);
    if (e != hipSuccess) {
      delete c;
      return hip_fail(e, "hipStreamCreate", __FILE__, __LINE__);
    }
    *out = c;
    return RH_OK;
  });
}

void rh_context_destroy(rh_context* ctx) {
  api_void([&] {
    if (!ctx) return;
    ctx_release(ctx);
  });
}

int rh_context_sync(rh_context* ctx) {
  return api_call([&]() -> int {
    CTX_GUARD(ctx);
    RH_HIP(hipStreamSynchronize(ctx->stream));
    return RH_OK;
  });
}

void* rh_context_stream(rh_context* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int rh_context_set_option(rh_context* ctx, int option, int value) {
  return api_call([&]() -> int {
    if (!ctx) return fail(RH_ERR_INVALID, "null context");
    std::lock_guard<std::mutex> lk(ctx->mu);
    ctx->generation++;
    switch (option) {
      case RH_CTX_F32_ALGO:
        if (value != F32_SPLIT3 && value != F32_NATIVE) return fail(RH_ERR_INVALID, "unknown fp32 algo");
        ctx->f32_algo = value;
        return RH_OK;
      case RH_CTX_W8_TERMS:
        if (value != 1 && value != 2) return fail(RH_ERR_INVALID, "w8 terms must be 1 or 2");
        ctx->w8_terms = value;
        return RH_OK;
      case RH_CTX_BF_ALGO:
        if (value < 0 || value > 1) return fail(RH_ERR_INVALID, "bf_algo must be 0 or 1");
        ctx->bf_algo = value;
        return RH_OK;
      case RH_CTX_TILE_GROUP:
        if (value < 1 || value > 64) return fail(RH_ERR_INVALID, "tile group must be 1..64");
        ctx->tile_group = value;
        return RH_OK;
      case RH_CTX_BF_TILE:
        if (value < 0 || value > kPlanesTileConfigs) return fail(RH_ERR_INVALID, "unknown planes tile");
        ctx->bf_tile = value;
        return RH_OK;
      case RH_CTX_I8_TILE:
        if (value < 0 || value > kI8TileConfigs) return fail(RH_ERR_INVALID, "unknown int8 tile");
        ctx->i8_tile = value;
        return RH_OK;
      default:
        return fail(RH_ERR_INVALID, "unknown context option");
    }
  });
}

int rh_malloc(rh_context* ctx, size_t bytes, void** dev) {
  return api_call([&]() -> int {
    if (!dev) return fail(RH_ERR_INVALID, "null out");
    CTX_GUARD(ctx);
    RH_HIP(hipMalloc(dev, bytes ? bytes : 1));
    return RH_OK;
  });
}

int rh_free(rh_context* ctx, void* dev) {
  return api_call([&]() -> int {
    CTX_GUARD(ctx);
    RH_HIP(hipStreamSynchronize(ctx->stream));
    RH_HIP(hipFree(dev));
    return RH_OK;
  });
}

int rh_memcpy_h2d(rh_context* ctx, void* dst, const void* src, size_t bytes) {
  return api_call([&]() -> int {
    CTX_GUARD(ctx);
    RH_HIP(hipStreamSynchronize(ctx->stream));
    RH_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return RH_OK;
  });
}

int rh_memcpy_d2h(rh_context* ctx, void* dst, const void* src, size_t bytes) {
  return api_call([&]() -> int {
    CTX_GUARD(ctx);
    RH_HIP(hipStreamSynchronize(ctx->stream));
    RH_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return RH_OK;
  });
}

int rh_profile_enable(rh_context* ctx, int on) {
  return api_call([&]() -> int {
    CTX_GUARD(ctx);
    RH_HIP(hipStreamSynchronize(ctx->stream));
    ctx->prof_clear();
    ctx->profiling = on != 0;
    return RH_OK;
  });
}

int rh_profile_read(rh_context* ctx, int kind, rh_profile_stat* out) {
  return api_call([&]() -> int {
    if (!out) return fail(RH_ERR_INVALID, "null out");
    CTX_GUARD(ctx);
    RH_HIP(hipStreamSynchronize(ctx->stream));
    rh_profile_stat st{};
    for (auto& r : ctx->recs) {
      if (r.kind != kind) continue;
      float ms = 0.0f;
      RH_HIP(hipEventElapsedTime(&ms, r.a, r.b));
      st.launches++;
      st.total_ms += ms;
      st.total_ops += r.ops;
      st.total_bytes += r.bytes;
    }
    *out = st;
    return RH_OK;
  });
}

int rh_attention_planes(rh_context* ctx, const void* qkv_hi, const void* qkv_lo, int ldqkv,
                        int q_off, int k_off, int v_off, const int32_t* cu, int batch,
                        int max_len, int heads, int kv_heads, int dh, float scale, int causal,
                        int window, float* out, int ldout) {
  return api_call([&]() -> int {
    if (!qkv_hi || !qkv_lo || !cu || !out) return fail(RH_ERR_INVALID, "null argument");
    if (dh != 32 && dh != 64 && dh != 128)
      return fail(RH_ERR_SHAPE, "planes attention head dim must be 32, 64 or 128");
    if (heads < 1 || kv_heads < 1 || heads % kv_heads)
      return fail(RH_ERR_SHAPE, "heads must be a positive multiple of kv_heads");
    if (batch < 0 || max_len < 0 || window < 0) return fail(RH_ERR_INVALID, "negative size");
    if (ldqkv % 8 || q_off % 8 || k_off % 8 || v_off % 8 || ldout % 4 || q_off < 0 ||
        k_off < 0 || v_off < 0 || ((uintptr_t)qkv_hi & 15) || ((uintptr_t)qkv_lo & 15) ||
        ((uintptr_t)out & 15))
      return fail(RH_ERR_SHAPE, "attention rows and offsets must be 16-byte aligned");
    CTX_GUARD(ctx);
    AttnArgs a{};
    a.qkv = qkv_hi;
    a.qkv_lo = qkv_lo;
    a.in_bf16 = 2;
    a.ldqkv = ldqkv;
    a.q_off = q_off;
    a.k_off = k_off;
    a.v_off = v_off;
    a.cu = cu;
    a.batch = batch;
    a.max_len = max_len;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.dh = dh;
    a.scale = scale;
    a.ctx = out;
    a.ldctx = ldout;
    a.causal = causal ? 1 : 0;
    a.window = window;
    int slot = -1;
    RH_HIP(ctx->prof_begin(3, 0.0, 0.0, &slot));
    RH_HIP(launch_attention(a, 3, ctx->stream));
    RH_HIP(ctx->prof_end(slot));
    return RH_OK;
  });
}

int rh_attention(rh_context* ctx, const void* qkv, int in_bf16, int ldqkv, int q_off,
                 int k_off, int v_off, const int32_t* cu, int batch, int max_len, int heads,
                 int kv_heads, int dh, float scale, int causal, int window, int precision,
                 float* out, int ldout) {
  return api_call([&]() -> int {
    if (!qkv || !cu || !out) return fail(RH_ERR_INVALID, "null argument");
    if (dh != 32 && dh != 64 && dh != 128 && dh != 256)
      return fail(RH_ERR_SHAPE, "attention head dim must be 32, 64, 128 or 256");
    if (heads < 1 || kv_heads < 1 || heads % kv_heads)
      return fail(RH_ERR_SHAPE, "heads must be a positive multiple of kv_heads");
    if (precision != 1 && precision != 3 && precision != 4)
      return fail(RH_ERR_INVALID, "precision must be 1, 3 or 4");
    if (in_bf16 && precision != 1) return fail(RH_ERR_INVALID, "bf16 input takes precision 1");
    if (precision == 4 && (causal || window || heads != kv_heads || dh == 256))
      return fail(RH_ERR_INVALID,
                  "reference-order attention: no mask, heads == kv_heads, dh 32, 64 or 128");
    if (batch < 0 || max_len < 0 || window < 0) return fail(RH_ERR_INVALID, "negative size");
    if (ldqkv % 8 || q_off % 8 || k_off % 8 || v_off % 8 || ldout % 4 || q_off < 0 ||
        k_off < 0 || v_off < 0 || ((uintptr_t)qkv & 15) || ((uintptr_t)out & 15))
      return fail(RH_ERR_SHAPE, "attention rows and offsets must be 16-byte aligned");
    CTX_GUARD(ctx);
    AttnArgs a{};
    a.qkv = qkv;
    a.in_bf16 = in_bf16 ? 1 : 0;
    a.ldqkv = ldqkv;
    a.q_off = q_off;
    a.k_off = k_off;
    a.v_off = v_off;
    a.cu = cu;
    a.batch = batch;
    a.max_len = max_len;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.dh = dh;
    a.scale = scale;
    a.ctx = out;
    a.ldctx = ldout;
    a.causal = causal ? 1 : 0;
    a.window = window;
    int slot = -1;
    RH_HIP(ctx->prof_begin(3, 0.0, 0.0, &slot));
    if (precision == 4) RH_HIP(launch_attention_exact(a, ctx->stream));
    else RH_HIP(launch_attention(a, precision, ctx->stream));
    RH_HIP(ctx->prof_end(slot));
    return RH_OK;
  });
}

int rh_pack_weight_gated(rh_context* ctx, int mode, const float* gate,
                                    const float* up, int k, int i, rh_weight** out) {
  return api_call([&]() -> int {
    if (!out || !gate || !up) return fail(RH_ERR_INVALID, "null argument");
    if (mode < RH_MODE_F32 || mode > RH_MODE_A8W8) return fail(RH_ERR_INVALID, "unknown mode");
    CTX_GUARD(ctx);
    return pack_weight_gated(ctx, mode, gate, up, k, i, out);
  });
}

int rh_pack_weight(rh_context* ctx, int mode, const float* bT, const float* bias,
                   int k, int n, rh_weight** out) {
  return api_call([&]() -> int {
    if (!out || !bT) return fail(RH_ERR_INVALID, "null argument");
    if (mode < RH_MODE_F32 || mode > RH_MODE_A8W8) return fail(RH_ERR_INVALID, "unknown mode");
    CTX_GUARD(ctx);
    return pack_weight(ctx, mode, bT, bias, k, n, out);
  });
}

void rh_weight_destroy(rh_weight* w) {
  api_void([&] {
    if (!w) return;
    Context* ctx = w->ctx;
    {
      std::lock_guard<std::mutex> lk(ctx->mu);
      (void)hipSetDevice(ctx->device);
      (void)hipStreamSynchronize(ctx->stream);
      destroy_weight(w);
    }
    ctx_release(ctx);
  });
}

int rh_weight_info(const rh_weight* w, int* mode, int* k, int* n) {
  return api_call([&]() -> int {
    if (!w) return fail(RH_ERR_INVALID, "null weight");
    if (mode) *mode = w->mode;
    if (k) *k = w->k;
    if (n) *n = w->n;
    return RH_OK;
  });
}

int rh_weight_export(const rh_weight* w, int8_t* q, float* scales, int32_t* colsum) {
  return api_call([&]() -> int {
    if (!w) return fail(RH_ERR_INVALID, "null weight");
    Context* ctx = w->ctx;
    CTX_GUARD(ctx);
    RH_HIP(hipStreamSynchronize(ctx->stream));
    if (q) {
      if (w->mode == RH_MODE_F32) return fail(RH_ERR_INVALID, "fp32 weight has no int8 image");
      std::vector<int8_t> img((size_t)w->np * w->kp);
      RH_HIP(hipMemcpy(img.data(), w->d_data, img.size(), hipMemcpyDeviceToHost));
      for (int j = 0; j < w->n; j++)
        memcpy(q + (size_t)j * w->k, img.data() + (size_t)j * w->kp, w->k);
    }
    if (scales) {
      if (!w->d_scales) return fail(RH_ERR_INVALID, "weight has no scales");
      RH_HIP(hipMemcpy(scales, w->d_scales, w->n * sizeof(float), hipMemcpyDeviceToHost));
    }
    if (colsum) {
      if (!w->d_colsum) return fail(RH_ERR_INVALID, "weight has no colsum");
      RH_HIP(hipMemcpy(colsum, w->d_colsum, w->n * sizeof(int32_t), hipMemcpyDeviceToHost));
    }
    return RH_OK;
  });
}

int rh_quantize_rows_u8(rh_context* ctx, const float* a, int m, int k, uint8_t* qa,
                        int ldq, float* row_scales) {
  return api_call([&]() -> int {
    if (m < 0 || k < 1) return fail(RH_ERR_INVALID, "bad m/k");
    if (ldq < k || ldq % 16 != 0) return fail(RH_ERR_INVALID, "ldq must be >= k and a multiple of 16");
    if (m > 0 && (!a || !qa || !row_scales)) return fail(RH_ERR_INVALID, "null argument");
    CTX_GUARD(ctx);
    RH_HIP(launch_quantize_rows_u8(a, k, m, k, qa, ldq, row_scales, ctx->stream));
    return RH_OK;
  });
}

int rh_gelu_quantize_rows_u8(rh_context* ctx, const float* a, int m, int k, uint8_t* qa,
                             int ldq, float* row_scales) {
  return api_call([&]() -> int {
    if (m < 0 || k < 8 || k % 8 != 0) return fail(RH_ERR_INVALID, "k must be a positive multiple of 8");
    if (ldq < k || ldq % 16 != 0) return fail(RH_ERR_INVALID, "ldq must be >= k and a multiple of 16");
    if (m > 0 && (!a || !qa || !row_scales)) return fail(RH_ERR_INVALID, "null argument");
    CTX_GUARD(ctx);
    RH_HIP(launch_quantize_rows_u8(a, k, m, k, qa, ldq, row_scales, ctx->stream, ACT_GELU));
    return RH_OK;
  });
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// A weight is used only on the context that packed it: its device copy lives
// on that context's device, and the context's mutex orders its use against
// rh_weight_destroy.
static int check_owner(const rh_context* ctx, const rh_weight* w) {
  if (!ctx) return fail(RH_ERR_INVALID, "null context");
  if (!w) return fail(RH_ERR_INVALID, "null weight");
  if (w->ctx != ctx) return fail(RH_ERR_INVALID, "weight belongs to another context");
  return RH_OK;
}

static int check_gemm(const rh_context* ctx, const rh_weight* w, int mode, const float* a,
                      const void* dst, int m) {
  if (int st = check_owner(ctx, w)) return st;
  if (mode >= 0 && w->mode != mode) return fail(RH_ERR_INVALID, "weight packed for another mode");
  if (mode >= 0 && w->glu) return fail(RH_ERR_INVALID, "gated weight: use rh_linear with a gated act");
  if (m < 0) return fail(RH_ERR_INVALID, "negative m");
  if (m > 0 && (!a || !dst)) return fail(RH_ERR_INVALID, "null argument");
  // the int8 epilogue writes 16-byte vectors
  if (w->mode == RH_MODE_A8W8 && !aligned16(dst))
    return fail(RH_ERR_INVALID, "output must be 16-byte aligned");
  return RH_OK;
}

// MatMulFunc / Default (tensor.go:16-70): dst[m x n] = a[m x k] · bTᵀ with raw
// fp32 weights bT [n][k] (no pack). Both operands are split into bf16 hi/lo
// planes in the context workspace for this call (B padded to 256 rows, zero
// past n and past k) and multiplied as the packed fp32 path does (three
// bf16 products). The fp32 epilogue stores 4 columns at a time, so an odd
// n or an unaligned dst goes through the workspace and a 2-D copy.
int rh_matmul(rh_context* ctx, float* dst, const float* a, const float* bT, int m, int k,
              int n) {
  return api_call([&]() -> int {
    if (m < 0 || k < 1 || n < 1) return fail(RH_ERR_SHAPE, "bad shape (m >= 0, k >= 1, n >= 1)");
    if (m > 0 && (!dst || !a || !bT)) return fail(RH_ERR_INVALID, "null argument");
    CTX_GUARD(ctx);
    if (m == 0) return RH_OK;
    const int ldk = (int)round_up(k, 64), np = (int)round_up(n, kWeightRowPad);
    const bool direct = n % 4 == 0 && aligned16(dst);
    const int ldc = direct ? n : (int)round_up(n, 4);
    if ((long long)std::max(m, np) * std::max(ldk, ldc) >= (1LL << 30))
      return fail(RH_ERR_SHAPE, "matrix too large for one call");
    const size_t ap = (size_t)m * ldk * 2, bp = (size_t)np * ldk * 2;
    const size_t cbytes = direct ? 0 : (size_t)m * ldc * 4;
    hipError_t e = ctx->ensure_ws(2 * ap + 2 * bp + cbytes);
    if (e != hipSuccess) return hip_fail(e, "matmul workspace", __FILE__, __LINE__);
    uint8_t* ws = static_cast<uint8_t*>(ctx->ws);
    __bf16* ah = reinterpret_cast<__bf16*>(ws);
    __bf16* al = reinterpret_cast<__bf16*>(ws + ap);
    __bf16* bh = reinterpret_cast<__bf16*>(ws + 2 * ap);
    __bf16* bl = reinterpret_cast<__bf16*>(ws + 2 * ap + bp);
    float* ct = direct ? dst : reinterpret_cast<float*>(ws + 2 * ap + 2 * bp);
    hipStream_t s = ctx->stream;
    RH_HIP(launch_split_bf16(a, k, m, k, ah, al, ldk, s));
    RH_HIP(launch_split_bf16(bT, k, n, k, bh, bl, ldk, s));
    if (np > n) {  // zero rows n..np of both B planes (rows are ldk*2 bytes)
      const int words = (np - n) * ldk / 2;
      RH_HIP(launch_fill_zero(reinterpret_cast<float*>(bh + (size_t)n * ldk), words, s));
      RH_HIP(launch_fill_zero(reinterpret_cast<float*>(bl + (size_t)n * ldk), words, s));
    }
    GemmPlArgs g{};
    g.Ah = ah;
    g.Al = al;
    g.lda = ldk;
    g.Bh = bh;
    g.Bl = bl;
    g.ldb = ldk;
    g.M = m;
    g.N = n;
    g.K = k;
    g.C = ct;
    g.ldc = ldc;
    g.act = ACT_NONE;
    g.tile_group = ctx->tile_group;
    int slot = -1;
    const double M = m, K = k, N = n;
    RH_HIP(ctx->prof_begin(2, 2.0 * M * K * N, 4.0 * (M * K + N * K + M * N), &slot));
    RH_HIP(launch_gemm_planes(g, 2, 2, ctx->bf_tile, s));
    RH_HIP(ctx->prof_end(slot));
    if (!direct)
      RH_HIP(hipMemcpy2DAsync(dst, (size_t)n * 4, ct, (size_t)ldc * 4, (size_t)n * 4, m,
                              hipMemcpyDeviceToDevice, s));
    return RH_OK;
  });
}

int rh_matmul_packed(rh_context* ctx, float* dst, const float* a, const rh_weight* w, int m) {
  return api_call([&]() -> int {
    int st = check_gemm(ctx, w, RH_MODE_F32, a, dst, m);
    if (st) return st;
    CTX_GUARD(ctx);
    return run_linear(ctx, w, a, w->k, m, dst, w->n, ACT_NONE, nullptr, nullptr, 0,
                      nullptr, false);
  });
}

int rh_matmul_packed8(rh_context* ctx, float* dst, const float* a, const rh_weight* w, int m) {
  return api_call([&]() -> int {
    int st = check_gemm(ctx, w, RH_MODE_W8, a, dst, m);
    if (st) return st;
    CTX_GUARD(ctx);
    return run_linear(ctx, w, a, w->k, m, dst, w->n, ACT_NONE, nullptr, nullptr, 0,
                      nullptr, false);
  });
}

int rh_matmul_packed_vnni(rh_context* ctx, float* dst, const float* a, const rh_weight* w,
                          int m, uint8_t* qa, int ldq, float* row_scales) {
  return api_call([&]() -> int {
    int st = check_gemm(ctx, w, RH_MODE_A8W8, a, dst, m);
    if (st) return st;
    if (m > 0 && (!qa || !row_scales)) return fail(RH_ERR_INVALID, "null scratch");
    if (ldq < w->k || ldq % 16 != 0)
      return fail(RH_ERR_INVALID, "ldq must be >= k and a multiple of 16");
    CTX_GUARD(ctx);
    return run_linear(ctx, w, a, w->k, m, dst, w->n, ACT_NONE, nullptr, qa, ldq,
                      row_scales, true);
  });
}

int rh_gemm_u8s8_i32(rh_context* ctx, int32_t* acc, const uint8_t* qa, int ldq,
                     const rh_weight* w, int m) {
  return api_call([&]() -> int {
    if (int st = check_owner(ctx, w)) return st;
    if (w->mode != RH_MODE_A8W8) return fail(RH_ERR_INVALID, "weight packed for another mode");
    if (m < 0) return fail(RH_ERR_INVALID, "negative m");
    if (m > 0 && (!acc || !qa)) return fail(RH_ERR_INVALID, "null argument");
    if (ldq < w->k || ldq % 16 != 0)
      return fail(RH_ERR_INVALID, "ldq must be >= k and a multiple of 16");
    if (!aligned16(acc) || !aligned16(qa)) return fail(RH_ERR_INVALID, "buffers must be 16-byte aligned");
    CTX_GUARD(ctx);
    return run_gemm_i8(ctx, w, qa, ldq, nullptr, m, EPI_ACC, acc, w->n, ACT_NONE, nullptr,
                       nullptr, nullptr, 2.0 * m * w->k * w->n);
  });
}

int rh_linear(rh_context* ctx, float* dst, const float* a, const rh_weight* w, int m,
              int act, uint8_t* qa, int ldq, float* row_scales) {
  return api_call([&]() -> int {
    int st = check_gemm(ctx, w, -1, a, dst, m);
    if (st) return st;
    if (act < RH_ACT_NONE || act > RH_ACT_GEGLU_ERF) return fail(RH_ERR_INVALID, "unknown act");
    if (w->glu != is_glu(act))
      return fail(RH_ERR_INVALID, "gated acts need a gated weight and vice versa");
    if (w->mode == RH_MODE_A8W8) {
      if (m > 0 && (!qa || !row_scales)) return fail(RH_ERR_INVALID, "null scratch");
      if (ldq < w->k || ldq % 16 != 0)
        return fail(RH_ERR_INVALID, "ldq must be >= k and a multiple of 16");
    }
    CTX_GUARD(ctx);
    return run_linear(ctx, w, a, w->k, m, dst, w->glu ? w->n / 2 : w->n, act, w->d_bias, qa,
                      ldq, row_scales, true);
  });
}

int rh_linear_u8(rh_context* ctx, const uint8_t* qa, int ldq, const float* row_scales,
                 const rh_weight* w, int m, int act, uint8_t* qa_out, int ldq_out,
                 float* rs_out, float* absmax_scratch) {
  return api_call([&]() -> int {
    if (int st = check_owner(ctx, w)) return st;
    if (w->mode != RH_MODE_A8W8) return fail(RH_ERR_INVALID, "weight must be RH_MODE_A8W8");
    if (m < 0) return fail(RH_ERR_INVALID, "negative m");
    // the re-quantizing epilogue has no gate/up pairing: gated weights go
    // through rh_linear (fp32 act(gate)*up rows) and rh_quantize_rows_u8
    if (w->glu || is_glu(act))
      return fail(RH_ERR_INVALID, "rh_linear_u8 takes no gated weight or gated act");
    if (act != RH_ACT_NONE && act != RH_ACT_GELU) return fail(RH_ERR_INVALID, "unknown act");
    if (m > 0 && (!qa || !row_scales || !qa_out || !rs_out || !absmax_scratch))
      return fail(RH_ERR_INVALID, "null argument");
    if (ldq < w->k || ldq % 16 != 0)
      return fail(RH_ERR_INVALID, "ldq must be >= k and a multiple of 16");
    if (ldq_out < w->n || ldq_out % 16 != 0)
      return fail(RH_ERR_INVALID, "ldq_out must be >= n and a multiple of 16");
    if (!aligned16(qa) || !aligned16(qa_out)) return fail(RH_ERR_INVALID, "buffers must be 16-byte aligned");
    CTX_GUARD(ctx);
    if (m == 0) return RH_OK;
    RH_HIP(launch_fill_zero(absmax_scratch, m, ctx->stream));
    int st = run_gemm_i8(ctx, w, qa, ldq, row_scales, m, EPI_ABSMAX, nullptr, 0, act, w->d_bias,
                         absmax_scratch, nullptr, 2.0 * m * w->k * w->n);
    if (st) return st;
    return run_gemm_i8(ctx, w, qa, ldq, row_scales, m, EPI_QUANT, qa_out, ldq_out, act,
                       w->d_bias, absmax_scratch, rs_out, 0.0);
  });
}

// Scratch bytes rh_linear_noalloc stages for m rows through w (256-byte
// aligned pieces): full int8 u8 rows [m][ldq] and row scales [m]; the bf16
// planes GEMM one or two planes [m][round_up(k, 64)]; the other weight-only
// int8 / fp32 algorithms read the fp32 rows directly and stage nothing.
static size_t noalloc_bytes(const rh_context* ctx, const rh_weight* w, int m) {
  if (w->mode == RH_MODE_A8W8)
    return round_up((size_t)m * round_up(w->k, 16), 256) + (size_t)m * 4;
  if (linear_on_planes(ctx, w))
    return round_up((size_t)m * round_up(w->k, 64) * 2, 256) * linear_a_terms(ctx, w);
  return 0;
}

int rh_linear_noalloc(rh_context* ctx, float* dst, const float* a, const rh_weight* w, int m,
                      int act) {
  return api_call([&]() -> int {
    int st = check_gemm(ctx, w, -1, a, dst, m);
    if (st) return st;
    if (act < RH_ACT_NONE || act > RH_ACT_GEGLU_ERF) return fail(RH_ERR_INVALID, "unknown act");
    if (w->glu != is_glu(act))
      return fail(RH_ERR_INVALID, "gated acts need a gated weight and vice versa");
    CTX_GUARD(ctx);
    if (m == 0) return RH_OK;
    const size_t need = noalloc_bytes(ctx, w, m);
    if (need > (size_t)RH_NOALLOC_SCRATCH_BYTES) {
      char buf[200];
      snprintf(buf, sizeof buf,
               "rh_linear_noalloc: %d rows of k=%d need %zu scratch bytes, the maximum is %zu",
               m, w->k, need, (size_t)RH_NOALLOC_SCRATCH_BYTES);
      return fail(RH_ERR_INVALID, buf);
    }
    uint8_t* base = static_cast<uint8_t*>(scratch_addr(ctx->device));
    if (!base) return fail(RH_ERR_INVALID, "scratch address of the device was not resolved");
    // per-launch event timing creates events: off for this call
    struct ProfOff {
      rh_context* c;
      bool was;
      ~ProfOff() { c->profiling = was; }
    } prof_off{ctx, ctx->profiling};
    ctx->profiling = false;
    const int ldc = w->glu ? w->n / 2 : w->n;
    if (w->mode == RH_MODE_A8W8) {
      const int ldq = (int)round_up(w->k, 16);
      uint8_t* qa = base;
      float* rs = reinterpret_cast<float*>(base + round_up((size_t)m * ldq, 256));
      return run_linear(ctx, w, a, w->k, m, dst, ldc, act, w->d_bias, qa, ldq, rs, true);
    }
    if (linear_on_planes(ctx, w)) {
      const int ldk = (int)round_up(w->k, 64);
      const size_t plane = round_up((size_t)m * ldk * 2, 256);
      Planes pin;
      pin.hi = reinterpret_cast<__bf16*>(base);
      pin.lo = linear_a_terms(ctx, w) == 2 ? reinterpret_cast<__bf16*>(base + plane) : nullptr;
      pin.ld = ldk;
      RH_HIP(launch_split_bf16(a, w->k, m, w->k, pin.hi, pin.lo, ldk, ctx->stream));
      return run_linear(ctx, w, a, w->k, m, dst, ldc, act, w->d_bias, nullptr, 0, nullptr,
                        false, &pin);
    }
    return run_linear(ctx, w, a, w->k, m, dst, ldc, act, w->d_bias, nullptr, 0, nullptr, false);
  });
}

int rh_gelu(rh_context* ctx, float* x, size_t n) {
  return api_call([&]() -> int {
    if (n > 0 && !x) return fail(RH_ERR_INVALID, "null x");
    CTX_GUARD(ctx);
    RH_HIP(launch_gelu(x, n, ctx->stream));
    return RH_OK;
  });
}

int rh_layernorm(rh_context* ctx, float* x, const float* gamma, const float* beta, int m,
                 int n, float eps) {
  return api_call([&]() -> int {
    if (m < 0 || n < 1 || n > 2048) return fail(RH_ERR_INVALID, "bad shape (n <= 2048)");
    if (m > 0 && (!x || !gamma || !beta)) return fail(RH_ERR_INVALID, "null argument");
    CTX_GUARD(ctx);
    // the reference's column-order sums where the row layout allows
    // (every model width); wave-parallel sums otherwise
    const bool exact = n % 4 == 0 && n <= 1024 &&
                       (((uintptr_t)x | (uintptr_t)gamma | (uintptr_t)beta) & 15) == 0;
    RH_HIP(launch_add_layernorm(x, nullptr, 0, gamma, beta, m, n, eps, nullptr, 0, nullptr,
                                ctx->stream, nullptr, nullptr, 0, exact));
    return RH_OK;
  });
}

}  // extern "C"
