// rh_internal.h — shared definitions for the rembed HIP backend (gfx950).
//
// Everything here is device-agnostic plumbing: status handling, vector
// types for the CDNA4 MFMA builtins, and the kernel launch entry points
// that the C-ABI layer (capi.cpp) and the model runtime (model.cpp) call.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <exception>
#include <new>
#include <string>

#include "../../include/rembed_hip.h"

namespace rh {

// Per-launch timing without extra stream packets: the profiler parks a
// start/stop event pair here and the next timed launch on this thread hands
// them to hipExtLaunchKernel, which stamps them from the kernel's own
// dispatch. Untimed launches pass null events (a plain launch).
struct LaunchTiming {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
LaunchTiming& launch_timing();

template <typename F, typename... Args>
inline void timed_launch(F kernel, dim3 grid, dim3 block, uint32_t shmem, hipStream_t s,
                         Args... args) {
  LaunchTiming& t = launch_timing();
  const LaunchTiming use = t;
  t = LaunchTiming{};
  hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, use.start, use.stop, 0u, args...);
}

// ---- status ----------------------------------------------------------------
// A thread-local message backs rh_last_error(); every C entry point returns
// one of the RH_* codes and never aborts the host. The message lives in a
// fixed thread-local buffer, so recording it never allocates or throws.
void set_error(const char* msg) noexcept;
int fail(int code, const char* msg) noexcept;
inline int fail(int code, const std::string& msg) noexcept { return fail(code, msg.c_str()); }
int hip_fail(hipError_t e, const char* what, const char* file, int line) noexcept;

// Exception barrier of the C ABI: every extern "C" body runs inside it, so no
// C++ exception unwinds into the (cgo) caller. A failed host allocation
// becomes RH_ERR_OOM, any other exception RH_ERR_INVALID, with a message.
int fail_exception(int code, const char* what) noexcept;
template <class F>
inline int api_call(F&& body) noexcept {
  try {
    return body();
  } catch (const std::bad_alloc&) {
    return fail(RH_ERR_OOM, "host memory allocation failed");
  } catch (const std::exception& e) {
    return fail_exception(RH_ERR_INVALID, e.what());
  } catch (...) {
    return fail(RH_ERR_INVALID, "internal error: unknown exception");
  }
}
// The same for entry points without a status (destroy calls): an exception
// is recorded for rh_last_error() and dropped.
template <class F>
inline void api_void(F&& body) noexcept {
  (void)api_call([&]() -> int {
    body();
    return 0;
  });
}

#define RH_HIP(call)                                                   \
  do {                                                                 \
    hipError_t rh_e_ = (call);                                         \
    if (rh_e_ != hipSuccess)                                           \
      return ::rh::hip_fail(rh_e_, #call, __FILE__, __LINE__);         \
  } while (0)

#define RH_CHECK(cond, code, msg)                                      \
  do {                                                                 \
    if (!(cond)) return ::rh::fail((code), (msg));                     \
  } while (0)

// ---- MFMA operand types ----------------------------------------------------
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v8s __attribute__((ext_vector_type(8)));

inline size_t round_up(size_t x, size_t m) { return (x + m - 1) / m * m; }
inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Padding of packed weights in HBM: rows (output channels) to a multiple of
// the widest N tile, columns (k) to a multiple of the deepest K tile, so
// every tile load of B stays inside the allocation with zero padding.
constexpr int kWeightRowPad = 256;
constexpr int kWeightKPad = 128;

// ---- GEMM launch descriptors -------------------------------------------------
// act codes for the fused epilogue (reference applies these as separate
// passes after AddBias: internal/model/bert.go:913-915, qwen3.go:530-539).
// ACT_SWIGLU / ACT_GEGLU apply to a gated weight (rows of gate and up
// interleaved in groups of 4, see kGluGroup): the epilogue writes
// act(gate) * up into n/2 output columns (qwen3.go:530-539, gemma3.go:365-374).
enum Act : int { ACT_NONE = 0, ACT_GELU = 1, ACT_SWIGLU = 2, ACT_GEGLU = 3, ACT_GEGLU_ERF = 4 };
constexpr int kGluGroup = 4;  // packed rows 8t..8t+3 = gate 4t.., 8t+4..8t+7 = up 4t..
__host__ __device__ inline bool is_glu(int act) {
  return act == ACT_SWIGLU || act == ACT_GEGLU || act == ACT_GEGLU_ERF;
}

// Epilogue variants of the int8 GEMM. value = act(float32(real)·rs·cs + bias)
enum I8Epi : int {
  EPI_F32 = 0,     // out fp32 [M][ldo] = value
  EPI_BF16 = 1,    // out bf16 [M][ldo] = value rounded to nearest even
  EPI_ABSMAX = 2,  // no out: row_absmax[row] = max over the row of |value|
                   // (atomic max on the float bits; zero it beforehand)
  EPI_QUANT = 3,   // out u8 [M][ldo] = QuantizeRowU8(value row) using
                   // row_absmax from a preceding EPI_ABSMAX pass; rs_out[M]
  EPI_ACC = 4,     // out int32 [M][ldo] = reference-form accumulators
  EPI_PLANES = 5,  // out / out_lo bf16 [M][ldo]: hi = bf16(value), lo =
                   // bf16(value - hi), both rounded to nearest even
  EPI_QSYNC = 6    // EPI_QUANT in one pass: the workgroups of a row block
                   // exchange their row maxima through `slots`
};

struct GemmI8Args {
  const uint8_t* A;  // u8 activations (+128 offset, QuantizeRowU8 format) [M][lda]
  int lda;           // bytes, multiple of 16
  const int8_t* B;   // s8 weights [Np][ldb], zero padded
  int ldb;           // bytes, multiple of kWeightKPad
  const int8_t* Bf;  // the same weights in B-fragment order (rh_weight::d_frag)
  int M, N, K;
  const float* row_scales;  // [M]
  const float* col_scales;  // [N]
  const int32_t* colsum;    // [N]
  const float* bias;        // [N] or null
  void* out;                // per epi; rows 16-byte aligned
  void* out_lo;             // EPI_PLANES: the lo plane (same layout as out)
  int ldo;                  // elements, multiple of 4
  int act;
  int epi;
  float* row_absmax;        // EPI_ABSMAX target / EPI_QUANT input
  float* rs_out;            // EPI_QUANT row scales
  int tile_group;           // row blocks per group of the tile order (tile_origin)
  // EPI_QSYNC: departures per 128-row block (zero on entry and on exit),
  // row maxima slots [M][slot_ld] per column tile (kSlotEmpty on entry and
  // on exit), bit 0 of sync_err set if a row's wait timed out
  unsigned* sync;
  unsigned* slots;
  int slot_ld;
  unsigned* sync_err;
};

// B formats of the bf16-MFMA GEMM family.
enum BKind : int {
  BK_I8 = 0,     // int8 weights, dequantised to bf16 on the way into LDS
  BK_BF16X2 = 1  // fp32 weights stored as bf16 hi + bf16 lo planes
};

struct GemmBfArgs {
  const float* A;  // fp32 activations [M][lda]
  int lda;         // floats, multiple of 4
  const void* B;   // BK_I8: int8 [Np][ldb]; BK_BF16X2: bf16 hi plane [Np][ldb]
  const void* Blo; // BK_BF16X2: bf16 lo plane
  int ldb;         // elements
  int M, N, K;
  const float* col_scales;  // BK_I8: [N]; else null
  const float* bias;        // [N] or null
  float* C;
  int ldc;
  int act;
};

// The bf16-planes GEMM (W8 and F32 modes): activations and weights arrive
// as bf16 planes (hi, optional lo), so the main loop only moves and
// multiplies. Products: Ah.Bh + [BT=2] Ah.Bl + [AT=2] Al.Bh.
struct GemmPlArgs {
  const __bf16* Ah;
  const __bf16* Al;  // AT == 2
  int lda;           // elements, >= round_up(K, 64), zero past K
  const __bf16* Bh;
  const __bf16* Bl;  // BT == 2
  int ldb;           // elements (kp)
  int M, N, K;
  const float* col_scales;  // W8: [N]; else null
  const float* bias;
  int tile_group;  // row blocks per group of the tile order (tile_origin)
  float* C;     // fp32 output, or null when the output goes to bf16 planes:
  __bf16* Ch;   // hi = bf16(c), lo = bf16(c - hi) of the output (the next
  __bf16* Cl;   // GEMM's activation planes; Cl may be null)
  int ldc;      // elements, for C or Ch/Cl
  int act;
  // QK-norm + RoPE epilogue of the decoders' q|k|v projection (qwen3.go /
  // gemma3.go): bf16 rows to qk_out [M][ldc] instead of C; heads of qk_dh
  // columns, the first qk_nq RMS-normed by qk_qg, the next qk_nkv by qk_kg,
  // both rotated by the tables at each row's position qk_pos[row]; the rest
  // (v) converted only.
  const float* qk_qg = nullptr;
  const float* qk_kg = nullptr;
  const float* qk_cos = nullptr;
  const float* qk_sin = nullptr;
  const int32_t* qk_pos = nullptr;
  __bf16* qk_out = nullptr;
  int qk_nq = 0, qk_nkv = 0, qk_dh = 0;
  float qk_eps = 0.0f;
};

// The split hi/lo of one value; every producer of activation planes uses
// exactly this, so planes written by a producer equal launch_split_bf16's.
__device__ __forceinline__ void split_hi_lo(float x, __bf16& hi, __bf16& lo) {
  hi = (__bf16)x;
  lo = (__bf16)(x - (float)hi);
}
// Four consecutive values -> four hi and (if lo) four lo bf16, 8-byte stores.
__device__ __forceinline__ void store_planes4(__bf16* hi, __bf16* lo, size_t off, const v4f& v) {
  typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
  v4bf h, l;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    __bf16 a, b;
    split_hi_lo(v[e], a, b);
    h[e] = a;
    l[e] = b;
  }
  *reinterpret_cast<v4bf*>(hi + off) = h;
  if (lo) *reinterpret_cast<v4bf*>(lo + off) = l;
}
// a fp32 [M][lda_f] -> hi, lo bf16 [M][ldk] (ldk = round_up(K, 64), zeros
// past K): hi = bf16(x), lo = bf16(x - float(hi)), both rounded to nearest even
hipError_t launch_split_bf16(const float* a, int lda_f, int M, int K, __bf16* hi, __bf16* lo,
                             int ldk, hipStream_t s);
constexpr int kPlanesTileConfigs = 10;
hipError_t launch_gemm_planes(const GemmPlArgs& a, int a_terms, int b_terms, int tile,
                              hipStream_t s);
// The q|k|v projection with the QK-norm + RoPE epilogue (a.qk_out set): one
// activation term, int8 weights as one bf16 plane, 256x256 tiles of 8 waves
// on two 128-byte stages; needs N % 256 == 0 and qk_dh in {64, 128, 256}.
hipError_t launch_gemm_planes_qk(const GemmPlArgs& a, hipStream_t s);

// fp32 GEMM strategies (selected per model/context; both kept so the
// choice can be re-measured): three bf16 products or native f32 MFMA.
enum F32Algo : int { F32_SPLIT3 = 0, F32_NATIVE = 1 };

// Launchers (gemm_i8.hip, gemm_bf16.hip). Return hipError_t of the launch.
// tile: 0 = automatic, else one of the configurations RH_CTX_I8_TILE lists.
constexpr int kI8TileConfigs = 15;
// EPI_QSYNC: column tiles per row at most (N <= 16 x 256)
constexpr int kQsyncMaxTiles = 16;
hipError_t launch_gemm_i8(const GemmI8Args& a, int tile, hipStream_t s);
// The residual + LayerNorm finish of a full-int8 linear whose N is the
// hidden width (the attention output and FFN2 projections of the BERT
// family, bert.go:905-907,916-918): x = LayerNorm(x + dense(a)), and
// optionally QuantizeRowU8 of the result for the next int8 GEMM.
struct I8LnArgs {
  float* x;             // [M][N] residual stream, replaced by the LayerNorm output
  const float* gamma;   // [N]
  const float* beta;    // [N]
  float eps;
  uint8_t* qa;          // [M][ldq] u8 of the result, or null (may alias the GEMM's A)
  int ldq;
  float* row_scales;    // [M] (may alias the GEMM's row scales)
};
// Whole output rows per workgroup (BM = 64, N in {384, 768, 1024}; needs
// the fragment-ordered weight, epi EPI_F32 and no activation): the dequant
// epilogue's values go through the same float operations, in the same
// order, as the EPI_F32 GEMM followed by launch_add_layernorm, so both give
// identical bits. hipErrorInvalidValue for a shape it does not cover.
hipError_t launch_gemm_i8_ln(const GemmI8Args& a, const I8LnArgs& f, hipStream_t s);
bool gemm_i8_ln_supported(int n, int k);
int pick_i8_tile(int M, int N, int K, int epi);
// fills n floats with zero (graph-capture safe, unlike hipMemsetAsync)
hipError_t launch_fill_zero(float* x, int n, hipStream_t s);
// a_terms: 1 or 2 bf16 terms for the fp32 activations.
hipError_t launch_gemm_w8(const GemmBfArgs& a, int a_terms, hipStream_t s);
hipError_t launch_gemm_f32(const GemmBfArgs& a, int algo, hipStream_t s);

// ---- elementwise / norm / attention launchers (kernels_misc.hip, attention.hip)
// QuantizeRowU8 of each row, optionally of act(row) (ACT_NONE or ACT_GELU)
hipError_t launch_quantize_rows_u8(const float* a, int lda, int m, int k,
                                   uint8_t* qa, int ldq, float* row_scales,
                                   hipStream_t s, int act = ACT_NONE);
hipError_t launch_gelu(float* x, size_t n, hipStream_t s);
hipError_t launch_add_bias(float* x, const float* bias, int m, int n, int ldx,
                           hipStream_t s);

// BERT embeddings: x[t] = word[id] + pos[t - start + pos_off] + type0, then
// LayerNorm; optionally also quantizes x rows for the next full-int8 GEMM.
struct EmbedArgs {
  const int32_t* ids;      // padded [batch][stride]
  int stride;
  const int32_t* cu;       // [batch+1] packed row offsets
  int batch;
  const float* word;       // [vocab][H]
  const float* pos;        // [max_pos][H]
  const float* type0;      // [H] or null
  const float* gamma;
  const float* beta;
  int H, vocab, pos_off;
  float eps;
  float* x;                // [M][H]
  uint8_t* qa;             // optional [M][ldq]
  int ldq;
  float* row_scales;       // optional [M]
  int* err_flag;           // set to 1 on an out-of-range id
  __bf16* ph = nullptr;    // optional bf16 hi/lo planes [M][ldp] of the first
  __bf16* pl = nullptr;    // weight-only int8 / fp32 GEMM's input (pl may be
  int ldp = 0;             // null)
  bool exact = false;      // LayerNorm's sums in the reference's column order
};
hipError_t launch_embed_layernorm(const EmbedArgs& a, int total_rows,
                                  hipStream_t s);

// x = LayerNorm(x + y) (bert.go:906-907,917-918); optional u8 quantization
// of the result for the next full-int8 GEMM, or its bf16 hi/lo planes
// [m][ldp] (ldp % 64 == 0, >= H) for the next weight-only int8 / fp32 GEMM.
// exact: the mean and variance are float32 sums in column order, as
// tensor.go:433-452 takes them (H % 4 == 0, 16-byte aligned rows), so the
// result is bit-identical to the reference's; otherwise wave-parallel sums.
hipError_t launch_add_layernorm(float* x, const float* y, int ldy,
                                const float* gamma, const float* beta, int m,
                                int H, float eps, uint8_t* qa, int ldq,
                                float* row_scales, hipStream_t s, __bf16* ph = nullptr,
                                __bf16* pl = nullptr, int ldp = 0, bool exact = false);
// standalone LayerNorm (tests)
hipError_t launch_layernorm(float* x, const float* gamma, const float* beta,
                            int m, int H, float eps, hipStream_t s);

// pooling + optional L2 per text (bert.go:669-703, tensor.go:542-554)
hipError_t launch_pool(const float* x, int H, const int32_t* cu, int batch,
                       int pooling, int normalize, float* out, hipStream_t s);

// Multi-head attention over a packed varlen batch (bert.go:853-902 per
// text): q/k/v read from the fused QKV rows, ctx written [M][H].
struct AttnArgs {
  const void* qkv;   // [M][ldqkv] fp32 (in_bf16 0), bf16 (1), or the bf16 hi plane (2)
  const void* qkv_lo;  // in_bf16 2: the bf16 lo plane, hi + lo = the fp32 rows' split
  int in_bf16;
  int ldqkv;
  int q_off, k_off, v_off;  // column offsets of head 0
  const int32_t* cu;        // [batch+1]
  int batch;
  int max_len;
  int heads, kv_heads, dh;
  float scale;
  float* ctx;  // [M][ldctx] fp32, or null when the output goes to planes:
  __bf16* ctx_hi;  // bf16 hi / lo planes [M][ldctx] of the output (the next
  __bf16* ctx_lo;  // GEMM's activations; ctx_lo may be null)
  int ldctx;
  int causal;  // key j visible to query i only if j <= i (qwen3.go:307-390)
  int window;  // > 0: key j visible only if |i - j| < window (gemma3.go:339-347)
  // MPNet: score(i, j) = score*scale + rel_bias[h * (2 * rel_center + 1) +
  // (j - i) + rel_center] (bert.go:876-890), or null
  const float* rel_bias;
  int rel_center;
};
// precision: 1 = bf16 MFMA, 3 = three-term bf16 split (fp32-grade; with
// in_bf16 2 the split arrives as hi/lo planes and runs on the pipelined
// kernel, dh <= 128)
hipError_t launch_attention(const AttnArgs& a, int precision, hipStream_t s);
// The same attention in the reference's float32 operation order
// (MatMulSerial/dot4, Softmax; attention_exact.hip): bit-identical context
// rows. fp32 q|k|v, no causal or window mask, heads == kv_heads, dh 32/64/128.
hipError_t launch_attention_exact(const AttnArgs& a, hipStream_t s);

// ---- RoPE-family row kernels (kernels_dec.hip) ------------------------------
// Token embeddings only (positions enter through RoPE): x[r] = word[id] * scale
// (+ add_row when given: nomic's segment-0 row, nomic.go:165-175) (scale 1 for
// Qwen3, nomic and ModernBERT, float32(sqrt(H)) for Gemma, gemma3.go:262-275);
// pos[r] = the token's index in its text.
hipError_t launch_embed_gather(const int32_t* ids, int stride, const int32_t* cu,
                               int batch, const float* word, const float* add_row, int H,
                               int vocab, float scale, float* x, int32_t* pos, int* err_flag,
                               int total_rows, hipStream_t s);
// Residual + norm sandwich per row (RMSNorm tensor.go:459-471, LayerNorm
// tensor.go:430-452):
//   y' = post_g ? RMSNorm(y, post_g) : y;  if (y) x += y';
//   out = RMSNorm(x, pre_g), or LayerNorm(x, pre_g, ln_b) with layer_norm
//   (out may alias x); optional u8 quantization of out.
struct RmsArgs {
  float* x;              // [m][H] residual stream, updated in place when y
  const float* y;        // sublayer output to add, or null
  const float* post_g;   // RMSNorm weight applied to y first, or null
  const float* pre_g;    // RMSNorm weight of out
  float* out;            // [m][H] fp32 out (may alias x), or null
  __bf16* ph;            // bf16 hi / lo planes of out [m][ldp], or null
  __bf16* pl;            // (pl may be null: one-term consumer)
  int ldp;               // multiple of 64, >= H (the columns past H are not written)
  int m, H;
  float eps;
  uint8_t* qa;           // QuantizeRowU8 of out [m][ldq], or null
  int ldq;
  float* row_scales;
  int layer_norm;        // 0: RMSNorm (pre_g); 1: LayerNorm (pre_g, ln_b), post_g unused
  const float* ln_b;     // LayerNorm beta, or null for a zero beta
};
hipError_t launch_rms_residual(const RmsArgs& a, hipStream_t s);
// QK-norm (RMSNorm over each head's dh values; none when q_g and k_g are
// null) then rotate-half RoPE at the row's position, in place on fused q|k
// rows (qwen3.go:484-516; nomic.go:210-211, modernbert.go:256-257).
hipError_t launch_qk_norm_rope(float* qkv, int ldqkv, int m, int nq, int nkv, int dh,
                               const float* q_g, const float* k_g, float eps,
                               const float* cos_t, const float* sin_t,
                               const int32_t* pos, __bf16* outh, hipStream_t s);
// EmbeddingGemma Dense head (gemma3.go:174-198) on pooled [batch][H] rows:
// out = W2 . (W1 . pooled), float32 sequential sums; optional L2. The
// weights are given transposed: w1T [H][D], w2T [D][H]; hid is [batch][D].
hipError_t launch_dense_head(const float* pooled, int batch, int H, int D, const float* w1T,
                             const float* w2T, int normalize, float* hid, float* out,
                             hipStream_t s);
// out[i] = act(gate[i]) * up[i] over n floats (act a gated ACT_*): the
// gated-MLP glue for gate and up packed as separate weights.
hipError_t launch_glu_rows(const float* gate, const float* up, float* out, size_t n, int act,
                           hipStream_t s);
// L2Normalize (tensor.go:540-554) of `rows` rows of [H] in place: the
// float64 sum of squares in column order, as the reference takes it.
hipError_t launch_l2_rows(float* y, int rows, int H, hipStream_t s);

}  // namespace rh
