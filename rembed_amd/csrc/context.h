// context.h — host-side objects behind the C ABI handles.
#pragma once

#include <atomic>
#include <mutex>
#include <vector>

#include "rh_internal.h"

// rh_context: one device, one stream (default priority), a mutex that
// serializes the calls made on it, GEMM strategy switches, and the optional
// per-launch event timing used by the benchmark.
struct rh_context {
  int device = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;
  // Weights and models created on the context hold a reference, so the
  // context (stream included) lives until rh_context_destroy has been called
  // AND every object created from it has been destroyed, in any order.
  std::atomic<int> refs{1};
  int f32_algo = rh::F32_SPLIT3;
  int w8_terms = 1;  // bf16 terms of the fp32 activations in weight-only int8
  int i8_tile = 0;   // 0 = automatic int8 GEMM tile choice
  int bf_algo = 0;   // W8/F32 GEMM: 0 = bf16 planes (pre-split), 1 = in-kernel split
  int bf_tile = 0;   // 0 = automatic bf16-planes GEMM tile choice
  int tile_group = 4;  // GEMM tile order: row blocks per group (1 = row-major)
  // bumped by every rh_context_set_option: forwards recorded as HIP graphs
  // under older settings are re-recorded
  int generation = 0;
  // grow-only device workspace (bf16 planes of the activations); the context
  // serializes its calls, so one buffer serves every GEMM on its stream
  void* ws = nullptr;
  size_t ws_bytes = 0;
  hipError_t ensure_ws(size_t bytes);

  struct ProfRec {
    hipEvent_t a, b;
    int kind;
    double ops, bytes;
  };
  bool profiling = false;
  std::vector<ProfRec> recs;

  hipError_t prof_begin(int kind, double ops, double bytes, int* slot);
  hipError_t prof_end(int slot);
  void prof_clear();
};

// rh_weight: a packed dense weight resident in HBM. d_data is [np][kp]
// (fp32 for RH_MODE_F32, int8 otherwise), zero outside the [n][k] corner.
struct rh_weight {
  rh_context* ctx = nullptr;
  int mode = 0;
  int k = 0, n = 0, kp = 0, np = 0;
  void* d_data = nullptr;
  float* d_scales = nullptr;
  int32_t* d_colsum = nullptr;
  float* d_bias = nullptr;
  // gated (SwiGLU/GeGLU) weight: n = 2 * i rows, gate and up interleaved in
  // groups of kGluGroup; rh_linear writes i = n / 2 output columns
  bool glu = false;
  // bf16 planes [np][kp] for the bf16-MFMA GEMMs: W8 holds the int8 values
  // (exact in bf16), F32 the hi/lo split of the fp32 weights
  void* d_bf = nullptr;
  void* d_bf_lo = nullptr;
  // A8W8: the s8 image again in v_mfma_i32_32x32x32_i8 B-fragment order
  // (kp % 128 == 0, np % 256 == 0): the 1 KiB for column block nb (32
  // columns) and k-step ks (32 bytes) sits at (nb * kp/32 + ks) * 1024, lane
  // l's 16 bytes (column nb*32 + l%32, k bytes ks*32 + (l/32)*16 ..) at l*16,
  // so a wave's fragment is one coalesced 16-byte load per lane
  void* d_frag = nullptr;
};

namespace rh {
using Context = rh_context;

void ctx_retain(Context* ctx);
void ctx_release(Context* ctx);  // frees the context on the last reference
// raw_ok: mode RH_MODE_F32 as newDense's last resort, the unpacked MatMulFunc
// weights (any k >= 1 and n % 4 == 0) rather than PackB's n % 16 rule.
int pack_weight(Context* ctx, int mode, const float* bT, const float* bias, int k,
                int n, rh_weight** out, bool raw_ok = false);
// The packers' refusal rules without packing: RH_OK when pack_weight(mode)
// would accept bT [n][k], else the status it would return (RH_ERR_SHAPE:
// PackB*'s n % 16 rule, or the unpacked rule with raw_ok; RH_ERR_NONFINITE:
// a NaN/Inf weight, pack8.go:43-48 / pack_vnni.go:48-56).
int pack_check(int mode, const float* bT, int k, int n, bool raw_ok = false);
void destroy_weight(rh_weight* w);
// gate/up [i][k] -> one interleaved [2i][k] weight (rows 8t..8t+3 = gate
// 4t..4t+3, rows 8t+4..8t+7 = up 4t..4t+3), packed in `mode`, glu = true
int pack_weight_gated(Context* ctx, int mode, const float* gate, const float* up, int k,
                      int i, rh_weight** out, bool raw_ok = false);
int quantize_b8(const float* bT, int k, int n, std::vector<int8_t>& q,
                std::vector<float>& scales);
int quantize_b8_vnni(const float* bT, int k, int n, std::vector<int8_t>& q,
                     std::vector<float>& scales, std::vector<int32_t>& colsum);
// bf16 planes of GEMM activations exchanged between producers and the
// planes GEMM: hi/lo [m][ld] (ld a multiple of 64 covering K, zero past K);
// lo may be null where the consumer takes one term.
struct Planes {
  __bf16* hi = nullptr;
  __bf16* lo = nullptr;
  int ld = 0;
};
// Does the linear of w run on bf16 planes in this context (weight-only int8
// or fp32, planes algorithm, not native-f32)? Then it can take its input as
// producer-written planes (`pin`) and write its output as planes (`pout`).
bool linear_on_planes(const Context* ctx, const rh_weight* w);
// Number of activation planes (1 or 2) the planes GEMM of w reads.
int linear_a_terms(const Context* ctx, const rh_weight* w);
int run_linear(Context* ctx, const rh_weight* w, const float* a, int lda, int m,
               float* dst, int ldc, int act, const float* bias, uint8_t* qa, int ldq,
               float* rs, bool quantize_first, const Planes* pin = nullptr,
               const Planes* pout = nullptr);
// QK-norm + RoPE applied in the epilogue of the decoders' q|k|v projection
// (GemmPlArgs::qk_*); pos is per row of the call.
struct QkEpilogue {
  const float *q_g, *k_g, *cos_t, *sin_t;
  const int32_t* pos;
  int nq, nkv, dh;
  float eps;
};
// The q|k|v linear of w on producer-written planes with the QK-norm + RoPE
// epilogue, bf16 rows to out [m][ldo]. *applied = false (nothing launched)
// when this form does not apply (another mode, a forced tile, a shape the
// fused tile does not cover): the caller then runs run_linear and the
// separate pass.
int run_linear_qk(Context* ctx, const rh_weight* w, const Planes& pin, int m,
                  const QkEpilogue& q, __bf16* out, int ldo, bool* applied);
int run_gemm_i8(Context* ctx, const rh_weight* w, const uint8_t* qa, int ldq,
                const float* rs, int m, int epi, void* out, int ldo, int act,
                const float* bias, float* row_absmax, float* rs_out, double ops,
                void* out_lo = nullptr, unsigned* sync = nullptr,
                unsigned* slots = nullptr, int slot_ld = 0, unsigned* sync_err = nullptr);
// run_gemm_i8 with the residual + LayerNorm finish (launch_gemm_i8_ln).
int run_gemm_i8_ln(Context* ctx, const rh_weight* w, const uint8_t* qa, int ldq,
                   const float* rs, int m, const I8LnArgs& f, double ops);
}  // namespace rh
