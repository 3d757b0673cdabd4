/*
 * rembed_hip.h — C ABI of the MI355X (gfx950) GEMM backend for rembed.
 *
 * Drop-in boundary for rembed's internal/tensor matmul family and the
 * encoder forward that calls it. Every entry point is plain C: opaque
 * handles, plain pointers and sizes, an int status (RH_OK == 0) and a
 * thread-local message from rh_last_error(). No entry point aborts the host:
 * no C++ exception crosses the ABI (a failed host allocation returns
 * RH_ERR_OOM, any other internal exception RH_ERR_INVALID).
 *
 * Pointer conventions
 *   "host"  — ordinary CPU memory, borrowed for the duration of the call.
 *   "dev"   — device memory from rh_malloc (or any HIP allocation on the
 *             context's device). Calls taking dev pointers are enqueued on
 *             the context's stream and return without waiting; call
 *             rh_context_sync before reading results back.
 *
 * Each declaration names the reference interface it replaces (file:line,
 * relative to the rembed source tree).
 */
#ifndef REMBED_HIP_H
#define REMBED_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------- */
#define RH_OK 0
#define RH_ERR_NO_DEVICE 1 /* no usable GPU: the host falls back to its CPU path */
#define RH_ERR_INVALID 2   /* contract violation (the reference panics on these) */
#define RH_ERR_SHAPE 3     /* PackB*: n%16 != 0, n < 16, k < 1 (pack.go:29-37) */
#define RH_ERR_NONFINITE 4 /* PackB8/PackB8VNNI: NaN/Inf weight (pack8.go:43-48) */
#define RH_ERR_HIP 5       /* HIP runtime failure */
#define RH_ERR_OOM 6       /* device allocation failed */
#define RH_ERR_VOCAB 7     /* token id out of vocab range (bert.go:797-800) */
#define RH_ERR_SEQ 8       /* empty or over-long sequence (bert.go:741-747) */
#define RH_ERR_MISSING 9   /* model tensor missing or misshapen (bert.go:345-360) */

/* Message for the last failing call on this thread ("" if none). */
const char *rh_last_error(void);
/* ABI version: major*10000 + minor*100 + patch. */
int rh_version(void);

/* ---- context ---------------------------------------------------------------
 * One context = one device + one HIP stream (default priority). A context
 * serializes the calls made on it; use one context per concurrent caller
 * (the reference's Model is safe for concurrent use, bert.go:54-56). */
typedef struct rh_context rh_context;

int rh_device_count(int *count);
int rh_context_create(int device, rh_context **out);
void rh_context_destroy(rh_context *ctx);
int rh_context_sync(rh_context *ctx);
/* The context's hipStream_t, for callers that time or order work around it. */
void *rh_context_stream(rh_context *ctx);
/* GEMM strategy switches of a context (kept so choices can be re-measured):
 *   RH_CTX_F32_ALGO  0 = three bf16 MFMA products (default), 1 = native f32
 *   RH_CTX_W8_TERMS  bf16 terms of the fp32 activations in the weight-only
 *                    int8 GEMM: 1 = bf16(a), the operand a bf16 MFMA takes
 *                    (default), 2 = bf16 hi + lo split (fp32-grade a)
 *   RH_CTX_I8_TILE   int8 GEMM tile: 0 = automatic, 1 = 256x256, 2 = 256x128,
 *                    3 = 128x128 (four stages), 4 = 256x128, 5 = 128x256
 *                    (three stages, two workgroups per CU), 6 = 256x256,
 *                    7 = 128x256 (eight waves), 8 = 256x256, 9 = 128x256
 *                    (eight waves, two 128-byte k stages), 10 = 128x256
 *                    (eight waves, three 128-byte k stages), 11-14 = 64x256
 *                    and 128x256 with B fragments loaded to registers (A8W8
 *                    weights), 15 = 256x256 on four 128x128 waves (a four-
 *                    or three-stage ring by ceil(K/64), else 9)
 *   RH_CTX_BF_ALGO   weight-only int8 / fp32 GEMMs: 0 = activations split
 *                    once into bf16 hi/lo planes and weights stored as bf16
 *                    planes (default), 1 = split inside the GEMM's main loop
 *   RH_CTX_BF_TILE   tile of the bf16-planes GEMM: 0 = automatic, 1 = 256x256,
 *                    2 = 256x128, 3 = 128x128, 4 = 256x256, 5 = 256x128
 *                    (eight waves), 6 = 256x256, 7 = 256x128 (eight waves,
 *                    128-byte k stages), 8 = 64x64, 9 = 128x64 (four waves),
 *                    10 = 128x256 (eight waves, three 64-byte k stages, two
 *                    workgroups per CU); 6, 7 and 10 for the one-term
 *                    weight-only int8 product only, the other products take 3
 *   RH_CTX_TILE_GROUP  GEMM tile order: consecutive workgroups walk this many
 *                    row blocks down a column block (1 = row-major; default 4) */
#define RH_CTX_F32_ALGO 1
#define RH_CTX_W8_TERMS 2
#define RH_CTX_I8_TILE 3
#define RH_CTX_BF_ALGO 4
#define RH_CTX_BF_TILE 5
#define RH_CTX_TILE_GROUP 6
int rh_context_set_option(rh_context *ctx, int option, int value);

/* Device memory helpers (the Go host has no other allocator for HBM). */
int rh_malloc(rh_context *ctx, size_t bytes, void **dev);
int rh_free(rh_context *ctx, void *dev);
int rh_memcpy_h2d(rh_context *ctx, void *dev_dst, const void *host_src, size_t bytes);
int rh_memcpy_d2h(rh_context *ctx, void *host_dst, const void *dev_src, size_t bytes);

/* Per-launch GEMM timing with HIP events on the context's stream.
 * kind: 0 = full-int8 GEMM, 1 = weight-only int8 GEMM, 2 = fp32 GEMM,
 * 3 = attention, 4 = bf16 split of GEMM activations (weight-only int8 and
 * fp32 GEMMs on bf16 planes), 5 = full-int8 GEMM with the GELU +
 * QuantizeRowU8 row pass in its epilogue (the one-pass FFN1; ops count the
 * GEMM only). Reading syncs the stream. */
typedef struct {
  int64_t launches;
  double total_ms;    /* sum of per-launch event durations */
  double total_ops;   /* algorithmic 2*M*K*N summed over launches */
  double total_bytes; /* algorithmic minimal HBM bytes summed over launches */
} rh_profile_stat;
int rh_profile_enable(rh_context *ctx, int on); /* also clears the tallies */
int rh_profile_read(rh_context *ctx, int kind, rh_profile_stat *out);

/* ---- attention (adjacent to the GEMMs; keeps activations on the device) -----
 * Softmax attention over a packed variable-length batch of fused q|k|v rows,
 * replacing the per-text, per-head loops of the model forwards: scores =
 * q·kᵀ·scale, row softmax, ctx = P·v (bert.go:853-902;
 * flashAttnCausalHead, qwen3.go:319-390; gemma3.go:318-356 with its
 * sliding window). Text b owns rows cu[b]..cu[b+1]-1 (cu: device int32
 * [batch+1]); max_len must be >= every text's length. qkv is [M][ldqkv] f32
 * (in_bf16 = 0) or bf16 (in_bf16 = 1); q head h starts at column
 * q_off + h*dh, its kv head h / (heads/kv_heads) at k_off / v_off.
 * causal: key j visible to query i only if j <= i; window > 0: only if
 * |i - j| < window. precision 1: bf16 MFMA operands; 3: hi/lo bf16 split,
 * fp32-grade (f32 input only); 4: the reference's own float32 order
 * (MatMulSerial's dot4 and remainder columns, Softmax with expNonPos;
 * tensor.go:284-330,389-428, dot_amd64.s:13-94), bit-identical to it (f32
 * input, no mask, heads == kv_heads, dh 32/64/128). out is f32 [M][ldout],
 * head h at h*dh.
 * dh in {32, 64, 128, 256}; ldqkv and the offsets multiples of 8, ldout of 4.
 * Enqueued on the context's stream. */
int rh_attention(rh_context *ctx, const void *qkv, int in_bf16, int ldqkv, int q_off,
                 int k_off, int v_off, const int32_t *cu, int batch, int max_len, int heads,
                 int kv_heads, int dh, float scale, int causal, int window, int precision,
                 float *out, int ldout);

/* rh_attention at fp32-grade precision with the q|k|v rows given as their
 * bf16 split: qkv_hi = bf16(x), qkv_lo = bf16(x - hi), both [M][ldqkv] bf16
 * (what the full-int8 q|k|v projection writes for this attention). Three
 * bf16 MFMA products per step (hi·hi + hi·lo + lo·hi), fp32 softmax and
 * accumulation; same masks and layout as rh_attention, dh 32/64/128.
 * Replaces: the per-text head loops of bert.go:853-902, qwen3.go:319-390,
 * gemma3.go:318-356, like rh_attention. */
int rh_attention_planes(rh_context *ctx, const void *qkv_hi, const void *qkv_lo, int ldqkv,
                        int q_off, int k_off, int v_off, const int32_t *cu, int batch,
                        int max_len, int heads, int kv_heads, int dh, float scale, int causal,
                        int window, float *out, int ldout);

/* ---- weights (tensor level) --------------------------------------------------
 * Quantize/pack on the host exactly as the reference does, then upload once
 * to HBM; the handle owns the device copy until rh_weight_destroy.
 *   mode RH_MODE_F32  replaces PackB       (internal/tensor/pack.go:25-50)
 *   mode RH_MODE_W8   replaces PackB8      (internal/tensor/pack8.go:25-76)
 *   mode RH_MODE_A8W8 replaces PackB8VNNI  (internal/tensor/pack_vnni.go:28-77)
 * bT is the HF [out=n][in=k] row-major matrix; bias (length n) may be NULL
 * and is applied by rh_linear only (newDense's bias, bert.go:263-278).
 * A weight is used only with the context that packed it: passing it to a
 * call on another context returns RH_ERR_INVALID. */
#define RH_MODE_F32 0
#define RH_MODE_W8 1
#define RH_MODE_A8W8 2
typedef struct rh_weight rh_weight;

int rh_pack_weight(rh_context *ctx, int mode, const float *bT, const float *bias,
                   int k, int n, rh_weight **out);
void rh_weight_destroy(rh_weight *w);
/* Gated-MLP weight (SwiGLU / GeGLU, qwen3.go:528-539, gemma3.go:363-374):
 * gate and up are each [i][k] (HF gate_proj / up_proj). They are quantized
 * per output channel exactly as two separate rh_pack_weight calls would, and
 * stored interleaved (4 gate rows, then the matching 4 up rows) so one GEMM
 * produces both halves and its epilogue writes act(gate) * up. Use it with
 * rh_linear and RH_ACT_SWIGLU / RH_ACT_GEGLU / RH_ACT_GEGLU_ERF; the output
 * has i columns. nomic's fc11 * silu(fc12) is gate = fc12, up = fc11 with
 * RH_ACT_SWIGLU (nomic.go:232-242); ModernBERT's gelu(Wi[:I]) * Wi[I:] is
 * gate = Wi[:I], up = Wi[I:] with RH_ACT_GEGLU_ERF (modernbert.go:292-301).
 * gate and up must each pass the packers' shape rule (i % 16 == 0, i >= 16,
 * k >= 1). No counterpart call in the reference, which runs two applyDense
 * calls and a loop. */
int rh_pack_weight_gated(rh_context *ctx, int mode, const float *gate, const float *up,
                         int k, int i, rh_weight **out);
/* Shape and mode of a packed weight. */
int rh_weight_info(const rh_weight *w, int *mode, int *k, int *n);
/* Host copies of the quantization results, for parity checks: q is
 * [n][k] row-major (RH_MODE_W8 / RH_MODE_A8W8), scales [n], colsum [n]
 * (RH_MODE_A8W8 only). Any output may be NULL. */
int rh_weight_export(const rh_weight *w, int8_t *q, float *scales, int32_t *colsum);

/* ---- activations and GEMMs (tensor level, dev pointers) ---------------------
 * QuantizeRowU8 over m rows (internal/tensor/pack_vnni.go:85-117, the row
 * loop of pack_vnni.go:129-140): qa is [m][ldq] bytes, ldq >= k and a
 * multiple of 16; bytes k..ldq-1 of each row are zeroed. a is [m][k]. */
int rh_quantize_rows_u8(rh_context *ctx, const float *a, int m, int k,
                        uint8_t *qa, int ldq, float *row_scales);
/* GELU then QuantizeRowU8: the full-int8 FFN's hand-over from the
 * intermediate dense to the output dense (internal/model/bert.go:910-916,
 * GELU as internal/tensor/gelu_amd64.s:37-123 computes it for whole 8-lane
 * groups). a is the pre-activation [m][k]; k a multiple of 8, qa and ldq as
 * above. a itself is not modified. */
int rh_gelu_quantize_rows_u8(rh_context *ctx, const float *a, int m, int k,
                             uint8_t *qa, int ldq, float *row_scales);

/* MatMulPacked (internal/tensor/pack.go:123-176): dst[m][n] = a[m][k]·Wᵀ. */
/* MatMulFunc / Default (tensor.go:16-70), the unpacked path: dst[m x n] =
 * a[m x k] · bTᵀ with raw fp32 weights bT [n][k] row-major (device
 * pointers; any m >= 0, k >= 1, n >= 1). Computed as the packed fp32 path
 * does, splitting both operands for this call. */
int rh_matmul(rh_context *ctx, float *dst, const float *a, const float *bT, int m, int k,
              int n);
int rh_matmul_packed(rh_context *ctx, float *dst, const float *a,
                     const rh_weight *w, int m);
/* MatMulPacked8 (internal/tensor/pack8.go:80-111). */
int rh_matmul_packed8(rh_context *ctx, float *dst, const float *a,
                      const rh_weight *w, int m);
/* MatMulPackedVNNI (internal/tensor/pack_vnni.go:124-176): quantizes a into
 * qa/row_scales (caller scratch, [m][ldq] and [m]) and writes
 * dst = float32(acc - 128·colSum)·rowScale·colScale. */
int rh_matmul_packed_vnni(rh_context *ctx, float *dst, const float *a,
                          const rh_weight *w, int m, uint8_t *qa, int ldq,
                          float *row_scales);
/* The int32 accumulators of gemm4x16vnni (internal/tensor/vnni_amd64.s:22-82)
 * over already-quantized rows: acc[m][n] = Σ_p u8(qa[i][p])·s8(q[j][p]),
 * wrapping. For bit-exact parity checks. */
int rh_gemm_u8s8_i32(rh_context *ctx, int32_t *acc, const uint8_t *qa, int ldq,
                     const rh_weight *w, int m);

/* applyDense (internal/model/bert.go:282-301) with the bias and activation
 * fused into the GEMM epilogue: dst = act(a·Wᵀ + bias). act: 0 none,
 * 1 erf-GELU (geluScalar, internal/tensor/tensor.go:508-538). For
 * RH_MODE_A8W8 the quantization scratch comes from qa/row_scales as in
 * rh_matmul_packed_vnni (both may be NULL for the other modes). */
#define RH_ACT_NONE 0
#define RH_ACT_GELU 1
#define RH_ACT_SWIGLU 2 /* silu(gate)*up, tensor.SiLU (tensor.go:477-481)       */
#define RH_ACT_GEGLU 3  /* gelu_tanh(gate)*up, tensor.GELUTanh (tensor.go:490-497) */
#define RH_ACT_GEGLU_ERF 4 /* gelu(gate)*up, erf-GELU as tensor.GELU (modernbert.go:292-301) */
int rh_linear(rh_context *ctx, float *dst, const float *a, const rh_weight *w,
              int m, int act, uint8_t *qa, int ldq, float *row_scales);

/* applyDense followed by QuantizeRowU8 of its output rows, for chaining
 * full-int8 linears (bert.go:910-916: FFN1, GELU, then FFN2's row
 * quantization) without an fp32 intermediate. Input rows are already
 * quantized (qa/row_scales as produced by rh_quantize_rows_u8); output rows
 * go to qa_out [m][ldq_out] (ldq_out >= n, multiple of 16) and rs_out [m].
 * absmax_scratch holds m floats of caller scratch. The weight must be
 * RH_MODE_A8W8 and not gated; act is RH_ACT_NONE or RH_ACT_GELU (a gated
 * weight or act returns RH_ERR_INVALID). Output bytes equal
 * QuantizeRowU8(act(a·Wᵀ + bias)) exactly. */
int rh_linear_u8(rh_context *ctx, const uint8_t *qa, int ldq, const float *row_scales,
                 const rh_weight *w, int m, int act, uint8_t *qa_out, int ldq_out,
                 float *rs_out, float *absmax_scratch);

/* rh_linear for callers that cannot allocate (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. It computes exactly what rh_linear computes, with the same
 * kernels, but stages its intermediate data (full int8: the u8 rows and row
 * scales; weight-only int8 / fp32: the bf16 planes of a) in a fixed device
 * array of RH_NOALLOC_SCRATCH_BYTES per GPU, held from library load until
 * the process ends, instead of caller scratch or a workspace it allocates.
 * It calls no hipMalloc/hipFree and times no launches. Sizes whose staging
 * exceeds the array (full int8: m*round_up(k,16) + 4m bytes; planes:
 * m*round_up(k,64)*2 bytes per plane) return RH_ERR_INVALID. Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (from
 * different contexts or threads) race and must be ordered by the caller. */
#define RH_NOALLOC_SCRATCH_BYTES (64u * 1024u * 1024u)
int rh_linear_noalloc(rh_context *ctx, float *dst, const float *a, const rh_weight *w,
                      int m, int act);

/* Elementwise entry points used by parity tests (dev pointers). */
int rh_gelu(rh_context *ctx, float *x, size_t n);          /* tensor.go:508-538 */
/* LayerNorm (tensor.go:433-452). Bit-identical to the reference (float32
 * sums in column order) for n % 4 == 0, n <= 1024 and 16-byte aligned
 * pointers; other shapes reduce across a wave (within float32 rounding). */
int rh_layernorm(rh_context *ctx, float *x, const float *gamma,
                 const float *beta, int m, int n, float eps);

/* ---- encoder model ------------------------------------------------------------
 * Replaces model.Load + Model.Forward/ForwardTokens + the Embed batch loop
 * (internal/model/bert.go:307-524,649-731; rembed.go:287-411) with one
 * device-resident forward over a packed variable-length batch. */
#define RH_ARCH_BERT 0   /* BERT / RoBERTa post-LN encoder (encoder.layer.N.* names) */
#define RH_ARCH_QWEN3 1  /* Qwen3 causal decoder embedder (qwen3.go:395-548) */
#define RH_ARCH_GEMMA3 2 /* EmbeddingGemma: Gemma 3 run bidirectionally (gemma3.go:206-384) */
#define RH_ARCH_NOMIC 3  /* nomic-embed (nomic_bert): post-LN, RoPE, SwiGLU, bias-free (nomic.go:113-250) */
#define RH_ARCH_MODERNBERT 4 /* ModernBERT: pre-LN, RoPE, global/local attention, GeGLU (modernbert.go:148-311) */
#define RH_ARCH_DISTILBERT 5 /* DistilBERT: the BERT flow on transformer.layer.N.* names, no token-type table (bert.go:399-470,491-493) */
#define RH_ARCH_MPNET 6      /* MPNet: the BERT flow on attention.attn.* names, no token-type table, a bucketed
                                relative-position bias added to the scaled scores (bert.go:123-150,439-452,495-503,816-830,876-890) */
#define RH_POOL_MEAN 0
#define RH_POOL_CLS 1
#define RH_POOL_LAST 2
/* Quantization requests, WithInt8 / WithInt8Activations (rembed.go:60-81,
 * 241-247). Per-matrix fallback as newDense (bert.go:263-278). */
#define RH_QUANT_NONE 0
#define RH_QUANT_WEIGHTS 1
#define RH_QUANT_FULL 2

typedef struct {
  int arch;
  int hidden;           /* H */
  int layers;
  int heads;
  int intermediate;     /* I */
  int vocab;
  int max_position;     /* rows of the position table */
  int position_offset;  /* Config.PositionOffset (config.go:84-89) */
  int type_vocab;       /* rows of token_type_embeddings (only row 0 used) */
  float layer_norm_eps; /* 0 means 1e-12 (config.go:228-230) */
  int pooling;          /* RH_POOL_* */
  int normalize;        /* L2-normalize pooled vectors */
  /* RoPE family (config.go:44-77); ignored for RH_ARCH_BERT. max_position
   * is the longest text (RoPE table rows); nomic and ModernBERT have no
   * kv head groups (kv_heads 0) and head_dim * heads == hidden. */
  int kv_heads;              /* NumKeyValueHeads (GQA); 0 = heads */
  int head_dim;              /* HeadDim; 0 = hidden / heads */
  double rope_theta;         /* Qwen3 / nomic RopeTheta; Gemma / ModernBERT GlobalRopeTheta */
  double rope_local_theta;   /* Gemma / ModernBERT LocalRopeTheta */
  int sliding_window;        /* Gemma: local layers attend where |i-j| < window;
                                ModernBERT: LocalAttention, |i-j| <= window / 2 */
  int sliding_pattern;       /* Gemma: layer l is global iff (l+1) % pattern == 0;
                                ModernBERT: GlobalAttnEveryNLayers, global iff l % n == 0 */
  int query_pre_attn_scalar; /* Gemma: scores scaled by 1/sqrt(scalar) */
  int dense_hidden;          /* Gemma Dense head width (2_Dense/3_Dense); 0 = none */
  int rel_buckets;           /* MPNet: relative_attention_num_buckets (32, config.go:219-221) */
  int reserved[7];           /* zero */
} rh_model_config;

typedef struct rh_model rh_model;

int rh_model_create(rh_context *ctx, const rh_model_config *cfg, int quant,
                    rh_model **out);
/* Hand one HF tensor (by its safetensors name, with or without the
 * "bert."/"roberta." prefix; decoders: embed_tokens.weight,
 * norm.weight, layers.N.*, with or without "model.", and Gemma's Dense head
 * as "2_Dense.linear.weight" / "3_Dense.linear.weight"; nomic:
 * embeddings.*, emb_ln.*, encoder.layers.N.*; ModernBERT: embeddings.*,
 * layers.N.*, final_norm.weight) to the model; data is copied. */
int rh_model_set_tensor(rh_model *m, const char *name, const float *host,
                        const int64_t *shape, int ndim);
/* Check every tensor is present, fuse Q|K|V (decoders: also gate|up into
 * one gated weight), quantize/pack and upload. */
int rh_model_finalize(rh_model *m);
/* A second handle on a finalized model's weights, bound to another context
 * on the same device. The weights stay in HBM once; each handle has its own
 * stream, workspace and lock, so calls on different handles run
 * concurrently (calls on one handle, or on handles sharing a context,
 * serialize). Options are copied from src and may then be set per handle
 * (not RH_OPT_FUSE_PROJECTIONS). Handles are destroyed in any order; the
 * weights go with the last. RH_ERR_INVALID for an unfinalized src or a
 * context on another device. Replaces: the reference Model's safety for
 * concurrent use with its weights held once (bert.go:52-56,
 * rembed.go:36-41), which a context-bound device model cannot give alone. */
int rh_model_share(rh_model *src, rh_context *ctx, rh_model **out);
void rh_model_destroy(rh_model *m);
/* Per-model switches. RH_OPT_ATTN_PRECISION: 1 = bf16 attention operands,
 * 3 = three-term bf16 split (fp32-grade; the default for RH_QUANT_NONE and,
 * in every mode, for the BERT family: RH_ARCH_BERT, RH_ARCH_DISTILBERT,
 * RH_ARCH_MPNET).
 * RH_OPT_FUSED_FFN1: full-int8 FFN1 + GELU + QuantizeRowU8 (bert.go:910-916).
 * 2 = one GEMM pass writes the u8 rows: its workgroups exchange each row's
 * |max| per row block (default; a bounded wait, and a wait that timed out
 * fails rh_model_embed / rh_model_embed_tokens and rh_model_check with
 * RH_ERR_HIP); 1 = two GEMM passes (row |max|, then the bytes); 0 = fp32
 * FFN1 rows, then GELU + QuantizeRowU8 as a separate pass. All give
 * identical bytes. RH_OPT_PRODUCER_PLANES: 1 = the
 * kernels that produce a weight-only int8 / fp32 GEMM's input (norms,
 * attention, the previous GEMM) write its bf16 hi/lo planes directly
 * (default), 0 = they write fp32 rows and each GEMM splits them; both give
 * identical values. RH_OPT_STREAMS: n = 1..4 (default 2): a batch runs as
 * up to n parts of whole texts (at least 2048 tokens each) on as many
 * streams, whose kernels overlap, when no GEMM of the model needs the
 * context's split workspace (full int8, or producer-written planes);
 * 1 = one stream. Every setting gives identical results.
 * RH_OPT_QK_EPILOGUE: 1 = a decoder's weight-only int8 q|k|v projection
 * applies QK-norm + RoPE in its GEMM epilogue and writes the bf16 rows
 * attention reads (where the shape allows; default: measured faster),
 * 0 = fp32 rows and a separate pass; both give identical results.
 * RH_OPT_FUSE_PROJECTIONS (set before rh_model_finalize): 1 = a decoder
 * layer's q, k, v (and gate, up) are packed as one weight where newDense
 * leaves all of them in one mode (default), 0 = always as separate weights,
 * as the reference packs them (qwen3.go:479-481,528-529); a group whose
 * matrices fall back to different modes is always separate. Identical
 * results either way.
 * RH_OPT_FUSED_LN: 1 = a BERT-family full-int8 attention-output or FFN2
 * projection whose output width is the hidden size (384, 768 or 1024)
 * finishes whole rows in its epilogue: residual add, LayerNorm and the next
 * int8 GEMM's u8 quantization in the same kernel, 0 = the linear writes
 * fp32 rows and a separate residual + LayerNorm pass follows (default:
 * measured faster); identical results.
 * RH_OPT_EXACT (BERT family): 1 = LayerNorm's mean and variance are float32
 * sums in column order (tensor.go:433-452) and attention runs in the
 * reference's float32 order on fp32 q|k|v rows (MatMulSerial/dot4,
 * Softmax; bert.go:853-902), so a full-int8 forward's activations, GEMM
 * inputs and vectors are byte-identical to the reference's; 0 = the
 * wave-parallel LayerNorm and the RH_OPT_ATTN_PRECISION attention (default).
 * The fused-LN epilogue is not used while it is set.
 * RH_OPT_GRAPH (BERT family): 1 = a forward's launches are recorded once
 * per batch shape (row offsets, ids and output buffers, model and context
 * settings) as a HIP graph and replayed on the next call with the same
 * shape; 0 = launched one by one. The graph holds kernels and stream
 * fork/join edges only (no memset or allocation); identical results. Used
 * where the forward needs no context split workspace and profiling is off. */
#define RH_OPT_ATTN_PRECISION 1
#define RH_OPT_FUSED_FFN1 2
#define RH_OPT_PRODUCER_PLANES 3
#define RH_OPT_STREAMS 4
#define RH_OPT_QK_EPILOGUE 5
#define RH_OPT_FUSE_PROJECTIONS 6
#define RH_OPT_FUSED_LN 7
#define RH_OPT_EXACT 8
#define RH_OPT_GRAPH 9
int rh_model_set_option(rh_model *m, int option, int value);
/* Model.Quantized / QuantizedActivations (bert.go:526-644). */
int rh_model_quantized(const rh_model *m);
int rh_model_quantized_activations(const rh_model *m);

/* Embed (rembed.go:287-332 + Forward bert.go:649-689): ids is [batch][stride]
 * host int64 as the reference's Forward takes them (bert.go:649), text b is
 * ids[b*stride .. b*stride+lens[b]); out is [batch][H] host. An id outside
 * [0, vocab) returns RH_ERR_VOCAB (bert.go:797-800); batch*stride must be
 * below 2^31. Synchronous: the call returns with out filled. */
int rh_model_embed(rh_model *m, const int64_t *ids, const int32_t *lens,
                   int batch, int stride, float *out);
/* EmbedTokens / ForwardTokens (rembed.go:370-411, bert.go:705-731): out is
 * [sum(lens)][H] host, texts concatenated in order. */
int rh_model_embed_tokens(rh_model *m, const int64_t *ids, const int32_t *lens,
                          int batch, int stride, float *out);
/* Device-resident variant: ids_dev [batch][stride] int32 and out_dev
 * [batch][H] in HBM, lens on the host; enqueued on the context stream (no
 * sync). Ids out of range are clamped and reported by the next
 * rh_model_check. */
int rh_model_embed_device(rh_model *m, const int32_t *ids_dev,
                          const int32_t *lens, int batch, int stride,
                          float *out_dev);
/* Sync and report a deferred device-side error (RH_ERR_VOCAB) of the
 * previous rh_model_embed_device calls. */
int rh_model_check(rh_model *m);

/* ---- tokenizer (host side: text -> the int64 ids rh_model_embed takes) ---- */
typedef struct rh_tokenizer rh_tokenizer;
/* tokenizer.New (tokenizer/tokenizer.go:39-72): a BERT WordPiece vocab, one
 * token per line, id = line number (a later duplicate line wins).
 * lower_case selects lowercasing + NFD accent stripping. cls_tok / sep_tok /
 * unk_tok name the framing tokens; NULL or "" selects "[CLS]" / "[SEP]" /
 * "[UNK]". RH_ERR_MISSING when one of them is not in the vocab,
 * RH_ERR_INVALID when the file cannot be read. */
int rh_tokenizer_wordpiece_load(const char *vocab_path, int lower_case, const char *cls_tok,
                                const char *sep_tok, const char *unk_tok, rh_tokenizer **out);
/* Byte-level BPE, bpe.New (tokenizer/bpe/bpe.go:104-157): RoBERTa / GPT-2's
 * vocab.json + merges.txt, GPT-2 pre-tokenizer, cls ... sep framing (the
 * three tokens must be in the vocab). RH_ERR_INVALID for an unreadable or
 * malformed file or a missing framing token. */
int rh_tokenizer_bpe_load(const char *vocab_json, const char *merges_txt, const char *cls_tok,
                          const char *sep_tok, const char *unk_tok, rh_tokenizer **out);
/* Byte-level BPE from a HuggingFace tokenizer.json: with qwen = 0,
 * NewFromTokenizerJSON (bpe.go:282-303, ModernBERT: NFC when declared, the
 * added tokens matched leftmost-longest before BPE with their lstrip /
 * rstrip whitespace rules, GPT-2 pre-tokenizer, cls ... sep); with
 * qwen = 1, NewQwenFromTokenizerJSON (bpe.go:305-324, Qwen3: the Qwen
 * pre-tokenizer and only a trailing eos, sep_tok; cls_tok and unk_tok may
 * be NULL). */
int rh_tokenizer_bpe_load_json(const char *tokenizer_json, int qwen, const char *cls_tok,
                               const char *sep_tok, const char *unk_tok, rh_tokenizer **out);
/* SentencePiece Unigram, sentencepiece.New (tokenizer/sentencepiece/
 * sentencepiece.go:47-103): an XLM-R-family sentencepiece.bpe.model (NMT-NFKC
 * charsmap normalizer, Viterbi over the normal pieces), ids in HF's fairseq
 * space (<s> 0, </s> 2, <unk> 3, pieces shifted by one). RH_ERR_INVALID for
 * an unreadable or malformed model or one with USER_DEFINED / UNUSED / BYTE
 * pieces. */
int rh_tokenizer_sentencepiece_load(const char *model_path, rh_tokenizer **out);
/* Normalize (sentencepiece.go:244), exposed for tests as the reference
 * exposes it: the NMT-NFKC text (U+2581 for spaces) of a SentencePiece
 * tokenizer, *n bytes into out; RH_ERR_SHAPE when capacity is short. */
int rh_tokenizer_sentencepiece_normalize(const rh_tokenizer *t, const char *text,
                                         size_t text_len, char *out, size_t capacity,
                                         size_t *n);
/* Gemma, gemma.New (tokenizer/gemma/gemma.go:58-111): a tokenizer.json with
 * a byte-fallback BPE ("<0xNN>" pieces), space -> U+2581, <bos> ... <eos>. */
int rh_tokenizer_gemma_load(const char *tokenizer_json, rh_tokenizer **out);
/* VocabSize (tokenizer.go:75, bpe.go:327, sentencepiece.go:109, gemma.go:114). */
int64_t rh_tokenizer_vocab_size(const rh_tokenizer *t);
/* Encode (tokenizer.go:198-216, bpe.go:648-742, sentencepiece.go:205-241,
 * gemma.go:235-254): the ids of one UTF-8 text (text_len bytes), framed, at
 * most max_len ids. WordPiece drops invalid UTF-8 and counts a max_len below
 * 2 as 2; the others read invalid bytes as U+FFFD and keep their framing
 * (two ids, or Qwen's eos alone) whatever max_len. *n receives the count; RH_ERR_SHAPE when it exceeds capacity
 * (nothing written). The attention mask of the reference is all ones over
 * the n ids. */
int rh_tokenizer_encode(const rh_tokenizer *t, const char *text, size_t text_len, int max_len,
                        int64_t *ids, int capacity, int *n);
/* Encode over a batch, in the layout rh_model_embed takes: ids is
 * [batch][max(max_len, 2)], each row padded with pad_id after its lens[b]
 * ids. No reference counterpart as one call (Embed encodes text by text,
 * rembed.go:287-332). */
int rh_tokenizer_encode_batch(const rh_tokenizer *t, const char *const *texts,
                              const size_t *text_lens, int batch, int max_len, int64_t pad_id,
                              int64_t *ids, int32_t *lens);
void rh_tokenizer_destroy(rh_tokenizer *t);

#ifdef __cplusplus
}
#endif
#endif /* REMBED_HIP_H */
