/*
 * oracle.h — CPU restatement of rembed's GEMM family and BERT forward pass.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library (rembed_amd/)
 * links, loads or calls this code: it is the reference that the parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP
 * path against. Each function cites the reference file:line it restates
 * (paths relative to the rembed source tree).
 *
 * Arithmetic discipline: compiled with -ffp-contract=off so only explicit
 * fmaf() fuses, matching Go on amd64 which never fuses scalar mul+add
 * (internal/tensor/tensor_test.go:126-131) while the packed GEMM assembly
 * uses explicit VFMADD231PS (internal/tensor/gemm_amd64.s:38-45).
 *
 * Pinning (what checks each function beyond retyping its formula):
 *   or_quantize_row_u8   known answers of TestQuantizeRowU8Rails
 *                        (internal/tensor/vnni_test.go:118-134) + rail inputs
 *   or_pack_b8_vnni /    vnniReference closed form (vnni_test.go:11-59)
 *   or_gemm_u8s8_i32     restated independently in tests, brute force int64
 *   or_pack_b8           |deq-w| <= maxAbs/254 (pack8_test.go:114-144),
 *                        zero-channel scale 1, NaN/Inf refusal
 *   or_matmul_f32/_w8    float64 reference within max(1e-5,1e-6*sqrt k)(1+|w|)
 *                        (pack_test.go:55-67), KAT {58,64,139,154}
 *   elementwise          KATs of tensor_test.go:154-268, float64 erf/tanh
 *   or_bert_*            composition pinned by source reading; invariants
 *                        (unit L2 norm, batch == single, mode agreement)
 *   or_dec_* / or_renc_* independent float64 numpy compositions of the
 *                        reference forwards, plus planted variants (operand
 *                        order, mask bounds, layer schedule) that must fail
 */
#ifndef REMBED_ORACLE_H
#define REMBED_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes (mirror the reference's error returns) */
#define OR_OK 0
#define OR_ERR_SHAPE 1
#define OR_ERR_NONFINITE 2
#define OR_ERR_VOCAB 3
#define OR_ERR_SEQ 4

/* ---- weight quantizers ------------------------------------------------ */
/* PackB8 (internal/tensor/pack8.go:25-76). q is [n][k] row-major. */
int or_pack_b8(const float *bT, int k, int n, int8_t *q, float *scales);
/* PackB8VNNI (internal/tensor/pack_vnni.go:28-77). q is [n][k] row-major. */
int or_pack_b8_vnni(const float *bT, int k, int n, int8_t *q, int32_t *colsum,
                    float *scales);

/* QuantizeRowU8 (internal/tensor/pack_vnni.go:85-117): dst holds dstlen >= k
 * bytes, bytes k..dstlen-1 are zeroed; returns the row scale. */
float or_quantize_row_u8(uint8_t *dst, int dstlen, const float *a, int k);

/* ---- the three GEMMs (dst[m][n] = a[m][k] . bT^T) ---------------------- */
/* MatMulPacked: one sequential fmaf chain per element, ascending k
 * (internal/tensor/pack.go:123-210, gemm_amd64.s:31-49). */
void or_matmul_f32(float *dst, const float *a, const float *bT, int m, int k,
                   int n);
/* MatMulPacked8: fmaf chain over float(q), then *scale
 * (internal/tensor/pack8.go:80-126, gemm8_amd64.s:32-64). */
void or_matmul_w8(float *dst, const float *a, const int8_t *q,
                  const float *scales, int m, int k, int n);
/* VPDPBUSD accumulators: acc[i][j] = sum_p u8(qa[i][p]) * s8(q[j][p]),
 * int32 wrapping (internal/tensor/vnni_amd64.s:22-82). qa row stride lda. */
void or_gemm_u8s8_i32(int32_t *acc, const uint8_t *qa, int lda,
                      const int8_t *q, int m, int k, int n);
/* MatMulPackedVNNI (internal/tensor/pack_vnni.go:124-176): quantize rows,
 * accumulate, epilogue (acc - 128*colSum)*rs*scale. qa_out ([m][k]),
 * rs_out ([m]) and acc_out ([m][n]) may be NULL. */
void or_matmul_vnni(float *dst, const float *a, const int8_t *q,
                    const int32_t *colsum, const float *scales, int m, int k,
                    int n, uint8_t *qa_out, float *rs_out, int32_t *acc_out);

/* ---- elementwise (internal/tensor/tensor.go:372-554, fastmath.go) ------ */
float or_expf32(float x);  /* fastmath.go:26-55 */
float or_erff32(float x);  /* fastmath.go:69-82 */
void or_add_bias(float *x, const float *bias, int m, int n);
void or_add(float *dst, const float *src, int n);
void or_softmax(float *x, int m, int n);
void or_layernorm(float *x, const float *g, const float *b, int m, int n,
                  float eps);
void or_rmsnorm(float *x, const float *g, int m, int n, float eps);
void or_gelu(float *x, int n);      /* geluScalar, tensor.go:508-538 */
float or_gelu_avx2_lane(float v);   /* geluAVX2 lane, gelu_amd64.s:37-123 */
void or_gelu_ref(float *x, int n);  /* GELU on amd64, gelu_amd64.go:16-26 */
void or_gelu_tanh(float *x, int n); /* tensor.go:490-497 */
void or_silu(float *x, int n);      /* tensor.go:477-481 */
void or_l2normalize(float *x, int n);
/* dot4 (internal/tensor/dot_amd64.s:13-94): 8-lane FMA body, fold, FMA
 * tail into lane 0, two horizontal adds. */
void or_dot4(float *dst, const float *a, const float *b0, const float *b1,
             const float *b2, const float *b3, int k);
/* MatMulSerial with the SIMD body (tensor.go:284-330). */
void or_matmul_serial(float *dst, const float *a, const float *bT, int m,
                      int k, int n);

/* ---- BERT-family encoder (internal/model/bert.go) ----------------------- */
#define OR_QUANT_NONE 0
#define OR_QUANT_WEIGHTS 1
#define OR_QUANT_FULL 2
#define OR_POOL_MEAN 0
#define OR_POOL_CLS 1
#define OR_POOL_LAST 2

typedef struct {
  int vocab, hidden, layers, heads, inter, max_pos, type_vocab;
  float eps;
  int pooling;   /* OR_POOL_* */
  int normalize; /* L2-normalize the pooled vector */
  int pos_off;   /* Config.PositionOffset (config.go:84-89): position row of
                    token i is i + pos_off; texts up to max_pos - pos_off */
  int rel_buckets; /* MPNet: buckets of the relative-position bias (0: none) */
} or_bert_config;

/* Per-layer tensor order inside `layer_tensors` (16 per layer, HF layouts):
 * q_w[H][H] q_b k_w k_b v_w v_b o_w[H][H] o_b ln1_g ln1_b
 * f1_w[I][H] f1_b f2_w[H][I] f2_b ln2_g ln2_b */
#define OR_BERT_TENSORS_PER_LAYER 16

typedef struct or_bert_model or_bert_model;

/* Load: fuse Q|K|V and pack/quantize every dense once (bert.go:307-524,
 * newDense bert.go:263-278). Weight pointers are borrowed for the model's
 * lifetime (embedding tables, norms and biases are not copied). */
or_bert_model *or_bert_create(const or_bert_config *cfg, int quant,
                              const float *word_emb, const float *pos_emb,
                              const float *type_emb, const float *emb_ln_g,
                              const float *emb_ln_b,
                              const float *const *layer_tensors);
void or_bert_free(or_bert_model *m);
/* MPNet's shared relative-position bias table [rel_buckets][heads]
 * (encoder.relative_attention_bias.weight, bert.go:511-519), borrowed. */
void or_bert_set_rel_bias(or_bert_model *m, const float *table);
/* relPosBucket (bert.go:123-150): the bias bucket of relative position
 * rel = j - i (HF's relative_position_bucket, max distance 128). */
int or_rel_pos_bucket(int rel, int num_buckets);

/* encodeWorkers (bert.go:740-923): one unpadded forward over seq ids,
 * writing the final hidden states [seq][H]. */
int or_bert_encode(const or_bert_model *m, const int32_t *ids, int seq,
                   float *hidden);
/* ...stopped after the first `layers` layers (0 <= layers <= cfg.layers). */
int or_bert_encode_layers(const or_bert_model *m, const int32_t *ids, int seq,
                          float *x, int layers);
/* Forward (bert.go:649-703): encode, pool, optional L2. out is [H]. */
int or_bert_forward(const or_bert_model *m, const int32_t *ids, int seq,
                    float *out);
/* Embed batch policy (rembed.go:309-330): one serial forward per text,
 * fanned out across texts on `threads` OS threads. ids is [batch][stride],
 * text b uses ids[b*stride .. b*stride+lens[b]). out is [batch][H]. */
int or_bert_embed_batch(const or_bert_model *m, const int32_t *ids,
                        const int32_t *lens, int batch, int stride,
                        float *out, int threads);
/* ...with each text's forward timed into secs[batch] (wall seconds). */
int or_bert_embed_batch_timed(const or_bert_model *m, const int32_t *ids,
                        const int32_t *lens, int batch, int stride,
                        float *out, int threads,
                        double *secs);

/* ---- decoder-family embedders (internal/model/qwen3.go, gemma3.go) ---- */
#define OR_ARCH_QWEN3 1
#define OR_ARCH_GEMMA3 2
typedef struct {
  int arch; /* OR_ARCH_* */
  int vocab, hidden, layers, heads, kv_heads, head_dim, inter;
  float eps;
  double rope_theta;         /* Qwen3 RopeTheta; Gemma GlobalRopeTheta */
  double rope_local_theta;   /* Gemma LocalRopeTheta */
  int sliding_window;        /* Gemma: local layers keep |i-j| < window */
  int sliding_pattern;       /* Gemma: layer l is global iff (l+1) % pattern == 0 */
  int query_pre_attn_scalar; /* Gemma: scores scaled by 1/sqrt(scalar) */
  int dense_hidden;          /* Gemma Dense head width (0: none) */
  int pooling, normalize;
  int max_seq;
} or_dec_config;

/* Per-layer tensors, HF layouts ([out][in] for projections):
 * Qwen3 (11):  input_layernorm q_proj k_proj v_proj o_proj q_norm k_norm
 *              post_attention_layernorm gate_proj up_proj down_proj
 * Gemma3 (13): input_layernorm q_proj k_proj v_proj o_proj q_norm k_norm
 *              post_attention_layernorm pre_feedforward_layernorm
 *              post_feedforward_layernorm gate_proj up_proj down_proj
 * Gemma norm weights are the checkpoint's (unit offset added at load). */
#define OR_QWEN3_TENSORS_PER_LAYER 11
#define OR_GEMMA3_TENSORS_PER_LAYER 13

typedef struct or_dec_model or_dec_model;
or_dec_model *or_dec_create(const or_dec_config *cfg, int quant,
                            const float *embed, const float *final_norm,
                            const float *const *layer_tensors,
                            const float *dense1, const float *dense2);
void or_dec_free(or_dec_model *m);
/* 0 fp32, 1 weight-only int8, 2 full int8: the mode layer 0's q_proj took */
int or_dec_quantized_kind(const or_dec_model *m);
int or_dec_encode(const or_dec_model *m, const int32_t *ids, int seq, float *x);
int or_dec_forward(const or_dec_model *m, const int32_t *ids, int seq, float *out);
int or_dec_embed_batch(const or_dec_model *m, const int32_t *ids,
                       const int32_t *lens, int batch, int stride, float *out,
                       int threads);
/* ...with each text's forward timed into secs[batch] (wall seconds). */
int or_dec_embed_batch_timed(const or_dec_model *m, const int32_t *ids,
                       const int32_t *lens, int batch, int stride, float *out,
                       int threads,
                        double *secs);

/* ---- bias-free RoPE encoders (internal/model/nomic.go, modernbert.go) ---- */
#define OR_ARCH_NOMIC 3
#define OR_ARCH_MODERNBERT 4
typedef struct {
  int arch; /* OR_ARCH_NOMIC / OR_ARCH_MODERNBERT */
  int vocab, hidden, layers, heads, inter;
  float eps;
  double rope_theta;       /* nomic RopeTheta; ModernBERT GlobalRopeTheta */
  double rope_local_theta; /* ModernBERT LocalRopeTheta */
  int local_attention;     /* ModernBERT: local layers keep |i-j| <= local_attention/2 */
  int global_every;        /* ModernBERT: layer l is global iff l % global_every == 0 */
  int pooling, normalize;
  int max_seq;
} or_renc_config;

/* Per-layer tensors, HF layouts ([out][in] for projections):
 * nomic (9):      attn.Wqkv attn.out_proj norm1.weight norm1.bias mlp.fc11
 *                 mlp.fc12 mlp.fc2 norm2.weight norm2.bias
 * ModernBERT (6): attn_norm (NULL for layer 0) attn.Wqkv attn.Wo mlp_norm
 *                 mlp.Wi [2I][H] mlp.Wo
 * Model tensors: embed (word / tok embeddings), nomic's token-type table
 * (row 0 used) and emb_ln weight/bias, ModernBERT's embeddings.norm (emb_g)
 * and final_norm; the others NULL. */
#define OR_NOMIC_TENSORS_PER_LAYER 9
#define OR_MODERNBERT_TENSORS_PER_LAYER 6

typedef struct or_renc_model or_renc_model;
or_renc_model *or_renc_create(const or_renc_config *cfg, int quant, const float *embed,
                              const float *type_emb, const float *emb_g, const float *emb_b,
                              const float *final_norm, const float *const *layer_tensors);
void or_renc_free(or_renc_model *m);
/* 0 fp32, 1 weight-only int8, 2 full int8: the mode layer 0's Wqkv took */
int or_renc_quantized_kind(const or_renc_model *m);
int or_renc_encode(const or_renc_model *m, const int32_t *ids, int seq, float *x);
int or_renc_forward(const or_renc_model *m, const int32_t *ids, int seq, float *out);
int or_renc_embed_batch_timed(const or_renc_model *m, const int32_t *ids,
                              const int32_t *lens, int batch, int stride, float *out,
                              int threads, double *secs);

/* building blocks (exported for the unit tests) */
void or_rope_table(float *cos_t, float *sin_t, int seq, int dh, double theta);
void or_apply_rope(float *x, int seq, int dh, const float *cos_t, const float *sin_t);
void or_flash_causal_head(const float *qh, const float *kh, const float *vh,
                          float *out, int seq, int dh, float scale);

/* Which int8 dot-product body the oracle picked at run time (for reports):
 * 2 = AVX-512-VNNI intrinsics, 0 = portable C. Both produce identical
 * integers. */
int or_vnni_kind(void);
/* The reference's full-int8 kernel shape: PackB8VNNI's panel layout
 * (pack_vnni.go:44-72) and gemm4x16vnni / gemm4x16vnni512's 4x16 tiles
 * (vnni_amd64.s:22-82, vnni512_amd64.s:16-76) over qa rows of lda >=
 * kg*4 bytes; same integers as or_gemm_u8s8_i32. or_vnni_panel_kind: 1 VEX
 * AVX-VNNI, 2 EVEX AVX-512-VNNI, 0 portable. or_set_gemm_impl(1) makes the
 * models' full-int8 denses run this path (the CPU baseline), 0 the default. */
void or_pack_vnni_panels(const int8_t *q, int k, int n, int8_t *pb);
void or_gemm_u8s8_panels(int32_t *acc, const uint8_t *qa, int lda, const int8_t *pb, int m,
                         int k, int n);
int or_vnni_panel_kind(void);
void or_set_gemm_impl(int impl);

#ifdef __cplusplus
}
#endif
#endif
