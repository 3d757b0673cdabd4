/*
 * oracle_renc.c — CPU restatement of rembed's bias-free RoPE encoders:
 * nomic-embed (nomic_bert: post-LayerNorm, RoPE, SwiGLU) and ModernBERT
 * (pre-LayerNorm, dual-theta RoPE, global / sliding-window attention,
 * erf-GELU GeGLU).
 *
 * TEST INFRASTRUCTURE ONLY (the parity reference, never the product); see oracle.h.
 * Every function cites the reference file:line it follows (paths relative
 * to the rembed source tree). Compiled with -ffp-contract=off, so a*b+c
 * rounds twice exactly as Go's float32 arithmetic does.
 */
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "oracle_int.h"

typedef struct {
  or_dense qkv, o, fc11, fc12, fc2; /* nomic; ModernBERT uses qkv, o, wi (fc11), wo (fc2) */
  const float *n1_g, *n1_b, *n2_g, *n2_b;
  const float *attn_norm, *mlp_norm; /* ModernBERT; attn_norm NULL on layer 0 */
  int global;
} or_renc_layer;

struct or_renc_model {
  or_renc_config cfg;
  int quant;
  const float *embed, *type0, *emb_g, *emb_b, *final_norm;
  float *zero_beta;
  or_renc_layer *layers;
};

/* loadNomic (internal/model/nomic.go:33-110) and loadModernBERT
 * (internal/model/modernbert.go:34-104): every projection through newDense,
 * no biases. Per-layer tensor order: see oracle.h. */
or_renc_model *or_renc_create(const or_renc_config *cfg, int quant, const float *embed,
                              const float *type_emb, const float *emb_g, const float *emb_b,
                              const float *final_norm, const float *const *lt) {
  int H = cfg->hidden, I = cfg->inter;
  int mb = cfg->arch == OR_ARCH_MODERNBERT;
  if (cfg->heads <= 0 || H % cfg->heads != 0 || (H / cfg->heads) % 2) return NULL;
  if (mb && (cfg->global_every < 1 || cfg->local_attention < 2)) return NULL;
  or_renc_model *m = (or_renc_model *)calloc(1, sizeof(*m));
  m->cfg = *cfg;
  m->quant = quant;
  m->embed = embed;
  m->type0 = type_emb;
  m->emb_g = emb_g;
  m->emb_b = emb_b;
  m->final_norm = final_norm;
  m->zero_beta = (float *)calloc((size_t)H, sizeof(float)); /* modernbert.go:67 */
  m->layers = (or_renc_layer *)calloc((size_t)cfg->layers, sizeof(or_renc_layer));
  int per = mb ? OR_MODERNBERT_TENSORS_PER_LAYER : OR_NOMIC_TENSORS_PER_LAYER;
  for (int l = 0; l < cfg->layers; l++) {
    const float *const *t = lt + (size_t)l * per;
    or_renc_layer *L = &m->layers[l];
    if (mb) {
      /* attn_norm Wqkv Wo mlp_norm Wi Wo(mlp) */
      L->attn_norm = l == 0 ? NULL : t[0];
      or__dense_init(&L->qkv, t[1], 0, NULL, 0, H, 3 * H, quant);
      or__dense_init(&L->o, t[2], 0, NULL, 0, H, H, quant);
      L->mlp_norm = t[3];
      or__dense_init(&L->fc11, t[4], 0, NULL, 0, H, 2 * I, quant); /* Wi */
      or__dense_init(&L->fc2, t[5], 0, NULL, 0, I, H, quant);
      L->global = l % cfg->global_every == 0; /* modernbert.go:73 */
    } else {
      /* Wqkv out_proj norm1.w norm1.b fc11 fc12 fc2 norm2.w norm2.b */
      or__dense_init(&L->qkv, t[0], 0, NULL, 0, H, 3 * H, quant);
      or__dense_init(&L->o, t[1], 0, NULL, 0, H, H, quant);
      L->n1_g = t[2];
      L->n1_b = t[3];
      or__dense_init(&L->fc11, t[4], 0, NULL, 0, H, I, quant);
      or__dense_init(&L->fc12, t[5], 0, NULL, 0, H, I, quant);
      or__dense_init(&L->fc2, t[6], 0, NULL, 0, I, H, quant);
      L->n2_g = t[7];
      L->n2_b = t[8];
      L->global = 1;
    }
  }
  return m;
}

void or_renc_free(or_renc_model *m) {
  if (!m) return;
  for (int l = 0; l < m->cfg.layers; l++) {
    or_renc_layer *L = &m->layers[l];
    or_dense *ds[5] = {&L->qkv, &L->o, &L->fc11, &L->fc12, &L->fc2};
    for (int i = 0; i < 5; i++) or__dense_free(ds[i]);
  }
  free(m->layers);
  free(m->zero_beta);
  free(m);
}

int or_renc_quantized_kind(const or_renc_model *m) {
  return m->cfg.layers > 0 ? m->layers[0].qkv.kind : 0;
}

/* The attention of both encoders (nomic.go:195-223, modernbert.go:239-281):
 * per head, q and k rotated by RoPE (v not), scores by MatMulSerial, scaled,
 * the sliding-window mask on ModernBERT's local layers (keys with
 * j < i - window or j > i + window filled with -1e30), Softmax, P.V against
 * V^T. qkv rows are [seq][3H]; ctx rows [seq][H]. */
static void renc_attention(const float *qkv, float *ctx, int seq, int H, int heads,
                           const float *cos_t, const float *sin_t, float scale, int window) {
  int dh = H / heads;
  float *qh = (float *)malloc(sizeof(float) * (size_t)seq * dh);
  float *kh = (float *)malloc(sizeof(float) * (size_t)seq * dh);
  float *vt = (float *)malloc(sizeof(float) * (size_t)seq * dh);
  float *ch = (float *)malloc(sizeof(float) * (size_t)seq * dh);
  float *sc = (float *)malloc(sizeof(float) * (size_t)seq * seq);
  for (int h = 0; h < heads; h++) {
    int off = h * dh;
    for (int i = 0; i < seq; i++) {
      const float *row = qkv + (size_t)i * 3 * H;
      memcpy(qh + (size_t)i * dh, row + off, sizeof(float) * dh);
      memcpy(kh + (size_t)i * dh, row + H + off, sizeof(float) * dh);
      for (int d = 0; d < dh; d++) vt[(size_t)d * seq + i] = row[2 * H + off + d];
    }
    or_apply_rope(qh, seq, dh, cos_t, sin_t);
    or_apply_rope(kh, seq, dh, cos_t, sin_t);
    or_matmul_serial(sc, qh, kh, seq, dh, seq);
    for (int i = 0; i < seq; i++) {
      float *r = sc + (size_t)i * seq;
      for (int j = 0; j < seq; j++) r[j] *= scale;
      if (window >= 0)
        for (int j = 0; j < seq; j++)
          if (j < i - window || j > i + window) r[j] = -1e30f;
    }
    or_softmax(sc, seq, seq);
    or_matmul_serial(ch, sc, vt, seq, seq, dh);
    for (int i = 0; i < seq; i++)
      memcpy(ctx + (size_t)i * H + off, ch + (size_t)i * dh, sizeof(float) * dh);
  }
  free(qh);
  free(kh);
  free(vt);
  free(ch);
  free(sc);
}

/* encodeNomic (internal/model/nomic.go:113-250) and encodeModernBERT
 * (internal/model/modernbert.go:148-311): one unpadded forward, final hidden
 * states [seq][H] into x. */
int or_renc_encode(const or_renc_model *m, const int32_t *ids, int seq, float *x) {
  const or_renc_config *c = &m->cfg;
  int mb = c->arch == OR_ARCH_MODERNBERT;
  int H = c->hidden, I = c->inter, heads = c->heads, dh = H / heads, half = dh / 2;
  float eps = c->eps;
  if (seq <= 0 || seq > c->max_seq) return OR_ERR_SEQ;
  for (int i = 0; i < seq; i++)
    if (ids[i] < 0 || ids[i] >= c->vocab) return OR_ERR_VOCAB;

  float *normed = (float *)malloc(sizeof(float) * (size_t)seq * H);
  float *qkv = (float *)malloc(sizeof(float) * (size_t)seq * 3 * H);
  float *ctx = (float *)malloc(sizeof(float) * (size_t)seq * H);
  float *att = (float *)malloc(sizeof(float) * (size_t)seq * H);
  float *w1 = (float *)malloc(sizeof(float) * (size_t)seq * 2 * I);
  float *w2 = (float *)malloc(sizeof(float) * (size_t)seq * I);
  float *act = (float *)malloc(sizeof(float) * (size_t)seq * I);
  float *cos_g = (float *)malloc(sizeof(float) * (size_t)seq * half);
  float *sin_g = (float *)malloc(sizeof(float) * (size_t)seq * half);
  float *cos_l = (float *)malloc(sizeof(float) * (size_t)seq * half);
  float *sin_l = (float *)malloc(sizeof(float) * (size_t)seq * half);
  or_rope_table(cos_g, sin_g, seq, dh, c->rope_theta);
  if (mb) or_rope_table(cos_l, sin_l, seq, dh, c->rope_local_theta);
  float scale = (float)(1.0 / sqrt((double)dh));

  if (mb) {
    /* token rows, LayerNorm with the zero beta (modernbert.go:203-211) */
    for (int i = 0; i < seq; i++)
      memcpy(x + (size_t)i * H, m->embed + (size_t)ids[i] * H, sizeof(float) * H);
    or_layernorm(x, m->emb_g, m->zero_beta, seq, H, eps);
    int window = c->local_attention / 2; /* modernbert.go:156 */
    for (int li = 0; li < c->layers; li++) {
      const or_renc_layer *L = &m->layers[li];
      /* pre-norm attention; layer 0's norm is an identity (modernbert.go:229-237) */
      memcpy(normed, x, sizeof(float) * (size_t)seq * H);
      if (L->attn_norm) or_layernorm(normed, L->attn_norm, m->zero_beta, seq, H, eps);
      or__dense_apply(&L->qkv, qkv, normed, seq);
      renc_attention(qkv, ctx, seq, H, heads, L->global ? cos_g : cos_l,
                     L->global ? sin_g : sin_l, scale, L->global ? -1 : window);
      or__dense_apply(&L->o, att, ctx, seq);
      or_add(x, att, seq * H);
      /* pre-norm GeGLU: gelu(Wi[:I]) * Wi[I:] (modernbert.go:286-302) */
      memcpy(normed, x, sizeof(float) * (size_t)seq * H);
      or_layernorm(normed, L->mlp_norm, m->zero_beta, seq, H, eps);
      or__dense_apply(&L->fc11, w1, normed, seq);
      for (int i = 0; i < seq; i++) {
        const float *in = w1 + (size_t)i * 2 * I, *gate = in + I;
        float *dst = act + (size_t)i * I;
        memcpy(dst, in, sizeof(float) * I);
        or_gelu_ref(dst, I);
        for (int d = 0; d < I; d++) dst[d] *= gate[d];
      }
      or__dense_apply(&L->fc2, att, act, seq);
      or_add(x, att, seq * H);
    }
    or_layernorm(x, m->final_norm, m->zero_beta, seq, H, eps); /* modernbert.go:307 */
  } else {
    /* word + segment-0 rows, LayerNorm (nomic.go:165-176) */
    for (int i = 0; i < seq; i++) {
      const float *w = m->embed + (size_t)ids[i] * H;
      float *row = x + (size_t)i * H;
      for (int j = 0; j < H; j++) row[j] = w[j] + m->type0[j];
    }
    or_layernorm(x, m->emb_g, m->emb_b, seq, H, eps);
    for (int li = 0; li < c->layers; li++) {
      const or_renc_layer *L = &m->layers[li];
      /* bidirectional RoPE attention, post-norm (nomic.go:192-227) */
      or__dense_apply(&L->qkv, qkv, x, seq);
      renc_attention(qkv, ctx, seq, H, heads, cos_g, sin_g, scale, -1);
      or__dense_apply(&L->o, att, ctx, seq);
      or_add(x, att, seq * H);
      or_layernorm(x, L->n1_g, L->n1_b, seq, H, eps);
      /* SwiGLU: fc11(x) * silu(fc12(x)), post-norm (nomic.go:229-245) */
      or__dense_apply(&L->fc11, w1, x, seq);
      or__dense_apply(&L->fc12, w2, x, seq);
      for (int i = 0; i < seq; i++) {
        const float *lin = w1 + (size_t)i * I;
        float *d = act + (size_t)i * I;
        memcpy(d, w2 + (size_t)i * I, sizeof(float) * I);
        or_silu(d, I);
        for (int j = 0; j < I; j++) d[j] *= lin[j];
      }
      or__dense_apply(&L->fc2, att, act, seq);
      or_add(x, att, seq * H);
      or_layernorm(x, L->n2_g, L->n2_b, seq, H, eps);
    }
  }
  free(normed); free(qkv); free(ctx); free(att); free(w1); free(w2); free(act);
  free(cos_g); free(sin_g); free(cos_l); free(sin_l);
  return OR_OK;
}

/* ForwardWorkers (internal/model/bert.go:657-689): pool, then L2. */
int or_renc_forward(const or_renc_model *m, const int32_t *ids, int seq, float *out) {
  int H = m->cfg.hidden;
  float *x = (float *)malloc(sizeof(float) * (size_t)(seq > 0 ? seq : 1) * H);
  int st = or_renc_encode(m, ids, seq, x);
  if (st != OR_OK) {
    free(x);
    return st;
  }
  if (m->cfg.pooling == OR_POOL_CLS) {
    memcpy(out, x, sizeof(float) * H);
  } else if (m->cfg.pooling == OR_POOL_LAST) {
    memcpy(out, x + (size_t)(seq - 1) * H, sizeof(float) * H);
  } else {
    for (int j = 0; j < H; j++) out[j] = 0.0f;
    for (int i = 0; i < seq; i++)
      for (int j = 0; j < H; j++) out[j] += x[(size_t)i * H + j];
    float inv = 1.0f / (float)seq;
    for (int j = 0; j < H; j++) out[j] *= inv;
  }
  if (m->cfg.normalize) or_l2normalize(out, H);
  free(x);
  return OR_OK;
}

/* Embed's batch path (rembed.go:309-330): texts fan out across threads, one
 * serial forward each, each timed into secs (wall seconds; may be NULL). */
int or_renc_embed_batch_timed(const or_renc_model *m, const int32_t *ids, const int32_t *lens,
                              int batch, int stride, float *out, int threads, double *secs) {
  int H = m->cfg.hidden;
  int err = OR_OK;
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
  for (int b = 0; b < batch; b++) {
    double t0 = omp_get_wtime();
    int st = or_renc_forward(m, ids + (size_t)b * stride, lens[b], out + (size_t)b * H);
    if (secs) secs[b] = omp_get_wtime() - t0;
    if (st != OR_OK) {
#pragma omp critical
      if (err == OR_OK) err = st;
    }
  }
  return err;
}
