/*
 * oracle_dec.c — CPU restatement of rembed's decoder-family embedders:
 * Qwen3 (causal, last-token pooled) and EmbeddingGemma (Gemma 3 run
 * bidirectionally, mean pooled through a Dense head).
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

/* ropeTable, internal/model/modernbert.go:112-122: inv_freq in float64,
 * float64 trig rounded to float32. cos/sin are [seq][dh/2]. */
void or_rope_table(float *cos_t, float *sin_t, int seq, int dh, double theta) {
  int half = dh / 2;
  for (int d = 0; d < half; d++) {
    double inv_freq = pow(theta, -2.0 * (double)d / (double)dh);
    for (int p = 0; p < seq; p++) {
      double ang = (double)p * inv_freq;
      cos_t[(size_t)p * half + d] = (float)cos(ang);
      sin_t[(size_t)p * half + d] = (float)sin(ang);
    }
  }
}

/* applyRoPE, internal/model/modernbert.go:130-143: rotate-half pairs
 * (d, d + dh/2), each product rounded to float32 before the add. */
void or_apply_rope(float *x, int seq, int dh, const float *cos_t,
                   const float *sin_t) {
  int half = dh / 2;
  for (int p = 0; p < seq; p++) {
    float *row = x + (size_t)p * dh;
    const float *c = cos_t + (size_t)p * half, *s = sin_t + (size_t)p * half;
    for (int d = 0; d < half; d++) {
      float x1 = row[d], x2 = row[d + half];
      float a = x1 * c[d], b = x2 * s[d];
      float e = x2 * c[d], f = x1 * s[d];
      row[d] = a - b;
      row[d + half] = e + f;
    }
  }
}

#define FLASH_BLK 64

/* flashAttnCausalHead, internal/model/qwen3.go:307-390: causal attention of
 * one head with online softmax over 64-key blocks, future blocks skipped.
 * qh/kh/vh/out are [seq][dh]. */
void or_flash_causal_head(const float *qh, const float *kh, const float *vh,
                          float *out, int seq, int dh, float scale) {
  const float neg_inf = -1e30f;
  int bq = seq < FLASH_BLK ? seq : FLASH_BLK;
  float *sblk = (float *)malloc(sizeof(float) * (size_t)bq * bq);
  float *acc = (float *)malloc(sizeof(float) * (size_t)bq * dh);
  float *mrow = (float *)malloc(sizeof(float) * bq);
  float *lrow = (float *)malloc(sizeof(float) * bq);
  for (int q0 = 0; q0 < seq; q0 += FLASH_BLK) {
    int q1 = q0 + FLASH_BLK < seq ? q0 + FLASH_BLK : seq;
    int nq = q1 - q0;
    for (int r = 0; r < nq; r++) {
      mrow[r] = neg_inf;
      lrow[r] = 0.0f;
    }
    memset(acc, 0, sizeof(float) * (size_t)nq * dh);
    for (int k0 = 0; k0 < q1; k0 += FLASH_BLK) {
      int k1 = k0 + FLASH_BLK < q1 ? k0 + FLASH_BLK : q1;
      int nk = k1 - k0;
      or_matmul_serial(sblk, qh + (size_t)q0 * dh, kh + (size_t)k0 * dh, nq, dh, nk);
      for (int r = 0; r < nq; r++) {
        int i = q0 + r;
        float *srow = sblk + (size_t)r * nk;
        float rmax = neg_inf;
        for (int c = 0; c < nk; c++) {
          if (k0 + c > i) {
            srow[c] = neg_inf;
          } else {
            srow[c] *= scale;
            if (srow[c] > rmax) rmax = srow[c];
          }
        }
        if (rmax == neg_inf) continue;
        float mprev = mrow[r], mnew = mprev;
        if (rmax > mnew) mnew = rmax;
        float *ar = acc + (size_t)r * dh;
        if (mprev != neg_inf && mnew != mprev) {
          float corr = or__exp_nonpos(mprev - mnew);
          lrow[r] *= corr;
          for (int d = 0; d < dh; d++) ar[d] *= corr;
        }
        float lr = lrow[r];
        for (int c = 0; c < nk; c++) {
          if (k0 + c > i) continue;
          float pv = or__exp_nonpos(srow[c] - mnew);
          lr += pv;
          const float *vk = vh + (size_t)(k0 + c) * dh;
          for (int d = 0; d < dh; d++) ar[d] += pv * vk[d];
        }
        lrow[r] = lr;
        mrow[r] = mnew;
      }
    }
    for (int r = 0; r < nq; r++) {
      const float *ar = acc + (size_t)r * dh;
      float inv = 1.0f / lrow[r];
      float *o = out + (size_t)(q0 + r) * dh;
      for (int d = 0; d < dh; d++) o[d] = ar[d] * inv;
    }
  }
  free(sblk);
  free(acc);
  free(mrow);
  free(lrow);
}

typedef struct {
  const float *in_norm, *q_norm, *k_norm, *post_attn, *pre_ffn, *post_ffn;
  float *owned[6]; /* unit-offset copies (Gemma) */
  or_dense q, k, v, o, gate, up, down;
  int global; /* Gemma: full attention layer */
} or_dec_layer;

struct or_dec_model {
  or_dec_config cfg;
  int quant;
  const float *embed;
  const float *final_norm;
  float *final_owned;
  const float *dense1, *dense2; /* Gemma Dense head [D][H], [H][D] */
  or_dec_layer *layers;
};

/* unitOffset, internal/model/gemma3.go:40-50: a copy with +1 folded in. */
static float *unit_offset(const float *v, int n) {
  float *o = (float *)malloc(sizeof(float) * n);
  for (int i = 0; i < n; i++) o[i] = v[i] + 1.0f;
  return o;
}

/* loadQwen3 (internal/model/qwen3.go:37-135) and loadGemma3
 * (internal/model/gemma3.go:57-158): bias-free projections through newDense,
 * Gemma norms stored unit-offset. Per-layer tensor order: see oracle.h. */
or_dec_model *or_dec_create(const or_dec_config *cfg, int quant,
                            const float *embed, const float *final_norm,
                            const float *const *lt, const float *dense1,
                            const float *dense2) {
  int H = cfg->hidden, I = cfg->inter, dh = cfg->head_dim;
  int qdim = cfg->heads * dh, kvdim = cfg->kv_heads * dh;
  if (cfg->kv_heads <= 0 || cfg->heads % cfg->kv_heads != 0 || dh % 2) return NULL;
  int gemma = cfg->arch == OR_ARCH_GEMMA3;
  int per = gemma ? OR_GEMMA3_TENSORS_PER_LAYER : OR_QWEN3_TENSORS_PER_LAYER;
  or_dec_model *m = (or_dec_model *)calloc(1, sizeof(*m));
  m->cfg = *cfg;
  m->quant = quant;
  m->embed = embed;
  if (gemma) {
    m->final_owned = unit_offset(final_norm, H);
    m->final_norm = m->final_owned;
  } else {
    m->final_norm = final_norm;
  }
  m->dense1 = dense1;
  m->dense2 = dense2;
  m->layers = (or_dec_layer *)calloc((size_t)cfg->layers, sizeof(or_dec_layer));
  for (int l = 0; l < cfg->layers; l++) {
    const float *const *t = lt + (size_t)l * per;
    or_dec_layer *L = &m->layers[l];
    if (gemma) {
      /* input_ln q k v o q_norm k_norm post_attn pre_ffn post_ffn gate up down */
      const float *norms[6] = {t[0], t[5], t[6], t[7], t[8], t[9]};
      const int dims[6] = {H, dh, dh, H, H, H};
      for (int n = 0; n < 6; n++) L->owned[n] = unit_offset(norms[n], dims[n]);
      L->in_norm = L->owned[0];
      L->q_norm = L->owned[1];
      L->k_norm = L->owned[2];
      L->post_attn = L->owned[3];
      L->pre_ffn = L->owned[4];
      L->post_ffn = L->owned[5];
      or__dense_init(&L->gate, t[10], 0, NULL, 0, H, I, quant);
      or__dense_init(&L->up, t[11], 0, NULL, 0, H, I, quant);
      or__dense_init(&L->down, t[12], 0, NULL, 0, I, H, quant);
      L->global = (l + 1) % cfg->sliding_pattern == 0; /* gemma3.go:87 */
    } else {
      /* input_ln q k v o q_norm k_norm post_attn gate up down */
      L->in_norm = t[0];
      L->q_norm = t[5];
      L->k_norm = t[6];
      L->post_attn = t[7];
      or__dense_init(&L->gate, t[8], 0, NULL, 0, H, I, quant);
      or__dense_init(&L->up, t[9], 0, NULL, 0, H, I, quant);
      or__dense_init(&L->down, t[10], 0, NULL, 0, I, H, quant);
      L->global = 1;
    }
    or__dense_init(&L->q, t[1], 0, NULL, 0, H, qdim, quant);
    or__dense_init(&L->k, t[2], 0, NULL, 0, H, kvdim, quant);
    or__dense_init(&L->v, t[3], 0, NULL, 0, H, kvdim, quant);
    or__dense_init(&L->o, t[4], 0, NULL, 0, qdim, H, quant);
  }
  return m;
}

void or_dec_free(or_dec_model *m) {
  if (!m) return;
  for (int l = 0; l < m->cfg.layers; l++) {
    or_dec_layer *L = &m->layers[l];
    or_dense *ds[7] = {&L->q, &L->k, &L->v, &L->o, &L->gate, &L->up, &L->down};
    for (int i = 0; i < 7; i++) or__dense_free(ds[i]);
    for (int i = 0; i < 6; i++) free(L->owned[i]);
  }
  free(m->layers);
  free(m->final_owned);
  free(m);
}

int or_dec_quantized_kind(const or_dec_model *m) {
  return m->cfg.layers > 0 ? m->layers[0].q.kind : 0;
}

/* encodeQwen3 (internal/model/qwen3.go:395-548) and encodeGemma3
 * (internal/model/gemma3.go:206-384): one unpadded forward, final hidden
 * states [seq][H] into x. */
int or_dec_encode(const or_dec_model *m, const int32_t *ids, int seq, float *x) {
  const or_dec_config *c = &m->cfg;
  int gemma = c->arch == OR_ARCH_GEMMA3;
  int H = c->hidden, I = c->inter, nq = c->heads, nkv = c->kv_heads, dh = c->head_dim;
  int qdim = nq * dh, kvdim = nkv * dh, group = nq / nkv, half = dh / 2;
  float eps = c->eps;
  if (seq <= 0 || seq > c->max_seq) return OR_ERR_SEQ;
  for (int i = 0; i < seq; i++)
    if (ids[i] < 0 || ids[i] >= c->vocab) return OR_ERR_VOCAB;

  float *normed = (float *)malloc(sizeof(float) * (size_t)seq * H);
  float *q = (float *)malloc(sizeof(float) * (size_t)seq * qdim);
  float *k = (float *)malloc(sizeof(float) * (size_t)seq * kvdim);
  float *v = (float *)malloc(sizeof(float) * (size_t)seq * kvdim);
  float *khead = (float *)malloc(sizeof(float) * (size_t)nkv * seq * dh);
  float *vhead = (float *)malloc(sizeof(float) * (size_t)nkv * seq * dh);
  float *qh = (float *)malloc(sizeof(float) * (size_t)seq * dh);
  float *ch = (float *)malloc(sizeof(float) * (size_t)seq * dh);
  float *ctx = (float *)malloc(sizeof(float) * (size_t)seq * qdim);
  float *att = (float *)malloc(sizeof(float) * (size_t)seq * H);
  float *gate = (float *)malloc(sizeof(float) * (size_t)seq * I);
  float *up = (float *)malloc(sizeof(float) * (size_t)seq * I);
  float *down = (float *)malloc(sizeof(float) * (size_t)seq * H);
  float *sc = gemma ? (float *)malloc(sizeof(float) * (size_t)seq * seq) : NULL;
  float *cos_g = (float *)malloc(sizeof(float) * (size_t)seq * half);
  float *sin_g = (float *)malloc(sizeof(float) * (size_t)seq * half);
  float *cos_l = (float *)malloc(sizeof(float) * (size_t)seq * half);
  float *sin_l = (float *)malloc(sizeof(float) * (size_t)seq * half);

  or_rope_table(cos_g, sin_g, seq, dh, c->rope_theta);
  if (gemma) or_rope_table(cos_l, sin_l, seq, dh, c->rope_local_theta);

  /* Embeddings: token rows only; Gemma scales them by float32(sqrt(H))
   * (qwen3.go:460-467, gemma3.go:262-275). */
  float emb_scale = (float)sqrt((double)H);
  for (int i = 0; i < seq; i++) {
    const float *src = m->embed + (size_t)ids[i] * H;
    float *dst = x + (size_t)i * H;
    for (int j = 0; j < H; j++) dst[j] = gemma ? src[j] * emb_scale : src[j];
  }
  float scale = gemma ? (float)(1.0 / sqrt((double)c->query_pre_attn_scalar))
                      : (float)(1.0 / sqrt((double)dh));

  for (int li = 0; li < c->layers; li++) {
    const or_dec_layer *L = &m->layers[li];
    const float *ct = cos_g, *st = sin_g;
    if (gemma && !L->global) {
      ct = cos_l;
      st = sin_l;
    }
    memcpy(normed, x, sizeof(float) * (size_t)seq * H);
    or_rmsnorm(normed, L->in_norm, seq, H, eps);
    or__dense_apply(&L->q, q, normed, seq);
    or__dense_apply(&L->k, k, normed, seq);
    or__dense_apply(&L->v, v, normed, seq);
    /* Per kv head: repack, QK-norm and RoPE K (qwen3.go:484-497). */
    for (int kv = 0; kv < nkv; kv++) {
      float *kh = khead + (size_t)kv * seq * dh, *vh = vhead + (size_t)kv * seq * dh;
      for (int i = 0; i < seq; i++) {
        memcpy(kh + (size_t)i * dh, k + (size_t)i * kvdim + kv * dh, sizeof(float) * dh);
        memcpy(vh + (size_t)i * dh, v + (size_t)i * kvdim + kv * dh, sizeof(float) * dh);
      }
      or_rmsnorm(kh, L->k_norm, seq, dh, eps);
      or_apply_rope(kh, seq, dh, ct, st);
    }
    for (int hh = 0; hh < nq; hh++) {
      for (int i = 0; i < seq; i++)
        memcpy(qh + (size_t)i * dh, q + (size_t)i * qdim + hh * dh, sizeof(float) * dh);
      or_rmsnorm(qh, L->q_norm, seq, dh, eps);
      or_apply_rope(qh, seq, dh, ct, st);
      int kv = hh / group;
      const float *kh = khead + (size_t)kv * seq * dh, *vh = vhead + (size_t)kv * seq * dh;
      if (!gemma) {
        or_flash_causal_head(qh, kh, vh, ch, seq, dh, scale);
      } else {
        /* Bidirectional scores, sliding window |i-j| < w on local layers,
         * Softmax, P.V against V^T (gemma3.go:331-351). */
        or_matmul_serial(sc, qh, kh, seq, dh, seq);
        int w = c->sliding_window;
        for (int i = 0; i < seq; i++) {
          float *row = sc + (size_t)i * seq;
          for (int j = 0; j < seq; j++) row[j] *= scale;
          if (!L->global)
            for (int j = 0; j < seq; j++)
              if (j <= i - w || j >= i + w) row[j] = -1e30f;
        }
        or_softmax(sc, seq, seq);
        float *vt = (float *)malloc(sizeof(float) * (size_t)seq * dh);
        for (int i = 0; i < seq; i++)
          for (int d = 0; d < dh; d++) vt[(size_t)d * seq + i] = vh[(size_t)i * dh + d];
        or_matmul_serial(ch, sc, vt, seq, seq, dh);
        free(vt);
      }
      for (int i = 0; i < seq; i++)
        memcpy(ctx + (size_t)i * qdim + hh * dh, ch + (size_t)i * dh, sizeof(float) * dh);
    }
    or__dense_apply(&L->o, att, ctx, seq);
    if (gemma) or_rmsnorm(att, L->post_attn, seq, H, eps);
    or_add(x, att, seq * H);
    /* MLP: pre-norm, gated activation, down projection. */
    memcpy(normed, x, sizeof(float) * (size_t)seq * H);
    or_rmsnorm(normed, gemma ? L->pre_ffn : L->post_attn, seq, H, eps);
    or__dense_apply(&L->gate, gate, normed, seq);
    or__dense_apply(&L->up, up, normed, seq);
    for (int i = 0; i < seq; i++) {
      float *g = gate + (size_t)i * I;
      const float *u = up + (size_t)i * I;
      if (gemma) or_gelu_tanh(g, I); /* gemma3.go:365-374 */
      else or_silu(g, I);            /* qwen3.go:530-539 */
      for (int j = 0; j < I; j++) g[j] *= u[j];
    }
    or__dense_apply(&L->down, down, gate, seq);
    if (gemma) or_rmsnorm(down, L->post_ffn, seq, H, eps);
    or_add(x, down, seq * H);
  }
  or_rmsnorm(x, m->final_norm, seq, H, eps);

  free(normed); free(q); free(k); free(v); free(khead); free(vhead);
  free(qh); free(ch); free(ctx); free(att); free(gate); free(up); free(down);
  free(sc); free(cos_g); free(sin_g); free(cos_l); free(sin_l);
  return OR_OK;
}

/* ForwardWorkers (internal/model/bert.go:657-689): pool, EmbeddingGemma's
 * Dense head (gemma3.go:174-198: two float32 matvecs, no FMA), then L2. */
int or_dec_forward(const or_dec_model *m, const int32_t *ids, int seq, float *out) {
  int H = m->cfg.hidden;
  float *x = (float *)malloc(sizeof(float) * (size_t)(seq > 0 ? seq : 1) * H);
  int st = or_dec_encode(m, ids, seq, x);
  if (st != OR_OK) {
    free(x);
    return st;
  }
  float *pooled = (float *)calloc((size_t)H, sizeof(float));
  if (m->cfg.pooling == OR_POOL_CLS) {
    memcpy(pooled, x, sizeof(float) * H);
  } else if (m->cfg.pooling == OR_POOL_LAST) {
    memcpy(pooled, x + (size_t)(seq - 1) * H, sizeof(float) * H);
  } else {
    for (int i = 0; i < seq; i++)
      for (int j = 0; j < H; j++) pooled[j] += x[(size_t)i * H + j];
    float inv = 1.0f / (float)seq;
    for (int j = 0; j < H; j++) pooled[j] *= inv;
  }
  if (m->dense1 && m->dense2 && m->cfg.dense_hidden > 0) {
    int D = m->cfg.dense_hidden;
    float *hid = (float *)malloc(sizeof(float) * D);
    for (int o = 0; o < D; o++) {
      const float *row = m->dense1 + (size_t)o * H;
      float acc = 0.0f;
      for (int i = 0; i < H; i++) acc += row[i] * pooled[i];
      hid[o] = acc;
    }
    for (int o = 0; o < H; o++) {
      const float *row = m->dense2 + (size_t)o * D;
      float acc = 0.0f;
      for (int i = 0; i < D; i++) acc += row[i] * hid[i];
      out[o] = acc;
    }
    free(hid);
  } else {
    memcpy(out, pooled, sizeof(float) * H);
  }
  if (m->cfg.normalize) or_l2normalize(out, H);
  free(pooled);
  free(x);
  return OR_OK;
}

int or_dec_embed_batch(const or_dec_model *m, const int32_t *ids,
                        const int32_t *lens, int batch, int stride,
                        float *out, int threads) {
  return or_dec_embed_batch_timed(m, ids, lens, batch, stride, out, threads, NULL);
}

/* The same with each text's forward timed (wall seconds; secs may be NULL). */
int or_dec_embed_batch_timed(const or_dec_model *m, const int32_t *ids,
                        const int32_t *lens, int batch, int stride,
                        float *out, int threads, double *secs) {
  int H = m->cfg.hidden;
  int err = OR_OK;
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
  for (int b = 0; b < batch; b++) {
    double t0 = omp_get_wtime();
    int st = or_dec_forward(m, ids + (size_t)b * stride, lens[b], out + (size_t)b * H);
    if (secs) secs[b] = omp_get_wtime() - t0;
    if (st != OR_OK) {
#pragma omp critical
      if (err == OR_OK) err = st;
    }
  }
  return err;
}
