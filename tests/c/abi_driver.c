/*
 * abi_driver.c — a plain C99 caller of librembed_hip.so, making the calls a
 * cgo binding of rembed makes, in the same order:
 *
 *   rh_device_count                   (WithDevice: is there a GPU at all?)
 *   rh_context_create(0)
 *   rh_model_create(cfg, quant)       (model.Load with WithInt8 / WithInt8Activations)
 *   rh_model_set_tensor  x N          (every raw float32 tensor, while Load has it)
 *   rh_model_finalize                 (quantize, pack, upload; raw weights may go)
 *   rh_model_quantized[_activations]  (Quantized / QuantizedActivations)
 *   rh_model_embed(int64 ids)         (Embed's batch forward)
 *   rh_context_create + rh_model_share (a second handle on the same weights,
 *                                       as a concurrent server's pool holds)
 *   rh_model_destroy, rh_context_destroy of the first handle, then an
 *   rh_model_embed on the second that must give the same bytes
 *   rh_model_destroy, rh_context_destroy  (Close)
 *
 * Usage: abi_driver <bundle> <out>
 *
 * The bundle (little-endian) holds what the Go side would hold after reading
 * a checkpoint and tokenizing a batch:
 *   "RHB1"; int32 config[22] (the int fields of rh_model_config in order, the
 *   eps as float bits); double rope_theta, rope_local_theta; int32 quant;
 *   int32 n_tensors; per tensor: int32 name_len, name bytes, int32 ndim,
 *   int64 dims[ndim], float32 data; int32 batch, stride; int32 lens[batch];
 *   int64 ids[batch * stride].
 * The output file holds int32 status, int32 quantized, int32
 * quantized_activations, int32 batch, int32 hidden, float32 vectors
 * [batch][hidden]. The exit code is the first failing status (0 = ok), with
 * rh_last_error() on stderr; no device is RH_ERR_NO_DEVICE, as a Go host
 * would see before falling back to its CPU path; 70 = the shared handle's
 * vectors differ from the first handle's.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "rembed_hip.h"

static FILE *g_in;

static int rd(void *dst, size_t size, size_t n) {
  return fread(dst, size, n, g_in) == n ? 0 : -1;
}

static int fail_status(const char *what, int st) {
  fprintf(stderr, "%s: status %d: %s\n", what, st, rh_last_error());
  return st;
}

int main(int argc, char **argv) {
  rh_model_config cfg;
  int32_t ci[22], quant = 0, ntensors = 0, batch = 0, stride = 0;
  int32_t *lens = NULL;
  int64_t *ids = NULL;
  float *vecs = NULL, *vecs2 = NULL;
  rh_context *ctx = NULL, *ctx2 = NULL;
  rh_model *model = NULL, *model2 = NULL;
  int st = RH_OK, ndev = 0, i;
  int32_t header[5];
  FILE *out;

  if (argc != 3) {
    fprintf(stderr, "usage: %s <bundle> <out>\n", argv[0]);
    return 64;
  }
  g_in = fopen(argv[1], "rb");
  if (!g_in) {
    perror(argv[1]);
    return 66;
  }
  {
    char magic[4];
    if (rd(magic, 1, 4) || memcmp(magic, "RHB1", 4) != 0 || rd(ci, 4, 22)) {
      fprintf(stderr, "bad bundle header\n");
      return 65;
    }
  }
  memset(&cfg, 0, sizeof cfg);
  cfg.arch = ci[0];
  cfg.hidden = ci[1];
  cfg.layers = ci[2];
  cfg.heads = ci[3];
  cfg.intermediate = ci[4];
  cfg.vocab = ci[5];
  cfg.max_position = ci[6];
  cfg.position_offset = ci[7];
  cfg.type_vocab = ci[8];
  memcpy(&cfg.layer_norm_eps, &ci[9], 4);
  cfg.pooling = ci[10];
  cfg.normalize = ci[11];
  cfg.kv_heads = ci[12];
  cfg.head_dim = ci[13];
  cfg.sliding_window = ci[14];
  cfg.sliding_pattern = ci[15];
  cfg.query_pre_attn_scalar = ci[16];
  cfg.dense_hidden = ci[17];
  if (rd(&cfg.rope_theta, 8, 1) || rd(&cfg.rope_local_theta, 8, 1) || rd(&quant, 4, 1) ||
      rd(&ntensors, 4, 1)) {
    fprintf(stderr, "bad bundle config\n");
    return 65;
  }

  st = rh_device_count(&ndev);
  if (st != RH_OK) return fail_status("rh_device_count", st);
  st = rh_context_create(0, &ctx);
  if (st != RH_OK) return fail_status("rh_context_create", st);
  st = rh_model_create(ctx, &cfg, quant, &model);
  if (st != RH_OK) {
    fail_status("rh_model_create", st);
    goto done;
  }

  /* Load: each raw tensor is handed over (and copied) by name, then freed
   * here, as model.Load drops the raw slices once they are packed. */
  for (i = 0; i < ntensors; i++) {
    int32_t name_len = 0, ndim = 0;
    int64_t dims[4];
    int64_t count = 1;
    char name[256];
    float *data;
    int d;
    if (rd(&name_len, 4, 1) || name_len <= 0 || name_len >= (int32_t)sizeof name ||
        rd(name, 1, (size_t)name_len) || rd(&ndim, 4, 1) || ndim < 0 || ndim > 4 ||
        rd(dims, 8, (size_t)ndim)) {
      fprintf(stderr, "bad tensor record %d\n", i);
      st = RH_ERR_INVALID;
      goto done;
    }
    name[name_len] = '\0';
    for (d = 0; d < ndim; d++) count *= dims[d];
    data = (float *)malloc((size_t)count * sizeof(float) + 4);
    if (!data || rd(data, 4, (size_t)count)) {
      fprintf(stderr, "bad tensor data %s\n", name);
      free(data);
      st = RH_ERR_INVALID;
      goto done;
    }
    st = rh_model_set_tensor(model, name, data, dims, ndim);
    free(data);
    if (st != RH_OK) {
      fail_status(name, st);
      goto done;
    }
  }
  st = rh_model_finalize(model);
  if (st != RH_OK) {
    fail_status("rh_model_finalize", st);
    goto done;
  }

  if (rd(&batch, 4, 1) || rd(&stride, 4, 1) || batch < 0 || stride < 1) {
    fprintf(stderr, "bad batch header\n");
    st = RH_ERR_INVALID;
    goto done;
  }
  lens = (int32_t *)malloc((size_t)batch * 4 + 4);
  ids = (int64_t *)malloc((size_t)batch * (size_t)stride * 8 + 8);
  vecs = (float *)malloc((size_t)batch * (size_t)cfg.hidden * 4 + 4);
  if (!lens || !ids || !vecs || rd(lens, 4, (size_t)batch) ||
      rd(ids, 8, (size_t)batch * (size_t)stride)) {
    fprintf(stderr, "bad batch data\n");
    st = RH_ERR_INVALID;
    goto done;
  }
  st = rh_model_embed(model, ids, lens, batch, stride, vecs);
  if (st != RH_OK) {
    fail_status("rh_model_embed", st);
    goto done;
  }

  /* A second handle on the same weights, on its own context; the first
   * handle and its context go before the second is used. */
  st = rh_context_create(0, &ctx2);
  if (st != RH_OK) {
    fail_status("rh_context_create (second)", st);
    goto done;
  }
  st = rh_model_share(model, ctx2, &model2);
  if (st != RH_OK) {
    fail_status("rh_model_share", st);
    goto done;
  }
  header[1] = rh_model_quantized(model);
  header[2] = rh_model_quantized_activations(model);
  rh_model_destroy(model);
  rh_context_destroy(ctx);
  model = NULL;
  ctx = NULL;
  vecs2 = (float *)malloc((size_t)batch * (size_t)cfg.hidden * 4 + 4);
  if (!vecs2) {
    st = RH_ERR_INVALID;
    goto done;
  }
  st = rh_model_embed(model2, ids, lens, batch, stride, vecs2);
  if (st != RH_OK) {
    fail_status("rh_model_embed (shared handle)", st);
    goto done;
  }
  if (rh_model_quantized(model2) != header[1] ||
      rh_model_quantized_activations(model2) != header[2] ||
      memcmp(vecs, vecs2, (size_t)batch * (size_t)cfg.hidden * 4) != 0) {
    fprintf(stderr, "the shared handle's vectors differ\n");
    st = 70;
    goto done;
  }

  out = fopen(argv[2], "wb");
  if (!out) {
    perror(argv[2]);
    st = RH_ERR_INVALID;
    goto done;
  }
  header[0] = st;
  header[3] = batch;
  header[4] = cfg.hidden;
  if (fwrite(header, 4, 5, out) != 5 ||
      fwrite(vecs, 4, (size_t)batch * (size_t)cfg.hidden, out) !=
          (size_t)batch * (size_t)cfg.hidden)
    st = RH_ERR_INVALID;
  if (fclose(out) != 0) st = RH_ERR_INVALID;

done:
  rh_model_destroy(model);
  rh_context_destroy(ctx);
  rh_model_destroy(model2);
  rh_context_destroy(ctx2);
  free(lens);
  free(ids);
  free(vecs);
  free(vecs2);
  fclose(g_in);
  return st;
}
