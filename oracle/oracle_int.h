/*
 * oracle_int.h — internals shared by the oracle's C files (test
 * infrastructure only; see oracle.h).
 */
#ifndef REMBED_ORACLE_INT_H
#define REMBED_ORACLE_INT_H

#include <stdint.h>

/* A dense weight as newDense leaves it (internal/model/bert.go:32-39,
 * 263-278): the mode that actually took plus its packed/quantized data. */
typedef struct {
  int kind; /* 0 fp32, 1 weight-only int8, 2 full int8 */
  int in, out;
  const float *raw; /* fp32: borrowed bT */
  float *rawcopy;   /* fp32 fused QKV copy owned here */
  int8_t *q;
  float *scales;
  int32_t *colsum;
  float *bias; /* owned (fused QKV) or NULL */
  const float *bias_ref;
  int8_t *panels; /* full int8: the same q in PackB8VNNI's panel layout */
} or_dense;

/* newDense (bert.go:263-278): full int8 -> weight-only int8 -> fp32 fallback. */
void or__dense_init(or_dense *d, const float *raw, int owned_raw,
                    const float *bias, int owned_bias, int in, int out, int quant);
void or__dense_free(or_dense *d);
/* applyDense (bert.go:282-301): dst[seq][out] = x[seq][in] . W^T (+ bias). */
void or__dense_apply(const or_dense *d, float *dst, const float *x, int seq);
/* expNonPos (internal/tensor/fastmath.go:93-109): e^x for x <= 0. */
float or__exp_nonpos(float x);

#endif
