// rows_common.h — row helpers shared by the row kernels (kernels_rows.hip)
// and the int8 GEMM whose epilogue finishes whole rows (gemm_i8.hip): wave
// reductions, QuantizeRowU8's byte step and the LayerNorm row finish, so a
// fused epilogue performs the same float operations in the same order as
// the separate pass.
#pragma once

#include "gemm_common.h"

namespace rh {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// QuantizeRowU8 (internal/tensor/pack_vnni.go:85-117) for one row already
// held by the wave: absmax, s = absmax/127 (1 if 0), inv = 1/s (IEEE float32
// divisions), q = clamp(rint(v*inv) + 128, 0, 255). rint is round-half-even
// as math.RoundToEven on the exactly-widened float32 product.
__device__ __forceinline__ uint8_t quant_u8(float v, float inv) {
  int q = (int)rintf(v * inv) + 128;
  q = q < 0 ? 0 : (q > 255 ? 255 : q);
  return (uint8_t)q;
}

// The elementwise half of LayerNorm (tensor.go:448-451) for the row held as
// float4 in v[] (lane l holds columns 4(l + 64e) .. +3; zeros past H), given
// its mean and inv = 1/float32(sqrt(var+eps)): out = (v-mean)*inv*g + b,
// written to xr, optionally to the bf16 hi/lo planes [..][ldp] of the next
// weight-only int8 / fp32 GEMM (pl may be null) and quantized into
// qa/row_scales (QuantizeRowU8).
template <int V>
__device__ __forceinline__ void ln_vec_apply(v4f (&v)[V], int lane, int row, int H, float mean,
                                             float inv, const float* __restrict__ gamma,
                                             const float* __restrict__ beta,
                                             float* __restrict__ xr, uint8_t* __restrict__ qa,
                                             int ldq, float* __restrict__ row_scales,
                                             __bf16* __restrict__ ph, __bf16* __restrict__ pl,
                                             int ldp) {
  float mx = 0.0f;
#pragma unroll
  for (int e = 0; e < V; e++) {
    const int j = (lane + 64 * e) * 4;
    if (j < H) {
      const v4f g = *reinterpret_cast<const v4f*>(gamma + j);
      const v4f b = *reinterpret_cast<const v4f*>(beta + j);
      v4f o;
#pragma unroll
      for (int c = 0; c < 4; c++) o[c] = (v[e][c] - mean) * inv * g[c] + b[c];
      v[e] = o;
      *reinterpret_cast<v4f*>(xr + j) = o;
      if (ph) store_planes4(ph, pl, (size_t)row * ldp + j, o);
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(o[0]), fabsf(o[1])), fmaxf(fabsf(o[2]), fabsf(o[3]))));
    }
  }
  if (qa) {
    mx = wave_max(mx);
    float scale = mx / 127.0f;
    if (scale == 0.0f) scale = 1.0f;
    const float qinv = 1.0f / scale;
    uint8_t* q = qa + (size_t)row * ldq;
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int j = (lane + 64 * e) * 4;
      if (j < H)
        *reinterpret_cast<uint32_t*>(q + j) =
            (uint32_t)quant_u8(v[e][0], qinv) | ((uint32_t)quant_u8(v[e][1], qinv) << 8) |
            ((uint32_t)quant_u8(v[e][2], qinv) << 16) | ((uint32_t)quant_u8(v[e][3], qinv) << 24);
    }
    for (int j = H + lane * 4; j < ldq; j += 256) *reinterpret_cast<uint32_t*>(q + j) = 0u;
    if (lane == 0) row_scales[row] = scale;
  }
}

// LayerNorm of the row held as float4 in v[] (layout as ln_vec_apply), with
// the mean and variance reduced across the wave (per lane over its float4
// groups, then a butterfly): biased variance, inv = 1/float32(sqrt(var+eps))
// (tensor.go:433-452). The sums' order differs from the reference's
// column-order loop; ln_exact_* keep that order.
template <int V>
__device__ __forceinline__ void ln_vec_finish(v4f (&v)[V], int lane, int row, int H,
                                              const float* __restrict__ gamma,
                                              const float* __restrict__ beta, float eps,
                                              float* __restrict__ xr, uint8_t* __restrict__ qa,
                                              int ldq, float* __restrict__ row_scales,
                                              __bf16* __restrict__ ph, __bf16* __restrict__ pl,
                                              int ldp) {
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < V; e++) s += (v[e][0] + v[e][1]) + (v[e][2] + v[e][3]);
  const float mean = wave_sum(s) / (float)H;
  float s2 = 0.0f;
#pragma unroll
  for (int e = 0; e < V; e++) {
    const int j = (lane + 64 * e) * 4;
    if (j < H) {
      const v4f d = v[e] - mean;
      s2 += (d[0] * d[0] + d[1] * d[1]) + (d[2] * d[2] + d[3] * d[3]);
    }
  }
  const float var = wave_sum(s2) / (float)H;
  const float inv = 1.0f / sqrtf(var + eps);
  ln_vec_apply<V>(v, lane, row, H, mean, inv, gamma, beta, xr, qa, ldq, row_scales, ph, pl, ldp);
}

}  // namespace rh
