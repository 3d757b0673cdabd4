// kernels_dec.hip — row kernels of the decoder-family embedders (Qwen3,
// EmbeddingGemma) that keep activations in HBM between the GEMMs: token
// embedding gather, the residual + RMSNorm sandwich, per-head QK-norm with
// rotate-half RoPE, and EmbeddingGemma's Dense head.
//
// One 64-lane wave owns one row (or one head of one row); rows are 16-byte
// aligned and every width here is a multiple of 4, so rows move as float4.
#include "gemm_common.h"

namespace rh {

namespace {

constexpr int kRows = 4;  // 256 threads = 4 waves = 4 rows

__device__ __forceinline__ float wsum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wmax(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ uint8_t qbyte(float v, float inv) {
  int q = (int)rintf(v * inv) + 128;
  return (uint8_t)(q < 0 ? 0 : (q > 255 ? 255 : q));
}

// RMSNorm's scale (tensor.go:459-471): 1 / float32(sqrt(float64(ss/n + eps))).
__device__ __forceinline__ float rms_inv(float ss, int n, float eps) {
  return 1.0f / (float)sqrt((double)(ss / (float)n + eps));
}

}  // namespace

// ---- embeddings ---------------------------------------------------------------
// embed_tokens rows (qwen3.go:460-467), scaled by float32(sqrt(H)) for Gemma
// (gemma3.go:262-275), plus each row's position in its text for RoPE.
__global__ __launch_bounds__(256) void embed_gather_kernel(
    const int32_t* __restrict__ ids, int stride, const int32_t* __restrict__ cu,
    int batch, const float* __restrict__ word, int H, int vocab, float scale,
    float* __restrict__ x, int32_t* __restrict__ pos, int* err_flag, int total) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRows + (threadIdx.x >> 6);
  if (row >= total) return;
  int lo = 0, hi = batch;  // text b with cu[b] <= row < cu[b+1]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (cu[mid] <= row) lo = mid;
    else hi = mid;
  }
  const int t = row - cu[lo];
  int id = ids[(size_t)lo * stride + t];
  if (id < 0 || id >= vocab) {
    if (lane == 0) *err_flag = 1;
    id = id < 0 ? 0 : vocab - 1;  // stay in bounds; the call reports failure
  }
  if (lane == 0) pos[row] = t;
  const float* src = word + (size_t)id * H;
  float* dst = x + (size_t)row * H;
  for (int j = lane * 4; j < H; j += 256) {
    v4f v = *reinterpret_cast<const v4f*>(src + j);
    if (scale != 1.0f) v = v * scale;
    *reinterpret_cast<v4f*>(dst + j) = v;
  }
}

hipError_t launch_embed_gather(const int32_t* ids, int stride, const int32_t* cu,
                               int batch, const float* word, int H, int vocab,
                               float scale, float* x, int32_t* pos, int* err_flag,
                               int total_rows, hipStream_t s) {
  if (total_rows <= 0) return hipSuccess;
  if (H % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(embed_gather_kernel, dim3(ceil_div(total_rows, kRows)), dim3(256), 0,
                     s, ids, stride, cu, batch, word, H, vocab, scale, x, pos, err_flag,
                     total_rows);
  return hipGetLastError();
}

// ---- residual + RMSNorm sandwich -------------------------------------------------
//   y' = post_g ? RMSNorm(y, post_g) : y   (Gemma post-norms, gemma3.go:357,376)
//   x += y'                                 (Add, tensor.go:383-387)
//   out = RMSNorm(x, pre_g)                 (the next sublayer's pre-norm)
// plus an optional QuantizeRowU8 of out for a full-int8 GEMM. V float4 per lane.
template <int V>
__global__ __launch_bounds__(256) void rms_residual_kernel(
    float* x, const float* __restrict__ y, const float* __restrict__ post_g,
    const float* __restrict__ pre_g, float* out, int m, int H, float eps,
    uint8_t* __restrict__ qa, int ldq, float* __restrict__ row_scales) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRows + (threadIdx.x >> 6);
  if (row >= m) return;
  float* xr = x + (size_t)row * H;
  v4f v[V];
#pragma unroll
  for (int e = 0; e < V; e++) {
    const int j = (lane + 64 * e) * 4;
    v[e] = j < H ? *reinterpret_cast<const v4f*>(xr + j) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
  }
  if (y) {
    const float* yr = y + (size_t)row * H;
    v4f w[V];
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int j = (lane + 64 * e) * 4;
      w[e] = j < H ? *reinterpret_cast<const v4f*>(yr + j) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
      ss += (w[e][0] * w[e][0] + w[e][1] * w[e][1]) + (w[e][2] * w[e][2] + w[e][3] * w[e][3]);
    }
    if (post_g) {
      const float inv = rms_inv(wsum(ss), H, eps);
#pragma unroll
      for (int e = 0; e < V; e++) {
        const int j = (lane + 64 * e) * 4;
        if (j < H) {
          const v4f g = *reinterpret_cast<const v4f*>(post_g + j);
#pragma unroll
          for (int c = 0; c < 4; c++) w[e][c] = w[e][c] * inv * g[c];
        }
      }
    }
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int j = (lane + 64 * e) * 4;
      if (j < H) {
        v[e] = v[e] + w[e];
        *reinterpret_cast<v4f*>(xr + j) = v[e];
      }
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < V; e++)
    ss += (v[e][0] * v[e][0] + v[e][1] * v[e][1]) + (v[e][2] * v[e][2] + v[e][3] * v[e][3]);
  const float inv = rms_inv(wsum(ss), H, eps);
  float* orow = out + (size_t)row * H;
  float mx = 0.0f;
#pragma unroll
  for (int e = 0; e < V; e++) {
    const int j = (lane + 64 * e) * 4;
    if (j < H) {
      const v4f g = *reinterpret_cast<const v4f*>(pre_g + j);
      v4f o;
#pragma unroll
      for (int c = 0; c < 4; c++) o[c] = v[e][c] * inv * g[c];
      v[e] = o;
      *reinterpret_cast<v4f*>(orow + j) = o;
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(o[0]), fabsf(o[1])), fmaxf(fabsf(o[2]), fabsf(o[3]))));
    }
  }
  if (qa) {  // QuantizeRowU8 (pack_vnni.go:85-117) of the normalized row
    mx = wmax(mx);
    float scale = mx / 127.0f;
    if (scale == 0.0f) scale = 1.0f;
    const float qinv = 1.0f / scale;
    uint8_t* q = qa + (size_t)row * ldq;
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int j = (lane + 64 * e) * 4;
      if (j < H)
        *reinterpret_cast<uint32_t*>(q + j) =
            (uint32_t)qbyte(v[e][0], qinv) | ((uint32_t)qbyte(v[e][1], qinv) << 8) |
            ((uint32_t)qbyte(v[e][2], qinv) << 16) | ((uint32_t)qbyte(v[e][3], qinv) << 24);
    }
    for (int j = H + lane * 4; j < ldq; j += 256) *reinterpret_cast<uint32_t*>(q + j) = 0u;
    if (lane == 0) row_scales[row] = scale;
  }
}

template <int V>
static void launch_rmsv(float* x, const float* y, const float* post_g, const float* pre_g,
                        float* out, int m, int H, float eps, uint8_t* qa, int ldq, float* rs,
                        hipStream_t s) {
  hipLaunchKernelGGL((rms_residual_kernel<V>), dim3(ceil_div(m, kRows)), dim3(256), 0, s, x,
                     y, post_g, pre_g, out, m, H, eps, qa, ldq, rs);
}

hipError_t launch_rms_residual(float* x, const float* y, const float* post_g,
                               const float* pre_g, float* out, int m, int H, float eps,
                               uint8_t* qa, int ldq, float* row_scales, hipStream_t s) {
  if (m <= 0) return hipSuccess;
  if (H % 4 || H > 4096 || (qa && ldq % 4)) return hipErrorInvalidValue;
  const int v = ceil_div(H, 256);
  if (v <= 1) launch_rmsv<1>(x, y, post_g, pre_g, out, m, H, eps, qa, ldq, row_scales, s);
  else if (v <= 2) launch_rmsv<2>(x, y, post_g, pre_g, out, m, H, eps, qa, ldq, row_scales, s);
  else if (v <= 3) launch_rmsv<3>(x, y, post_g, pre_g, out, m, H, eps, qa, ldq, row_scales, s);
  else if (v <= 4) launch_rmsv<4>(x, y, post_g, pre_g, out, m, H, eps, qa, ldq, row_scales, s);
  else if (v <= 8) launch_rmsv<8>(x, y, post_g, pre_g, out, m, H, eps, qa, ldq, row_scales, s);
  else launch_rmsv<16>(x, y, post_g, pre_g, out, m, H, eps, qa, ldq, row_scales, s);
  return hipGetLastError();
}

// ---- QK-norm + RoPE -----------------------------------------------------------------
// One wave per (row, head) over the q heads then the k heads of a fused
// q|k|v row: RMSNorm of the head's dh values with its norm weight, then
// rotate-half RoPE at the row's position (applyRoPE, modernbert.go:130-143:
// each product rounded to float32 before the add). With `outh` the results
// go to bf16 rows of the same layout instead (round to nearest even), and
// the v heads are converted too: the operands of a bf16 attention.
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    float* __restrict__ qkv, int ldqkv, int m, int nq, int nkv, int dh,
    const float* __restrict__ q_g, const float* __restrict__ k_g, float eps,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const int32_t* __restrict__ pos, __bf16* __restrict__ outh) {
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * kRows + (threadIdx.x >> 6);
  const int nh = nq + nkv + (outh ? nkv : 0);
  if (item >= m * nh) return;
  const int row = item / nh, h = item % nh;
  float* v = qkv + (size_t)row * ldqkv + h * dh;  // q heads, k heads, [v heads]
  if (h >= nq + nkv) {  // v head: conversion only
    __bf16* o = outh + (size_t)row * ldqkv + h * dh;
    for (int d = lane; d < dh; d += 64) o[d] = (__bf16)v[d];
    return;
  }
  const float* g = h < nq ? q_g : k_g;
  const int half = dh >> 1;
  // lane holds pairs (d, d + half) for d = lane, lane + 64 (dh <= 256)
  float x1[2], x2[2];
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const int d = lane + 64 * e;
    x1[e] = d < half ? v[d] : 0.0f;
    x2[e] = d < half ? v[d + half] : 0.0f;
    ss += x1[e] * x1[e] + x2[e] * x2[e];
  }
  const float inv = rms_inv(wsum(ss), dh, eps);
  const int p = pos[row];
  const float* c = cos_t + (size_t)p * half;
  const float* sn = sin_t + (size_t)p * half;
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const int d = lane + 64 * e;
    if (d < half) {
      const float a = x1[e] * inv * g[d];
      const float b = x2[e] * inv * g[d + half];
      const float cc = c[d], ssn = sn[d];
      const float t0 = a * cc, t1 = b * ssn, t2 = b * cc, t3 = a * ssn;
      if (outh) {
        __bf16* o = outh + (size_t)row * ldqkv + h * dh;
        o[d] = (__bf16)(t0 - t1);
        o[d + half] = (__bf16)(t2 + t3);
      } else {
        v[d] = t0 - t1;
        v[d + half] = t2 + t3;
      }
    }
  }
}

hipError_t launch_qk_norm_rope(float* qkv, int ldqkv, int m, int nq, int nkv, int dh,
                               const float* q_g, const float* k_g, float eps,
                               const float* cos_t, const float* sin_t,
                               const int32_t* pos, __bf16* outh, hipStream_t s) {
  if (m <= 0) return hipSuccess;
  if (dh % 2 || dh > 256) return hipErrorInvalidValue;
  const int items = m * (nq + nkv + (outh ? nkv : 0));
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(ceil_div(items, kRows)), dim3(256), 0, s, qkv,
                     ldqkv, m, nq, nkv, dh, q_g, k_g, eps, cos_t, sin_t, pos, outh);
  return hipGetLastError();
}

// ---- EmbeddingGemma Dense head --------------------------------------------------------
// applyGemmaDenseHead (gemma3.go:174-198): hid[o] = sum_i w1[o][i] * pooled[i],
// out[o] = sum_i w2[o][i] * hid[i], each a sequential float32 sum in ascending
// i (no FMA), then L2Normalize (tensor.go:542-554) with a float64 sum.
// One workgroup per text; hid lives in LDS.
__global__ __launch_bounds__(256) void dense_head_kernel(const float* __restrict__ pooled,
                                                         int H, int D,
                                                         const float* __restrict__ w1,
                                                         const float* __restrict__ w2,
                                                         int normalize, float* __restrict__ out) {
  extern __shared__ float hid[];  // D floats
  __shared__ double red[256];
  const int b = blockIdx.x;
  const float* x = pooled + (size_t)b * H;
  for (int o = threadIdx.x; o < D; o += 256) {
    const float* row = w1 + (size_t)o * H;
    float acc = 0.0f;
    for (int i = 0; i < H; i++) acc = acc + row[i] * x[i];
    hid[o] = acc;
  }
  __syncthreads();
  float* y = out + (size_t)b * H;
  double ss = 0.0;
  for (int o = threadIdx.x; o < H; o += 256) {
    const float* row = w2 + (size_t)o * D;
    float acc = 0.0f;
    for (int i = 0; i < D; i++) acc = acc + row[i] * hid[i];
    y[o] = acc;
    ss += (double)acc * (double)acc;
  }
  if (!normalize) return;
  red[threadIdx.x] = ss;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  const double sum = red[0];
  if (sum == 0.0) return;
  const float inv = (float)(1.0 / sqrt(sum));
  for (int o = threadIdx.x; o < H; o += 256) y[o] = y[o] * inv;
}

hipError_t launch_dense_head(const float* pooled, int batch, int H, int D, const float* w1,
                             const float* w2, int normalize, float* out, hipStream_t s) {
  if (batch <= 0) return hipSuccess;
  if ((size_t)D * sizeof(float) > 64 * 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(dense_head_kernel, dim3(batch), dim3(256), D * sizeof(float), s, pooled,
                     H, D, w1, w2, normalize, out);
  return hipGetLastError();
}

}  // namespace rh
