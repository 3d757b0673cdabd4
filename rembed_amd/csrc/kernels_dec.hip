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

}  // namespace

// ---- embeddings ---------------------------------------------------------------
// embed_tokens rows (qwen3.go:460-467), scaled by float32(sqrt(H)) for Gemma
// (gemma3.go:262-275), plus an optional row added to each (nomic's segment-0
// row: w[j] + t[j], nomic.go:177-188), and each row's position in its text
// for RoPE.
__global__ __launch_bounds__(256) void embed_gather_kernel(
    const int32_t* __restrict__ ids, int stride, const int32_t* __restrict__ cu,
    int batch, const float* __restrict__ word, const float* __restrict__ add_row, int H,
    int vocab, float scale, float* __restrict__ x, int32_t* __restrict__ pos, int* err_flag,
    int total) {
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
    if (add_row) v = v + *reinterpret_cast<const v4f*>(add_row + j);
    *reinterpret_cast<v4f*>(dst + j) = v;
  }
}

hipError_t launch_embed_gather(const int32_t* ids, int stride, const int32_t* cu,
                               int batch, const float* word, const float* add_row, int H,
                               int vocab, float scale, float* x, int32_t* pos, int* err_flag,
                               int total_rows, hipStream_t s) {
  if (total_rows <= 0) return hipSuccess;
  if (H % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(embed_gather_kernel, dim3(ceil_div(total_rows, kRows)), dim3(256), 0,
                     s, ids, stride, cu, batch, word, add_row, H, vocab, scale, x, pos,
                     err_flag, total_rows);
  return hipGetLastError();
}

// ---- residual + norm sandwich ----------------------------------------------------
//   y' = post_g ? RMSNorm(y, post_g) : y   (Gemma post-norms, gemma3.go:357,376)
//   x += y'                                 (Add, tensor.go:383-387)
//   out = RMSNorm(x, pre_g)                 (the next sublayer's pre-norm)
// or, with layer_norm set, out = LayerNorm(x, pre_g, ln_b) (tensor.go:430-452:
// biased variance, 1 / float32(sqrt(var + eps)), (v - mean) * inv * g + b;
// a null ln_b adds zero, as ModernBERT's shared zero beta does). out goes to
// fp32 rows and/or to the bf16 hi/lo planes of the next GEMM's input, plus
// an optional QuantizeRowU8 of it for a full-int8 GEMM. When out is x itself
// (a post-norm block, or the final norm) the sum is not stored first. V
// float4 per lane.
template <int V>
__global__ __launch_bounds__(256) void rms_residual_kernel(RmsArgs p) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRows + (threadIdx.x >> 6);
  if (row >= p.m) return;
  const int H = p.H;
  float* xr = p.x + (size_t)row * H;
  v4f v[V];
#pragma unroll
  for (int e = 0; e < V; e++) {
    const int j = (lane + 64 * e) * 4;
    v[e] = j < H ? *reinterpret_cast<const v4f*>(xr + j) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
  }
  if (p.y) {
    const float* yr = p.y + (size_t)row * H;
    v4f w[V];
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int j = (lane + 64 * e) * 4;
      w[e] = j < H ? *reinterpret_cast<const v4f*>(yr + j) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
      ss += (w[e][0] * w[e][0] + w[e][1] * w[e][1]) + (w[e][2] * w[e][2] + w[e][3] * w[e][3]);
    }
    if (p.post_g) {
      const float inv = rms_inv(wsum(ss), H, p.eps);
#pragma unroll
      for (int e = 0; e < V; e++) {
        const int j = (lane + 64 * e) * 4;
        if (j < H) {
          const v4f g = *reinterpret_cast<const v4f*>(p.post_g + j);
#pragma unroll
          for (int c = 0; c < 4; c++) w[e][c] = w[e][c] * inv * g[c];
        }
      }
    }
    const bool store_sum = p.out != p.x;
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int j = (lane + 64 * e) * 4;
      if (j < H) {
        v[e] = v[e] + w[e];
        if (store_sum) *reinterpret_cast<v4f*>(xr + j) = v[e];
      }
    }
  }
  float inv, mean = 0.0f;
  if (p.layer_norm) {
    float s = 0.0f;  // lanes past H hold zeros
#pragma unroll
    for (int e = 0; e < V; e++) s += (v[e][0] + v[e][1]) + (v[e][2] + v[e][3]);
    mean = wsum(s) / (float)H;
    float s2 = 0.0f;
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int j = (lane + 64 * e) * 4;
      if (j < H) {
        const v4f d = v[e] - mean;
        s2 += (d[0] * d[0] + d[1] * d[1]) + (d[2] * d[2] + d[3] * d[3]);
      }
    }
    inv = 1.0f / sqrtf(wsum(s2) / (float)H + p.eps);
  } else {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < V; e++)
      ss += (v[e][0] * v[e][0] + v[e][1] * v[e][1]) + (v[e][2] * v[e][2] + v[e][3] * v[e][3]);
    inv = rms_inv(wsum(ss), H, p.eps);
  }
  float mx = 0.0f;
#pragma unroll
  for (int e = 0; e < V; e++) {
    const int j = (lane + 64 * e) * 4;
    if (j < H) {
      const v4f g = *reinterpret_cast<const v4f*>(p.pre_g + j);
      v4f o;
      if (p.layer_norm) {
        const v4f b = p.ln_b ? *reinterpret_cast<const v4f*>(p.ln_b + j)
                             : v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < 4; c++) o[c] = (v[e][c] - mean) * inv * g[c] + b[c];
      } else {
#pragma unroll
        for (int c = 0; c < 4; c++) o[c] = v[e][c] * inv * g[c];
      }
      v[e] = o;
      if (p.out) *reinterpret_cast<v4f*>(p.out + (size_t)row * H + j) = o;
      if (p.ph) store_planes4(p.ph, p.pl, (size_t)row * p.ldp + j, o);
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(o[0]), fabsf(o[1])), fmaxf(fabsf(o[2]), fabsf(o[3]))));
    }
  }
  if (p.qa) {  // QuantizeRowU8 (pack_vnni.go:85-117) of the normalized row
    mx = wmax(mx);
    float scale = mx / 127.0f;
    if (scale == 0.0f) scale = 1.0f;
    const float qinv = 1.0f / scale;
    uint8_t* q = p.qa + (size_t)row * p.ldq;
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int j = (lane + 64 * e) * 4;
      if (j < H)
        *reinterpret_cast<uint32_t*>(q + j) =
            (uint32_t)qbyte(v[e][0], qinv) | ((uint32_t)qbyte(v[e][1], qinv) << 8) |
            ((uint32_t)qbyte(v[e][2], qinv) << 16) | ((uint32_t)qbyte(v[e][3], qinv) << 24);
    }
    for (int j = H + lane * 4; j < p.ldq; j += 256) *reinterpret_cast<uint32_t*>(q + j) = 0u;
    if (lane == 0) p.row_scales[row] = scale;
  }
}

hipError_t launch_rms_residual(const RmsArgs& a, hipStream_t s) {
  if (a.m <= 0) return hipSuccess;
  if (a.H % 4 || a.H > 4096 || (a.qa && a.ldq % 4) || (a.ph && (a.ldp % 64 || a.ldp < a.H)) ||
      (a.layer_norm && a.post_g))
    return hipErrorInvalidValue;
  const dim3 grid(ceil_div(a.m, kRows)), block(256);
  const int v = ceil_div(a.H, 256);
  if (v <= 1) hipLaunchKernelGGL((rms_residual_kernel<1>), grid, block, 0, s, a);
  else if (v <= 2) hipLaunchKernelGGL((rms_residual_kernel<2>), grid, block, 0, s, a);
  else if (v <= 3) hipLaunchKernelGGL((rms_residual_kernel<3>), grid, block, 0, s, a);
  else if (v <= 4) hipLaunchKernelGGL((rms_residual_kernel<4>), grid, block, 0, s, a);
  else if (v <= 8) hipLaunchKernelGGL((rms_residual_kernel<8>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((rms_residual_kernel<16>), grid, block, 0, s, a);
  return hipGetLastError();
}

// ---- QK-norm + RoPE -----------------------------------------------------------------
// Items are (row, head) over the q heads then the k heads of a fused q|k|v
// row: RMSNorm of the head's dh values with its norm weight (none when the
// norm weights are null: nomic and ModernBERT rotate the raw projections,
// nomic.go:210-211, modernbert.go:256-257), then rotate-half RoPE at the
// row's position (applyRoPE, modernbert.go:130-143: each product rounded to
// float32 before the add). With `outh` the results
// go to bf16 rows of the same layout instead (round to nearest even), and
// the v heads are converted too: the operands of a bf16 attention.
// A wave takes kQkItems consecutive items, loading all of them before it
// reduces, so their memory latencies overlap.
constexpr int kQkItems = 4;

__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    float* __restrict__ qkv, int ldqkv, int m, int nq, int nkv, int dh,
    const float* __restrict__ q_g, const float* __restrict__ k_g, float eps,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const int32_t* __restrict__ pos, __bf16* __restrict__ outh) {
  const int lane = threadIdx.x & 63;
  const int item0 = (blockIdx.x * kRows + (threadIdx.x >> 6)) * kQkItems;
  const int nh = nq + nkv + (outh ? nkv : 0);
  const int total = m * nh;
  const int half = dh >> 1;
  // lane holds pairs (d, d + half) for d = lane, lane + 64 (dh <= 256)
  float x1[kQkItems][2], x2[kQkItems][2];
#pragma unroll
  for (int it = 0; it < kQkItems; it++) {
    const int item = min(item0 + it, total - 1);
    const float* v = qkv + (size_t)(item / nh) * ldqkv + (item % nh) * dh;
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const int d = lane + 64 * e;
      x1[it][e] = d < half ? v[d] : 0.0f;
      x2[it][e] = d < half ? v[d + half] : 0.0f;
    }
  }
#pragma unroll
  for (int it = 0; it < kQkItems; it++) {
    const int item = item0 + it;
    if (item >= total) return;
    const int row = item / nh, h = item % nh;
    float* v = qkv + (size_t)row * ldqkv + h * dh;
    __bf16* o = outh ? outh + (size_t)row * ldqkv + h * dh : nullptr;
    if (h >= nq + nkv) {  // v head: conversion only
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const int d = lane + 64 * e;
        if (d < half) {
          o[d] = (__bf16)x1[it][e];
          o[d + half] = (__bf16)x2[it][e];
        }
      }
      continue;
    }
    const float* g = h < nq ? q_g : k_g;  // null: no QK-norm, RoPE only
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 2; e++) ss += x1[it][e] * x1[it][e] + x2[it][e] * x2[it][e];
    const float inv = rms_inv(wsum(ss), dh, eps);
    const int p = pos[row];
    const float* c = cos_t + (size_t)p * half;
    const float* sn = sin_t + (size_t)p * half;
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const int d = lane + 64 * e;
      if (d < half) {
        const float a = g ? x1[it][e] * inv * g[d] : x1[it][e];
        const float b = g ? x2[it][e] * inv * g[d + half] : x2[it][e];
        const float cc = c[d], ssn = sn[d];
        const float t0 = a * cc, t1 = b * ssn, t2 = b * cc, t3 = a * ssn;
        if (o) {
          o[d] = (__bf16)(t0 - t1);
          o[d + half] = (__bf16)(t2 + t3);
        } else {
          v[d] = t0 - t1;
          v[d + half] = t2 + t3;
        }
      }
    }
  }
}

// Vector form for dh in {64, 128, 256}: one workgroup per row; a head is
// dh/4 consecutive lanes holding 4 columns each (16-byte loads, 8- or
// 16-byte stores), so a wave covers 64/(dh/4) heads at once. The head's
// sum of squares reduces over its lanes; lane l and l ^ (dh/8) hold the
// RoPE pair (d, d + dh/2). Same per-element operations as the scalar form
// (only the sum of squares is added in another order).
template <int DH>
__global__ __launch_bounds__(256) void qk_norm_rope_vec_kernel(
    float* __restrict__ qkv, int ldqkv, int nq, int nkv, const float* __restrict__ q_g,
    const float* __restrict__ k_g, float eps, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, const int32_t* __restrict__ pos,
    __bf16* __restrict__ outh) {
  typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
  constexpr int LPH = DH / 4;    // lanes per head
  constexpr int HPW = 64 / LPH;  // heads per wave
  constexpr int HALF = DH / 2;
  constexpr int IT = 4;          // passes whose loads are issued together
  const int row = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l = lane % LPH, d = l * 4;
  const int nh = nq + nkv + (outh ? nkv : 0);
  float* rowp = qkv + (size_t)row * ldqkv;
  const int p = pos[row];
  for (int base = 0; base < nh; base += IT * 4 * HPW) {
    v4f x[IT];
#pragma unroll
    for (int it = 0; it < IT; it++) {
      const int h = base + (it * 4 + wave) * HPW + lane / LPH;
      x[it] = h < nh ? *reinterpret_cast<const v4f*>(rowp + h * DH + d)
                     : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int it = 0; it < IT; it++) {
      const int h0 = base + (it * 4 + wave) * HPW;  // first head of this wave's pass
      if (h0 >= nh) break;
      const int h = h0 + lane / LPH;
      const size_t off = (size_t)row * ldqkv + h * DH + d;
      float ss = (x[it][0] * x[it][0] + x[it][1] * x[it][1]) +
                 (x[it][2] * x[it][2] + x[it][3] * x[it][3]);
#pragma unroll
      for (int o = LPH / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
      if (h >= nh) continue;
      if (h >= nq + nkv) {  // v head: conversion only
        *reinterpret_cast<v4bf*>(outh + off) =
            v4bf{(__bf16)x[it][0], (__bf16)x[it][1], (__bf16)x[it][2], (__bf16)x[it][3]};
        continue;
      }
      const float inv = rms_inv(ss, DH, eps);
      const float* gp = h < nq ? q_g : k_g;  // null: no QK-norm, RoPE only
      v4f xn, pn;
      if (gp) {
        const v4f g = *reinterpret_cast<const v4f*>(gp + d);
#pragma unroll
        for (int c = 0; c < 4; c++) xn[c] = x[it][c] * inv * g[c];
      } else {
        xn = x[it];
      }
#pragma unroll
      for (int c = 0; c < 4; c++) pn[c] = __shfl_xor(xn[c], LPH / 2, 64);
      const bool first = l < LPH / 2;  // columns d < dh/2
      const int dp = first ? d : d - HALF;
      const v4f cc = *reinterpret_cast<const v4f*>(cos_t + (size_t)p * HALF + dp);
      const v4f sn = *reinterpret_cast<const v4f*>(sin_t + (size_t)p * HALF + dp);
      v4f o;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float a = first ? xn[c] : pn[c], b = first ? pn[c] : xn[c];
        o[c] = first ? a * cc[c] - b * sn[c] : b * cc[c] + a * sn[c];
      }
      if (outh)
        *reinterpret_cast<v4bf*>(outh + off) =
            v4bf{(__bf16)o[0], (__bf16)o[1], (__bf16)o[2], (__bf16)o[3]};
      else
        *reinterpret_cast<v4f*>(qkv + off) = o;
    }
  }
}

hipError_t launch_qk_norm_rope(float* qkv, int ldqkv, int m, int nq, int nkv, int dh,
                               const float* q_g, const float* k_g, float eps,
                               const float* cos_t, const float* sin_t,
                               const int32_t* pos, __bf16* outh, hipStream_t s) {
  if (m <= 0) return hipSuccess;
  if (dh % 2 || dh > 256) return hipErrorInvalidValue;
  const bool vec = ldqkv % 4 == 0 && ((reinterpret_cast<uintptr_t>(qkv) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(outh) & 7) == 0);
  if (vec && (dh == 64 || dh == 128 || dh == 256)) {
    if (dh == 64)
      hipLaunchKernelGGL((qk_norm_rope_vec_kernel<64>), dim3(m), dim3(256), 0, s, qkv, ldqkv, nq,
                         nkv, q_g, k_g, eps, cos_t, sin_t, pos, outh);
    else if (dh == 128)
      hipLaunchKernelGGL((qk_norm_rope_vec_kernel<128>), dim3(m), dim3(256), 0, s, qkv, ldqkv,
                         nq, nkv, q_g, k_g, eps, cos_t, sin_t, pos, outh);
    else
      hipLaunchKernelGGL((qk_norm_rope_vec_kernel<256>), dim3(m), dim3(256), 0, s, qkv, ldqkv,
                         nq, nkv, q_g, k_g, eps, cos_t, sin_t, pos, outh);
    return hipGetLastError();
  }
  const int items = m * (nq + nkv + (outh ? nkv : 0));
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(ceil_div(items, kRows * kQkItems)), dim3(256), 0,
                     s, qkv, ldqkv, m, nq, nkv, dh, q_g, k_g, eps, cos_t, sin_t, pos, outh);
  return hipGetLastError();
}

// ---- EmbeddingGemma Dense head --------------------------------------------------------
// applyGemmaDenseHead (gemma3.go:174-198): hid[o] = sum_i w1[o][i] * pooled[i],
// out[o] = sum_i w2[o][i] * hid[i], each a sequential float32 sum in ascending
// i (no FMA). One thread per (text, output) over transposed weights
// (wT[i][o], so a wave's loads of one i are contiguous); the text's input
// vector is staged in LDS.
__global__ __launch_bounds__(256) void dense_matvec_kernel(const float* __restrict__ wT,
                                                           int in, int outn,
                                                           const float* __restrict__ x,
                                                           float* __restrict__ y) {
  extern __shared__ float xs[];  // in floats
  const int b = blockIdx.y;
  for (int i = threadIdx.x; i < in; i += 256) xs[i] = x[(size_t)b * in + i];
  __syncthreads();
  const int o = blockIdx.x * 256 + threadIdx.x;
  if (o >= outn) return;
  const float* w = wT + o;
  // The sum runs i = 0, 1, ... as in the reference; only the loads run
  // ahead: two register blocks of U weights, the next block's loads in
  // flight while the current one is summed (each thread's chain waited on
  // every block's memory latency before).
  constexpr int U = 32;
  float acc = 0.0f;
  int i = 0;
  float ta[U], tb[U];
  auto fill = [&](float (&t)[U], int i0) {
#pragma unroll
    for (int e = 0; e < U; e++) t[e] = w[(size_t)(i0 + e) * outn];
  };
  auto sum = [&](const float (&t)[U], int i0) {
#pragma unroll
    for (int e = 0; e < U; e++) acc = acc + t[e] * xs[i0 + e];
  };
  if (in >= U) fill(ta, 0);
  for (; i + 2 * U <= in; i += 2 * U) {
    fill(tb, i + U);
    sum(ta, i);
    if (i + 3 * U <= in) fill(ta, i + 2 * U);
    sum(tb, i + U);
  }
  if (i + U <= in) {  // one loaded block left
    sum(ta, i);
    i += U;
  }
  for (; i < in; i++) acc = acc + w[(size_t)i * outn] * xs[i];
  y[(size_t)b * outn + o] = acc;
}

hipError_t launch_dense_head(const float* pooled, int batch, int H, int D, const float* w1T,
                             const float* w2T, int normalize, float* hid, float* out,
                             hipStream_t s) {
  if (batch <= 0) return hipSuccess;
  if ((size_t)std::max(H, D) * sizeof(float) > 64 * 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(dense_matvec_kernel, dim3(ceil_div(D, 256), batch), dim3(256),
                     H * sizeof(float), s, w1T, H, D, pooled, hid);
  hipLaunchKernelGGL(dense_matvec_kernel, dim3(ceil_div(H, 256), batch), dim3(256),
                     D * sizeof(float), s, w2T, D, H, hid, out);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess && normalize) e = launch_l2_rows(out, batch, H, s);
  return e;
}

// Gated-MLP glue over separate gate and up rows (qwen3.go:530-539,
// gemma3.go:365-374): out = act(gate) * up element by element, with the same
// float32 glu_act the fused gated epilogues apply, so the result equals the
// fused form bit for bit. Used when newDense packed gate and up in different
// modes. out may alias gate.
__global__ void glu_rows_kernel(const float* gate, const float* up, float* out, size_t n,
                                int act) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = glu_act(gate[i], up[i], act);
}

hipError_t launch_glu_rows(const float* gate, const float* up, float* out, size_t n, int act,
                           hipStream_t s) {
  if (n == 0) return hipSuccess;
  if (!is_glu(act)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(glu_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, gate,
                     up, out, n, act);
  return hipGetLastError();
}

}  // namespace rh
