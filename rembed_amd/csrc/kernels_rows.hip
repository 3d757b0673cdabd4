// kernels_rows.hip — row-wise kernels that keep activations in HBM between
// the GEMMs: activation quantization, embeddings + LayerNorm, residual add +
// LayerNorm (each optionally fused with the next GEMM's u8 quantization),
// pooling + L2 normalization, and the standalone GELU / bias passes.
//
// One 64-lane wave owns one row; lane l holds columns l, l+64, l+128, ...
#include "gemm_common.h"
#include "rows_common.h"

namespace rh {

constexpr int kRowsPerBlock = 4;  // 256 threads = 4 waves = 4 rows
constexpr int kMaxPerLane = 32;   // rows up to 2048 wide stay in registers

// Generic quantizer over rows of any width (two passes over the row; the
// second pass hits L2). Writes ldq bytes per row: k quantized + zero tail.
// `act` is applied to each element first (the activation of the GEMM that
// produced the row, moved here where the kernel has VALU to spare).
__global__ __launch_bounds__(256) void quantize_rows_kernel(
    const float* __restrict__ a, int lda, int m, int k, uint8_t* __restrict__ qa,
    int ldq, float* __restrict__ row_scales, int vec, int act) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= m) return;
  const float* src = a + (size_t)row * lda;
  float mx = 0.0f;
  for (int i = lane; i < k; i += 64) mx = fmaxf(mx, fabsf(apply_act(src[i], act)));
  mx = wave_max(mx);
  float scale = mx / 127.0f;
  if (scale == 0.0f) scale = 1.0f;
  const float inv = 1.0f / scale;
  uint8_t* dst = qa + (size_t)row * ldq;
  if (vec) {
    for (int i = lane * 4; i < k; i += 256) {
      v4f v = *reinterpret_cast<const v4f*>(src + i);
#pragma unroll
      for (int e = 0; e < 4; e++) v[e] = apply_act(v[e], act);
      uint32_t w = (uint32_t)quant_u8(v[0], inv) | ((uint32_t)quant_u8(v[1], inv) << 8) |
                   ((uint32_t)quant_u8(v[2], inv) << 16) |
                   ((uint32_t)quant_u8(v[3], inv) << 24);
      *reinterpret_cast<uint32_t*>(dst + i) = w;
    }
  } else {
    for (int i = lane; i < k; i += 64) dst[i] = quant_u8(apply_act(src[i], act), inv);
  }
  for (int i = k + lane; i < ldq; i += 64) dst[i] = 0;
  if (lane == 0) row_scales[row] = scale;
}

// Single-pass variant for 16-byte aligned rows with k % 4 == 0 and
// k <= 256 * V: the row stays in registers (V float4 per lane), so HBM sees
// one read of the row and one write of its bytes.
template <int V, bool GELU>
__global__ __launch_bounds__(256) void quantize_rows_vec_kernel(
    const float* __restrict__ a, int lda, int m, int k, uint8_t* __restrict__ qa,
    int ldq, float* __restrict__ row_scales) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= m) return;
  const float* src = a + (size_t)row * lda;
  v4f x[V];
  float mx = 0.0f;
#pragma unroll
  for (int e = 0; e < V; e++) {
    const int i = (lane + 64 * e) * 4;
    x[e] = i < k ? *reinterpret_cast<const v4f*>(src + i) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (GELU) {
#pragma unroll
      for (int c = 0; c < 4; c++) x[e][c] = apply_act(x[e][c], ACT_GELU);
    }
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(x[e][0]), fabsf(x[e][1])), fmaxf(fabsf(x[e][2]), fabsf(x[e][3]))));
  }
  mx = wave_max(mx);
  float scale = mx / 127.0f;
  if (scale == 0.0f) scale = 1.0f;
  const float inv = 1.0f / scale;
  uint8_t* dst = qa + (size_t)row * ldq;
#pragma unroll
  for (int e = 0; e < V; e++) {
    const int i = (lane + 64 * e) * 4;
    if (i < k)
      *reinterpret_cast<uint32_t*>(dst + i) =
          (uint32_t)quant_u8(x[e][0], inv) | ((uint32_t)quant_u8(x[e][1], inv) << 8) |
          ((uint32_t)quant_u8(x[e][2], inv) << 16) | ((uint32_t)quant_u8(x[e][3], inv) << 24);
  }
  for (int i = k + lane * 4; i < ldq; i += 256) *reinterpret_cast<uint32_t*>(dst + i) = 0u;
  if (lane == 0) row_scales[row] = scale;
}

template <int V>
static void launch_qvec(const float* a, int lda, int m, int k, uint8_t* qa, int ldq,
                        float* rs, int act, hipStream_t s) {
  if (act == ACT_GELU)
    hipLaunchKernelGGL((quantize_rows_vec_kernel<V, true>), dim3(ceil_div(m, kRowsPerBlock)),
                       dim3(256), 0, s, a, lda, m, k, qa, ldq, rs);
  else
    hipLaunchKernelGGL((quantize_rows_vec_kernel<V, false>), dim3(ceil_div(m, kRowsPerBlock)),
                       dim3(256), 0, s, a, lda, m, k, qa, ldq, rs);
}

hipError_t launch_quantize_rows_u8(const float* a, int lda, int m, int k,
                                   uint8_t* qa, int ldq, float* row_scales,
                                   hipStream_t s, int act) {
  if (m <= 0) return hipSuccess;
  if (act != ACT_NONE && act != ACT_GELU) return hipErrorInvalidValue;
  // 16-byte row loads and 4-byte stores need aligned rows.
  const int vec = (k % 4 == 0) && (lda % 4 == 0) && (ldq % 4 == 0) &&
                  ((reinterpret_cast<uintptr_t>(a) & 15) == 0) &&
                  ((reinterpret_cast<uintptr_t>(qa) & 3) == 0);
  if (vec && k <= 4096) {
    const int v = ceil_div(k, 256);
    if (v <= 1) launch_qvec<1>(a, lda, m, k, qa, ldq, row_scales, act, s);
    else if (v <= 2) launch_qvec<2>(a, lda, m, k, qa, ldq, row_scales, act, s);
    else if (v <= 3) launch_qvec<3>(a, lda, m, k, qa, ldq, row_scales, act, s);
    else if (v <= 4) launch_qvec<4>(a, lda, m, k, qa, ldq, row_scales, act, s);
    else if (v <= 6) launch_qvec<6>(a, lda, m, k, qa, ldq, row_scales, act, s);
    else if (v <= 8) launch_qvec<8>(a, lda, m, k, qa, ldq, row_scales, act, s);
    else if (v <= 12) launch_qvec<12>(a, lda, m, k, qa, ldq, row_scales, act, s);
    else launch_qvec<16>(a, lda, m, k, qa, ldq, row_scales, act, s);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(quantize_rows_kernel, dim3(ceil_div(m, kRowsPerBlock)),
                     dim3(256), 0, s, a, lda, m, k, qa, ldq, row_scales, vec, act);
  return hipGetLastError();
}

// LayerNorm of the row held in v[] (tensor.go:433-452: biased variance,
// inv = 1/float32(sqrt(var+eps)), out = (v-mean)*inv*g + b), then optional
// quantization of the normalized row into qa/row_scales.
__device__ __forceinline__ void ln_row_finish(float (&v)[kMaxPerLane], int lane,
                                              int H, const float* gamma,
                                              const float* beta, float eps,
                                              float* out, uint8_t* qa, int ldq,
                                              float* rs_out) {
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < kMaxPerLane; e++)
    if (lane + 64 * e < H) s += v[e];
  const float mean = wave_sum(s) / (float)H;
  float s2 = 0.0f;
#pragma unroll
  for (int e = 0; e < kMaxPerLane; e++)
    if (lane + 64 * e < H) {
      const float d = v[e] - mean;
      s2 += d * d;
    }
  const float var = wave_sum(s2) / (float)H;
  const float inv = 1.0f / sqrtf(var + eps);
  float mx = 0.0f;
#pragma unroll
  for (int e = 0; e < kMaxPerLane; e++) {
    const int j = lane + 64 * e;
    if (j < H) {
      const float y = (v[e] - mean) * inv * gamma[j] + beta[j];
      v[e] = y;
      out[j] = y;
      mx = fmaxf(mx, fabsf(y));
    }
  }
  if (qa) {
    mx = wave_max(mx);
    float scale = mx / 127.0f;
    if (scale == 0.0f) scale = 1.0f;
    const float qinv = 1.0f / scale;
#pragma unroll
    for (int e = 0; e < kMaxPerLane; e++) {
      const int j = lane + 64 * e;
      if (j < H) qa[j] = quant_u8(v[e], qinv);
    }
    for (int j = H + lane; j < ldq; j += 64) qa[j] = 0;
    if (lane == 0) *rs_out = scale;
  }
}

__global__ __launch_bounds__(256) void embed_ln_kernel(EmbedArgs p, int total) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= total) return;
  // text b with cu[b] <= row < cu[b+1]
  int lo = 0, hi = p.batch;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (p.cu[mid] <= row) lo = mid;
    else hi = mid;
  }
  const int b = lo, t = row - p.cu[b];
  int id = p.ids[(size_t)b * p.stride + t];
  if (id < 0 || id >= p.vocab) {
    if (lane == 0) *p.err_flag = 1;
    id = id < 0 ? 0 : p.vocab - 1;  // stay in bounds; the call reports failure
  }
  const float* w = p.word + (size_t)id * p.H;
  const float* ps = p.pos + (size_t)(t + p.pos_off) * p.H;
  float v[kMaxPerLane];
#pragma unroll
  for (int e = 0; e < kMaxPerLane; e++) {
    const int j = lane + 64 * e;
    // bert.go:801-812: row = w + p (+ t)
    if (j < p.H) v[e] = p.type0 ? (w[j] + ps[j]) + p.type0[j] : w[j] + ps[j];
    else v[e] = 0.0f;
  }
  ln_row_finish(v, lane, p.H, p.gamma, p.beta, p.eps, p.x + (size_t)row * p.H,
                p.qa ? p.qa + (size_t)row * p.ldq : nullptr, p.ldq,
                p.row_scales ? p.row_scales + row : nullptr);
}


__global__ __launch_bounds__(256) void add_ln_kernel(
    float* __restrict__ x, const float* __restrict__ y, int ldy,
    const float* __restrict__ gamma, const float* __restrict__ beta, int m,
    int H, float eps, uint8_t* __restrict__ qa, int ldq,
    float* __restrict__ row_scales) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= m) return;
  float* xr = x + (size_t)row * H;
  const float* yr = y ? y + (size_t)row * ldy : nullptr;
  float v[kMaxPerLane];
#pragma unroll
  for (int e = 0; e < kMaxPerLane; e++) {
    const int j = lane + 64 * e;
    v[e] = j < H ? (yr ? xr[j] + yr[j] : xr[j]) : 0.0f;  // Add, tensor.go:383-387
  }
  ln_row_finish(v, lane, H, gamma, beta, eps, xr,
                qa ? qa + (size_t)row * ldq : nullptr, ldq,
                row_scales ? row_scales + row : nullptr);
}

// float4 variant for H % 4 == 0 (every encoder width): lane l holds columns
// 4(l + 64e) .. +3. With ph the normalized row also goes to the bf16 hi/lo
// planes [m][ldp] of the next weight-only int8 / fp32 GEMM's input (pl may
// be null).
// R rows per wave: every row's loads are issued before the first row's
// reductions.
template <int V, int R = 1>
__global__ __launch_bounds__(256) void add_ln_vec_kernel(
    float* __restrict__ x, const float* __restrict__ y, int ldy,
    const float* __restrict__ gamma, const float* __restrict__ beta, int m,
    int H, float eps, uint8_t* __restrict__ qa, int ldq,
    float* __restrict__ row_scales, __bf16* __restrict__ ph, __bf16* __restrict__ pl,
    int ldp) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6)) * R;
  if (row0 >= m) return;
  v4f v[R][V];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int row = row0 + r < m ? row0 + r : row0;
    const float* xr = x + (size_t)row * H;
    const float* yr = y ? y + (size_t)row * ldy : nullptr;
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int j = (lane + 64 * e) * 4;
      v4f t = {0.0f, 0.0f, 0.0f, 0.0f};
      if (j < H) {
        t = *reinterpret_cast<const v4f*>(xr + j);
        if (yr) t = t + *reinterpret_cast<const v4f*>(yr + j);  // Add, tensor.go:383-387
      }
      v[r][e] = t;
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int row = row0 + r;
    if (row < m)
      ln_vec_finish<V>(v[r], lane, row, H, gamma, beta, eps, x + (size_t)row * H, qa, ldq,
                       row_scales, ph, pl, ldp);
  }
}

// Embeddings + LayerNorm, float4 rows (H % 4 == 0, 16-byte aligned tables).
// The row's text is the number of text starts cu[1..batch-1] at or before
// it, counted by one ballot per 64 texts (no dependent loads).
template <int V>
__global__ __launch_bounds__(256) void embed_ln_vec_kernel(EmbedArgs p, int total) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= total) return;
  int b = 0;
  for (int base = 1; base < p.batch; base += 64) {
    const int i = base + lane;
    b += __popcll(__ballot(i < p.batch && p.cu[i] <= row));
  }
  const int t = row - p.cu[b];
  int id = p.ids[(size_t)b * p.stride + t];
  if (id < 0 || id >= p.vocab) {
    if (lane == 0) *p.err_flag = 1;
    id = id < 0 ? 0 : p.vocab - 1;  // stay in bounds; the call reports failure
  }
  const float* w = p.word + (size_t)id * p.H;
  const float* ps = p.pos + (size_t)(t + p.pos_off) * p.H;
  v4f v[V];
#pragma unroll
  for (int e = 0; e < V; e++) {
    const int j = (lane + 64 * e) * 4;
    v4f r = {0.0f, 0.0f, 0.0f, 0.0f};
    if (j < p.H) {
      // bert.go:801-812: row = w + p (+ t)
      r = *reinterpret_cast<const v4f*>(w + j) + *reinterpret_cast<const v4f*>(ps + j);
      if (p.type0) r = r + *reinterpret_cast<const v4f*>(p.type0 + j);
    }
    v[e] = r;
  }
  ln_vec_finish<V>(v, lane, row, p.H, p.gamma, p.beta, p.eps, p.x + (size_t)row * p.H,
                   p.qa, p.ldq, p.row_scales, p.ph, p.pl, p.ldp);
}

// ---- LayerNorm in the reference's own order ---------------------------------
// tensor.go:433-452 sums each row left to right in float32: once for the mean,
// once for the variance (d*d rounded, then added). R rows per one-wave
// workgroup: the rows arrive coalesced in registers (lane l holds columns
// 4(l + 64e) .. +3) and are parked in LDS; lane r < R walks row r's two sums
// serially (the only serial part); the normalization itself runs coalesced
// again (ln_vec_apply). inv = 1/float32(sqrt(float64(var+eps))).
// s += the 32 values of a, one at a time in index order.
__device__ __forceinline__ void add_in_order(float& s, const v4f (&a)[8]) {
#pragma unroll
  for (int u = 0; u < 8; u++) {
    s = s + a[u][0];
    s = s + a[u][1];
    s = s + a[u][2];
    s = s + a[u][3];
  }
}

__device__ __forceinline__ void load32(v4f (&a)[8], const float* p) {
#pragma unroll
  for (int u = 0; u < 8; u++) a[u] = *reinterpret_cast<const v4f*>(p + 4 * u);
}

// Float32 sum of rp[0..n) in column order, one dependent add per element
// (n % 4 == 0, rp 16-byte aligned, in LDS). The next 32 values are read
// while the current 32 are added, so the LDS latency stays off the chain.
__device__ __forceinline__ float serial_sum(const float* rp, int n) {
  float s = 0.0f;
  v4f a[8], b[8];  // two blocks of 32 values in turn
  const int n32 = n & ~31;
  if (n32) load32(a, rp);
  for (int j = 0; j < n32; j += 64) {
    if (j + 32 < n32) load32(b, rp + j + 32);
    add_in_order(s, a);
    if (j + 32 >= n32) break;
    if (j + 64 < n32) load32(a, rp + j + 64);
    add_in_order(s, b);
  }
  for (int j = n32; j < n; j += 4) {
    const v4f v = *reinterpret_cast<const v4f*>(rp + j);
    s = s + v[0];
    s = s + v[1];
    s = s + v[2];
    s = s + v[3];
  }
  return s;
}

template <int V, int R>
__device__ __forceinline__ void ln_exact_rows(v4f (&v)[R][V], int row0, int nrows, int H,
                                              float eps, const float* __restrict__ gamma,
                                              const float* __restrict__ beta, float* x,
                                              uint8_t* qa, int ldq, float* rs, __bf16* ph,
                                              __bf16* pl, int ldp) {
  // row pitch: 16 bytes past a multiple of 1 KiB, so the R lanes' float4
  // reads of one column group fall in distinct banks
  constexpr int S = V * 256 + 4;
  __shared__ __attribute__((aligned(16))) float rowbuf[R * S];
  __shared__ float stat[2 * R];
  const int lane = threadIdx.x;
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int j = (lane + 64 * e) * 4;
      if (j < H) *reinterpret_cast<v4f*>(rowbuf + r * S + j) = v[r][e];
    }
  __syncthreads();
  if (lane < R) stat[lane] = serial_sum(rowbuf + lane * S, H) / (float)H;  // mean
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; r++) {
    const float mean = stat[r];
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int j = (lane + 64 * e) * 4;
      if (j < H) {
        const v4f d = v[r][e] - mean;
        *reinterpret_cast<v4f*>(rowbuf + r * S + j) = d * d;
      }
    }
  }
  __syncthreads();
  if (lane < R) {  // variance: the rounded squares summed in column order
    const float var = serial_sum(rowbuf + lane * S, H) / (float)H;
    stat[R + lane] = 1.0f / (float)sqrt((double)(var + eps));
  }
  __syncthreads();
  // ln_vec_apply's arithmetic for the R rows at once: gamma and beta loaded
  // once, the rows' |max| reductions interleaved (one row at a time left
  // each row's loads and shuffles waiting on the previous row's)
  v4f g[V], bb[V];
#pragma unroll
  for (int e = 0; e < V; e++) {
    const int j = min((lane + 64 * e) * 4, H - 4);
    g[e] = *reinterpret_cast<const v4f*>(gamma + j);
    bb[e] = *reinterpret_cast<const v4f*>(beta + j);
  }
  float mx[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    mx[r] = 0.0f;
    const float mean = stat[r], inv = stat[R + r];
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int j = (lane + 64 * e) * 4;
      if (j < H) {
        v4f o;
#pragma unroll
        for (int c = 0; c < 4; c++) o[c] = (v[r][e][c] - mean) * inv * g[e][c] + bb[e][c];
        v[r][e] = o;
        mx[r] = fmaxf(mx[r], fmaxf(fmaxf(fabsf(o[0]), fabsf(o[1])), fmaxf(fabsf(o[2]), fabsf(o[3]))));
        if (r < nrows) {
          const int row = row0 + r;
          *reinterpret_cast<v4f*>(x + (size_t)row * H + j) = o;
          if (ph) store_planes4(ph, pl, (size_t)row * ldp + j, o);
        }
      }
    }
  }
  if (qa) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
#pragma unroll
      for (int r = 0; r < R; r++) mx[r] = fmaxf(mx[r], __shfl_xor(mx[r], o, 64));
#pragma unroll
    for (int r = 0; r < R; r++) {
      if (r >= nrows) continue;
      const int row = row0 + r;
      float scale = mx[r] / 127.0f;
      if (scale == 0.0f) scale = 1.0f;
      const float qinv = 1.0f / scale;
      uint8_t* q = qa + (size_t)row * ldq;
#pragma unroll
      for (int e = 0; e < V; e++) {
        const int j = (lane + 64 * e) * 4;
        if (j < H)
          *reinterpret_cast<uint32_t*>(q + j) =
              (uint32_t)quant_u8(v[r][e][0], qinv) | ((uint32_t)quant_u8(v[r][e][1], qinv) << 8) |
              ((uint32_t)quant_u8(v[r][e][2], qinv) << 16) |
              ((uint32_t)quant_u8(v[r][e][3], qinv) << 24);
      }
      for (int j = H + lane * 4; j < ldq; j += 256) *reinterpret_cast<uint32_t*>(q + j) = 0u;
      if (lane == 0) rs[row] = scale;
    }
  }
}

template <int V, int R>
__global__ __launch_bounds__(64) void add_ln_exact_kernel(
    float* __restrict__ x, const float* __restrict__ y, int ldy,
    const float* __restrict__ gamma, const float* __restrict__ beta, int m, int H, float eps,
    uint8_t* __restrict__ qa, int ldq, float* __restrict__ row_scales,
    __bf16* __restrict__ ph, __bf16* __restrict__ pl, int ldp) {
  const int lane = threadIdx.x;
  const int row0 = blockIdx.x * R;
  // Every load of the workgroup's rows is issued before any is used (clamped
  // in-bounds addresses, out-of-range slots zeroed afterwards): a load
  // guarded together with its use would wait for each row in turn.
  v4f v[R][V];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int j = min((lane + 64 * e) * 4, H - 4);
      v[r][e] = *reinterpret_cast<const v4f*>(x + (size_t)min(row0 + r, m - 1) * H + j);
    }
  if (y) {  // Add
    v4f w[R][V];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
      for (int e = 0; e < V; e++) {
        const int j = min((lane + 64 * e) * 4, H - 4);
        w[r][e] = *reinterpret_cast<const v4f*>(y + (size_t)min(row0 + r, m - 1) * ldy + j);
      }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
      for (int e = 0; e < V; e++) v[r][e] = v[r][e] + w[r][e];
  }
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int e = 0; e < V; e++)
      if (row0 + r >= m || (lane + 64 * e) * 4 >= H) v[r][e] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  ln_exact_rows<V, R>(v, row0, min(R, m - row0), H, eps, gamma, beta, x, qa, ldq, row_scales,
                      ph, pl, ldp);
}

template <int V, int R>
__global__ __launch_bounds__(64) void embed_ln_exact_kernel(EmbedArgs p, int total) {
  const int lane = threadIdx.x;
  const int row0 = blockIdx.x * R;
  v4f v[R][V];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int row = min(row0 + r, total - 1);
    int b = 0;
    for (int base = 1; base < p.batch; base += 64) {
      const int i = base + lane;
      b += __popcll(__ballot(i < p.batch && p.cu[i] <= row));
    }
    const int t = row - p.cu[b];
    int id = p.ids[(size_t)b * p.stride + t];
    if (id < 0 || id >= p.vocab) {
      if (lane == 0) *p.err_flag = 1;
      id = id < 0 ? 0 : p.vocab - 1;  // stay in bounds; the call reports failure
    }
    const float* w = p.word + (size_t)id * p.H;
    const float* ps = p.pos + (size_t)(t + p.pos_off) * p.H;
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int j = (lane + 64 * e) * 4;
      v4f a = {0.0f, 0.0f, 0.0f, 0.0f};
      if (j < p.H) {
        // bert.go:801-812: row = w + p (+ t)
        a = *reinterpret_cast<const v4f*>(w + j) + *reinterpret_cast<const v4f*>(ps + j);
        if (p.type0) a = a + *reinterpret_cast<const v4f*>(p.type0 + j);
      }
      v[r][e] = a;
    }
  }
  ln_exact_rows<V, R>(v, row0, min(R, total - row0), p.H, p.eps, p.gamma, p.beta, p.x, p.qa,
                      p.ldq, p.row_scales, p.ph, p.pl, p.ldp);
}

// rows per one-wave workgroup of the exact LayerNorm: each row's serial sums
// set a wave's critical path whatever R is, and fewer rows per wave shorten
// its apply phase (BERT-base at M = 10102: 25.4 µs with 4, 29.9 with 2, 28.8
// with 8, 35.3 with 16)
constexpr int kExactRows = 4;

hipError_t launch_embed_layernorm(const EmbedArgs& a, int total, hipStream_t s) {
  if (total <= 0) return hipSuccess;
  if (a.H > 64 * kMaxPerLane) return hipErrorInvalidValue;
  const bool vec = a.H % 4 == 0 && (!a.qa || a.ldq % 4 == 0) &&
                   ((reinterpret_cast<uintptr_t>(a.word) | reinterpret_cast<uintptr_t>(a.pos) |
                     reinterpret_cast<uintptr_t>(a.type0) | reinterpret_cast<uintptr_t>(a.gamma) |
                     reinterpret_cast<uintptr_t>(a.beta) | reinterpret_cast<uintptr_t>(a.x)) &
                    15) == 0;
  if (a.ph && (!vec || a.ldp % 64 || a.ldp < a.H)) return hipErrorInvalidValue;
  const int v = ceil_div(a.H, 256);
  if (a.exact) {
    if (!vec || v > 4) return hipErrorInvalidValue;
    constexpr int R = kExactRows;
    const dim3 g(ceil_div(total, R)), b(64);
    if (v <= 1) hipLaunchKernelGGL((embed_ln_exact_kernel<1, R>), g, b, 0, s, a, total);
    else if (v <= 2) hipLaunchKernelGGL((embed_ln_exact_kernel<2, R>), g, b, 0, s, a, total);
    else if (v <= 3) hipLaunchKernelGGL((embed_ln_exact_kernel<3, R>), g, b, 0, s, a, total);
    else hipLaunchKernelGGL((embed_ln_exact_kernel<4, R>), g, b, 0, s, a, total);
    return hipGetLastError();
  }
  const dim3 grid(ceil_div(total, kRowsPerBlock)), block(256);
  if (vec && v <= 1) hipLaunchKernelGGL((embed_ln_vec_kernel<1>), grid, block, 0, s, a, total);
  else if (vec && v <= 2) hipLaunchKernelGGL((embed_ln_vec_kernel<2>), grid, block, 0, s, a, total);
  else if (vec && v <= 3) hipLaunchKernelGGL((embed_ln_vec_kernel<3>), grid, block, 0, s, a, total);
  else if (vec && v <= 4) hipLaunchKernelGGL((embed_ln_vec_kernel<4>), grid, block, 0, s, a, total);
  else hipLaunchKernelGGL(embed_ln_kernel, grid, block, 0, s, a, total);
  return hipGetLastError();
}

template <int V>
static void launch_alnv(float* x, const float* y, int ldy, const float* gamma,
                        const float* beta, int m, int H, float eps, uint8_t* qa, int ldq,
                        float* rs, __bf16* ph, __bf16* pl, int ldp, hipStream_t s) {
  constexpr int R = 2;
  hipLaunchKernelGGL((add_ln_vec_kernel<V, R>), dim3(ceil_div(m, kRowsPerBlock * R)),
                     dim3(256), 0, s, x, y, ldy, gamma, beta, m, H, eps, qa, ldq, rs, ph, pl,
                     ldp);
}

hipError_t launch_add_layernorm(float* x, const float* y, int ldy,
                                const float* gamma, const float* beta, int m,
                                int H, float eps, uint8_t* qa, int ldq,
                                float* row_scales, hipStream_t s, __bf16* ph, __bf16* pl,
                                int ldp, bool exact) {
  if (m <= 0) return hipSuccess;
  if (H > 64 * kMaxPerLane) return hipErrorInvalidValue;
  const bool vec = H % 4 == 0 && (!y || ldy % 4 == 0) && (!qa || ldq % 4 == 0) &&
                   ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y) |
                     reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(beta)) &
                    15) == 0;
  if (ph && (!vec || ldp % 64 || ldp < H)) return hipErrorInvalidValue;
  if (exact) {
    const int v = ceil_div(H, 256);
    if (!vec || v > 4) return hipErrorInvalidValue;
    constexpr int R = kExactRows;
    const dim3 g(ceil_div(m, R)), b(64);
#define RH_ALNX(V)                                                                         \
  hipLaunchKernelGGL((add_ln_exact_kernel<V, R>), g, b, 0, s, x, y, ldy, gamma, beta, m, H, \
                     eps, qa, ldq, row_scales, ph, pl, ldp)
    if (v <= 1) RH_ALNX(1);
    else if (v <= 2) RH_ALNX(2);
    else if (v <= 3) RH_ALNX(3);
    else RH_ALNX(4);
#undef RH_ALNX
    return hipGetLastError();
  }
  if (vec) {
    const int v = ceil_div(H, 256);
    if (v <= 1) launch_alnv<1>(x, y, ldy, gamma, beta, m, H, eps, qa, ldq, row_scales, ph, pl, ldp, s);
    else if (v <= 2) launch_alnv<2>(x, y, ldy, gamma, beta, m, H, eps, qa, ldq, row_scales, ph, pl, ldp, s);
    else if (v <= 3) launch_alnv<3>(x, y, ldy, gamma, beta, m, H, eps, qa, ldq, row_scales, ph, pl, ldp, s);
    else if (v <= 4) launch_alnv<4>(x, y, ldy, gamma, beta, m, H, eps, qa, ldq, row_scales, ph, pl, ldp, s);
    else launch_alnv<8>(x, y, ldy, gamma, beta, m, H, eps, qa, ldq, row_scales, ph, pl, ldp, s);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(add_ln_kernel, dim3(ceil_div(m, kRowsPerBlock)), dim3(256),
                     0, s, x, y, ldy, gamma, beta, m, H, eps, qa, ldq, row_scales);
  return hipGetLastError();
}

hipError_t launch_layernorm(float* x, const float* gamma, const float* beta,
                            int m, int H, float eps, hipStream_t s) {
  return launch_add_layernorm(x, nullptr, 0, gamma, beta, m, H, eps, nullptr, 0,
                              nullptr, s);
}

// Pooling (bert.go:657-703): one thread per (text, column). CLS / last token
// copy a row; mean sums the column over the text's rows in ascending order
// in float32 (poolMean's order), then multiplies by float32(1/len). The
// row loads run a register block ahead of the sum.
__global__ __launch_bounds__(256) void pool_kernel(const float* __restrict__ x, int H,
                                                   const int32_t* __restrict__ cu,
                                                   int pooling, float* __restrict__ out) {
  const int b = blockIdx.y;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= H) return;
  const int r0 = cu[b], len = cu[b + 1] - cu[b];
  float v;
  if (pooling == RH_POOL_CLS) {
    v = x[(size_t)r0 * H + j];
  } else if (pooling == RH_POOL_LAST) {
    v = x[(size_t)(r0 + len - 1) * H + j];
  } else {
    const float* col = x + (size_t)r0 * H + j;
    // ascending rows; the loads run a block of U rows ahead of the sum
    constexpr int U = 32;
    float s = 0.0f;
    int i = 0;
    float ta[U], tb[U];
    auto fill = [&](float (&t)[U], int i0) {
#pragma unroll
      for (int e = 0; e < U; e++) t[e] = col[(size_t)(i0 + e) * H];
    };
    auto sum = [&](const float (&t)[U]) {
#pragma unroll
      for (int e = 0; e < U; e++) s += t[e];
    };
    if (len >= U) fill(ta, 0);
    for (; i + 2 * U <= len; i += 2 * U) {
      fill(tb, i + U);
      sum(ta);
      if (i + 3 * U <= len) fill(ta, i + 2 * U);
      sum(tb);
    }
    if (i + U <= len) {  // one loaded block left
      sum(ta);
      i += U;
    }
    for (; i < len; i++) s += col[(size_t)i * H];
    v = s * (1.0f / (float)len);
  }
  out[(size_t)b * H + j] = v;
}

// L2Normalize (tensor.go:540-554) of each [H] row in place: float64 sum of
// squares in column order (the squares of float32 values are exact in
// float64; one lane adds them as the reference's loop does), scale by
// float32(1/sqrt(sum)); an all-zero row is left as is.
__global__ __launch_bounds__(256) void l2_rows_kernel(float* __restrict__ y, int H) {
  __shared__ double sq[2048];
  __shared__ float inv_s;
  __shared__ int zero_s;
  float* o = y + (size_t)blockIdx.x * H;
  double sum = 0.0;
  for (int j0 = 0; j0 < H; j0 += 2048) {  // 2048 columns at a time through LDS
    const int n = min(2048, H - j0);
    for (int j = threadIdx.x; j < n; j += 256) sq[j] = (double)o[j0 + j] * (double)o[j0 + j];
    __syncthreads();
    if (threadIdx.x == 0)
      for (int j = 0; j < n; j++) sum = sum + sq[j];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    zero_s = sum == 0.0;
    inv_s = (float)(1.0 / sqrt(sum));
  }
  __syncthreads();
  if (zero_s) return;
  const float inv = inv_s;
  for (int j = threadIdx.x; j < H; j += 256) o[j] = o[j] * inv;
}

hipError_t launch_l2_rows(float* y, int rows, int H, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(l2_rows_kernel, dim3(rows), dim3(256), 0, s, y, H);
  return hipGetLastError();
}

hipError_t launch_pool(const float* x, int H, const int32_t* cu, int batch,
                       int pooling, int normalize, float* out, hipStream_t s) {
  if (batch <= 0) return hipSuccess;
  hipLaunchKernelGGL(pool_kernel, dim3(ceil_div(H, 256), batch), dim3(256), 0, s, x, H, cu,
                     pooling, out);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess && normalize) e = launch_l2_rows(out, batch, H, s);
  return e;
}

__global__ void fill_zero_kernel(float* x, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = 0.0f;
}

hipError_t launch_fill_zero(float* x, int n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, s, x, n);
  return hipGetLastError();
}

// GELU over a flat array as tensor.GELU does on amd64 (gelu_amd64.go:16-26):
// the geluAVX2 sequence for whole 8-element groups, geluScalar for the tail.
__global__ void gelu_kernel(float* x, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  x[i] = i < (n & ~(size_t)7) ? gelu_avx2(x[i]) : gelu_ref(x[i]);
}

hipError_t launch_gelu(float* x, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(gelu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     s, x, n);
  return hipGetLastError();
}

__global__ void add_bias_kernel(float* x, const float* bias, int m, int n,
                                int ldx) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)m * n) return;
  const int r = (int)(i / n), c = (int)(i % n);
  x[(size_t)r * ldx + c] += bias[c];
}

hipError_t launch_add_bias(float* x, const float* bias, int m, int n, int ldx,
                           hipStream_t s) {
  const size_t tot = (size_t)m * n;
  if (tot == 0) return hipSuccess;
  hipLaunchKernelGGL(add_bias_kernel, dim3((unsigned)((tot + 255) / 256)),
                     dim3(256), 0, s, x, bias, m, n, ldx);
  return hipGetLastError();
}

}  // namespace rh
