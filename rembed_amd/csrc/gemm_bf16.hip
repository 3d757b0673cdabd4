// gemm_bf16.hip — the floating-point GEMMs for gfx950 on bf16 MFMA
// (v_mfma_f32_32x32x16_bf16, fp32 accumulation), plus a native
// v_mfma_f32_32x32x2_f32 variant of the fp32 GEMM.
//
//  * Weight-only int8 (replaces MatMulPacked8, internal/tensor/pack8.go:80-126
//    and gemm4x16i8, gemm8_amd64.s:14-79): int8 weight tiles are dequantised
//    to bf16 (exact: |q| <= 127 needs 7 significant bits) while they are
//    staged into LDS; the fp32 activations are split into A_TERMS bf16 terms
//    (hi, lo) so a·q keeps ~16 significant bits of a; the per-channel scale
//    multiplies the fp32 accumulator in the epilogue, as the reference does.
//  * fp32 (replaces MatMulPacked, pack.go:123-210 and gemm4x16,
//    gemm_amd64.s:14-64): both operands split into bf16 hi + lo, three MFMA
//    products hi·hi + hi·lo + lo·hi (the lo·lo term is below fp32 rounding
//    of the sum for these magnitudes), or native f32 MFMA.
//
// Same tiling scheme as gemm_i8.hip: 256 threads as 2x2 waves, LDS rows of
// 128 bytes (64 bf16 of k per stage), XOR swizzle, double buffering.
#include "gemm_common.h"

namespace rh {

__device__ __forceinline__ void split_bf16(float x, __bf16& hi, __bf16& lo) {
  hi = (__bf16)x;
  lo = (__bf16)(x - (float)hi);
}

// Load 8 consecutive fp32 activations of row r starting at column k (k a
// multiple of 8). Vector path (K and lda multiples of 4, 16-byte aligned
// base): two unconditional 16-byte loads from clamped in-bounds addresses,
// so a stage's loads all issue before any wait; halves past M or K are
// zeroed later through the returned mask bits. Scalar path otherwise.
__device__ __forceinline__ uint32_t load_a8(const float* A, int lda, int r, int M,
                                            int k, int K, bool vec, v4f& x0,
                                            v4f& x1) {
  if (vec) {
    const bool rok = r < M;
    const float* row = A + (size_t)(rok ? r : M - 1) * lda;
    const bool h0 = rok && k < K;      // k+4 <= K since both are multiples of 4
    const bool h1 = rok && k + 4 < K;  // k+8 <= K
    x0 = *reinterpret_cast<const v4f*>(row + (h0 ? k : 0));
    x1 = *reinterpret_cast<const v4f*>(row + (h1 ? k + 4 : 0));
    return (uint32_t)h0 | ((uint32_t)h1 << 1);
  }
#pragma unroll
  for (int e = 0; e < 4; e++) {
    x0[e] = (r < M && k + e < K) ? A[(size_t)r * lda + k + e] : 0.0f;
    x1[e] = (r < M && k + 4 + e < K) ? A[(size_t)r * lda + k + 4 + e] : 0.0f;
  }
  return 3u;
}

template <int BM, int BN, int A_TERMS, bool B_INT8, bool GLU>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(GemmBfArgs p, int a_vec) {
  constexpr int B_TERMS = B_INT8 ? 1 : 2;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int AP = BM / 32, BP = BN / 32;
  constexpr int kA = BM * 128, kB = BN * 128;
  constexpr int kStage = A_TERMS * kA + B_TERMS * kB;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  const int tiles_n = (p.N + BN - 1) / BN;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int row0 = (tile / tiles_n) * BM;
  const int col0 = (tile % tiles_n) * BN;

  const int lrow = tid >> 3, lchunk = tid & 7;
  const int nk = (p.K + 63) >> 6;
  const bool vec = a_vec != 0;

  v4f ra0[AP], ra1[AP];
  uint32_t amask = 0;
  // B staging registers: int8 -> 8 bytes (2 dwords); fp32 -> 8 floats.
  int rbi[B_INT8 ? BP : 1][2];
  v4f rbf0[B_INT8 ? 1 : BP], rbf1[B_INT8 ? 1 : BP];

  auto gload = [&](int kt) {
    const int k = (kt << 6) + (lchunk << 3);
    amask = 0;
#pragma unroll
    for (int i = 0; i < AP; i++)
      amask |= load_a8(p.A, p.lda, row0 + i * 32 + lrow, p.M, k, p.K, vec, ra0[i],
                       ra1[i]) << (2 * i);
#pragma unroll
    for (int i = 0; i < BP; i++) {
      const int c = col0 + i * 32 + lrow;  // zero-padded rows, in bounds
      if constexpr (B_INT8) {
        const int* src = reinterpret_cast<const int*>(
            static_cast<const int8_t*>(p.B) + (size_t)c * p.ldb + k);
        rbi[i][0] = src[0];
        rbi[i][1] = src[1];
      } else {
        const v4f* src = reinterpret_cast<const v4f*>(
            static_cast<const float*>(p.B) + (size_t)c * p.ldb + k);
        rbf0[i] = src[0];
        rbf1[i] = src[1];
      }
    }
  };
  auto lstore = [&](int buf) {
    uint8_t* s = lds + buf * kStage;
#pragma unroll
    for (int i = 0; i < AP; i++) {
      const int r = i * 32 + lrow;
      const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
      const v4f x0 = ((amask >> (2 * i)) & 1) ? ra0[i] : z;
      const v4f x1 = ((amask >> (2 * i + 1)) & 1) ? ra1[i] : z;
      v8bf hi, lo;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        __bf16 h, l;
        split_bf16(e < 4 ? x0[e] : x1[e - 4], h, l);
        hi[e] = h;
        lo[e] = l;
      }
      *reinterpret_cast<v8bf*>(s + lds_off(r, lchunk)) = hi;
      if constexpr (A_TERMS == 2)
        *reinterpret_cast<v8bf*>(s + kA + lds_off(r, lchunk)) = lo;
    }
    uint8_t* sb = s + A_TERMS * kA;
#pragma unroll
    for (int i = 0; i < BP; i++) {
      const int r = i * 32 + lrow;
      if constexpr (B_INT8) {
        v8bf q;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const int byte = (rbi[i][e >> 2] >> (8 * (e & 3))) & 0xff;
          q[e] = (__bf16)(float)(int)(int8_t)byte;
        }
        *reinterpret_cast<v8bf*>(sb + lds_off(r, lchunk)) = q;
      } else {
        v8bf hi, lo;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          __bf16 h, l;
          split_bf16(e < 4 ? rbf0[i][e] : rbf1[i][e - 4], h, l);
          hi[e] = h;
          lo[e] = l;
        }
        *reinterpret_cast<v8bf*>(sb + lds_off(r, lchunk)) = hi;
        *reinterpret_cast<v8bf*>(sb + kB + lds_off(r, lchunk)) = lo;
      }
    }
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

  gload(0);
  lstore(0);
  __syncthreads();

  const int fr = lane & 31, fg = lane >> 5;
  for (int kt = 0; kt < nk; kt++) {
    if (kt + 1 < nk) gload(kt + 1);
    const uint8_t* s = lds + (kt & 1) * kStage;
    const uint8_t* sB = s + A_TERMS * kA;
#pragma unroll
    for (int st = 0; st < 4; st++) {
      const int c = 2 * st + fg;
      v8bf fah[TM], fal[TM], fbh[TN], fbl[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int r = wm * WM + i * 32 + fr;
        fah[i] = *reinterpret_cast<const v8bf*>(s + lds_off(r, c));
        if constexpr (A_TERMS == 2)
          fal[i] = *reinterpret_cast<const v8bf*>(s + kA + lds_off(r, c));
      }
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int r = wn * WN + j * 32 + fr;
        fbh[j] = *reinterpret_cast<const v8bf*>(sB + lds_off(r, c));
        if constexpr (!B_INT8)
          fbl[j] = *reinterpret_cast<const v8bf*>(sB + kB + lds_off(r, c));
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fah[i], fbh[j],
                                                              acc[i][j], 0, 0, 0);
          if constexpr (!B_INT8)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                fah[i], fbl[j], acc[i][j], 0, 0, 0);
          if constexpr (A_TERMS == 2)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                fal[i], fbh[j], acc[i][j], 0, 0, 0);
        }
    }
    if (kt + 1 < nk) lstore((kt + 1) & 1);
    __syncthreads();
  }

  if constexpr (GLU) {
    // Gated weight (rows 8t..8t+3 gate, 8t+4..8t+7 up): lane fr holds one
    // packed column; the gate lanes (fr % 8 < 4) fetch their up partner from
    // lane + 4 and write act(gate) * up at column (packed / 8) * 4 + fr % 4.
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int col = col0 + wn * WN + j * 32 + fr;
      const bool cok = col < p.N;
      const float cs = (p.col_scales && cok) ? p.col_scales[col] : 1.0f;
      const float b = (p.bias && cok) ? p.bias[col] : 0.0f;
      const int ocol = (col >> 3) * 4 + (fr & 3);
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int ii = 0; ii < 4; ii++)
#pragma unroll
          for (int jj = 0; jj < 4; jj++) {
            const int row = row0 + wm * WM + i * 32 + ii * 8 + fg * 4 + jj;
            float v = acc[i][j][ii * 4 + jj];
            if (p.col_scales) v = v * cs;
            if (p.bias) v = v + b;
            const float u = __shfl(v, lane + 4, 64);
            if ((fr & 4) == 0 && cok && row < p.M) p.C[(size_t)row * p.ldc + ocol] = glu_act(v, u, p.act);
          }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < TN; j++) {
    const int col = col0 + wn * WN + j * 32 + fr;
    if (col >= p.N) continue;
    const float cs = p.col_scales ? p.col_scales[col] : 1.0f;
    const float b = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int ii = 0; ii < 4; ii++)
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
          const int row = row0 + wm * WM + i * 32 + ii * 8 + fg * 4 + jj;
          if (row >= p.M) continue;
          float v = acc[i][j][ii * 4 + jj];
          if (p.col_scales) v = v * cs;
          if (p.bias) v = v + b;
          p.C[(size_t)row * p.ldc + col] = apply_act(v, p.act);
        }
  }
}

// Native fp32: v_mfma_f32_32x32x2_f32. LDS rows hold 32 fp32 of k per stage
// (8 chunks of 4); lane half g takes chunk 2s+g and feeds its 4 elements to
// 4 consecutive MFMAs, identically for A and B, so the k pairing agrees.
template <int BM, int BN, bool GLU>
__global__ __launch_bounds__(256) void gemm_f32_native_kernel(GemmBfArgs p,
                                                              int a_vec) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int AP = BM / 32, BP = BN / 32;
  constexpr int kStage = (BM + BN) * 128;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int row0 = (tile / tiles_n) * BM;
  const int col0 = (tile % tiles_n) * BN;
  const int lrow = tid >> 3, lchunk = tid & 7;
  const int nk = (p.K + 31) >> 5;
  const bool vec = a_vec != 0;

  v4f ra[AP], rb[BP];
  uint32_t amask = 0;
  auto gload = [&](int kt) {
    const int k = (kt << 5) + (lchunk << 2);
    amask = 0;
#pragma unroll
    for (int i = 0; i < AP; i++) {
      const int r = row0 + i * 32 + lrow;
      if (vec) {  // unconditional load from a clamped address, masked later
        const bool ok = r < p.M && k < p.K;
        const float* row = p.A + (size_t)(r < p.M ? r : p.M - 1) * p.lda;
        ra[i] = *reinterpret_cast<const v4f*>(row + (ok ? k : 0));
        amask |= (uint32_t)ok << i;
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++)
          ra[i][e] = (r < p.M && k + e < p.K) ? p.A[(size_t)r * p.lda + k + e] : 0.0f;
        amask |= 1u << i;
      }
    }
#pragma unroll
    for (int i = 0; i < BP; i++) {
      const int c = col0 + i * 32 + lrow;
      rb[i] = *reinterpret_cast<const v4f*>(static_cast<const float*>(p.B) +
                                            (size_t)c * p.ldb + k);
    }
  };
  auto lstore = [&](int buf) {
    uint8_t* s = lds + buf * kStage;
    const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < AP; i++)
      *reinterpret_cast<v4f*>(s + lds_off(i * 32 + lrow, lchunk)) =
          ((amask >> i) & 1) ? ra[i] : z;
#pragma unroll
    for (int i = 0; i < BP; i++)
      *reinterpret_cast<v4f*>(s + lds_off(BM + i * 32 + lrow, lchunk)) = rb[i];
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

  gload(0);
  lstore(0);
  __syncthreads();
  const int fr = lane & 31, fg = lane >> 5;
  for (int kt = 0; kt < nk; kt++) {
    if (kt + 1 < nk) gload(kt + 1);
    const uint8_t* sA = lds + (kt & 1) * kStage;
    const uint8_t* sB = sA + BM * 128;
#pragma unroll
    for (int st = 0; st < 4; st++) {
      const int c = 2 * st + fg;
      v4f fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; i++)
        fa[i] = *reinterpret_cast<const v4f*>(sA + lds_off(wm * WM + i * 32 + fr, c));
#pragma unroll
      for (int j = 0; j < TN; j++)
        fb[j] = *reinterpret_cast<const v4f*>(sB + lds_off(wn * WN + j * 32 + fr, c));
#pragma unroll
      for (int e = 0; e < 4; e++)
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
          for (int j = 0; j < TN; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][e], fb[j][e],
                                                             acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) lstore((kt + 1) & 1);
    __syncthreads();
  }

  if constexpr (GLU) {  // gated weight, as in gemm_bf16_kernel
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int col = col0 + wn * WN + j * 32 + fr;
      const bool cok = col < p.N;
      const float b = (p.bias && cok) ? p.bias[col] : 0.0f;
      const int ocol = (col >> 3) * 4 + (fr & 3);
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int ii = 0; ii < 4; ii++)
#pragma unroll
          for (int jj = 0; jj < 4; jj++) {
            const int row = row0 + wm * WM + i * 32 + ii * 8 + fg * 4 + jj;
            float v = acc[i][j][ii * 4 + jj];
            if (p.bias) v = v + b;
            const float u = __shfl(v, lane + 4, 64);
            if ((fr & 4) == 0 && cok && row < p.M) p.C[(size_t)row * p.ldc + ocol] = glu_act(v, u, p.act);
          }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < TN; j++) {
    const int col = col0 + wn * WN + j * 32 + fr;
    if (col >= p.N) continue;
    const float b = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int ii = 0; ii < 4; ii++)
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
          const int row = row0 + wm * WM + i * 32 + ii * 8 + fg * 4 + jj;
          if (row >= p.M) continue;
          float v = acc[i][j][ii * 4 + jj];
          if (p.bias) v = v + b;
          p.C[(size_t)row * p.ldc + col] = apply_act(v, p.act);
        }
  }
}

// The vector load path needs 16-byte aligned rows and K a multiple of 4 (so a
// 4-float group is either wholly inside [0, K) or wholly past it).
static int a_vec_ok(const GemmBfArgs& a) {
  return (a.lda % 4 == 0) && (a.K % 4 == 0) &&
         ((reinterpret_cast<uintptr_t>(a.A) & 15) == 0);
}

template <int BM, int BN, int AT, bool BI8>
static hipError_t launch_bf(const GemmBfArgs& a, hipStream_t s) {
  const int tiles = ceil_div(a.M, BM) * ceil_div(a.N, BN);
  if (is_glu(a.act))
    timed_launch((gemm_bf16_kernel<BM, BN, AT, BI8, true>), dim3(tiles), dim3(256),
                       0, s, a, a_vec_ok(a));
  else
    timed_launch((gemm_bf16_kernel<BM, BN, AT, BI8, false>), dim3(tiles), dim3(256),
                       0, s, a, a_vec_ok(a));
  return hipGetLastError();
}

// Prefer the larger tile when it still fills the 256 CUs.
static bool big_tile(const GemmBfArgs& a, int bm, int bn) {
  return ceil_div(a.M, bm) * ceil_div(a.N, bn) >= 256;
}

hipError_t launch_gemm_w8(const GemmBfArgs& a, int a_terms, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (a_terms == 1) {
    if (big_tile(a, 256, 256)) return launch_bf<256, 256, 1, true>(a, s);
    return launch_bf<128, 128, 1, true>(a, s);
  }
  if (big_tile(a, 256, 128)) return launch_bf<256, 128, 2, true>(a, s);
  return launch_bf<128, 128, 2, true>(a, s);
}

hipError_t launch_gemm_f32(const GemmBfArgs& a, int algo, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (algo == F32_NATIVE) {
    const int tiles = ceil_div(a.M, 128) * ceil_div(a.N, 128);
    if (is_glu(a.act))
      timed_launch((gemm_f32_native_kernel<128, 128, true>), dim3(tiles), dim3(256),
                         0, s, a, a_vec_ok(a));
    else
      timed_launch((gemm_f32_native_kernel<128, 128, false>), dim3(tiles), dim3(256),
                         0, s, a, a_vec_ok(a));
    return hipGetLastError();
  }
  return launch_bf<128, 128, 2, false>(a, s);
}

}  // namespace rh
