// gemm_i8.hip — full-int8 GEMM for gfx950: u8 activations x s8 weights on
// v_mfma_i32_32x32x32_i8 with int32 accumulation.
//
// Replaces MatMulPackedVNNI's integer core (internal/tensor/pack_vnni.go:
// 142-175, gemm4x16vnni vnni_amd64.s:22-82). The reference feeds VPDPBUSD
// u8 = q+128 and subtracts 128·colSum afterwards; the MFMA takes s8 x s8, so
// each activation byte is flipped to u8 ^ 0x80 = q (the same integer minus
// 128) while it is staged into LDS. The int32 sum is then directly
// real = acc_ref − 128·colSum (exact mod 2^32), and acc_ref is recovered
// as real + 128·colSum when the raw accumulators are requested.
//
// Tiling: BM x BN output tile per 256-thread workgroup (2x2 waves), K staged
// through double-buffered LDS in 128-byte slabs with an XOR swizzle; each
// wave owns (BM/2) x (BN/2) as a grid of 32x32 MFMA tiles.
#include "gemm_common.h"

namespace rh {

template <int BM, int BN>
__global__ __launch_bounds__(256) void gemm_i8_kernel(GemmI8Args p) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int AP = BM / 32, BP = BN / 32;  // 32-row load passes
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
  const int nk = (p.K + 127) >> 7;

  v4i ra[AP], rb[BP];
  auto gload = [&](int kt) {
    const int kb = (kt << 7) + (lchunk << 4);
#pragma unroll
    for (int i = 0; i < AP; i++) {
      const int r = row0 + i * 32 + lrow;
      if (r < p.M && kb < p.lda) {
        v4i v = *reinterpret_cast<const v4i*>(p.A + (size_t)r * p.lda + kb);
        ra[i] = v ^ (int)0x80808080;  // u8 (q+128) -> s8 q
      } else {
        ra[i] = v4i{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int i = 0; i < BP; i++) {
      const int c = col0 + i * 32 + lrow;  // inside the zero-padded rows
      rb[i] = *reinterpret_cast<const v4i*>(p.B + (size_t)c * p.ldb + kb);
    }
  };
  auto lstore = [&](int buf) {
    uint8_t* s = lds + buf * kStage;
#pragma unroll
    for (int i = 0; i < AP; i++) {
      const int r = i * 32 + lrow;
      *reinterpret_cast<v4i*>(s + lds_off(r, lchunk)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BP; i++) {
      const int r = BM + i * 32 + lrow;
      *reinterpret_cast<v4i*>(s + lds_off(r, lchunk)) = rb[i];
    }
  };

  v16i acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0;

  gload(0);
  lstore(0);
  __syncthreads();

  const int fr = lane & 31, fg = lane >> 5;
  for (int kt = 0; kt < nk; kt++) {
    if (kt + 1 < nk) gload(kt + 1);
    const uint8_t* sA = lds + (kt & 1) * kStage;
    const uint8_t* sB = sA + BM * 128;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const int c = 2 * s + fg;
      v4i fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int r = wm * WM + i * 32 + fr;
        fa[i] = *reinterpret_cast<const v4i*>(sA + lds_off(r, c));
      }
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int r = wn * WN + j * 32 + fr;
        fb[j] = *reinterpret_cast<const v4i*>(sB + lds_off(r, c));
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j],
                                                            acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) lstore((kt + 1) & 1);
    __syncthreads();
  }

  // Epilogue: lane holds column (lane & 31) and rows ii*8 + (lane>>5)*4 + jj
  // of each 32x32 tile. Reference order: float32(real)·rs·cs, then + bias
  // (AddBias pass), then the activation (bert.go:297-300, 913-915).
#pragma unroll
  for (int j = 0; j < TN; j++) {
    const int col = col0 + wn * WN + j * 32 + fr;
    if (col >= p.N) continue;
    const float cs = p.col_scales ? p.col_scales[col] : 1.0f;
    const uint32_t corr = 128u * (uint32_t)(p.colsum ? p.colsum[col] : 0);
    const float b = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
      for (int ii = 0; ii < 4; ii++) {
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
          const int row = row0 + wm * WM + i * 32 + ii * 8 + fg * 4 + jj;
          if (row >= p.M) continue;
          const int real = acc[i][j][ii * 4 + jj];
          const size_t o = (size_t)row * p.ldc + col;
          if (p.Cacc) p.Cacc[o] = (int)((uint32_t)real + corr);
          if (p.C) {
            float v = (float)real * p.row_scales[row];
            v = v * cs;
            if (p.bias) v = v + b;
            p.C[o] = apply_act(v, p.act);
          }
        }
      }
    }
  }
}

template <int BM, int BN>
static hipError_t launch_i8(const GemmI8Args& a, hipStream_t s) {
  const int tiles = ceil_div(a.M, BM) * ceil_div(a.N, BN);
  hipLaunchKernelGGL((gemm_i8_kernel<BM, BN>), dim3(tiles), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_gemm_i8(const GemmI8Args& a, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  // Tile choice: fewest CU rounds x tile work, with a mild penalty for the
  // smaller tiles' lower operand reuse (256 CUs on MI355X).
  struct Cand { int bm, bn; double eff; };
  const Cand cands[] = {{256, 256, 1.0}, {256, 128, 1.12}, {128, 128, 1.35}};
  int best = 0;
  double best_cost = 1e300;
  for (int i = 0; i < 3; i++) {
    const int tiles = ceil_div(a.M, cands[i].bm) * ceil_div(a.N, cands[i].bn);
    const double rounds = (double)ceil_div(tiles, 256);
    const double cost = rounds * cands[i].bm * cands[i].bn * cands[i].eff;
    if (cost < best_cost) {
      best_cost = cost;
      best = i;
    }
  }
  switch (best) {
    case 0: return launch_i8<256, 256>(a, s);
    case 1: return launch_i8<256, 128>(a, s);
    default: return launch_i8<128, 128>(a, s);
  }
}

}  // namespace rh
