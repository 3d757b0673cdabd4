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

  // Loads are unconditional (out-of-range rows/columns read a clamped,
  // in-bounds address) so that all of a stage's loads are in flight at once;
  // the validity mask is applied when the data is written to LDS.
  v4i ra[AP], rb[BP];
  uint32_t amask = 0;
  auto gload = [&](int kt) {
    const int kb = (kt << 7) + (lchunk << 4);
    const bool kok = kb < p.lda;
    const int kbc = kok ? kb : 0;
    amask = 0;
#pragma unroll
    for (int i = 0; i < AP; i++) {
      const int r = row0 + i * 32 + lrow;
      const bool ok = kok && r < p.M;
      const int rc = r < p.M ? r : p.M - 1;
      ra[i] = *reinterpret_cast<const v4i*>(p.A + (size_t)rc * p.lda + kbc);
      amask |= (uint32_t)ok << i;
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
      // u8 (q+128) -> s8 q; rows past M and columns past lda contribute 0
      const v4i v = ((amask >> i) & 1) ? (ra[i] ^ (int)0x80808080) : v4i{0, 0, 0, 0};
      *reinterpret_cast<v4i*>(s + lds_off(r, lchunk)) = v;
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

// ---- v2: direct-to-LDS multi-stage pipeline ------------------------------
//
// Stage = BK = 64 bytes of k. Tiles reach LDS through global_load_lds_dwordx4
// (no register staging): lane l of a wave instruction writes LDS bytes
// [16l, 16l+16) of a 1 KiB block, so each lane loads the global 16-byte chunk
// that belongs at that LDS slot. A slot holds (row, chunk ^ ((row>>1)&3)),
// which keeps the 32-row fragment reads free of bank conflicts. NS stages
// are in flight; one barrier per stage orders the ring. u8 activations are
// flipped to s8 (xor 0x80) after the fragment read.
__device__ __forceinline__ int v2_slot(int row, int chunk) {
  return (row << 2) + (chunk ^ ((row >> 1) & 3));
}

// 16-byte global -> LDS copy (global_load_lds_dwordx4). The builtin exists
// only for the device target; the host pass of the kernel template must
// still see a valid body to emit its launch stub.
__device__ __forceinline__ void lds_dma16(const void* src, void* lds_dst) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(src, lds_dst, 16, 0, 0);
#endif
}

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] and
// [15:14], expcnt[6:4] and lgkmcnt[11:8] left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | (((N >> 4) & 3) << 14));
}

template <int BM, int BN, int NS>
__global__ __launch_bounds__(256) void gemm_i8_v2_kernel(GemmI8Args p) {
  constexpr int BK = 64;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int kA = BM * BK, kB = BN * BK, kStage = kA + kB;
  constexpr int LA = kA / (256 * 16), LB = kB / (256 * 16);  // loads per thread
  constexpr int kLoads = LA + LB;
  constexpr int kEpiStride = WN + 4;  // ints per row of the epilogue transpose
  static_assert(NS * kStage >= 4 * 32 * kEpiStride * 4, "epilogue LDS");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int row0 = (tile / tiles_n) * BM;
  const int col0 = (tile % tiles_n) * BN;
  const int nk = (p.K + BK - 1) / BK;

  // Per-lane source rows/chunks of this thread's loads (fixed across stages).
  const uint8_t* asrc[LA];
  int achunk[LA];
#pragma unroll
  for (int j = 0; j < LA; j++) {
    const int slot = (wave * LA + j) * 64 + lane;
    const int r = slot >> 2;
    achunk[j] = (slot & 3) ^ ((r >> 1) & 3);
    const int gr = row0 + r;
    asrc[j] = p.A + (size_t)(gr < p.M ? gr : p.M - 1) * p.lda;
  }
  const int8_t* bsrc[LB];
  int bchunk[LB];
#pragma unroll
  for (int j = 0; j < LB; j++) {
    const int slot = (wave * LB + j) * 64 + lane;
    const int r = slot >> 2;
    bchunk[j] = (slot & 3) ^ ((r >> 1) & 3);
    bsrc[j] = p.B + (size_t)(col0 + r) * p.ldb;  // zero-padded rows
  }

  auto issue = [&](int kt) {
    uint8_t* s = lds + (kt % NS) * kStage;
    const int k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < LA; j++) {
      int kb = k0 + achunk[j] * 16;
      kb = kb < p.lda ? kb : 0;  // past the row: any in-bounds bytes (B is 0 there)
      lds_dma16(asrc[j] + kb, s + (wave * LA + j) * 1024);
    }
#pragma unroll
    for (int j = 0; j < LB; j++)
      lds_dma16(bsrc[j] + k0 + bchunk[j] * 16, s + kA + (wave * LB + j) * 1024);
  };

  v16i acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = v16i{};

#pragma unroll
  for (int st = 0; st < NS - 1; st++)
    if (st < nk) issue(st);

  const int fr = lane & 31, fg = lane >> 5;
  for (int kt = 0; kt < nk; kt++) {
    // Stage kt landed once at most min(NS-2, nk-1-kt) later stages are pending.
    const int later = nk - 1 - kt;
    if (later >= NS - 2) wait_vmcnt<(NS - 2) * kLoads>();
    else if (NS > 3 && later == 1) wait_vmcnt<kLoads>();
    else wait_vmcnt<0>();
    // A bare s_barrier: __syncthreads() would add a release fence that waits
    // for every outstanding load (vmcnt(0)), draining the ring each stage.
    // This wave's stage-kt data is in LDS (vmcnt above); its reads of the
    // previous stage have completed (their MFMAs consumed them).
    __builtin_amdgcn_s_barrier();
    if (kt + NS - 1 < nk) issue(kt + NS - 1);
    const uint8_t* sA = lds + (kt % NS) * kStage;
    const uint8_t* sB = sA + kA;
#pragma unroll
    for (int s = 0; s < BK / 32; s++) {
      const int c = 2 * s + fg;
      v4i fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int r = wm * WM + i * 32 + fr;
        fa[i] = *reinterpret_cast<const v4i*>(sA + v2_slot(r, c) * 16) ^ (int)0x80808080;
      }
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int r = wn * WN + j * 32 + fr;
        fb[j] = *reinterpret_cast<const v4i*>(sB + v2_slot(r, c) * 16);
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  }

  // Epilogue: per 32-row band, the wave parks its int32 accumulators in its
  // own LDS region, then reads rows back 4 columns per lane and writes
  // 16-byte vectors. Dequant order matches the reference: float32(real)·rs,
  // ·cs, then + bias (AddBias), then the activation.
  __syncthreads();
  int* ep = reinterpret_cast<int*>(lds) + wave * 32 * kEpiStride;
  const int gcol_base = col0 + wn * WN;
#pragma unroll
  for (int i = 0; i < TM; i++) {
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++)
        ep[((r >> 2) * 8 + fg * 4 + (r & 3)) * kEpiStride + j * 32 + fr] = acc[i][j][r];
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    const int grow_base = row0 + wm * WM + i * 32;
    constexpr int kLanesPerRow = WN / 4;
    constexpr int kRowsPerPass = 64 / kLanesPerRow;
    const int c4 = (lane % kLanesPerRow) * 4;
    const int gcol = gcol_base + c4;
    const bool col_ok = gcol < p.N;
    v4f cs = {1.0f, 1.0f, 1.0f, 1.0f}, bs = {0.0f, 0.0f, 0.0f, 0.0f};
    v4i corr = {0, 0, 0, 0};
    if (col_ok) {
      if (p.col_scales) cs = *reinterpret_cast<const v4f*>(p.col_scales + gcol);
      if (p.bias) bs = *reinterpret_cast<const v4f*>(p.bias + gcol);
      if (p.colsum) corr = *reinterpret_cast<const v4i*>(p.colsum + gcol) * 128;
    }
#pragma unroll 2
    for (int rr = lane / kLanesPerRow; rr < 32; rr += kRowsPerPass) {
      const int grow = grow_base + rr;
      const v4i a = *reinterpret_cast<const v4i*>(ep + rr * kEpiStride + c4);
      if (grow < p.M && col_ok) {
        const size_t o = (size_t)grow * p.ldc + gcol;
        if (p.Cacc) {
          v4i w;
#pragma unroll
          for (int e = 0; e < 4; e++) w[e] = (int)((uint32_t)a[e] + (uint32_t)corr[e]);
          *reinterpret_cast<v4i*>(p.Cacc + o) = w;
        }
        if (p.C) {
          const float rs = p.row_scales[grow];
          v4f w;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            float v = (float)a[e] * rs;
            v = v * cs[e];
            if (p.bias) v = v + bs[e];
            w[e] = apply_act(v, p.act);
          }
          *reinterpret_cast<v4f*>(p.C + o) = w;
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

template <int BM, int BN>
static hipError_t launch_i8_v2(const GemmI8Args& a, hipStream_t s) {
  const int tiles = ceil_div(a.M, BM) * ceil_div(a.N, BN);
  hipLaunchKernelGGL((gemm_i8_v2_kernel<BM, BN, 4>), dim3(tiles), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int BM, int BN>
static hipError_t launch_i8(const GemmI8Args& a, hipStream_t s) {
  const int tiles = ceil_div(a.M, BM) * ceil_div(a.N, BN);
  hipLaunchKernelGGL((gemm_i8_kernel<BM, BN>), dim3(tiles), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_gemm_i8(const GemmI8Args& a, int tile, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  switch (tile) {
    case 1: return launch_i8<256, 256>(a, s);
    case 2: return launch_i8<256, 128>(a, s);
    case 3: return launch_i8<128, 128>(a, s);
    case 4: return launch_i8_v2<256, 256>(a, s);
    case 5: return launch_i8_v2<256, 128>(a, s);
    case 6: return launch_i8_v2<128, 128>(a, s);
    default: break;
  }
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
