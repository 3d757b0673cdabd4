// gemm_planes.hip — the weight-only int8 and fp32 GEMMs on bf16 MFMA
// (v_mfma_f32_32x32x16_bf16, fp32 accumulation) with every operand already
// in bf16 "planes", so the main loop only moves bytes and multiplies.
//
//  * Weight-only int8 (replaces MatMulPacked8, internal/tensor/pack8.go:80-126
//    and gemm4x16i8, gemm8_amd64.s:14-79): the int8 weights are stored once,
//    at pack time, as a bf16 plane of the same integers (exact: |q| <= 127
//    needs 7 significant bits). The fp32 activations are split by one light
//    pass into hi = bf16(a) and lo = bf16(a - hi), so a·q keeps ~16
//    significant bits of a; the per-channel scale multiplies the fp32
//    accumulator in the epilogue, as the reference does.
//  * fp32 (replaces MatMulPacked, pack.go:123-210 and gemm4x16,
//    gemm_amd64.s:14-64): weights split into hi/lo planes at pack time,
//    activations by the same pass; three products hi·hi + hi·lo + lo·hi (the
//    lo·lo term is ~2^-16 of the others, below the fp32 rounding of the sum
//    at these magnitudes).
//
// Main loop (same scheme as the int8 GEMM): BM x BN tile per 256-thread
// workgroup, 2x2 waves of 32x32 MFMA tiles, K in stages of 32 bf16 = 64
// bytes per row and plane. Stages reach LDS by global_load_lds_dwordx4 (no
// register staging): lane l of a wave instruction writes LDS bytes
// [16l, 16l+16) of a 1 KiB block, so each lane loads the global 16-byte chunk
// that belongs at that slot, rows permuted by i8_slot (conflict-free fragment
// reads). NS stages in flight, one barrier per stage.
//
// The epilogue parks each 32-row band of accumulators in LDS and reads rows
// back 4 columns per lane: scale, bias, activation (or the gated pair) and a
// 4-wide vector store.
#include "gemm_common.h"

namespace rh {

// WGN waves along N (2: a 2x2 grid of 4 waves; 4: a 2x4 grid of 8 waves, two
// per SIMD, so one wave's LDS waits overlap the other's MFMAs).
// BK: k elements per stage and row, 32 (64-byte rows, i8_slot permutation)
// or 64 (128-byte rows, lds_off permutation; half the barriers).
// QKN: the QK-norm + RoPE epilogue of the decoders' q|k|v projection (bf16
// rows to p.qk_out; see GemmPlArgs).
template <int BM, int BN, int NS, int AT, int BT, bool GLU, int WGN = 2, int BK = 32,
          bool QKN = false>
__global__ __launch_bounds__(128 * WGN) void gemm_planes_kernel(GemmPlArgs p) {
  constexpr int NT = 128 * WGN;  // threads
  constexpr int NW = 2 * WGN;    // waves
  constexpr int CPR = BK / 8;    // 16-byte chunks per row
  static_assert(BK == 32 || BK == 64, "stage depth");
  constexpr int WM = BM / 2, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int kA = BM * BK * 2, kB = BN * BK * 2;  // bytes per plane
  constexpr int kStage = AT * kA + BT * kB;
  constexpr int LA = kA / (NT * 16), LB = kB / (NT * 16);  // loads per thread and plane
  constexpr int kLoads = AT * LA + BT * LB;
  constexpr int kEpiStride = WN + 4;  // floats per row of the epilogue transpose
  static_assert(LA >= 1 && LB >= 1 && TN >= 1, "tile too small for the wave grid");
  // A stage's slot is refilled right after the barrier that follows the
  // last reads of it, so two slots suffice (one stage in flight).
  static_assert(NS >= 2, "ring");
  static_assert(NS * kStage <= 160 * 1024, "LDS");
  static_assert(NS * kStage >= NW * 32 * kEpiStride * 4, "epilogue LDS");
  static_assert((NS - 2) * kLoads < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  int rb, cb;
  tile_origin(tile, (p.M + BM - 1) / BM, tiles_n, p.tile_group, rb, cb);
  const int row0 = rb * BM;
  const int col0 = cb * BN;
  const int nk = (p.K + BK - 1) / BK;

  // Element offsets of this thread's loads (fixed across stages). Rows past
  // M read row M-1 (their outputs are never stored); weight rows are
  // zero-padded to a multiple of 256; both operands are zero past K up to a
  // multiple of 64, so a stage never masks.
  int aoff[LA], boff[LB];
#pragma unroll
  for (int j = 0; j < LA; j++) {
    const int slot = (wave * LA + j) * 64 + lane;
    const int r = slot / CPR;
    const int chunk = stage_slot_chunk<BK * 2>(r, slot % CPR);
    const int gr = row0 + r;
    aoff[j] = (gr < p.M ? gr : p.M - 1) * p.lda + chunk * 8;
  }
#pragma unroll
  for (int j = 0; j < LB; j++) {
    const int slot = (wave * LB + j) * 64 + lane;
    const int r = slot / CPR;
    const int chunk = stage_slot_chunk<BK * 2>(r, slot % CPR);
    boff[j] = (col0 + r) * p.ldb + chunk * 8;
  }

  auto issue = [&](int kt) {
    uint8_t* s = lds + (kt % NS) * kStage;
    const int k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < LA; j++) {
      lds_dma16(p.Ah + aoff[j] + k0, s + (wave * LA + j) * 1024);
      if constexpr (AT == 2) lds_dma16(p.Al + aoff[j] + k0, s + kA + (wave * LA + j) * 1024);
    }
#pragma unroll
    for (int j = 0; j < LB; j++) {
      lds_dma16(p.Bh + boff[j] + k0, s + AT * kA + (wave * LB + j) * 1024);
      if constexpr (BT == 2)
        lds_dma16(p.Bl + boff[j] + k0, s + AT * kA + kB + (wave * LB + j) * 1024);
    }
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

#pragma unroll
  for (int st = 0; st < NS - 1; st++)
    if (st < nk) issue(st);

  const int fr = lane & 31, fg = lane >> 5;
  for (int kt = 0; kt < nk; kt++) {
    // Stage kt has landed once at most min(NS-2, nk-1-kt) later stages are
    // still pending for this wave.
    const int later = nk - 1 - kt;
    if (later >= NS - 2) wait_vmcnt<(NS - 2) * kLoads>();
    else if (NS > 3 && later == 1) wait_vmcnt<kLoads>();
    else wait_vmcnt<0>();
    // A bare s_barrier (a __syncthreads() fence would drain the whole ring):
    // every wave's stage-kt data is in LDS and its reads of stage kt-1 are
    // done, so the slot of stage kt-1 can be refilled.
    __builtin_amdgcn_s_barrier();
    if (kt + NS - 1 < nk) issue(kt + NS - 1);
    const uint8_t* sA = lds + (kt % NS) * kStage;
    const uint8_t* sB = sA + AT * kA;
#pragma unroll
    for (int s = 0; s < BK / 16; s++) {
      const int c = 2 * s + fg;
      v8bf fah[TM], fal[TM], fbh[TN], fbl[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int off = stage_frag_off<BK * 2>(wm * WM + i * 32 + fr, c);
        fah[i] = *reinterpret_cast<const v8bf*>(sA + off);
        if constexpr (AT == 2) fal[i] = *reinterpret_cast<const v8bf*>(sA + kA + off);
      }
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int off = stage_frag_off<BK * 2>(wn * WN + j * 32 + fr, c);
        fbh[j] = *reinterpret_cast<const v8bf*>(sB + off);
        if constexpr (BT == 2) fbl[j] = *reinterpret_cast<const v8bf*>(sB + kB + off);
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fah[i], fbh[j], acc[i][j], 0, 0, 0);
          if constexpr (BT == 2)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fah[i], fbl[j], acc[i][j], 0, 0, 0);
          if constexpr (AT == 2)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fal[i], fbh[j], acc[i][j], 0, 0, 0);
        }
    }
  }

  // ---- epilogue ----------------------------------------------------------
  // applyDense order (bert.go:282-301, pack8.go:118-122): fp32 sum, ·scale
  // (weight-only int8), + bias, then the activation.
  __syncthreads();
  float* ep = reinterpret_cast<float*>(lds) + wave * 32 * kEpiStride;
  // QKN: this lane's column scales, bias and norm weights (fixed columns
  // 4*lane..+3 of the tile for every row)
  v4f qk_cs = {1.0f, 1.0f, 1.0f, 1.0f}, qk_bs = {0.0f, 0.0f, 0.0f, 0.0f};
  v4f qk_g = {1.0f, 1.0f, 1.0f, 1.0f};
  // and the positions of this wave row's WM rows (lane r: rows r, 64 + r),
  // read per row with readlane: no dependent global load before a row's
  // cos/sin loads
  int qk_pos0 = 0, qk_pos1 = 0;
  if constexpr (QKN) {
    static_assert(WM == 128, "two position registers cover the wave row");
    const int r = row0 + wm * WM + lane;
    qk_pos0 = r < p.M ? p.qk_pos[r] : 0;
    qk_pos1 = r + 64 < p.M ? p.qk_pos[r + 64] : 0;
    const int gcol = col0 + lane * 4, h = gcol / p.qk_dh, d = gcol % p.qk_dh;
    if (p.col_scales) qk_cs = *reinterpret_cast<const v4f*>(p.col_scales + gcol);
    if (p.bias) qk_bs = *reinterpret_cast<const v4f*>(p.bias + gcol);
    if (h < p.qk_nq + p.qk_nkv)
      qk_g = *reinterpret_cast<const v4f*>((h < p.qk_nq ? p.qk_qg : p.qk_kg) + d);
  }
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
    if constexpr (QKN) {
      // The band's 32 rows x BN columns are parked across the WGN waves of
      // this wave row (wave wn holds columns [wn*WN, wn*WN + WN)). A pass
      // takes one tile row: lane l holds columns 4l..4l+3, a head is dh/4
      // consecutive lanes (the separate QK-norm pass's layout), and wave wn
      // takes rows wn, wn + WGN, ... of the band. The arithmetic is the
      // separate pass's, element for element (the sum of squares adds lane
      // pairs, then a butterfly over the head's lanes).
      static_assert(BN == 256, "a pass is one 256-column tile row of 64 lanes");
      __syncthreads();  // every wave of the band row has parked its columns
      const int dh = p.qk_dh, lph = dh >> 2, half = dh >> 1;
      const int c = lane * 4, l = lane % lph, d = l * 4;
      const int gcol = col0 + c, h = gcol / dh;
      const bool vh = h >= p.qk_nq + p.qk_nkv;  // v head: conversion only
      const bool first = l < (lph >> 1);        // columns d < dh/2
      const int dp = first ? d : d - half;
      const float* src0 = reinterpret_cast<const float*>(lds) +
                          (wm * WGN + c / WN) * 32 * kEpiStride + c % WN;
      typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
      // This wave's rows of the band: their cos/sin pieces are loaded before
      // the first row's store, so no table load queues behind a store
      // (vmcnt counts both in order).
      constexpr int RPW = 32 / WGN;
      v4f ccs[RPW], sns[RPW];
#pragma unroll
      for (int k = 0; k < RPW; k++) {
        const int wr = i * 32 + wn + k * WGN;  // row within the wave row (uniform)
        const int pos = __builtin_amdgcn_readlane(wr < 64 ? qk_pos0 : qk_pos1, wr & 63);
        ccs[k] = *reinterpret_cast<const v4f*>(p.qk_cos + (size_t)pos * half + dp);
        sns[k] = *reinterpret_cast<const v4f*>(p.qk_sin + (size_t)pos * half + dp);
      }
#pragma unroll
      for (int k = 0; k < RPW; k++) {
        const int rr = wn + k * WGN;
        v4f x = *reinterpret_cast<const v4f*>(src0 + rr * kEpiStride);
        const int grow = grow_base + rr;
        const bool ok = grow < p.M;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          if (p.col_scales) x[e] = x[e] * qk_cs[e];
          if (p.bias) x[e] = x[e] + qk_bs[e];
        }
        float ss = (x[0] * x[0] + x[1] * x[1]) + (x[2] * x[2] + x[3] * x[3]);
        for (int o = lph >> 1; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
        v4bf* out = reinterpret_cast<v4bf*>(p.qk_out + (size_t)grow * p.ldc + gcol);
        const v4f cc = ccs[k], sn = sns[k];
        const float inv = rms_inv(ss, dh, p.qk_eps);
        v4f xn, pn;
#pragma unroll
        for (int e = 0; e < 4; e++) xn[e] = x[e] * inv * qk_g[e];
#pragma unroll
        for (int e = 0; e < 4; e++) pn[e] = __shfl_xor(xn[e], lph >> 1, 64);
        v4f o;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float a = first ? xn[e] : pn[e], b = first ? pn[e] : xn[e];
          o[e] = first ? a * cc[e] - b * sn[e] : b * cc[e] + a * sn[e];
        }
        if (vh) o = x;
        if (ok) *out = v4bf{(__bf16)o[0], (__bf16)o[1], (__bf16)o[2], (__bf16)o[3]};
      }
      __syncthreads();  // the next band overwrites the parked columns
    } else if constexpr (GLU) {
      // Gated weight: tile columns 8t..8t+3 are gate rows, 8t+4..8t+7 the
      // matching up rows. A lane reads both halves of one group of 8 and
      // writes act(gate) * up at output column (packed column) / 2.
      constexpr int kL8 = WN / 8, kR8 = 64 / kL8;
      const int c8 = (lane % kL8) * 8;
      const int gpk = col0 + wn * WN + c8;
      const bool pk_ok = gpk < p.N;
      v4f csg = {1.0f, 1.0f, 1.0f, 1.0f}, csu = csg;
      v4f bg = {0.0f, 0.0f, 0.0f, 0.0f}, bu = bg;
      if (pk_ok) {
        if (p.col_scales) {
          csg = *reinterpret_cast<const v4f*>(p.col_scales + gpk);
          csu = *reinterpret_cast<const v4f*>(p.col_scales + gpk + 4);
        }
        if (p.bias) {
          bg = *reinterpret_cast<const v4f*>(p.bias + gpk);
          bu = *reinterpret_cast<const v4f*>(p.bias + gpk + 4);
        }
      }
      for (int rr = lane / kL8; rr < 32; rr += kR8) {
        const int grow = grow_base + rr;
        const v4f ag = *reinterpret_cast<const v4f*>(ep + rr * kEpiStride + c8);
        const v4f au = *reinterpret_cast<const v4f*>(ep + rr * kEpiStride + c8 + 4);
        if (grow < p.M && pk_ok) {
          v4f o;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            float g = ag[e], u = au[e];
            if (p.col_scales) {
              g = g * csg[e];
              u = u * csu[e];
            }
            if (p.bias) {
              g = g + bg[e];
              u = u + bu[e];
            }
            o[e] = glu_act(g, u, p.act);
          }
          if (p.Ch) store_planes4(p.Ch, p.Cl, (size_t)grow * p.ldc + gpk / 2, o);
          else *reinterpret_cast<v4f*>(p.C + (size_t)grow * p.ldc + gpk / 2) = o;
        }
      }
    } else {
      constexpr int kLanesPerRow = WN / 4;
      constexpr int kRowsPerPass = 64 / kLanesPerRow;
      const int c4 = (lane % kLanesPerRow) * 4;
      const int gcol = col0 + wn * WN + c4;
      const bool col_ok = gcol < p.N;
      v4f cs = {1.0f, 1.0f, 1.0f, 1.0f}, bs = {0.0f, 0.0f, 0.0f, 0.0f};
      if (col_ok) {
        if (p.col_scales) cs = *reinterpret_cast<const v4f*>(p.col_scales + gcol);
        if (p.bias) bs = *reinterpret_cast<const v4f*>(p.bias + gcol);
      }
#pragma unroll 2
      for (int rr = lane / kLanesPerRow; rr < 32; rr += kRowsPerPass) {
        const int grow = grow_base + rr;
        const v4f a = *reinterpret_cast<const v4f*>(ep + rr * kEpiStride + c4);
        if (grow < p.M && col_ok) {
          v4f v;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            float x = a[e];
            if (p.col_scales) x = x * cs[e];
            if (p.bias) x = x + bs[e];
            v[e] = apply_act(x, p.act);
          }
          if (p.Ch) store_planes4(p.Ch, p.Cl, (size_t)grow * p.ldc + gcol, v);
          else *reinterpret_cast<v4f*>(p.C + (size_t)grow * p.ldc + gcol) = v;
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// a [M][lda_f] fp32 -> hi/lo [M][ldk] bf16 planes, zero in [K, ldk). One
// thread per 4 columns; rows with 16-byte aligned 4-groups load as float4.
__global__ __launch_bounds__(256) void split_bf16_kernel(const float* __restrict__ a,
                                                         int lda_f, int M, int K,
                                                         __bf16* __restrict__ hi,
                                                         __bf16* __restrict__ lo, int ldk,
                                                         int vec) {
  typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
  const int groups = ldk >> 2;
  const size_t total = (size_t)M * groups;
  for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < total;
       g += (size_t)gridDim.x * blockDim.x) {
    const int row = (int)(g / groups);
    const int c = (int)(g % groups) * 4;
    const float* src = a + (size_t)row * lda_f + c;
    v4f x;
    if (vec && c + 4 <= K) {
      x = *reinterpret_cast<const v4f*>(src);
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) x[e] = c + e < K ? src[e] : 0.0f;
    }
    v4bf h, l;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      __bf16 a, b;
      split_hi_lo(x[e], a, b);
      h[e] = a;
      l[e] = b;
    }
    *reinterpret_cast<v4bf*>(hi + (size_t)row * ldk + c) = h;
    if (lo) *reinterpret_cast<v4bf*>(lo + (size_t)row * ldk + c) = l;
  }
}

hipError_t launch_split_bf16(const float* a, int lda_f, int M, int K, __bf16* hi, __bf16* lo,
                             int ldk, hipStream_t s) {
  if (M <= 0) return hipSuccess;
  if (ldk % 64 != 0 || ldk < K) return hipErrorInvalidValue;
  const int vec = (lda_f % 4 == 0) && ((reinterpret_cast<uintptr_t>(a) & 15) == 0);
  const size_t total = (size_t)M * (ldk / 4);
  const size_t blocks = std::min<size_t>((total + 255) / 256, 256 * 16);
  timed_launch(split_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a, lda_f, M, K,
                     hi, lo, ldk, vec);
  return hipGetLastError();
}

template <int BM, int BN, int NS, int AT, int BT, int WGN = 2, int BK = 32>
static hipError_t launch_pl(const GemmPlArgs& a, hipStream_t s) {
  const int tiles = ceil_div(a.M, BM) * ceil_div(a.N, BN);
  if (is_glu(a.act))
    timed_launch((gemm_planes_kernel<BM, BN, NS, AT, BT, true, WGN, BK>), dim3(tiles),
                 dim3(128 * WGN), 0, s, a);
  else
    timed_launch((gemm_planes_kernel<BM, BN, NS, AT, BT, false, WGN, BK>), dim3(tiles),
                 dim3(128 * WGN), 0, s, a);
  return hipGetLastError();
}

// Tiles: 1 = 256x256, 2 = 256x128, 3 = 128x128 with 4 waves (2x2); 4 =
// 256x256 and 5 = 256x128 with 8 waves (2x4, two per SIMD); for one
// activation term and int8 weights also 6 = 256x256 and 7 = 256x128 on
// 128-byte stages (two and three); 8 = 64x64 and 9 = 128x64 with 4 waves;
// 10 = 128x256 with 8 waves on three 64-byte stages (72 KiB: two workgroups
// per CU), for one term.
// Stages: as many as fit in 160 KiB of LDS. fp32's four planes leave no room
// for 256x256 (1 and 4 fall back to 2 and 5). Automatic choice (measured on
// MI355X at M = 16384 over the Qwen3/BERT linears; 8 waves 2-15% faster than
// 4 at the same tile): tile 6 for one-term W8 when the 256x256 grid gives
// at least every other CU a workgroup, 4 for the other products when it
// gives every CU one, else 5 down to 96 tiles, else 128x128
// while its grid has at least 192 workgroups; below that (MiniLM's M ~ 2300,
// or N = 384) 64x64, which keeps the CUs busy: at M = 2304 the weight-only
// int8 linears take 9.8 / 5.6 / 11.6 µs (384x1152, 384x384, 1536x384)
// against 10.6 / 9.5 / 20.0 with 128x128.
int pick_planes_tile(int M, int N, int K, int a_terms, int b_terms) {
  // one term: at M = 16384, K = 3072, N = 768 the 192 tiles of tile 6 take
  // 91 µs against 120 for the 384 tiles of 256x128
  if (a_terms == 1 && b_terms == 1 && ceil_div(M, 256) * ceil_div(N, 256) >= 128) {
    // Past one round, with the last round at most half full and a short K,
    // tile 6's tail is one 256x256 workgroup per busy CU; the 128x256 tile
    // with two workgroups per CU halves it. K = 768: M = 24576, N = 768
    // (1.125 rounds) 47.9 against 56.1 µs; M = 16384, N = 1280 (1.25) 48.5
    // against 57.4; N = 2304 (2.25) 84.4 against 89.1. At 1.875 rounds, whole
    // rounds, below one round and K = 2048 tile 6 stays ahead.
    const int t6 = ceil_div(M, 256) * ceil_div(N, 256), tail = t6 % 256;
    return t6 > 256 && tail != 0 && tail <= 128 && K <= 1536 ? 10 : 6;
  }
  if (a_terms + b_terms < 4 && ceil_div(M, 256) * ceil_div(N, 256) >= 256) return 4;
  // 256x128 down to 96 tiles (fp32 at M = 10102, N = 768: 240 tiles, 43.5 /
  // 154 µs at K = 768 / 3072 against 53.6 / 190 on 128x128; the two-stream
  // fp32 BERT-base forward's parts, ~5050 rows, give 120 tiles at N = 768:
  // 1.49 against 1.41 M tokens/s end to end with 128x128 there)
  if (ceil_div(M, 256) * ceil_div(N, 128) >= 96) return 5;
  return ceil_div(M, 128) * ceil_div(N, 128) >= 192 ? 3 : 8;
}

hipError_t launch_gemm_planes_qk(const GemmPlArgs& a, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (a.N % 256 != 0 || a.lda % 64 != 0 || a.ldb % 64 != 0 || a.ldc % 4 != 0 || !a.qk_out ||
      !(a.qk_dh == 64 || a.qk_dh == 128 || a.qk_dh == 256) || is_glu(a.act))
    return hipErrorInvalidValue;
  const int tiles = ceil_div(a.M, 256) * (a.N / 256);
  timed_launch((gemm_planes_kernel<256, 256, 2, 1, 1, false, 4, 64, true>), dim3(tiles),
               dim3(512), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_gemm_planes(const GemmPlArgs& a, int a_terms, int b_terms, int tile,
                              hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (a.lda % 64 != 0 || a.ldb % 64 != 0) return hipErrorInvalidValue;
  if (tile <= 0 || tile > kPlanesTileConfigs)
    tile = pick_planes_tile(a.M, a.N, a.K, a_terms, b_terms);
  if (a_terms == 1 && b_terms == 1) {
    switch (tile) {
      case 1: return launch_pl<256, 256, 4, 1, 1>(a, s);
      case 2: return launch_pl<256, 128, 4, 1, 1>(a, s);
      case 4: return launch_pl<256, 256, 4, 1, 1, 4>(a, s);
      case 5: return launch_pl<256, 128, 4, 1, 1, 4>(a, s);
      case 6: return launch_pl<256, 256, 2, 1, 1, 4, 64>(a, s);
      case 7: return launch_pl<256, 128, 3, 1, 1, 4, 64>(a, s);
      case 8: return launch_pl<64, 64, 4, 1, 1>(a, s);
      case 9: return launch_pl<128, 64, 4, 1, 1>(a, s);
      case 10: return launch_pl<128, 256, 3, 1, 1, 4>(a, s);
      default: return launch_pl<128, 128, 4, 1, 1>(a, s);
    }
  }
  if (a_terms == 2 && b_terms == 1) {
    switch (tile) {
      case 1: return launch_pl<256, 256, 3, 2, 1>(a, s);
      case 2: return launch_pl<256, 128, 4, 2, 1>(a, s);
      case 4: return launch_pl<256, 256, 3, 2, 1, 4>(a, s);
      case 5: return launch_pl<256, 128, 4, 2, 1, 4>(a, s);
      case 8: return launch_pl<64, 64, 4, 2, 1>(a, s);
      case 9: return launch_pl<128, 64, 4, 2, 1>(a, s);
      default: return launch_pl<128, 128, 3, 2, 1>(a, s);
    }
  }
  if (a_terms == 2 && b_terms == 2) {
    switch (tile) {
      case 1:
      case 2: return launch_pl<256, 128, 3, 2, 2>(a, s);
      case 4:
      case 5: return launch_pl<256, 128, 3, 2, 2, 4>(a, s);
      case 8: return launch_pl<64, 64, 4, 2, 2>(a, s);
      case 9: return launch_pl<128, 64, 4, 2, 2>(a, s);
      default: return launch_pl<128, 128, 3, 2, 2>(a, s);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace rh
