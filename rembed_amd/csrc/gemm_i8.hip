// gemm_i8.hip — full-int8 GEMM for gfx950: u8 activations x s8 weights on
// v_mfma_i32_32x32x32_i8 with int32 accumulation.
//
// Replaces MatMulPackedVNNI's integer core (internal/tensor/pack_vnni.go:
// 142-175, gemm4x16vnni vnni_amd64.s:22-82). The reference feeds VPDPBUSD
// u8 = q+128 and subtracts 128·colSum afterwards; the MFMA takes s8 x s8, so
// each activation byte is flipped to u8 ^ 0x80 = q (the same integer minus
// 128) after its fragment is read from LDS. The int32 sum is then directly
// real = acc_ref − 128·colSum (exact mod 2^32), and acc_ref is recovered as
// real + 128·colSum when the raw accumulators are requested.
//
// Main loop: BM x BN tile per workgroup of 2x2 or 2x4 waves, each wave a
// grid of 32x32 MFMA tiles. K advances in 64-byte stages that reach LDS by
// global_load_lds_dwordx4 (no register staging): lane l of a wave
// instruction writes LDS bytes [16l, 16l+16) of a 1 KiB block, so each lane
// loads the global 16-byte chunk that belongs at that slot. A slot holds
// (row, chunk permuted by i8_slot), which keeps the fragment reads free of
// bank conflicts. NS stages are in flight, one barrier per stage orders the
// ring.
//
// A second family (gemm_i8f_kernel, further down) stages only A in LDS and
// loads B fragments straight into registers from a fragment-ordered copy of
// the weight.
//
// Epilogue (shared by both): per 32-row band a wave parks its accumulators
// in LDS and reads rows back 4 columns per lane, so every output is a
// 4-wide vector store. Variants (EPI): fp32 or bf16 values, bf16 hi/lo
// planes, the raw accumulators, the two passes of a fused row quantization
// (row |max| by atomics, then u8 bytes), or that quantization in one pass
// (i8_epilogue_qsync: the workgroups of a row block exchange the row
// maxima).
#include "gemm_common.h"
#include "rows_common.h"

namespace rh {

// QuantizeRowU8's per-element step (internal/tensor/pack_vnni.go:103-111).
__device__ __forceinline__ uint32_t quant_byte(float v, float inv) {
  int q = (int)rintf(v * inv) + 128;
  q = q < 0 ? 0 : (q > 255 ? 255 : q);
  return (uint32_t)q;
}

// Epilogue shared by the int8 kernels: per 32-row band each wave parks its
// accumulators in LDS and reads rows back 4 columns per lane, so every output
// is a 4-wide vector store. Dequant order matches the reference:
// float32(real)·rs, ·cs, then + bias (AddBias), then the activation
// (bert.go:297-300, 913-915). `lds` must hold NW·32·(WN+4) ints plus 3·BM
// floats; the caller has finished every LDS read and DMA of its main loop.
template <int BM, int WM, int WN, int TM, int TN, int NW, int NT, int EPI>
__device__ __forceinline__ void i8_epilogue(const GemmI8Args& p, v16i (&acc)[TM][TN],
                                            uint8_t* lds, int row0, int col0, int wave,
                                            int wm, int wn, int tid) {
  constexpr int kEpiStride = WN + 4;  // ints per row of the epilogue transpose
  constexpr int kEpiBytes = NW * 32 * kEpiStride * 4;
  const int lane = tid & 63;
  const int fr = lane & 31, fg = lane >> 5;
  __syncthreads();
  int* ep = reinterpret_cast<int*>(lds) + wave * 32 * kEpiStride;
  // Per-row operands of the tile (row scale; for EPI_QUANT the output row's
  // scale and its reciprocal), fetched once per tile by one thread per row
  // and read from LDS in the store loops: a global load per stored row would
  // put one memory latency per row pass on the epilogue's critical path.
  float* rs_l = reinterpret_cast<float*>(lds + kEpiBytes);
  float* sc_l = rs_l + BM;
  float* inv_l = sc_l + BM;
  if constexpr (EPI != EPI_ACC) {
    for (int r = tid; r < BM; r += NT) {
      const int gr = row0 + r;
      float rs = 0.0f, sc = 1.0f;
      if (gr < p.M) {
        rs = p.row_scales[gr];
        if constexpr (EPI == EPI_QUANT) {
          sc = p.row_absmax[gr] / 127.0f;
          if (sc == 0.0f) sc = 1.0f;
        }
      }
      rs_l[r] = rs;
      if constexpr (EPI == EPI_QUANT) {
        sc_l[r] = sc;
        inv_l[r] = 1.0f / sc;
      }
    }
    __syncthreads();
  }
  constexpr int kLanesPerRow = WN / 4;
  constexpr int kRowsPerPass = 64 / kLanesPerRow;
  const int c4 = (lane % kLanesPerRow) * 4;
  const int gcol = col0 + wn * WN + c4;
  const bool col_ok = gcol < p.N;
  v4f cs = {1.0f, 1.0f, 1.0f, 1.0f}, bs = {0.0f, 0.0f, 0.0f, 0.0f};
  v4i corr = {0, 0, 0, 0};
  if (col_ok) {
    if (p.col_scales) cs = *reinterpret_cast<const v4f*>(p.col_scales + gcol);
    if (p.bias) bs = *reinterpret_cast<const v4f*>(p.bias + gcol);
    if (EPI == EPI_ACC && p.colsum) corr = *reinterpret_cast<const v4i*>(p.colsum + gcol) * 128;
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
    if constexpr (EPI == EPI_F32) {
      if (is_glu(p.act)) {
        // Gated weight: tile columns 8t..8t+3 are gate rows, 8t+4..8t+7 the
        // matching up rows. A lane reads both halves of one group of 8 and
        // writes 4 outputs act(gate) * up at column (packed column) / 2.
        constexpr int kL8 = WN / 8, kR8 = 64 / kL8;
        const int c8 = (lane % kL8) * 8;
        const int gpk = col0 + wn * WN + c8;
        const bool pk_ok = gpk < p.N;
        v4f csg = {1.0f, 1.0f, 1.0f, 1.0f}, csu = csg;
        v4f bg = {0.0f, 0.0f, 0.0f, 0.0f}, bu = bg;
        if (pk_ok) {
          csg = *reinterpret_cast<const v4f*>(p.col_scales + gpk);
          csu = *reinterpret_cast<const v4f*>(p.col_scales + gpk + 4);
          if (p.bias) {
            bg = *reinterpret_cast<const v4f*>(p.bias + gpk);
            bu = *reinterpret_cast<const v4f*>(p.bias + gpk + 4);
          }
        }
        for (int rr = lane / kL8; rr < 32; rr += kR8) {
          const int grow = grow_base + rr;
          const v4i ag = *reinterpret_cast<const v4i*>(ep + rr * kEpiStride + c8);
          const v4i au = *reinterpret_cast<const v4i*>(ep + rr * kEpiStride + c8 + 4);
          if (grow < p.M && pk_ok) {
            const float rs = rs_l[grow - row0];
            v4f o;
#pragma unroll
            for (int e = 0; e < 4; e++) {
              float g = (float)ag[e] * rs;
              g = g * csg[e];
              float u = (float)au[e] * rs;
              u = u * csu[e];
              if (p.bias) {
                g = g + bg[e];
                u = u + bu[e];
              }
              o[e] = glu_act(g, u, p.act);
            }
            *reinterpret_cast<v4f*>(static_cast<float*>(p.out) + (size_t)grow * p.ldo + gpk / 2) = o;
          }
        }
        __builtin_amdgcn_wave_barrier();
        continue;
      }
    }
#pragma unroll 2
    for (int it = 0; it < 32 / kRowsPerPass; it++) {
      const int rr = lane / kLanesPerRow + it * kRowsPerPass;
      const int grow = grow_base + rr;
      const bool ok = grow < p.M && col_ok;
      const v4i a = *reinterpret_cast<const v4i*>(ep + rr * kEpiStride + c4);
      if constexpr (EPI == EPI_ACC) {
        if (ok) {
          v4i w;
#pragma unroll
          for (int e = 0; e < 4; e++) w[e] = (int)((uint32_t)a[e] + (uint32_t)corr[e]);
          *reinterpret_cast<v4i*>(static_cast<int32_t*>(p.out) + (size_t)grow * p.ldo + gcol) = w;
        }
      } else {
        v4f v = {0.0f, 0.0f, 0.0f, 0.0f};
        if (ok) {
          const float rs = rs_l[grow - row0];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            float x = (float)a[e] * rs;
            x = x * cs[e];
            if (p.bias) x = x + bs[e];
            v[e] = apply_act(x, p.act);
          }
        }
        if constexpr (EPI == EPI_F32) {
          if (ok) *reinterpret_cast<v4f*>(static_cast<float*>(p.out) + (size_t)grow * p.ldo + gcol) = v;
        } else if constexpr (EPI == EPI_BF16) {
          if (ok) {
            typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
            v4bf w = {(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
            *reinterpret_cast<v4bf*>(static_cast<__bf16*>(p.out) + (size_t)grow * p.ldo + gcol) = w;
          }
        } else if constexpr (EPI == EPI_PLANES) {
          if (ok)
            store_planes4(static_cast<__bf16*>(p.out), static_cast<__bf16*>(p.out_lo),
                          (size_t)grow * p.ldo + gcol, v);
        } else if constexpr (EPI == EPI_ABSMAX) {
          // |value| max over this row's columns of the tile; every lane takes
          // part in the shuffles (invalid lanes contribute 0).
          float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
          for (int o = kLanesPerRow / 2; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
          if (grow < p.M && (lane % kLanesPerRow) == 0)
            atomicMax(reinterpret_cast<unsigned int*>(p.row_absmax) + grow, __float_as_uint(m));
        } else {  // EPI_QUANT: QuantizeRowU8 with the row's |max| from pass 1
          if (ok) {
            const float scale = sc_l[grow - row0];
            const float inv = inv_l[grow - row0];
            const uint32_t w = quant_byte(v[0], inv) | (quant_byte(v[1], inv) << 8) |
                               (quant_byte(v[2], inv) << 16) | (quant_byte(v[3], inv) << 24);
            *reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(p.out) + (size_t)grow * p.ldo + gcol) = w;
            if (gcol == 0) p.rs_out[grow] = scale;
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// Single-pass GELU + QuantizeRowU8 epilogue (EPI_QSYNC), for FFN1 feeding
// FFN2's u8 rows (bert.go:910-916, pack_vnni.go:85-117) without the fp32
// intermediate. Sweep 1 dequantizes the tile through the LDS transpose (the
// same float32 operations as the other epilogues), keeps the values in
// registers and publishes each row's |max| over the tile's columns in the
// row's slot for this column tile. Each row's thread then reads the row's
// tiles_n slots until none holds the empty mark: their max is the |max|
// over the whole row, as QuantizeRowU8 takes it. Sweep 2 quantizes the held
// values and stores the bytes. The last workgroup of a row block to leave
// (a departure count per row block) empties the block's slots and zeroes
// its count for the next launch.
//
// A row block's column tiles are consecutive workgroups of one XCD
// (qsync_tile), which starts its workgroups in order: once a row block's
// first tile runs, the tiles it waits for are the next ones queued on that
// XCD, and at most tiles_n - 1 workgroups of one launch wait at a time (two
// launches on two streams leave most of an XCD's 64 slots to workgroups
// that finish), so every wait ends. It is bounded all the same: past
// kSyncWaitTicks of the 100 MHz clock the row is taken as complete and
// sync_err is set. Slots are written and read by device-scope atomic
// stores and loads, coherent across the XCDs.
constexpr uint64_t kSyncWaitTicks = 20000000;  // 200 ms
constexpr unsigned kSlotEmpty = 0xFFFFFFFFu;   // never the bits of a |max|

template <int BM, int WM, int WN, int TM, int TN, int NW, int NT>
__device__ __forceinline__ void i8_epilogue_qsync(const GemmI8Args& p, v16i (&acc)[TM][TN],
                                                  uint8_t* lds, int row0, int col0, int rb,
                                                  int cb, int tiles_n, int wave, int wm, int wn,
                                                  int tid) {
  constexpr int WGN = NW / 2;
  constexpr int kEpiStride = WN + 4;
  constexpr int kEpiBytes = NW * 32 * kEpiStride * 4;
  constexpr int kLanesPerRow = WN / 4;
  constexpr int kRowsPerPass = 64 / kLanesPerRow;
  constexpr int kPasses = 32 / kRowsPerPass;
  static_assert(TM * kPasses * 4 <= 64, "values held per lane");
  static_assert(BM <= NT, "one thread per row gathers the row's slots");
  const int lane = tid & 63;
  const int fr = lane & 31, fg = lane >> 5;
  __syncthreads();
  int* ep = reinterpret_cast<int*>(lds) + wave * 32 * kEpiStride;
  float* rs_l = reinterpret_cast<float*>(lds + kEpiBytes);  // [BM] row scales
  float* mx_l = rs_l + BM;                                   // [BM][WGN] per-wave row |max|
  float* sc_l = mx_l + BM * WGN;                             // [BM] output row scales
  float* inv_l = sc_l + BM;                                  // [BM] their reciprocals
  unsigned* last_l = reinterpret_cast<unsigned*>(inv_l + BM);
  for (int r = tid; r < BM; r += NT) rs_l[r] = row0 + r < p.M ? p.row_scales[row0 + r] : 0.0f;
  __syncthreads();
  const int c4 = (lane % kLanesPerRow) * 4;
  const int gcol = col0 + wn * WN + c4;
  const bool col_ok = gcol < p.N;
  v4f cs = {1.0f, 1.0f, 1.0f, 1.0f}, bs = {0.0f, 0.0f, 0.0f, 0.0f};
  if (col_ok) {
    cs = *reinterpret_cast<const v4f*>(p.col_scales + gcol);
    if (p.bias) bs = *reinterpret_cast<const v4f*>(p.bias + gcol);
  }
  v4f val[TM][kPasses];
#pragma unroll
  for (int i = 0; i < TM; i++) {
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++)
        ep[((r >> 2) * 8 + fg * 4 + (r & 3)) * kEpiStride + j * 32 + fr] = acc[i][j][r];
    wait_lgkmcnt0();
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int it = 0; it < kPasses; it++) {
      const int rr = lane / kLanesPerRow + it * kRowsPerPass;
      const int trow = wm * WM + i * 32 + rr;
      const v4i a = *reinterpret_cast<const v4i*>(ep + rr * kEpiStride + c4);
      v4f v = {0.0f, 0.0f, 0.0f, 0.0f};
      if (row0 + trow < p.M && col_ok) {
        const float rs = rs_l[trow];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float x = (float)a[e] * rs;
          x = x * cs[e];
          if (p.bias) x = x + bs[e];
          v[e] = apply_act(x, p.act);
        }
      }
      val[i][it] = v;
      // invalid lanes contribute 0; every lane takes part in the shuffles
      float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
      for (int o = kLanesPerRow / 2; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      if (lane % kLanesPerRow == 0) mx_l[trow * WGN + wn] = m;
    }
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  if (tid < BM && row0 + tid < p.M) {
    // publish this tile's |max| of the row, then gather the row's slots
    float m = mx_l[tid * WGN];
#pragma unroll
    for (int w = 1; w < WGN; w++) m = fmaxf(m, mx_l[tid * WGN + w]);
    unsigned* slot = p.slots + (size_t)(row0 + tid) * p.slot_ld;
    __hip_atomic_store(slot + cb, __float_as_uint(m), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    unsigned mx = 0;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
      unsigned v[kQsyncMaxTiles];
#pragma unroll
      for (int c = 0; c < kQsyncMaxTiles; c++)
        v[c] = c < tiles_n
                   ? __hip_atomic_load(slot + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                   : 0u;
      bool full = true;
      mx = 0;
#pragma unroll
      for (int c = 0; c < kQsyncMaxTiles; c++) {
        full = full && v[c] != kSlotEmpty;
        mx = max(mx, v[c] == kSlotEmpty ? 0u : v[c]);
      }
      if (full) break;
      if (__builtin_amdgcn_s_memrealtime() - t0 > kSyncWaitTicks) {
        atomicOr(p.sync_err, 1u);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    // QuantizeRowU8's scale (pack_vnni.go:94-101); |max| bits order as floats
    float sc = __uint_as_float(mx) / 127.0f;
    if (sc == 0.0f) sc = 1.0f;
    sc_l[tid] = sc;
    inv_l[tid] = 1.0f / sc;
  }
  __syncthreads();
  // every read of the slots has returned: count this workgroup out
  // (the count's value is needed only after the stores below)
  unsigned dep = 0;
  if (tid == 0) dep = atomicAdd(p.sync + rb, 1u);
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int it = 0; it < kPasses; it++) {
      const int trow = wm * WM + i * 32 + lane / kLanesPerRow + it * kRowsPerPass;
      const int grow = row0 + trow;
      if (grow < p.M && col_ok) {
        const float inv = inv_l[trow];
        const v4f v = val[i][it];
        const uint32_t w = quant_byte(v[0], inv) | (quant_byte(v[1], inv) << 8) |
                           (quant_byte(v[2], inv) << 16) | (quant_byte(v[3], inv) << 24);
        *reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(p.out) + (size_t)grow * p.ldo + gcol) = w;
        if (gcol == 0) p.rs_out[grow] = sc_l[trow];
      }
    }
  if (tid == 0) last_l[0] = dep == (unsigned)tiles_n - 1;
  __syncthreads();
  if (last_l[0]) {
    for (int i = tid; i < BM * tiles_n; i += NT) {
      const int r = i / tiles_n, c = i - r * tiles_n;
      if (row0 + r < p.M)
        __hip_atomic_store(p.slots + (size_t)(row0 + r) * p.slot_ld + c, kSlotEmpty,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid == 0) __hip_atomic_store(p.sync + rb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// EPI_QSYNC workgroup -> tile: workgroup b runs on XCD b % 8 (the dispatch
// order) as that XCD's (b / 8)-th; each XCD owns ceil(tiles_m / 8)
// consecutive row blocks and runs them one after another, a row block's
// column tiles in a row. Workgroups past the last row block have no tile
// (rb >= tiles_m). Pairs of row blocks down each column (the order of the
// other tiles) took 101 against 86 µs at M = 10102, N = 3072: a row
// block's tiles then spread over twice as many workgroups, which wait
// longer for the last of them.
__device__ __forceinline__ void qsync_tile(int b, int tiles_m, int tiles_n, int& rb, int& cb) {
  constexpr int kXcd = 8;
  const int per_xcd = (tiles_m + kXcd - 1) / kXcd;
  const int k = b / kXcd;
  rb = (b % kXcd) * per_xcd + k / tiles_n;
  cb = k % tiles_n;
}

// WGN waves along N: 2 = a 2x2 grid of 4 waves, 4 = a 2x4 grid of 8 (two per
// SIMD when one workgroup fills a CU).
// BK: k bytes per stage and row, 64 (i8_slot rows) or 128 (lds_off rows;
// half the barriers, four k-steps per stage).
template <int BM, int BN, int NS, int EPI, int WGN = 2, int BK = 64>
__global__ __launch_bounds__(128 * WGN) void gemm_i8_kernel(GemmI8Args p) {
  constexpr int NT = 128 * WGN, NW = 2 * WGN;
  constexpr int CPR = BK / 16;  // 16-byte chunks per row
  constexpr int WM = BM / 2, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int kA = BM * BK, kB = BN * BK, kStage = kA + kB;
  constexpr int LA = kA / (NT * 16), LB = kB / (NT * 16);  // loads per thread
  constexpr int kLoads = LA + LB;
  constexpr int kEpiStride = WN + 4;  // ints per row of the epilogue transpose
  constexpr int kEpiBytes = NW * 32 * kEpiStride * 4;
  static_assert(LA >= 1 && LB >= 1 && TN >= 1, "tile too small for the wave grid");
  static_assert(NS * kStage >= kEpiBytes + 3 * BM * 4, "epilogue LDS");
  static_assert(EPI != EPI_QSYNC || NS * kStage >= kEpiBytes + (3 + WGN) * BM * 4 + 4,
                "single-pass epilogue LDS");
  static_assert(NS * kStage <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int tiles_n = (p.N + BN - 1) / BN;
  int rb, cb;
  if constexpr (EPI == EPI_QSYNC) {
    qsync_tile(blockIdx.x, (p.M + BM - 1) / BM, tiles_n, rb, cb);
    if (rb >= (p.M + BM - 1) / BM) return;
  } else {
    tile_origin(xcd_remap(blockIdx.x, gridDim.x), (p.M + BM - 1) / BM, tiles_n, p.tile_group,
                rb, cb);
  }
  const int row0 = rb * BM;
  const int col0 = cb * BN;
  const int nk = (p.K + BK - 1) / BK;

  // Per-lane source rows/chunks of this thread's loads (fixed across stages).
  // Rows past M read row M-1 (any in-bounds bytes: their outputs are never
  // stored); B rows are zero-padded to a multiple of 256.
  const uint8_t* asrc[LA];
  int achunk[LA];
#pragma unroll
  for (int j = 0; j < LA; j++) {
    const int slot = (wave * LA + j) * 64 + lane;
    const int r = slot / CPR;
    achunk[j] = stage_slot_chunk<BK>(r, slot % CPR);
    const int gr = row0 + r;
    asrc[j] = p.A + (size_t)(gr < p.M ? gr : p.M - 1) * p.lda;
  }
  const int8_t* bsrc[LB];
  int bchunk[LB];
#pragma unroll
  for (int j = 0; j < LB; j++) {
    const int slot = (wave * LB + j) * 64 + lane;
    const int r = slot / CPR;
    bchunk[j] = stage_slot_chunk<BK>(r, slot % CPR);
    bsrc[j] = p.B + (size_t)(col0 + r) * p.ldb;
  }

  auto issue = [&](int kt, int slot) {
    uint8_t* s = lds + slot * kStage;
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

  // Fragments of one 32-byte k-step, double-buffered in registers: the LDS
  // reads of step s+1 are in flight while the MFMAs of step s run, and at a
  // stage's end the next stage's first reads go out right after its barrier.
  constexpr int S = BK / 32;
  static_assert(S % 2 == 0 && NS <= 4, "k-steps per stage / ring depth");
  const int fr = lane & 31, fg = lane >> 5;
  v4i fa[2][TM], fb[2][TN];
  auto load = [&](int slot, int s, v4i (&a)[TM], v4i (&b)[TN]) {
    const uint8_t* sA = lds + slot * kStage;
    const uint8_t* sB = sA + kA;
    const int c = 2 * s + fg;
#pragma unroll
    for (int i = 0; i < TM; i++)
      a[i] = *reinterpret_cast<const v4i*>(sA + stage_frag_off<BK>(wm * WM + i * 32 + fr, c));
#pragma unroll
    for (int j = 0; j < TN; j++)
      b[j] = *reinterpret_cast<const v4i*>(sB + stage_frag_off<BK>(wn * WN + j * 32 + fr, c));
  };
  auto mma = [&](const v4i (&a)[TM], const v4i (&b)[TN]) {
#pragma unroll
    for (int i = 0; i < TM; i++) {
      const v4i ai = a[i] ^ (int)0x80808080;
#pragma unroll
      for (int j = 0; j < TN; j++)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ai, b[j], acc[i][j], 0, 0, 0);
    }
  };
  // This wave's DMA of stage `st` has landed once at most min(NS-2, later)
  // younger stages are pending (later = stages issued after it).
  auto wait_stage = [&](int later) {
    if (later >= NS - 2) wait_vmcnt<(NS - 2) * kLoads>();
    else if (NS > 3 && later == 1) wait_vmcnt<kLoads>();
    else wait_vmcnt<0>();
  };

#pragma unroll
  for (int st = 0; st < NS - 1; st++)
    if (st < nk) issue(st, st);
  wait_stage(nk - 1);
  stage_barrier();
  if (NS - 1 < nk) issue(NS - 1, NS - 1);
  load(0, 0, fa[0], fb[0]);

  // Unrolled by the ring depth, so every slot offset is a constant.
  for (int kt0 = 0; kt0 < nk; kt0 += NS) {
#pragma unroll
    for (int u = 0; u < NS; u++) {
      const int kt = kt0 + u;
      if (kt >= nk) break;
#pragma unroll
      for (int s = 0; s < S; s++) {
        if (s + 1 < S) {
          load(u, s + 1, fa[(s + 1) & 1], fb[(s + 1) & 1]);
        } else {
          // The last step's fragments have returned (on every path, so the
          // MFMAs below need no wait that would also cover the next stage's
          // reads). Slot u (= kt % NS) is refilled after the barrier, which is safe
          // once every wave is past this point; stage kt+1 must have landed
          // for every wave.
          wait_lgkmcnt0();
        }
        if (s + 1 == S && kt + 1 < nk) {
          wait_stage(nk - 2 - kt);
          stage_barrier();
          if (kt + NS < nk) issue(kt + NS, u);
          load((u + 1) % NS, 0, fa[0], fb[0]);
        }
        mma(fa[s & 1], fb[s & 1]);
        // keep each step's MFMAs ahead of the next step's waits
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  if constexpr (EPI == EPI_QSYNC)
    i8_epilogue_qsync<BM, WM, WN, TM, TN, NW, NT>(p, acc, lds, row0, col0, rb, cb, tiles_n,
                                                  wave, wm, wn, tid);
  else
    i8_epilogue<BM, WM, WN, TM, TN, NW, NT, EPI>(p, acc, lds, row0, col0, wave, wm, wn, tid);
}

// ---- 128x128 wave tiles for the long-K problems ---------------------------------
// 256 x 256 tile on 4 waves (2 x 2), each wave 128 x 128 = 4 x 4 MFMA tiles with
// its 256 accumulators in AGPRs: 0.5 KiB of LDS fragment reads per MFMA
// against 1 KiB for the 64 x 64 waves above. K in 64-byte stages (i8_slot
// rows), an NS-slot ring refilled right after each stage's barrier. The loop
// body has no branch: stages past the last are clamped to it (a reload of
// real bytes into a slot nobody reads again), so each stage is followed by
// the same number of younger loads and every wait count is a constant — a
// branch in the body made the compiler copy the 256 accumulators through
// VGPRs at every back edge. The stage's DMA and the next k-step's fragment
// reads are spread one per MFMA (sched_group_barrier), so their issue hides
// behind the matrix core. Requires ceil(K / 64) % NS == 0 (launch_w4 checks).
// The same products in the same k order as the other tiles: the same int32
// accumulators.
template <int NS, int EPI>
__global__ __launch_bounds__(256, 1) void gemm_i8_w4_kernel(GemmI8Args p) {
  constexpr int BM = 256, BN = 256, BK = 64, WGN = 2;
  constexpr int NT = 256, NW = 4, CPR = BK / 16;
  constexpr int WM = 128, WN = 128, TM = 4, TN = 4;
  constexpr int kA = BM * BK, kB = BN * BK, kStage = kA + kB;
  constexpr int LA = kA / (NT * 16), LB = kB / (NT * 16);  // 4 + 4
  constexpr int kLoads = LA + LB;
  constexpr int S = BK / 32;  // k-steps per stage
  static_assert(NS >= 3 && NS * kStage <= 160 * 1024, "ring");
  static_assert(NS * kStage >= NW * 32 * (WN + 4) * 4 + 3 * BM * 4, "epilogue LDS");
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
  const int row0 = rb * BM, col0 = cb * BN;
  const int nk = (p.K + BK - 1) / BK;

  // Per-lane sources (rows past M read row M-1; B rows are zero-padded to
  // a multiple of 256, and B is zero past K).
  const uint8_t* asrc[LA];
  int achunk[LA];
#pragma unroll
  for (int j = 0; j < LA; j++) {
    const int slot = (wave * LA + j) * 64 + lane;
    const int r = slot / CPR;
    achunk[j] = stage_slot_chunk<BK>(r, slot % CPR) * 16;
    const int gr = row0 + r;
    asrc[j] = p.A + (size_t)(gr < p.M ? gr : p.M - 1) * p.lda;
  }
  const int8_t* bsrc[LB];
#pragma unroll
  for (int j = 0; j < LB; j++) {
    const int slot = (wave * LB + j) * 64 + lane;
    const int r = slot / CPR;
    bsrc[j] = p.B + (size_t)(col0 + r) * p.ldb + stage_slot_chunk<BK>(r, slot % CPR) * 16;
  }
  auto issue = [&](int kt, int slot) {
    kt = kt < nk ? kt : nk - 1;
    uint8_t* st = lds + slot * kStage;
    const int k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < LA; j++) {
      int kb = k0 + achunk[j];
      kb = kb < p.lda ? kb : 0;  // past the row: any in-bounds bytes (B is 0 there)
      lds_dma16(asrc[j] + kb, st + (wave * LA + j) * 1024);
    }
#pragma unroll
    for (int j = 0; j < LB; j++) lds_dma16(bsrc[j] + k0, st + kA + (wave * LB + j) * 1024);
  };

  v16i acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = v16i{};
  // Fragment offsets: rows 32 apart sit 2 KiB apart (i8_slot's permutation
  // depends on (r >> 2) & 3 only) and k-step s XORs the chunk index by 2s,
  // so one base per operand serves every fragment.
  const int fr = lane & 31, fg = lane >> 5;
  const int abase = stage_frag_off<BK>(wm * WM + fr, fg);
  const int bbase = kA + stage_frag_off<BK>(wn * WN + fr, fg);
  v4i fa[2][TM], fb[2][TN];
  auto load = [&](int slot, int s, v4i (&a)[TM], v4i (&b)[TN]) {
    const uint8_t* st = lds + slot * kStage;
    const int ab = abase ^ (32 * s), bb = bbase ^ (32 * s);
#pragma unroll
    for (int i = 0; i < TM; i++) a[i] = *reinterpret_cast<const v4i*>(st + ab + i * 32 * BK);
#pragma unroll
    for (int j = 0; j < TN; j++) b[j] = *reinterpret_cast<const v4i*>(st + bb + j * 32 * BK);
  };
  auto mma = [&](v4i (&a)[TM], const v4i (&b)[TN]) {
#pragma unroll
    for (int i = 0; i < TM; i++) a[i] ^= (int)0x80808080;  // u8 -> s8 (q = u8 - 128)
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
  };

#pragma unroll
  for (int st = 0; st < NS - 1; st++) issue(st, st);
  wait_vmcnt<(NS - 2) * kLoads>();
  stage_barrier();
  issue(NS - 1, NS - 1);
  load(0, 0, fa[0], fb[0]);
  for (int kt0 = 0; kt0 < nk; kt0 += NS) {
#pragma unroll
    for (int u = 0; u < NS; u++) {
      const int kt = kt0 + u;
#pragma unroll
      for (int s = 0; s < S; s++) {
        if (s + 1 < S) {
          load(u, s + 1, fa[(s + 1) & 1], fb[(s + 1) & 1]);
          mma(fa[s & 1], fb[s & 1]);
#pragma unroll
          for (int g = 0; g < TM + TN; g++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
          }
          __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - (TM + TN), 0);
        } else {
          wait_lgkmcnt0();
          // stage kt+1 has landed for this wave: NS-2 younger stages pending
          wait_vmcnt<(NS - 2) * kLoads>();
          stage_barrier();  // ... for every wave; slot u is free
          issue(kt + NS, u);
          load((u + 1) % NS, 0, fa[0], fb[0]);
          mma(fa[s & 1], fb[s & 1]);
#pragma unroll
          for (int g = 0; g < kLoads; g++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM (DMA)
          }
#pragma unroll
          for (int g = 0; g < TM + TN; g++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  wait_vmcnt<0>();  // clamped refills may still be landing
  i8_epilogue<BM, WM, WN, TM, TN, NW, NT, EPI>(p, acc, lds, row0, col0, wave, wm, wn, tid);
}

// ---- B fragments straight to registers ------------------------------------
// 64 x 256 tile on 4 waves side by side (each 64 rows x 64 columns: 2 x 2
// MFMA tiles). Only A goes through LDS (128-byte stage rows by
// global_load_lds_dwordx4, NS-slot ring, one barrier per stage); each wave
// loads its own B fragments from the fragment-ordered image (rh_weight::
// d_frag) with one 16-byte global load per lane and fragment, D k-steps ahead
// into a register ring. Per MFMA the CU's LDS then serves 0.5 KiB of A
// fragment reads instead of 1 KiB of A and B, and no B byte is written to
// LDS at all: the main loop of the LDS-staged kernel above is bound by LDS
// bandwidth.
//
// Every stage issues the same loads in the same order (a compiler and
// scheduler fence follows each A DMA, so no B load moves above it), so the
// count of loads younger than a stage's A DMA is one constant: the ring is
// primed as stages -(NS-1)..-1 would have issued it. Past the last stage the
// k indices are clamped (an A reload into a freed slot, B reloads nobody
// reads). Those B reloads may be dropped by the compiler as dead or merged
// as duplicates, which would leave fewer younger loads than the constant
// assumes, so the stages that follow one that issued them (the last NS-1)
// wait for every outstanding load instead.
// The B ring holds NS stages of k-steps, so with the stage loop unrolled by
// NS every ring slot is a constant register set. NK > 0: the kernel is built
// for exactly NK stages and the stage loop is unrolled completely; the
// compiler then counts every B register's outstanding loads exactly (across
// a loop back-edge it waits for all loads to drain, which empties the
// prefetch ring once per NS stages). NK = 0: any K, a loop.
// Compiler and scheduler fence: no memory access moves across it.
__device__ __forceinline__ void load_fence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// The main loop of the fragment-B kernels: A (BM rows of 128-byte stages)
// by DMA into an NS-slot LDS ring, this wave's TN B fragments per k-step
// straight to registers from the fragment-ordered weight, D = 4·NS k-steps
// ahead; acc receives the wave's WM x (32·TN) int32 block at rows
// row0 + wm·WM and columns colw. On return every load has landed and the
// caller may reuse the LDS.
template <int NS, int NK, int BM, int NT, int TM, int TN>
__device__ __forceinline__ void i8f_main_loop(const GemmI8Args& p, uint8_t* lds,
                                              v16i (&acc)[TM][TN], int row0, int colw,
                                              int wave, int wm, int lane) {
  constexpr int BK = 128, CPR = BK / 16;  // A stage row bytes, 16-byte chunks per row
  constexpr int WM = 32 * TM;
  constexpr int KPS = BK / 32;               // k-steps per stage
  constexpr int D = KPS * NS;                // B ring depth in k-steps
  constexpr int kA = BM * BK;                // A bytes per stage
  constexpr int LA = kA / (NT * 16);         // A DMA instructions per thread per stage
  // loads younger than stage t's A DMA when stage t begins: the B loads of
  // the NS-1 stages before it and the A DMAs of the NS-2 between
  constexpr int kWaitA = (NS - 1) * KPS * TN + (NS - 2) * LA;
  static_assert(LA >= 1 && kWaitA <= 63 && NS >= 2, "ring");
  const int nk = NK > 0 ? NK : (p.K + BK - 1) / BK;  // stages
  const int nks = nk * KPS;  // k-steps (= kp / 32 of the weight)
  // A DMA sources, as in gemm_i8_kernel (rows past M read row M-1).
  const uint8_t* asrc[LA];
  int achunk[LA];
#pragma unroll
  for (int j = 0; j < LA; j++) {
    const int slot = (wave * LA + j) * 64 + lane;
    const int r = slot / CPR;
    achunk[j] = stage_slot_chunk<BK>(r, slot % CPR);
    const int gr = row0 + r;
    asrc[j] = p.A + (size_t)(gr < p.M ? gr : p.M - 1) * p.lda;
  }
  auto issue_a = [&](int kt, int slot) {
    kt = kt < nk ? kt : nk - 1;
    uint8_t* s = lds + slot * kA;
    const int k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < LA; j++) {
      int kb = k0 + achunk[j] * 16;
      kb = kb < p.lda ? kb : 0;  // past the row: any in-bounds bytes (B is 0 there)
      lds_dma16(asrc[j] + kb, s + (wave * LA + j) * 1024);
    }
  };
  // This lane's 16 bytes of each of the wave's column blocks; k-step ks is
  // ks KiB further (np % 256 == 0 keeps every block of the tile in the image).
  const int8_t* bsrc[TN];
#pragma unroll
  for (int j = 0; j < TN; j++)
    bsrc[j] = p.Bf + (size_t)((colw + j * 32) >> 5) * nks * 1024 + lane * 16;
  v4i bq[D][TN];
  auto load_b = [&](int ks, v4i (&dst)[TN]) {
    ks = ks < nks ? ks : nks - 1;
#pragma unroll
    for (int j = 0; j < TN; j++) dst[j] = *reinterpret_cast<const v4i*>(bsrc[j] + (size_t)ks * 1024);
  };

#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = v16i{};
  const int fr = lane & 31, fg = lane >> 5;

  // Prime: stage 0's B k-steps, then for each virtual stage v = -(NS-1)..-1
  // the A DMA of stage v + NS - 1 and the B loads of its k-steps + D.
#pragma unroll
  for (int s = 0; s < KPS; s++) load_b(s, bq[s]);
#pragma unroll
  for (int v = 0; v < NS - 1; v++) {
    load_fence();
    issue_a(v, v);
    load_fence();
#pragma unroll
    for (int s = 0; s < KPS; s++) load_b((v + 1) * KPS + s, bq[(v + 1) * KPS + s]);
  }

  constexpr int kUnroll = NK > 0 ? (NK + NS - 1) / NS : 1;
#pragma unroll kUnroll
  for (int t0 = 0; t0 < nk; t0 += NS) {
#pragma unroll
    for (int u = 0; u < NS; u++) {
      const int t = t0 + u;
      if (t >= nk) break;
      load_fence();
      // this wave's A DMA of stage t has landed
      if (t + NS - 1 >= nk) wait_vmcnt<0>();
      else wait_vmcnt<kWaitA>();
      stage_barrier();  // every wave's has; slot (t-1) % NS is free
      issue_a(t + NS - 1, (u + NS - 1) % NS);
      load_fence();
      const uint8_t* sA = lds + u * kA;
#pragma unroll
      for (int s = 0; s < KPS; s++) {
        const int rs = u * KPS + s;  // = (t * KPS + s) % D
        v4i fa[TM];
#pragma unroll
        for (int i = 0; i < TM; i++)
          fa[i] = *reinterpret_cast<const v4i*>(
                      sA + stage_frag_off<BK>(wm * WM + i * 32 + fr, 2 * s + fg)) ^
                  (int)0x80808080;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
          for (int j = 0; j < TN; j++)
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], bq[rs][j], acc[i][j], 0, 0, 0);
        load_b(t * KPS + s + D, bq[rs]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // The clamped refills past the last stage may still be landing in LDS.
  wait_vmcnt<0>();
}

template <int NS, int EPI, int NK, int WGM = 1>
__global__ __launch_bounds__(256 * WGM, 2 / WGM) void gemm_i8f_kernel(GemmI8Args p) {
  constexpr int BM = 64 * WGM, BN = 256, NT = 256 * WGM, NW = 4 * WGM;
  constexpr int WM = 64, WN = 64, TM = WM / 32, TN = WN / 32;
  constexpr int kA = BM * 128;  // A bytes per stage
  constexpr int kEpiBytes = NW * 32 * (WN + 4) * 4;
  constexpr int kLds = NS * kA > kEpiBytes + 3 * BM * 4 ? NS * kA : kEpiBytes + 3 * BM * 4;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kLds];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / 4, wn = wave % 4;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  int rb, cb;
  tile_origin(tile, (p.M + BM - 1) / BM, tiles_n, p.tile_group, rb, cb);
  const int row0 = rb * BM;
  const int col0 = cb * BN;
  v16i acc[TM][TN];
  i8f_main_loop<NS, NK, BM, NT, TM, TN>(p, lds, acc, row0, col0 + wn * WN, wave, wm, lane);
  i8_epilogue<BM, WM, WN, TM, TN, NW, NT, EPI>(p, acc, lds, row0, col0, wave, wm, wn, tid);
}

// ---- whole rows per workgroup, with the residual + LayerNorm epilogue ---------------
// 64 rows x all N columns on NWN waves side by side (each 64 x 32·TN: 2 x TN
// MFMA tiles), the main loop of the fragment-B kernels. The epilogue, per
// 32-row band: every wave parks y = f32(acc)·rs·cs (+ bias) — the EPI_F32
// epilogue's operations — in an LDS band [32][N + 8] (the two half-waves'
// rows land 32 banks apart), then each wave takes whole rows: v = x + y and
// ln_vec_finish, exactly add_ln_vec_kernel's steps. So the layer's two
// passes (the linear's fp32 rows to HBM and back, then the residual add and
// LayerNorm) become one kernel with identical results, and the fp32 y never
// leaves the CU. With N the hidden width the grid has ceil(M / 64)
// workgroups (158 at M = 10102): each streams the whole B image from L2.
template <int NS, int NK, int NWN, int TN>
__global__ __launch_bounds__(64 * NWN, 1) void gemm_i8_ln_kernel(GemmI8Args p, I8LnArgs f) {
  constexpr int BM = 64, TM = 2, NT = 64 * NWN, WN = 32 * TN, N = NWN * WN;
  constexpr int V = (N + 255) / 256;  // float4 groups per lane of a row
  constexpr int kA = BM * 128;
  constexpr int kStride = N + 8;      // floats per band row
  constexpr int kBand = 32 * kStride * 4;
  constexpr int kLds = NS * kA > kBand ? NS * kA : kBand;
  static_assert(kLds <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kLds];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row0 = blockIdx.x * BM;
  v16i acc[TM][TN];
  i8f_main_loop<NS, NK, BM, NT, TM, TN>(p, lds, acc, row0, wave * WN, wave, 0, lane);

  const int fr = lane & 31, fg = lane >> 5;
  float cs[TN], bs[TN];
#pragma unroll
  for (int j = 0; j < TN; j++) {
    const int col = wave * WN + j * 32 + fr;
    cs[j] = p.col_scales[col];
    bs[j] = p.bias ? p.bias[col] : 0.0f;
  }
  float* band = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int i = 0; i < TM; i++) {
    __syncthreads();  // the ring's last reads / the previous band's rows are done
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int lr = (r >> 2) * 8 + fg * 4 + (r & 3);  // the MFMA tile's row of element r
      const int gr = row0 + i * 32 + lr;
      const float rs = gr < p.M ? p.row_scales[gr] : 0.0f;
#pragma unroll
      for (int j = 0; j < TN; j++) {
        float y = (float)acc[i][j][r] * rs;
        y = y * cs[j];
        if (p.bias) y = y + bs[j];
        band[lr * kStride + wave * WN + j * 32 + fr] = y;
      }
    }
    __syncthreads();
    for (int lr = wave; lr < 32; lr += NWN) {
      const int grow = row0 + i * 32 + lr;
      if (grow >= p.M) break;
      float* xr = f.x + (size_t)grow * N;
      v4f v[V];
#pragma unroll
      for (int e = 0; e < V; e++) {
        const int j = (lane + 64 * e) * 4;
        v4f t = {0.0f, 0.0f, 0.0f, 0.0f};
        if (j < N) {
          t = *reinterpret_cast<const v4f*>(xr + j);
          t = t + *reinterpret_cast<const v4f*>(band + lr * kStride + j);  // Add
        }
        v[e] = t;
      }
      ln_vec_finish<V>(v, lane, grow, N, f.gamma, f.beta, f.eps, xr, f.qa, f.ldq,
                       f.row_scales, nullptr, nullptr, 0);
    }
  }
}

template <int NWN, int TN>
static hipError_t launch_ln(const GemmI8Args& a, const I8LnArgs& f, hipStream_t s) {
  const dim3 g(ceil_div(a.M, 64)), b(64 * NWN);
  switch (ceil_div(a.K, 128)) {  // fully unrolled builds for the encoder widths
    case 3: timed_launch((gemm_i8_ln_kernel<2, 3, NWN, TN>), g, b, 0, s, a, f); break;
    case 6: timed_launch((gemm_i8_ln_kernel<2, 6, NWN, TN>), g, b, 0, s, a, f); break;
    case 12: timed_launch((gemm_i8_ln_kernel<2, 12, NWN, TN>), g, b, 0, s, a, f); break;
    case 24: timed_launch((gemm_i8_ln_kernel<2, 24, NWN, TN>), g, b, 0, s, a, f); break;
    default: timed_launch((gemm_i8_ln_kernel<2, 0, NWN, TN>), g, b, 0, s, a, f);
  }
  return hipGetLastError();
}

bool gemm_i8_ln_supported(int n, int k) {
  return (n == 384 || n == 768 || n == 1024) && k >= 1;
}

hipError_t launch_gemm_i8_ln(const GemmI8Args& a, const I8LnArgs& f, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (!a.Bf || a.epi != EPI_F32 || a.act != ACT_NONE || !f.x || !f.gamma || !f.beta ||
      (f.qa && (!f.row_scales || f.ldq % 4)) || !gemm_i8_ln_supported(a.N, a.K))
    return hipErrorInvalidValue;
  switch (a.N) {
    case 384: return launch_ln<4, 3>(a, f, s);
    case 768: return launch_ln<8, 3>(a, f, s);
    default: return launch_ln<8, 4>(a, f, s);  // 1024
  }
}

template <int NS, int EPI, int WGM = 1>
static hipError_t launch_frag(const GemmI8Args& a, hipStream_t s) {
  const int tiles = ceil_div(a.M, 64 * WGM) * ceil_div(a.N, 256);
  const dim3 g(tiles), b(256 * WGM);
  // fully unrolled builds for the encoder widths (K = 768 and 3072)
  switch (ceil_div(a.K, 128)) {
    case 6: timed_launch((gemm_i8f_kernel<NS, EPI, 6, WGM>), g, b, 0, s, a); break;
    case 24: timed_launch((gemm_i8f_kernel<NS, EPI, 24, WGM>), g, b, 0, s, a); break;
    default: timed_launch((gemm_i8f_kernel<NS, EPI, 0, WGM>), g, b, 0, s, a);
  }
  return hipGetLastError();
}

template <int BM, int BN, int NS, int EPI, int WGN = 2, int BK = 64>
static hipError_t launch_tile(const GemmI8Args& a, hipStream_t s) {
  const int tiles = ceil_div(a.M, BM) * ceil_div(a.N, BN);
  timed_launch((gemm_i8_kernel<BM, BN, NS, EPI, WGN, BK>), dim3(tiles), dim3(128 * WGN), 0, s,
               a);
  return hipGetLastError();
}

// Tile 15: the 128x128-wave kernel with a four-slot ring where the stage
// count allows it, else three, else tile 9.
template <int EPI>
static hipError_t launch_w4(const GemmI8Args& a, hipStream_t s) {
  const int nk = ceil_div(a.K, 64);
  const dim3 g(ceil_div(a.M, 256) * ceil_div(a.N, 256)), b(256);
  if (nk % 4 == 0) timed_launch((gemm_i8_w4_kernel<4, EPI>), g, b, 0, s, a);
  else if (nk % 3 == 0) timed_launch((gemm_i8_w4_kernel<3, EPI>), g, b, 0, s, a);
  else return launch_tile<128, 256, 2, EPI, 4, 128>(a, s);
  return hipGetLastError();
}

// 1 = 256x256, 2 = 256x128 and 3 = 128x128 with 4 stages; 4 = 256x128 and
// 5 = 128x256 with 3 stages; 6 = 256x256 (4 stages) and 7 = 128x256 (3
// stages) on 8 waves. Tiles 4, 5 and 7 take 72 KiB of LDS and <= 256
// registers per lane, so two workgroups share a CU.
template <int EPI>
static hipError_t launch_epi(const GemmI8Args& a, int tile, hipStream_t s) {
  switch (tile) {
    case 1: return launch_tile<256, 256, 4, EPI>(a, s);
    case 2: return launch_tile<256, 128, 4, EPI>(a, s);
    case 4: return launch_tile<256, 128, 3, EPI>(a, s);
    case 5: return launch_tile<128, 256, 3, EPI>(a, s);
    case 6: return launch_tile<256, 256, 4, EPI, 4>(a, s);
    case 7: return launch_tile<128, 256, 3, EPI, 4>(a, s);
    case 8: return launch_tile<256, 256, 2, EPI, 4, 128>(a, s);
    case 9: return launch_tile<128, 256, 2, EPI, 4, 128>(a, s);
    case 10: return launch_tile<128, 256, 3, EPI, 4, 128>(a, s);
    case 11: return a.Bf ? launch_frag<3, EPI>(a, s) : hipErrorInvalidValue;
    case 12: return a.Bf ? launch_frag<4, EPI>(a, s) : hipErrorInvalidValue;
    case 13: return a.Bf ? launch_frag<2, EPI, 2>(a, s) : hipErrorInvalidValue;
    case 14: return a.Bf ? launch_frag<3, EPI, 2>(a, s) : hipErrorInvalidValue;
    case 15: return launch_w4<EPI>(a, s);
    default: return launch_tile<128, 128, 4, EPI>(a, s);
  }
}

// Automatic tile, measured on MI355X over the BERT-base linears at M = 10102
// and 16384: 128x256 with 8 waves (two workgroups and four waves per SIMD
// per CU; ahead of 256x256 by 7-12% at N = 3072), or its 128-byte-stage
// form where that occupancy cannot be had or does not pay: a grid of at
// most one workgroup per CU (N = 768 at M = 10102) or deep K (3072), where
// the halved barrier count wins. Small problems keep 128x128 so the grid
// still covers the CUs.
int pick_i8_tile(int M, int N, int K, int epi) {
  (void)epi;
  const int tiles = ceil_div(M, 128) * ceil_div(N, 256);
  // The fragment-B 128x256 tile (B fragments straight to registers halve
  // the LDS reads) for deep K on a grid of at most one such workgroup per CU
  // (the BERT-base FFN2 at M = 10102: 34.2 against 35.5 µs fp32 out, 31.9
  // against 33.2 int32 out), and for any K on 64..127 of them: the
  // two-stream headline runs its parts of ~5050 rows, where O and FFN2 give
  // 120 such tiles; against 128x128 there the whole forward went from 3.28
  // to 3.34 M tokens/s with FFN2 on it and from 3.47 to 3.51 with O as well
  // (interleaved runs)
  if ((K >= 2048 || tiles < 128) && tiles <= 256 && tiles >= 64) return 13;
  if (tiles < 128) return 3;
  // deep K on a grid of at least one 256x256 tile per CU: the 128x128-wave
  // tile (4-12 % ahead of tiles 7 and 9 at M = 16384, K = 2048 and 3072)
  const int nk = ceil_div(K, 64);
  if (K >= 2048 && ceil_div(M, 256) * ceil_div(N, 256) >= 256 && (nk % 4 == 0 || nk % 3 == 0))
    return 15;
  return (K >= 2048 || tiles <= 256) ? 9 : 7;
}

// EPI_QSYNC on the 128x256 tiles of gemm_i8_kernel (7, 9, 10; any other
// choice takes 7), on the grid qsync_tile maps: 8 XCDs x ceil(tiles_m / 8)
// row blocks x tiles_n.
template <int BN, int NS, int WGN = 2, int BK = 64>
static hipError_t launch_qsync_tile(const GemmI8Args& a, hipStream_t s) {
  const int g = 8 * ceil_div(ceil_div(a.M, 128), 8) * ceil_div(a.N, BN);
  timed_launch((gemm_i8_kernel<128, BN, NS, EPI_QSYNC, WGN, BK>), dim3(g), dim3(128 * WGN), 0,
               s, a);
  return hipGetLastError();
}

static hipError_t launch_qsync(const GemmI8Args& a, int tile, hipStream_t s) {
  if (!a.sync || !a.sync_err || !a.slots || !a.rs_out || !a.out || !a.col_scales ||
      is_glu(a.act) || ceil_div(a.N, 256) > kQsyncMaxTiles || a.slot_ld < ceil_div(a.N, 256))
    return hipErrorInvalidValue;
  switch (tile) {
    case 9: return launch_qsync_tile<256, 2, 4, 128>(a, s);
    case 10: return launch_qsync_tile<256, 3, 4, 128>(a, s);
    default: return launch_qsync_tile<256, 3, 4>(a, s);
  }
}

hipError_t launch_gemm_i8(const GemmI8Args& a, int tile, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (a.epi == EPI_QSYNC) return launch_qsync(a, tile > 0 && tile <= kI8TileConfigs ? tile : 7, s);
  if (tile <= 0 || tile > kI8TileConfigs) {
    tile = pick_i8_tile(a.M, a.N, a.K, a.epi);
    if (tile == 13 && !a.Bf) tile = 9;  // no fragment-ordered image of B
  }
  switch (a.epi) {
    case EPI_F32: return launch_epi<EPI_F32>(a, tile, s);
    case EPI_BF16: return launch_epi<EPI_BF16>(a, tile, s);
    case EPI_ABSMAX: return launch_epi<EPI_ABSMAX>(a, tile, s);
    case EPI_QUANT: return launch_epi<EPI_QUANT>(a, tile, s);
    case EPI_ACC: return launch_epi<EPI_ACC>(a, tile, s);
    case EPI_PLANES: return launch_epi<EPI_PLANES>(a, tile, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rh
