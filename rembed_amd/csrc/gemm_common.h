// gemm_common.h — device helpers shared by the GEMM kernels.
#pragma once

#include "rh_internal.h"

namespace rh {

// Workgroups are handed to the 8 XCDs of an MI355X round-robin
// (workgroup b runs on XCD b % 8). Remap so each XCD owns a contiguous range
// of logical tile ids: with tiles ordered row-block-major, the N tiles that
// share one A row block then run on the same XCD and hit its L2.
__device__ __forceinline__ int xcd_remap(int b, int nwg) {
  constexpr int kXcd = 8;
  int q = nwg / kXcd, r = nwg % kXcd;
  int xcd = b % kXcd, idx = b / kXcd;
  return xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}

// Logical tile -> (row block, column block), grouped: consecutive tiles walk
// `group` row blocks down one column block before moving right. The tiles an
// XCD runs at once (a contiguous range after xcd_remap) then share both A row
// blocks and B column blocks in its L2 (group 1 = plain row-major order).
__device__ __forceinline__ void tile_origin(int t, int tiles_m, int tiles_n, int group,
                                            int& rb, int& cb) {
  const int per = group * tiles_n;
  const int g = t / per;
  const int first = g * group;
  const int gm = min(tiles_m - first, group);
  const int r = t - g * per;
  rb = first + r % gm;
  cb = r / gm;
}

// LDS tiles hold rows of 128 bytes = 8 chunks of 16 bytes. A 16-byte
// fragment read serves 16 consecutive rows per LDS cycle on gfx950 (64 banks
// = 256 bytes, i.e. two rows per bank window), so chunk c of row r lives at
// slot c ^ ((r ^ (r >> 3)) & 7): rows r and r+8 of one window then differ in
// slot, and any 8 aligned rows stay distinct for a 32-bank phase too.
__device__ __forceinline__ int lds_off(int r, int c) {
  return (r << 7) + ((c ^ ((r ^ (r >> 3)) & 7)) << 4);
}

// 64-byte rows of 4 chunks, chunk c of row r at slot c ^ ((r >> 2) & 3): the
// four rows of a 256-byte bank window keep their chunks in place and the
// next windows rotate them. Measured with SQ_LDS_BANK_CONFLICT on the int8
// GEMM's fragment reads (32 rows x 2 chunks per ds_read_b128): 0.4 conflict
// cycles per MFMA (the epilogue's share) against 4.4 for
// ((r >> 1) ^ (r >> 3)) & 3 and 12.4 unpermuted.
__device__ __forceinline__ int i8_slot(int row, int chunk) {
  return (row << 2) + (chunk ^ ((row >> 2) & 3));
}

// LDS layout of a stage row of RB bytes (64: i8_slot, 128: lds_off): the
// byte offset of logical 16-byte chunk c of row r, and the inverse the DMA
// needs (the logical chunk that belongs at physical slot pc of row r). Both
// permutations are involutions on the chunk index.
template <int RB>
__device__ __forceinline__ int stage_frag_off(int r, int c) {
  static_assert(RB == 64 || RB == 128, "row bytes");
  if constexpr (RB == 64) return i8_slot(r, c) * 16;
  else return lds_off(r, c);
}
template <int RB>
__device__ __forceinline__ int stage_slot_chunk(int r, int pc) {
  if constexpr (RB == 64) return pc ^ ((r >> 2) & 3);
  else return pc ^ ((r ^ (r >> 3)) & 7);
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
// s_waitcnt lgkmcnt(0) alone: this wave's LDS reads have returned.
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x3 << 14));
}
// Workgroup barrier that orders no memory by itself: no vmcnt/lgkmcnt wait
// is attached (callers wait for exactly what they need), and the empty asm
// statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// erf-GELU with exactly the float32 operation sequence of the reference's
// geluScalar (internal/tensor/tensor.go:508-538; exp body fastmath.go:93-109).
// The library is compiled with -ffp-contract=off, so no FMA is formed here.
__device__ __forceinline__ float gelu_ref(float v) {
  const float invSqrt2 = 0.7071067811865476f;
  float a = v * invSqrt2;
  float sign = 1.0f;
  if (a < 0.0f) {
    sign = -1.0f;
    a = -a;
  }
  float t = 1.0f / (1.0f + 0.3275911f * a);
  float poly =
      t * (0.254829592f +
           t * (-0.284496736f +
                t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
  float xe = -a * a;
  if (xe < -87.33f) xe = -87.33f;
  float nf = (float)(int)(xe * 1.44269504088896341f - 0.5f);
  xe -= nf * 0.693359375f;
  xe -= nf * -2.12194440e-4f;
  float z = xe * xe;
  float y = 1.9875691500e-4f;
  y = y * xe + 1.3981999507e-3f;
  y = y * xe + 8.3334519073e-3f;
  y = y * xe + 4.1665795894e-2f;
  y = y * xe + 1.6666665459e-1f;
  y = y * xe + 5.0000001201e-1f;
  float e = (y * z + xe + 1.0f) * __int_as_float(((int)nf + 127) << 23);
  float erf = sign * (1.0f - poly * e);
  return 0.5f * v * (1.0f + erf);
}

// RMSNorm's inverse scale (tensor.go:459-471): 1/float32(sqrt(float64(ss/n + eps))).
__device__ __forceinline__ float rms_inv(float ss, int n, float eps) {
  return 1.0f / (float)sqrt((double)(ss / (float)n + eps));
}

// 1/d rounded to nearest for finite d >= 1: the hardware reciprocal (within
// 1 ulp) and one Newton step with fused multiply-adds. Over every float
// input of gelu_avx2 below (all 2^32 bit patterns) this gives the same
// results as the IEEE division sequence (v_div_scale/fmas/fixup), whose
// operand scaling and special-case fixups never act for such d; the caller
// keeps d finite.
__device__ __forceinline__ float recip_ge1(float d) {
  const float r = __builtin_amdgcn_rcpf(d);
  return __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
}

// erf-GELU as rembed computes it on amd64 for every whole 8-lane group of a
// row (geluAVX2, internal/tensor/gelu_amd64.s:37-123): geluScalar's
// constants with fused multiply-adds exactly where the assembly fuses them,
// a correctly rounded reciprocal for t and trunc-toward-zero exponent
// rounding. |a| enters the reciprocal clamped to FLT_MAX (a = ±inf would
// make the Newton step NaN); past |a| ~ 4 the product poly·e is below half
// an ulp of 1, so erf is ±1 either way. 2^n scales by ldexp, which equals
// the multiplication by the power of two for every n the clamp allows.
__device__ __forceinline__ float gelu_avx2(float v) {
  const float a = v * 0.7071067811865476f;
  const float aa = fabsf(a);
  const float t = recip_ge1(__builtin_fmaf(0.3275911f, fminf(aa, 3.40282347e38f), 1.0f));
  float h = 1.061405429f;
  h = __builtin_fmaf(h, t, -1.453152027f);
  h = __builtin_fmaf(h, t, 1.421413741f);
  h = __builtin_fmaf(h, t, -0.284496736f);
  h = __builtin_fmaf(h, t, 0.254829592f);
  const float poly = h * t;
  // fmaxf instead of the reference's compare-and-set: the same value except
  // for a NaN input, whose result is NaN either way
  float xe = fmaxf(-(aa * aa), -87.33f);
  const float nf = __builtin_truncf(__builtin_fmaf(1.44269504088896341f, xe, -0.5f));
  xe = __builtin_fmaf(-0.693359375f, nf, xe);
  xe = __builtin_fmaf(2.12194440e-4f, nf, xe);
  const float z = xe * xe;
  float y = 1.9875691500e-4f;
  y = __builtin_fmaf(y, xe, 1.3981999507e-3f);
  y = __builtin_fmaf(y, xe, 8.3334519073e-3f);
  y = __builtin_fmaf(y, xe, 4.1665795894e-2f);
  y = __builtin_fmaf(y, xe, 1.6666665459e-1f);
  y = __builtin_fmaf(y, xe, 5.0000001201e-1f);
  y = __builtin_fmaf(y, z, xe);
  y = y + 1.0f;
  const float e = __builtin_amdgcn_ldexpf(y, (int)nf);
  const float val = __builtin_fmaf(-poly, e, 1.0f);
  // the sign bit of a is xor-ed into val (covers a == -0 as well)
  const float erf = __int_as_float(__float_as_int(val) ^ (__float_as_int(a) & 0x80000000));
  return (v * 0.5f) * (1.0f + erf);
}

// SiLU and the tanh-approximation GELU of the gated MLPs. The reference
// evaluates them in float64 and rounds once (tensor.SiLU: v /
// float32(1 + exp(-v)), tensor.go:477-481; tensor.GELUTanh: 0.5·x·(1 +
// tanh(c·(x + 0.044715·x³))), tensor.go:490-497). Here they run in float32
// on the accurate expf, GELUTanh in the equivalent form x / (1 + e^(-2t))
// (no cancellation where tanh(t) -> -1): within a few float32 ulp of the
// reference's values, at a fraction of the epilogue's float64 cost.
__device__ __forceinline__ float silu_f32(float v) { return v / (1.0f + expf(-v)); }

__device__ __forceinline__ float gelu_tanh_f32(float v) {
  const float t = 0.7978845608028654f * (v + 0.044715f * v * v * v);
  return v / (1.0f + expf(-2.0f * t));
}

// Gated activation of one output: act(gate) * up, the float32 product of
// the model loops: SiLU (qwen3.go:530-539; nomic.go:232-242 with gate = fc12,
// up = fc11), GELUTanh (gemma3.go:365-374) or the erf-GELU of tensor.GELU on
// a row whose length is a multiple of 8, i.e. geluAVX2 (modernbert.go:292-301,
// gate = Wi[:I], up = Wi[I:]).
__device__ __forceinline__ float glu_act(float g, float u, int act) {
  const float a = act == ACT_SWIGLU ? silu_f32(g)
                  : act == ACT_GEGLU ? gelu_tanh_f32(g)
                                     : gelu_avx2(g);
  return a * u;
}

// GEMM epilogue activation. Output rows always have n % 16 == 0 columns
// (the packers require it), so every element lies in a whole 8-lane group and
// takes the geluAVX2 sequence, as the reference's GELU(row) does.
__device__ __forceinline__ float apply_act(float v, int act) {
  return act == ACT_GELU ? gelu_avx2(v) : v;
}

}  // namespace rh
