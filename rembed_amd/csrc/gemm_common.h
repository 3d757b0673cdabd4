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

// LDS tiles hold rows of 128 bytes = 8 chunks of 16 bytes; chunk c of row r
// lives at slot c ^ (r & 7) so that the 32 rows one MFMA fragment read
// touches spread over all slots (bank-conflict avoidance).
__device__ __forceinline__ int lds_off(int r, int c) {
  return (r << 7) + ((c ^ (r & 7)) << 4);
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

__device__ __forceinline__ float apply_act(float v, int act) {
  return act == ACT_GELU ? gelu_ref(v) : v;
}

}  // namespace rh
