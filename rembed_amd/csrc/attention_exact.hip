// attention_exact.hip — bidirectional softmax attention in the reference's
// own float32 operation order, for the byte-exact encoder forward.
//
// Reference (internal/model/bert.go:853-902, one text, one head):
//   scores = MatMulSerial(Qh, Kh)        (matMulSIMDCols, tensor.go:295-330)
//   scores *= scale                      (bert.go:884-886)
//   Softmax(scores)                      (tensor.go:389-428)
//   ctx    = MatMulSerial(P, Vhᵀ)
// MatMulSerial takes output columns four at a time through dot4
// (dot_amd64.s:13-94): eight lane accumulators, lane l an FMA chain over
// k = l, l+8, ...; lanes l and l+4 added; the k % 8 tail FMA'd into lane 0
// in order; then (x0+x1) + (x2+x3). The n % 4 remainder columns are plain
// in-order sums of rounded products. Softmax takes the row max, then
// expNonPos (fastmath.go:93-109, written out in the loop) per element, a
// float32 sum in column order, inv = 1/sum and P *= inv.
//
// Every float operation here is that sequence on the same values, so the
// context rows are bit-identical to the reference's. The arithmetic is
// float32 VALU work (an FMA chain's intermediate roundings cannot be
// reproduced by a matrix instruction's internal sums): ~2·L²·dh FMAs per
// text and head.
//
// Workgroup: one (text, head, block of 32 queries), 256 threads.
//   scores:  thread (queries i and i+16, key group g of 16) computes the
//            whole dot4 of both queries against keys g, g+16, ... in-lane
//            (q in registers, K staged in LDS 64 keys at a time; each key
//            value read serves two queries);
//   softmax: the same threads exponentiate; one lane per query then sums
//            its row in column order;
//   P·V:     thread (queries i and i+16, half of dh, dot4 lane l) runs dot4
//            lane l's FMA chains for its dh/2 outputs of both queries (keys
//            l, l+8, ..., V staged 64 keys at a time), and the 8 lanes of a
//            group fold as dot4 does.
// The arithmetic is bound by VALU FMAs and LDS reads (one float read per
// two FMAs).
#include "gemm_common.h"

namespace rh {

constexpr int kXQ = 32;  // queries per workgroup
constexpr int kXK = 64;  // keys per LDS chunk

// Score row pitch in floats: a multiple of 64 plus 8, so the queries of one
// wave's P reads fall in distinct banks.
__host__ __device__ inline int exact_pitch(int max_len) { return ((max_len + 63) / 64) * 64 + 8; }
// Staged key/value row pitch: dh + 4 floats, so rows 16 bytes apart in bank
// terms (the rows one instruction reads are conflict-free).
__host__ __device__ constexpr int exact_cpitch(int dh) { return dh + 4; }

__host__ inline size_t exact_lds_bytes(int max_len, int dh) {
  return sizeof(float) * ((size_t)kXQ * exact_pitch(max_len) + (size_t)kXK * exact_cpitch(dh) +
                          17 * kXQ);
}

// expNonPos (fastmath.go:93-109) as Softmax writes it (tensor.go:407-420):
// clamp at -87.33, n = trunc(x·log2e - 0.5), Cody-Waite reduction by C1 and
// C2, the degree-5 Cephes polynomial, scale by 2^n. No contraction: each
// product and sum rounds, as Go's amd64 float32 code does.
__device__ __forceinline__ float exp_nonpos_ref(float xe) {
  if (xe < -87.33f) xe = -87.33f;
  const float nf = (float)(int)(xe * 1.44269504088896341f - 0.5f);
  xe = xe - nf * 0.693359375f;
  xe = xe - nf * -2.12194440e-4f;
  const float z = xe * xe;
  float y = 1.9875691500e-4f;
  y = y * xe + 1.3981999507e-3f;
  y = y * xe + 8.3334519073e-3f;
  y = y * xe + 4.1665795894e-2f;
  y = y * xe + 1.6666665459e-1f;
  y = y * xe + 5.0000001201e-1f;
  const float p2 = __int_as_float(((int)nf + 127) << 23);
  return (y * z + xe + 1.0f) * p2;
}

// dot4 (DH % 8 == 0: no tail) of two query rows a, a2 with one key row b
// read from LDS as float4 groups: lane accumulators, fold, horizontal adds.
// Each key value read serves both queries.
template <int DH>
__device__ __forceinline__ void dot4_ref2(const float (&a)[DH], const float (&a2)[DH],
                                          const float* __restrict__ b, float& s, float& s2) {
  float acc[8], acc2[8];
#pragma unroll
  for (int l = 0; l < 8; l++) acc[l] = acc2[l] = 0.0f;
#pragma unroll
  for (int blk = 0; blk < DH / 8; blk++) {
    const v4f b0 = *reinterpret_cast<const v4f*>(b + blk * 8);
    const v4f b1 = *reinterpret_cast<const v4f*>(b + blk * 8 + 4);
#pragma unroll
    for (int l = 0; l < 4; l++) {
      acc[l] = __builtin_fmaf(a[blk * 8 + l], b0[l], acc[l]);
      acc[4 + l] = __builtin_fmaf(a[blk * 8 + 4 + l], b1[l], acc[4 + l]);
      acc2[l] = __builtin_fmaf(a2[blk * 8 + l], b0[l], acc2[l]);
      acc2[4 + l] = __builtin_fmaf(a2[blk * 8 + 4 + l], b1[l], acc2[4 + l]);
    }
  }
  s = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
  s2 = ((acc2[0] + acc2[4]) + (acc2[1] + acc2[5])) + ((acc2[2] + acc2[6]) + (acc2[3] + acc2[7]));
}

// matMulSIMDCols' remainder columns (tensor.go:318-328): s += a·b in order.
template <int DH>
__device__ __forceinline__ float dot_serial_ref(const float (&a)[DH], const float* __restrict__ b) {
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < DH / 4; c++) {
    const v4f bv = *reinterpret_cast<const v4f*>(b + c * 4);
#pragma unroll
    for (int e = 0; e < 4; e++) s = s + a[c * 4 + e] * bv[e];
  }
  return s;
}

// Rows c0 .. c0+63 of the (text-local) key or value head, staged through
// registers: fetch() issues this thread's 16-byte loads (zeros past the
// text's last row) so they fly while the previous chunk is consumed,
// commit() writes them to chunk[64][exact_cpitch(DH)].
template <int DH>
struct ExactChunk {
  static constexpr int kPer = kXK * DH / 4 / 256;  // float4 per thread
  v4f x[kPer];
  __device__ __forceinline__ void fetch(const float* __restrict__ src, int ld, int c0, int len) {
#pragma unroll
    for (int u = 0; u < kPer; u++) {
      const int v = threadIdx.x + u * 256;
      const int r = v / (DH / 4), c = v % (DH / 4);
      x[u] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      if (c0 + r < len) x[u] = *reinterpret_cast<const v4f*>(src + (size_t)(c0 + r) * ld + c * 4);
    }
  }
  __device__ __forceinline__ void commit(float* __restrict__ chunk) const {
#pragma unroll
    for (int u = 0; u < kPer; u++) {
      const int v = threadIdx.x + u * 256;
      const int r = v / (DH / 4), c = v % (DH / 4);
      *reinterpret_cast<v4f*>(chunk + r * exact_cpitch(DH) + c * 4) = x[u];
    }
  }
};

template <int DH>
__device__ __forceinline__ void load_row(const float* __restrict__ src, float (&q)[DH]) {
#pragma unroll
  for (int c = 0; c < DH / 4; c++) {
    const v4f v = *reinterpret_cast<const v4f*>(src + c * 4);
#pragma unroll
    for (int e = 0; e < 4; e++) q[c * 4 + e] = v[e];
  }
}

template <int DH>
__global__ __launch_bounds__(256) void attention_exact_kernel(AttnArgs p) {
  constexpr int CP = exact_cpitch(DH);
  constexpr int H2 = kXQ / 2;  // each thread carries queries i and i + H2
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int lp = exact_pitch(p.max_len);
  float* P = lds;                       // [kXQ][lp] scores, then exponentials
  float* chunk = lds + kXQ * lp;        // [kXK][CP] keys, then values
  float* red = chunk + kXK * CP;        // [16][kXQ] partial row maxima
  float* rinv = red + 16 * kXQ;         // [kXQ] 1/sum per query

  const int nqb = (p.max_len + kXQ - 1) / kXQ;
  const int qb = blockIdx.x % nqb;
  const int bh = blockIdx.x / nqb;
  const int h = bh % p.heads, b = bh / p.heads;
  if (b >= p.batch) return;
  const int r0 = p.cu[b], len = p.cu[b + 1] - r0;
  const int q0 = qb * kXQ;
  if (q0 >= len) return;  // uniform over the workgroup
  const int nq = min(kXQ, len - q0);
  const int t = threadIdx.x;
  const float* base = static_cast<const float*>(p.qkv) + (size_t)r0 * p.ldqkv;
  const float* kbase = base + p.k_off + h * DH;
  const float* vbase = base + p.v_off + h * DH;

  ExactChunk<DH> stage;
  stage.fetch(kbase, p.ldqkv, 0, len);

  // ---- scores: thread (queries i and i + 16, key group g of 16) -------------
  {
    const int i = t % H2, g = t / H2;
    float qa[DH], qb2[DH];
    const float* qcol = base + p.q_off + h * DH;
    load_row<DH>(qcol + (size_t)(q0 + min(i, nq - 1)) * p.ldqkv, qa);
    load_row<DH>(qcol + (size_t)(q0 + min(i + H2, nq - 1)) * p.ldqkv, qb2);
    const int l4 = len & ~3;  // dot4 columns; the rest are serial sums
    float mxa = -INFINITY, mxb = -INFINITY;
    for (int c0 = 0; c0 < len; c0 += kXK) {
      __syncthreads();  // the previous chunk's reads are done
      stage.commit(chunk);
      // the next chunk's loads fly while this one is consumed: the next key
      // chunk, or after the last one the first value chunk
      if (c0 + kXK < len) stage.fetch(kbase, p.ldqkv, c0 + kXK, len);
      else stage.fetch(vbase, p.ldqkv, 0, len);
      __syncthreads();
      for (int kk = g; kk < kXK; kk += 16) {
        const int j = c0 + kk;
        if (j >= len) break;
        const float* kr = chunk + kk * CP;
        float sa, sb;
        if (j < l4) {
          dot4_ref2<DH>(qa, qb2, kr, sa, sb);
        } else {
          sa = dot_serial_ref<DH>(qa, kr);
          sb = dot_serial_ref<DH>(qb2, kr);
        }
        sa = sa * p.scale;  // scores *= scale (bert.go:884-886)
        sb = sb * p.scale;
        if (p.rel_bias) {  // MPNet: + the bias of bucket(j - i), after the scale
          const float* rb = p.rel_bias + (size_t)h * (2 * p.rel_center + 1) + p.rel_center + j;
          sa = sa + rb[-(q0 + min(i, nq - 1))];
          sb = sb + rb[-(q0 + min(i + H2, nq - 1))];
        }
        P[i * lp + j] = sa;
        P[(i + H2) * lp + j] = sb;
        mxa = fmaxf(mxa, sa);
        mxb = fmaxf(mxb, sb);
      }
    }
    red[g * kXQ + i] = mxa;
    red[g * kXQ + i + H2] = mxb;
    __syncthreads();
    float ma = red[i], mb = red[i + H2];
#pragma unroll
    for (int gg = 1; gg < 16; gg++) {
      ma = fmaxf(ma, red[gg * kXQ + i]);
      mb = fmaxf(mb, red[gg * kXQ + i + H2]);
    }
    // Softmax's exponentials (tensor.go:407-420), x - max <= 0
    for (int j = g; j < len; j += 16) {
      P[i * lp + j] = exp_nonpos_ref(P[i * lp + j] - ma);
      P[(i + H2) * lp + j] = exp_nonpos_ref(P[(i + H2) * lp + j] - mb);
    }
  }
  __syncthreads();
  if (t < kXQ) {  // the row sum in column order, then inv = 1/sum
    const float* pr = P + t * lp;
    float s = 0.0f;
    int j = 0;
    for (; j + 4 <= len; j += 4) {
      const v4f e = *reinterpret_cast<const v4f*>(pr + j);
      s = s + e[0];
      s = s + e[1];
      s = s + e[2];
      s = s + e[3];
    }
    for (; j < len; j++) s = s + pr[j];
    rinv[t] = 1.0f / s;
  }

  // ---- P·V: thread (queries i and i + 16, half of dh, dot4 lane l) ------------
  constexpr int D2 = DH / 2;
  const int l = t & 7, hf = (t >> 3) & 1, i = t >> 4;
  float acc[D2], acc2[D2];
#pragma unroll
  for (int d = 0; d < D2; d++) acc[d] = acc2[d] = 0.0f;
  const int nb8 = len & ~7;  // keys in whole blocks of 8; the rest are dot4's tail
  const float* pa = P + i * lp;
  const float* pb = P + (i + H2) * lp;
  for (int c0 = 0; c0 < len; c0 += kXK) {
    __syncthreads();  // previous chunk's reads (and, first time, the row sums) done
    stage.commit(chunk);
    if (c0 + kXK < len) stage.fetch(vbase, p.ldqkv, c0 + kXK, len);
    __syncthreads();
    const float ia = rinv[i], ib = rinv[i + H2];
    const int kend = min(kXK, nb8 - c0);
    for (int kk = l; kk < kend; kk += 8) {
      const float pva = pa[c0 + kk] * ia;  // P *= inv (tensor.go:424-427)
      const float pvb = pb[c0 + kk] * ib;
      const float* vr = chunk + kk * CP + hf * D2;
#pragma unroll
      for (int c = 0; c < D2 / 4; c++) {
        const v4f v = *reinterpret_cast<const v4f*>(vr + c * 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          acc[c * 4 + e] = __builtin_fmaf(pva, v[e], acc[c * 4 + e]);
          acc2[c * 4 + e] = __builtin_fmaf(pvb, v[e], acc2[c * 4 + e]);
        }
      }
    }
    if (c0 + kXK >= len) {
      // fold lanes l and l+4, the tail into lane 0 in key order, then
      // (x0 + x1) + (x2 + x3); lanes 0-3 of each group end with the result
#pragma unroll
      for (int d = 0; d < D2; d++) {
        acc[d] = acc[d] + __shfl_xor(acc[d], 4, 64);
        acc2[d] = acc2[d] + __shfl_xor(acc2[d], 4, 64);
      }
      if (l == 0) {
        for (int j = nb8; j < len; j++) {
          const float pva = pa[j] * ia, pvb = pb[j] * ib;
          const float* vr = chunk + (j - c0) * CP + hf * D2;
#pragma unroll
          for (int d = 0; d < D2; d++) {
            acc[d] = __builtin_fmaf(pva, vr[d], acc[d]);
            acc2[d] = __builtin_fmaf(pvb, vr[d], acc2[d]);
          }
        }
      }
#pragma unroll
      for (int d = 0; d < D2; d++) {
        acc[d] = acc[d] + __shfl_xor(acc[d], 1, 64);
        acc2[d] = acc2[d] + __shfl_xor(acc2[d], 1, 64);
      }
#pragma unroll
      for (int d = 0; d < D2; d++) {
        acc[d] = acc[d] + __shfl_xor(acc[d], 2, 64);
        acc2[d] = acc2[d] + __shfl_xor(acc2[d], 2, 64);
      }
    }
  }
  // lanes 0-3 of a group each store a quarter of its outputs (indices kept
  // constant per branch: a lane-dependent index would put acc in scratch)
  constexpr int kPer = D2 / 4;  // outputs per lane and query
#pragma unroll
  for (int ll = 0; ll < 4; ll++) {
    if (l != ll) continue;
#pragma unroll
    for (int qq = 0; qq < 2; qq++) {
      const int iq = i + qq * H2;
      if (iq >= nq) continue;
      const size_t row = (size_t)r0 + q0 + iq;
#pragma unroll
      for (int c = 0; c < kPer / 4; c++) {
        v4f o;
#pragma unroll
        for (int e = 0; e < 4; e++)
          o[e] = qq ? acc2[ll * kPer + c * 4 + e] : acc[ll * kPer + c * 4 + e];
        const size_t off = row * p.ldctx + h * DH + hf * D2 + ll * kPer + c * 4;
        if (p.ctx) *reinterpret_cast<v4f*>(p.ctx + off) = o;
        else store_planes4(p.ctx_hi, p.ctx_lo, off, o);
      }
    }
  }
}

template <int DH>
static hipError_t launch_exact_dh(const AttnArgs& a, hipStream_t s) {
  const size_t shmem = exact_lds_bytes(a.max_len, DH);
  if (shmem > 160 * 1024) return hipErrorInvalidValue;
  static bool attr_set = false;  // past 64 KiB: raise the dynamic LDS limit once
  if (shmem > 64 * 1024 && !attr_set) {
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&attention_exact_kernel<DH>),
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const dim3 grid(a.batch * a.heads * ceil_div(a.max_len, kXQ));
  timed_launch((attention_exact_kernel<DH>), grid, dim3(256), (uint32_t)shmem, s, a);
  return hipGetLastError();
}

hipError_t launch_attention_exact(const AttnArgs& a, hipStream_t s) {
  if (a.batch <= 0 || a.max_len <= 0) return hipSuccess;
  // the reference order is the BERT family's attention: every head its own
  // key/value head, no mask past the text, fp32 q|k|v rows
  if (a.in_bf16 || a.causal || a.window > 0 || a.kv_heads != a.heads) return hipErrorInvalidValue;
  if ((!a.ctx && !a.ctx_hi) || a.ldqkv % 4 || a.ldctx % 4) return hipErrorInvalidValue;
  switch (a.dh) {
    case 32: return launch_exact_dh<32>(a, s);
    case 64: return launch_exact_dh<64>(a, s);
    case 128: return launch_exact_dh<128>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rh
