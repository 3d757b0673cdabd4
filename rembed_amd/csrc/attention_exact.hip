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
//   scores:  thread (query i, key group g of 8) computes the whole dot4 of
//            its query against keys g, g+8, ..., two keys per step (q in
//            registers, K staged in LDS 64 keys at a time; one query per
//            thread keeps the registers at three waves per SIMD, measured
//            294 against 351 µs with two queries per thread at the BERT-base
//            batch);
//   softmax: the same threads exponentiate; one lane per query then sums
//            its row in column order;
//   P·V:     thread (queries i and i+16, half of dh, dot4 lane l) runs dot4
//            lane l's FMA chains for its dh/2 outputs of both queries (keys
//            l, l+8, ..., V staged 64 keys at a time), and the 8 lanes of a
//            group fold as dot4 does.
// The arithmetic is bound by VALU FMAs and LDS reads (one float read per
// one FMA in the scores, per two in P·V).
#include "gemm_common.h"

namespace rh {

constexpr int kXQ = 32;  // queries per workgroup
constexpr int kXK = 64;  // keys per LDS chunk

// Score row pitch in floats: a multiple of 64 plus 2, so a wave's score
// writes and the exponentials' pass (32 queries x 2 key groups, one float
// each) hit 64 distinct banks (plus 8 put four queries on each bank: 1.73
// against 1.79 M tokens/s for the exact BERT-base forward). The rows are
// then only 8-byte aligned, so the row sums read single floats.
__host__ __device__ inline int exact_pitch(int max_len) { return ((max_len + 63) / 64) * 64 + 2; }
// Staged key/value row pitch: dh + 4 floats, so rows 16 bytes apart in bank
// terms (the rows one instruction reads are conflict-free).
__host__ __device__ constexpr int exact_cpitch(int dh) { return dh + 4; }

__host__ inline size_t exact_lds_bytes(int max_len, int dh) {
  return sizeof(float) * ((size_t)kXQ * exact_pitch(max_len) + (size_t)kXK * exact_cpitch(dh) +
                          9 * kXQ);
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

// dot4 (DH % 8 == 0: no tail) of one query row a with two key rows b, b2
// read from LDS as float4 groups: lane accumulators, fold, horizontal adds;
// the two dot products' chains interleave.
template <int DH>
__device__ __forceinline__ void dot4_ref1x2(const float (&a)[DH], const float* __restrict__ b,
                                            const float* __restrict__ b2, float& s, float& s2) {
  float acc[8], acc2[8];
#pragma unroll
  for (int l = 0; l < 8; l++) acc[l] = acc2[l] = 0.0f;
#pragma unroll
  for (int blk = 0; blk < DH / 8; blk++) {
    const v4f b0 = *reinterpret_cast<const v4f*>(b + blk * 8);
    const v4f b1 = *reinterpret_cast<const v4f*>(b + blk * 8 + 4);
    const v4f c0 = *reinterpret_cast<const v4f*>(b2 + blk * 8);
    const v4f c1 = *reinterpret_cast<const v4f*>(b2 + blk * 8 + 4);
#pragma unroll
    for (int l = 0; l < 4; l++) {
      acc[l] = __builtin_fmaf(a[blk * 8 + l], b0[l], acc[l]);
      acc[4 + l] = __builtin_fmaf(a[blk * 8 + 4 + l], b1[l], acc[4 + l]);
      acc2[l] = __builtin_fmaf(a[blk * 8 + l], c0[l], acc2[l]);
      acc2[4 + l] = __builtin_fmaf(a[blk * 8 + 4 + l], c1[l], acc2[4 + l]);
    }
  }
  s = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
  s2 = ((acc2[0] + acc2[4]) + (acc2[1] + acc2[5])) + ((acc2[2] + acc2[6]) + (acc2[3] + acc2[7]));
}

// dot4 of one query row with one key row.
template <int DH>
__device__ __forceinline__ float dot4_ref1(const float (&a)[DH], const float* __restrict__ b) {
  float acc[8];
#pragma unroll
  for (int l = 0; l < 8; l++) acc[l] = 0.0f;
#pragma unroll
  for (int blk = 0; blk < DH / 8; blk++) {
    const v4f b0 = *reinterpret_cast<const v4f*>(b + blk * 8);
    const v4f b1 = *reinterpret_cast<const v4f*>(b + blk * 8 + 4);
#pragma unroll
    for (int l = 0; l < 4; l++) {
      acc[l] = __builtin_fmaf(a[blk * 8 + l], b0[l], acc[l]);
      acc[4 + l] = __builtin_fmaf(a[blk * 8 + 4 + l], b1[l], acc[4 + l]);
    }
  }
  return ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
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

// Three workgroups per CU at head dim <= 64 and texts up to 256 tokens
// (53 KB of LDS each): registers capped for three waves per SIMD.
template <int DH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DH <= 64 ? 3 : 1)))
void attention_exact_kernel(AttnArgs p) {
  constexpr int CP = exact_cpitch(DH);
  constexpr int H2 = kXQ / 2;  // P·V: each thread carries queries i and i + H2
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int lp = exact_pitch(p.max_len);
  float* P = lds;                       // [kXQ][lp] scores, then exponentials
  float* chunk = lds + kXQ * lp;        // [kXK][CP] keys, then values
  float* red = chunk + kXK * CP;        // [8][kXQ] partial row maxima
  float* rinv = red + 8 * kXQ;          // [kXQ] 1/sum per query

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

  {
    // ---- scores: thread (query i, key group g of 8), two keys per step -------
    constexpr int NG = 256 / kXQ;  // key groups: the rows of red
    const int i = t % kXQ, g = t / kXQ;
    float qa[DH];
    load_row<DH>(base + p.q_off + h * DH + (size_t)(q0 + min(i, nq - 1)) * p.ldqkv, qa);
    const int l4 = len & ~3;  // dot4 columns; the rest are serial sums
    const float* rb = p.rel_bias
                          ? p.rel_bias + (size_t)h * (2 * p.rel_center + 1) + p.rel_center -
                                (q0 + min(i, nq - 1))
                          : nullptr;
    float mx = -INFINITY;
    for (int c0 = 0; c0 < len; c0 += kXK) {
      __syncthreads();  // the previous chunk's reads are done
      stage.commit(chunk);
      if (c0 + kXK < len) stage.fetch(kbase, p.ldqkv, c0 + kXK, len);
      else stage.fetch(vbase, p.ldqkv, 0, len);
      __syncthreads();
      for (int kk = g; kk < kXK; kk += 2 * NG) {
        const int j = c0 + kk, j2 = j + NG;
        if (j >= len) break;
        const float* kr = chunk + kk * CP;
        const float* kr2 = chunk + (kk + NG) * CP;
        float sa, sb = 0.0f;
        if (j2 < l4) {
          dot4_ref1x2<DH>(qa, kr, kr2, sa, sb);
        } else {
          sa = j < l4 ? dot4_ref1<DH>(qa, kr) : dot_serial_ref<DH>(qa, kr);
          if (j2 < len) sb = dot_serial_ref<DH>(qa, kr2);
        }
        sa = sa * p.scale;  // scores *= scale (bert.go:884-886)
        sb = sb * p.scale;
        if (rb) {  // MPNet: + the bias of bucket(j - i), after the scale
          sa = sa + rb[j];
          if (j2 < len) sb = sb + rb[j2];
        }
        P[i * lp + j] = sa;
        mx = fmaxf(mx, sa);
        if (j2 < len) {
          P[i * lp + j2] = sb;
          mx = fmaxf(mx, sb);
        }
      }
    }
    red[g * kXQ + i] = mx;
    __syncthreads();
    float m = red[i];
#pragma unroll
    for (int gg = 1; gg < NG; gg++) m = fmaxf(m, red[gg * kXQ + i]);
    for (int j = g; j < len; j += NG) P[i * lp + j] = exp_nonpos_ref(P[i * lp + j] - m);
  }
  __syncthreads();
  if (t < kXQ) {  // the row sum in column order, then inv = 1/sum
    const float* pr = P + t * lp;
    float s = 0.0f;
    int j = 0;
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
