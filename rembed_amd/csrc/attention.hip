// attention.hip — multi-head softmax attention over a packed variable-length
// batch, for gfx950 bf16 MFMA (v_mfma_f32_32x32x16_bf16).
//
// Reference semantics (internal/model/bert.go:853-902, per text, unpadded):
// scores = Qh·Khᵀ · (1/√dh), row softmax, ctx = P·Vh. Texts are packed
// back to back (rows cu[b]..cu[b+1]) so no pad token is ever attended and
// the result per text equals an unpadded forward.
//
// Layout trick: each wave computes Sᵀ = K·Qᵀ for 32 queries, so in the
// 32x32 accumulator lane l owns query l%32 and 16 of the 32 keys of the tile;
// the other 16 sit in lane l^32. Online softmax then needs one cross-lane
// exchange per row statistic, and Pᵀ already sits in the MFMA B-operand
// registers for Oᵀ = Vᵀ·Pᵀ, with V's keys read in the matching order.
// precision 1: bf16 operands; precision 3: hi/lo bf16 split with three
// products per MFMA step (fp32-grade scores and context).
#include "gemm_common.h"

namespace rh {

constexpr int kAttnQ = 128;   // queries per workgroup (4 waves x 32)
constexpr int kAttnKV = 64;   // keys per LDS block

// 8 consecutive activations as floats, from fp32 (two 16-byte loads) or bf16
// (one 16-byte load; widening is exact).
__device__ __forceinline__ void load8(const float* src, float (&x)[8]) {
  const v4f a = reinterpret_cast<const v4f*>(src)[0], b = reinterpret_cast<const v4f*>(src)[1];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    x[e] = a[e];
    x[4 + e] = b[e];
  }
}
__device__ __forceinline__ void load8(const __bf16* src, float (&x)[8]) {
  const v8bf a = *reinterpret_cast<const v8bf*>(src);
#pragma unroll
  for (int e = 0; e < 8; e++) x[e] = (float)a[e];
}

template <int DH, int PREC, typename TIn>
__global__ __launch_bounds__(256) void attention_kernel(AttnArgs p) {
  const TIn* qkv = static_cast<const TIn*>(p.qkv);
  constexpr int T = PREC == 3 ? 2 : 1;        // bf16 planes per operand
  constexpr int KS = DH / 16;                 // k-steps over dh
  constexpr int DT = DH / 32;                 // 32-wide d tiles of O^T
  constexpr int kK = kAttnKV * DH * 2;        // bytes of one K plane
  constexpr int kV = DH * kAttnKV * 2;        // bytes of one V^T plane
  // XOR swizzle of 16-byte chunks inside a K row, kept inside the row
  // (a row holds DH/8 chunks: 4 for dh 32, 8 or more otherwise).
  constexpr int kSwz = DH / 8 >= 8 ? 7 : DH / 8 - 1;
  __shared__ __attribute__((aligned(16))) uint8_t lds[T * (kK + kV)];
  uint8_t* sK = lds;
  uint8_t* sV = lds + T * kK;

  const int b = blockIdx.z, h = blockIdx.y;
  const int r0 = p.cu[b], len = p.cu[b + 1] - r0;
  const int q0 = blockIdx.x * kAttnQ;
  if (q0 >= len) return;
  const int kvh = h / (p.heads / p.kv_heads);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fg = lane >> 5;
  const int qi = q0 + wave * 32 + fr;  // this lane's query (text-local)

  // Q fragments (B operand of S^T): lane (query fr, half fg) holds
  // Q[q][s*16 + fg*8 + e].
  v8bf qh[KS], ql[KS];
  {
    // rows past the text read its last row; their outputs are not stored
    const TIn* qrow = qkv + (size_t)(r0 + (qi < len ? qi : len - 1)) * p.ldqkv + p.q_off + h * DH;
#pragma unroll
    for (int s = 0; s < KS; s++) {
      float xq[8];
      load8(qrow + s * 16 + fg * 8, xq);
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const __bf16 hi = (__bf16)xq[e];
        qh[s][e] = hi;
        if constexpr (PREC == 3) ql[s][e] = (__bf16)(xq[e] - (float)hi);
      }
    }
  }

  v16f o[DT];
#pragma unroll
  for (int t = 0; t < DT; t++)
#pragma unroll
    for (int e = 0; e < 16; e++) o[t][e] = 0.0f;
  float mrun = -INFINITY, lrun = 0.0f;
  const float l2e = 1.44269504088896341f;

  // Key blocks this workgroup's queries can see: causal stops after the
  // last query; a window bounds both ends (|i - j| < window).
  int kb_lo = 0, kb_hi = (len + kAttnKV - 1) / kAttnKV;
  const int qlast = min(q0 + kAttnQ, len) - 1;
  if (p.causal) kb_hi = min(kb_hi, qlast / kAttnKV + 1);
  if (p.window > 0) {
    kb_lo = max(0, q0 - p.window + 1) / kAttnKV;
    kb_hi = min(kb_hi, (qlast + p.window - 1) / kAttnKV + 1);
  }
  for (int kb = kb_lo; kb < kb_hi; kb++) {
    const int key0 = kb * kAttnKV;
    __syncthreads();  // previous block's LDS reads are done
    // Stage K (row-major [key][d], swizzled 16B chunks) and V^T ([d][key]).
    constexpr int kChunksPerRow = DH / 8;
    for (int it = tid; it < kAttnKV * kChunksPerRow; it += 256) {
      const int key = it / kChunksPerRow, ch = it % kChunksPerRow;
      const int kg = key0 + key;
      // Unconditional loads from a clamped in-text row; keys past the text
      // are zeroed after the loads (and masked out of the softmax below).
      const bool kok = kg < len;
      const size_t rowk = (size_t)(r0 + (kok ? kg : len - 1)) * p.ldqkv;
      float kx[8], vx[8];
      load8(qkv + rowk + p.k_off + kvh * DH + ch * 8, kx);
      load8(qkv + rowk + p.v_off + kvh * DH + ch * 8, vx);
#pragma unroll
      for (int e = 0; e < 8; e++) {
        kx[e] = kok ? kx[e] : 0.0f;
        vx[e] = kok ? vx[e] : 0.0f;
      }
      v8bf khi, klo;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const __bf16 hi = (__bf16)kx[e];
        khi[e] = hi;
        if constexpr (PREC == 3) klo[e] = (__bf16)(kx[e] - (float)hi);
      }
      const int koff = key * (DH * 2) + ((ch ^ (key & kSwz)) << 4);
      *reinterpret_cast<v8bf*>(sK + koff) = khi;
      if constexpr (PREC == 3) *reinterpret_cast<v8bf*>(sK + kK + koff) = klo;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int d = ch * 8 + e;
        const int voff = d * (kAttnKV * 2) + (((key >> 3) ^ (d & 7)) << 4) + ((key & 7) << 1);
        const __bf16 hi = (__bf16)vx[e];
        *reinterpret_cast<__bf16*>(sV + voff) = hi;
        if constexpr (PREC == 3)
          *reinterpret_cast<__bf16*>(sV + kV + voff) = (__bf16)(vx[e] - (float)hi);
      }
    }
    __syncthreads();

    // S^T for the two 32-key tiles of this block.
    v16f sc[2];
#pragma unroll
    for (int t2 = 0; t2 < 2; t2++) {
#pragma unroll
      for (int e = 0; e < 16; e++) sc[t2][e] = 0.0f;
      const int key = t2 * 32 + fr;
#pragma unroll
      for (int s = 0; s < KS; s++) {
        const int ch = 2 * s + fg;
        const int koff = key * (DH * 2) + ((ch ^ (key & kSwz)) << 4);
        const v8bf kh = *reinterpret_cast<const v8bf*>(sK + koff);
        sc[t2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, qh[s], sc[t2], 0, 0, 0);
        if constexpr (PREC == 3) {
          const v8bf kl = *reinterpret_cast<const v8bf*>(sK + kK + koff);
          sc[t2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, ql[s], sc[t2], 0, 0, 0);
          sc[t2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kl, qh[s], sc[t2], 0, 0, 0);
        }
      }
    }
    // Scale, mask keys past the text, running max shared by lanes l, l^32.
    float mloc = -INFINITY;
#pragma unroll
    for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int key = key0 + t2 * 32 + i * 8 + fg * 4 + j;
          float v = sc[t2][i * 4 + j] * p.scale;
          if (key >= len || (p.causal && key > qi) ||
              (p.window > 0 && (key <= qi - p.window || key >= qi + p.window)))
            v = -INFINITY;
          sc[t2][i * 4 + j] = v;
          mloc = fmaxf(mloc, v);
        }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    // A masked query can see no key of this block yet (mnew = -inf): use a
    // finite reference so alpha = exp(-inf) = 0 and every p = 0, not NaN.
    const float mnew = fmaxf(mrun, mloc);
    const float mref = mnew == -INFINITY ? 0.0f : mnew;
    const float alpha = exp2f((mrun - mref) * l2e);
    mrun = mnew;
    float psum = 0.0f;
#pragma unroll
    for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const float pv = exp2f((sc[t2][e] - mref) * l2e);
        sc[t2][e] = pv;
        psum += pv;
      }
    lrun = lrun * alpha + psum;
#pragma unroll
    for (int t = 0; t < DT; t++)
#pragma unroll
      for (int e = 0; e < 16; e++) o[t][e] *= alpha;

    // O^T += V^T · P^T over 4 chunks of 16 keys. Chunk kc, lane half g,
    // element e <-> key kc*16 + (e/4)*8 + g*4 + e%4 = register
    // sc[kc/2][(kc%2)*8 + e].
#pragma unroll
    for (int kc = 0; kc < 4; kc++) {
      v8bf ph, pl;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float x = sc[kc >> 1][(kc & 1) * 8 + e];
        const __bf16 hi = (__bf16)x;
        ph[e] = hi;
        if constexpr (PREC == 3) pl[e] = (__bf16)(x - (float)hi);
      }
#pragma unroll
      for (int t = 0; t < DT; t++) {
        const int d = t * 32 + fr;
        const int base = d * (kAttnKV * 2);
        const int c0 = 2 * kc, c1 = 2 * kc + 1;
        const int off0 = base + ((c0 ^ (d & 7)) << 4) + fg * 8;
        const int off1 = base + ((c1 ^ (d & 7)) << 4) + fg * 8;
        v8bf vh;
        {
          typedef short v4s __attribute__((ext_vector_type(4)));
          const v4s a = *reinterpret_cast<const v4s*>(sV + off0);
          const v4s c = *reinterpret_cast<const v4s*>(sV + off1);
          v8s w = {a[0], a[1], a[2], a[3], c[0], c[1], c[2], c[3]};
          vh = __builtin_bit_cast(v8bf, w);
        }
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vh, ph, o[t], 0, 0, 0);
        if constexpr (PREC == 3) {
          typedef short v4s __attribute__((ext_vector_type(4)));
          const v4s a = *reinterpret_cast<const v4s*>(sV + kV + off0);
          const v4s c = *reinterpret_cast<const v4s*>(sV + kV + off1);
          v8s w = {a[0], a[1], a[2], a[3], c[0], c[1], c[2], c[3]};
          const v8bf vl = __builtin_bit_cast(v8bf, w);
          o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vh, pl, o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vl, ph, o[t], 0, 0, 0);
        }
      }
    }
  }

  const float ltot = lrun + __shfl_xor(lrun, 32, 64);
  if (qi >= len) return;
  const float inv = 1.0f / ltot;
  float* orow = p.ctx + (size_t)(r0 + qi) * p.ldctx + h * DH;
#pragma unroll
  for (int t = 0; t < DT; t++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v4f w;
#pragma unroll
      for (int j = 0; j < 4; j++) w[j] = o[t][i * 4 + j] * inv;
      *reinterpret_cast<v4f*>(orow + t * 32 + i * 8 + fg * 4) = w;
    }
}

template <int DH>
static hipError_t launch_attn_dh(const AttnArgs& a, int precision, hipStream_t s) {
  dim3 grid(ceil_div(a.max_len, kAttnQ), a.heads, a.batch);
  if (a.in_bf16)  // bf16 input carries no low half: one-term products
    timed_launch((attention_kernel<DH, 1, __bf16>), grid, dim3(256), 0, s, a);
  else if (precision == 3)
    timed_launch((attention_kernel<DH, 3, float>), grid, dim3(256), 0, s, a);
  else
    timed_launch((attention_kernel<DH, 1, float>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& a, int precision, hipStream_t s) {
  if (a.batch <= 0 || a.max_len <= 0) return hipSuccess;
  switch (a.dh) {
    case 32: return launch_attn_dh<32>(a, precision, s);
    case 64: return launch_attn_dh<64>(a, precision, s);
    case 128: return launch_attn_dh<128>(a, precision, s);
    case 256: return launch_attn_dh<256>(a, precision, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rh
