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

// Visible keys of query qi (text-local): [klo, khi]. Keys past the text,
// after the query (causal, qwen3.go:319-390) or at distance >= window
// (gemma3.go:339-347) are excluded.
__device__ __forceinline__ void attn_key_range(const AttnArgs& p, int qi, int len, int& klo,
                                               int& khi) {
  khi = len - 1;
  if (p.causal) khi = min(khi, qi);
  klo = 0;
  if (p.window > 0) {
    khi = min(khi, qi + p.window - 1);
    klo = qi - p.window + 1;
  }
}

// Online-softmax step for one 64-key block held as S^T tiles (lane: query
// fr, keys key0 + t2*32 + i*8 + fg*4 + j in register t2, i*4 + j). Scores
// go to log2 units through cs = scale·log2 e, folded into the exponent:
// the block max of s·cs is max(s)·cs exactly (rounding is monotonic and
// cs > 0), and p = 2^fma(s, cs, -m). `masked` (uniform over the wave)
// applies the per-key range test. P = 2^(s·cs - mref) against a reference
// that moves only when a block's max exceeds it by more than 8: P stays
// <= 256 (no overflow in fp32), and the running output is rescaled (by the
// returned alpha, when `rescale`) only on those moves. sc becomes P.
__device__ __forceinline__ float attn_softmax_block(v16f (&sc)[2], int key0, int fg, int klo,
                                                    int khi, bool masked, float cs,
                                                    float& mref, float& lrun, bool& rescale) {
  // One uniform branch around the whole mask (a per-element condition is
  // if-converted into selects that every block pays for). key is outside
  // [klo, khi] iff key - klo, as unsigned, exceeds khi - klo: exact when
  // klo <= khi, which holds for every query inside its text (the query sees
  // itself); queries past the text only feed outputs that are not stored.
  if (masked) {
    const unsigned span = (unsigned)(khi - klo);
    const int base = key0 + fg * 4 - klo;
#pragma unroll
    for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const unsigned off = (unsigned)(base + t2 * 32 + i * 8 + j);
          sc[t2][i * 4 + j] = off > span ? -INFINITY : sc[t2][i * 4 + j];
        }
  }
  float smax = -INFINITY;
#pragma unroll
  for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
    for (int e = 0; e < 16; e++) smax = fmaxf(smax, sc[t2][e]);
  smax = fmaxf(smax, __shfl_xor(smax, 32, 64));
  const float mloc = smax * cs;
  // -inf + 8 = -inf: a lane's first visible key always moves the reference
  // (alpha = 2^-inf = 0 then); a lane with no visible key keeps -inf.
  const bool up = mloc > mref + 8.0f;
  rescale = __any(up);
  float alpha = 1.0f;
  if (up) {
    alpha = __builtin_amdgcn_exp2f(mref - mloc);
    mref = mloc;
  }
  const float m = mref == -INFINITY ? 0.0f : mref;  // all-masked lanes: every p = 0
  float psum = 0.0f;
#pragma unroll
  for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[t2][e], cs, -m));
      sc[t2][e] = pv;
      psum += pv;
    }
  lrun = lrun * alpha + psum;
  return alpha;
}

// P's bf16 split for the fp32-grade products: hi = bf16(x), lo = bf16(x -
// hi), both rounded to nearest even, two scores per conversion; hi as a float
// is its half of the packed pair moved to the upper 16 bits (exact).
__device__ __forceinline__ void attn_split8(const v16f& s, int base, v8bf& ph, v8bf& pl) {
  typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
  typedef float v2f __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const float x0 = s[base + e], x1 = s[base + e + 1];
    const v2bf h = __builtin_convertvector((v2f){x0, x1}, v2bf);
    const uint32_t u = __builtin_bit_cast(uint32_t, h);
    const float h0 = __uint_as_float(u << 16), h1 = __uint_as_float(u & 0xffff0000u);
    const float l0 = x0 - h0, l1 = x1 - h1;
    const v2bf l = __builtin_convertvector((v2f){l0, l1}, v2bf);
    ph[e] = h[0];
    ph[e + 1] = h[1];
    pl[e] = l[0];
    pl[e + 1] = l[1];
  }
}

// MPNet (bert.go:876-890): scores become score·scale + bias(j - i), the
// bias of the head's relative-position bucket; the softmax then takes them
// with cs = log2 e. Lane layout as attn_softmax_block (query qi; keys key0 +
// t2*32 + i*8 + fg*4 + j). Relative positions outside the table belong to
// masked keys or unstored queries and are clamped into it.
__device__ __forceinline__ void attn_rel_bias(const AttnArgs& p, v16f (&sc)[2], int h, int qi,
                                              int key0, int fg) {
  const int c = p.rel_center;
  const float* rb = p.rel_bias + (size_t)h * (2 * c + 1) + c;
#pragma unroll
  for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int d = min(max(key0 + t2 * 32 + i * 8 + fg * 4 + j - qi, -c), c);
        sc[t2][i * 4 + j] = sc[t2][i * 4 + j] * p.scale + rb[d];
      }
}

// Workgroup -> (text b, head h, query block). Workgroups are dealt to the 8
// XCDs round-robin (workgroup w runs on XCD w % 8), and the query blocks
// of one text read the same K and V rows, as do the q heads of one kv head
// (GQA): ids are laid out so that all workgroups of one (text, kv head)
// unit share an XCD and its L2, units spread over the XCDs. Returns false
// past the last unit.
__device__ __forceinline__ bool attn_block(const AttnArgs& p, int& b, int& h, int& qb) {
  const int nqb = (p.max_len + kAttnQ - 1) / kAttnQ;
  const int G = p.heads / p.kv_heads;
  const int nv = G * nqb;  // workgroups per unit
  const int w = blockIdx.x;
  const int t = w >> 3;
  const int v = t % nv;
  const int u = (t / nv) * 8 + (w & 7);
  if (u >= p.batch * p.kv_heads) return false;
  qb = v % nqb;
  b = u / p.kv_heads;
  h = (u % p.kv_heads) * G + v / nqb;
  return true;
}

// Output rows of one wave's 32 queries: O^T leaves the MFMAs with lane
// (query fr, half fg) holding d = t*32 + i*8 + fg*4 + j, i.e. 32-byte pieces
// of 32 different rows per store instruction. The wave parks its rows in its
// own LDS region (row stride DH + 4 floats) and writes them back DH/4 lanes
// per row, so every store instruction covers whole 128-byte lines of
// consecutive rows. The caller has finished every LDS read of the key loop
// on all waves (the region overlaps the K/V blocks).
template <int DH>
__device__ __forceinline__ void attn_store_rows(const AttnArgs& p, const v16f (&o)[DH / 32],
                                                float inv, uint8_t* lds, int wave, int lane,
                                                int r0, int qw0, int len, int h) {
  constexpr int DT = DH / 32, kStride = DH + 4;
  constexpr int LPR = DH / 4, RPI = 64 / LPR;  // lanes per row, rows per instruction
  const int fr = lane & 31, fg = lane >> 5;
  float* st = reinterpret_cast<float*>(lds) + wave * 32 * kStride;
#pragma unroll
  for (int t = 0; t < DT; t++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v4f w;
#pragma unroll
      for (int j = 0; j < 4; j++) w[j] = o[t][i * 4 + j] * inv;
      *reinterpret_cast<v4f*>(st + fr * kStride + t * 32 + i * 8 + fg * 4) = w;
    }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's rows are in LDS
  __builtin_amdgcn_wave_barrier();
  const int c4 = (lane % LPR) * 4;
#pragma unroll
  for (int k = 0; k < 32 / RPI; k++) {
    const int rr = lane / LPR + k * RPI;
    const int q = qw0 + rr;
    const v4f w = *reinterpret_cast<const v4f*>(st + rr * kStride + c4);
    if (q < len) {
      const size_t off = (size_t)(r0 + q) * p.ldctx + h * DH + c4;
      if (p.ctx_hi) store_planes4(p.ctx_hi, p.ctx_lo, off, w);
      else *reinterpret_cast<v4f*>(p.ctx + off) = w;
    }
  }
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
  constexpr int kOut = 4 * 32 * (DH + 4) * 4;  // output staging (attn_store_rows)
  __shared__ __attribute__((aligned(16))) uint8_t lds[T * (kK + kV) > kOut ? T * (kK + kV) : kOut];
  uint8_t* sK = lds;
  uint8_t* sV = lds + T * kK;

  int b, h, qb;
  if (!attn_block(p, b, h, qb)) return;
  const int r0 = p.cu[b], len = p.cu[b + 1] - r0;
  const int q0 = qb * kAttnQ;
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
  const float cs = p.scale * 1.44269504088896341f;  // scores in log2 units
  int klo, khi;
  attn_key_range(p, qi, len, klo, khi);

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
    // Scale, mask, online softmax; the output is rescaled only when some
    // query's reference max moved.
    const bool masked = __any(key0 < klo || key0 + kAttnKV - 1 > khi);
    bool rescale;
    if (p.rel_bias) attn_rel_bias(p, sc, h, qi, key0, fg);
    const float alpha = attn_softmax_block(sc, key0, fg, klo, khi, masked,
                                           p.rel_bias ? 1.44269504088896341f : cs, mrun,
                                           lrun, rescale);
    if (rescale) {
#pragma unroll
      for (int t = 0; t < DT; t++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[t][e] *= alpha;
    }

    // O^T += V^T · P^T over 4 chunks of 16 keys. Chunk kc, lane half g,
    // element e <-> key kc*16 + (e/4)*8 + g*4 + e%4 = register
    // sc[kc/2][(kc%2)*8 + e].
#pragma unroll
    for (int kc = 0; kc < 4; kc++) {
      v8bf ph, pl;
      if constexpr (PREC == 3) {
        attn_split8(sc[kc >> 1], (kc & 1) * 8, ph, pl);
      } else {
#pragma unroll
        for (int e = 0; e < 8; e++) ph[e] = (__bf16)sc[kc >> 1][(kc & 1) * 8 + e];
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
  // rows past the text divide by 1 (their values are never stored)
  const float inv = 1.0f / (qi < len ? ltot : 1.0f);
  __syncthreads();  // every wave's reads of the last key block are done
  attn_store_rows<DH>(p, o, inv, lds, wave, lane, r0, q0 + wave * 32, len, h);
}

// ---- bf16 operands, pipelined --------------------------------------------------
// The same algorithm and fragment layouts for bf16 q|k|v rows, with the key
// blocks double-buffered: while a block is multiplied, the next block's K
// and V rows stream into LDS by global_load_lds_dwordx4.
//
// K block: [64 keys][DH] bf16, 16-byte chunk c of row r at slot c ^ kswz(r)
// (16 consecutive rows of one fragment read land in 16 distinct bank
// groups). V block: [64 keys][DH] bf16 as well, 64-byte pieces swizzled by
// attn_vswz; the PV products read it transposed (ds_read_b64_tr_b16), so
// each lane's V^T fragment holds the keys in the order its P^T registers
// do (see below).
template <int DH>
__device__ __forceinline__ int attn_kswz(int r) {
  constexpr int C = DH / 8;                       // chunks per K row
  constexpr int W = DH * 2 < 256 ? 256 / (DH * 2) : 1;  // rows per 256-B bank window
  return (r / W) & ((C < 16 ? C : 16) - 1);
}

// Two ds_read_b64_tr_b16 (CDNA4's transposing LDS read) make one 8-element
// bf16 A fragment of a PV product from row-major V: within each 16-lane
// group, lane i element e is element i % 4 of the 8 bytes lane 4e + i / 4
// addressed (checked on the GPU). `lo` gives elements 0..3, `hi` 4..7.
typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));
__device__ __forceinline__ v8bf attn_vt_frag(const uint8_t* lo, const uint8_t* hi) {
  typedef __attribute__((address_space(3))) v4s* lds_v4s;
  const v4s a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(lo));
  const v4s b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s)(hi));
  return __builtin_bit_cast(v8bf, (v8s)__builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

// V rows in LDS, row-major as DMA-staged: 64-byte piece q of row r sits at
// piece q ^ attn_vswz<DH>(r). A transposed read of the 32x32 kernel covers 8
// consecutive rows x 64 bytes; the swizzle spreads them two per 64-byte bank
// window (head dim 32 needs none).
template <int DH>
__device__ __forceinline__ int attn_vswz(int r) {
  return DH == 64 ? (r >> 1) & 1 : DH >= 128 ? r & 3 : 0;
}

template <int DH, int T>
__global__ __launch_bounds__(256) void attention_bf16_kernel(AttnArgs p) {
  const __bf16* qkv = static_cast<const __bf16*>(p.qkv);
  const __bf16* qkv_lo = static_cast<const __bf16*>(p.qkv_lo);  // T == 2
  constexpr int KS = DH / 16, DT = DH / 32;
  constexpr int kRowB = DH * 2;               // bytes of one K row
  constexpr int kKB = kAttnKV * kRowB;        // K block bytes
  constexpr int kStage = 2 * kKB * T;         // K + V (same size), per plane
  constexpr int kKLoads = kKB / (4 * 1024);   // DMA instructions per wave per block
  static_assert(kKLoads >= 1 && kKB % 4096 == 0, "K block must split into 4 waves x 1 KiB");
  constexpr int kOut = 4 * 32 * (DH + 4) * 4;  // output staging (attn_store_rows)
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * kStage > kOut ? 2 * kStage : kOut];

  int b, h, qb;
  if (!attn_block(p, b, h, qb)) return;
  const int r0 = p.cu[b], len = p.cu[b + 1] - r0;
  const int q0 = qb * kAttnQ;
  if (q0 >= len) return;
  const int kvh = h / (p.heads / p.kv_heads);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fg = lane >> 5;
  const int qi = q0 + wave * 32 + fr;

  // Q fragments (B operand of S^T), straight from the bf16 rows.
  v8bf qf[KS], ql[KS];
  {
    const size_t qo = (size_t)(r0 + (qi < len ? qi : len - 1)) * p.ldqkv + p.q_off + h * DH;
#pragma unroll
    for (int s = 0; s < KS; s++) {
      qf[s] = *reinterpret_cast<const v8bf*>(qkv + qo + s * 16 + fg * 8);
      if constexpr (T == 2) ql[s] = *reinterpret_cast<const v8bf*>(qkv_lo + qo + s * 16 + fg * 8);
    }
  }

  // K DMA: this lane's slot in each of its 1 KiB blocks -> (row, chunk).
  int k_row[kKLoads], k_chunk[kKLoads];
#pragma unroll
  for (int j = 0; j < kKLoads; j++) {
    const int off = (wave * kKLoads + j) * 1024 + lane * 16;
    k_row[j] = off / kRowB;
    k_chunk[j] = ((off % kRowB) >> 4) ^ attn_kswz<DH>(k_row[j]);
  }
  // plane t of a stage: K at t * 2 * kKB, V^T right after it
  const size_t kvo = (size_t)p.k_off + kvh * DH, vvo = (size_t)p.v_off + kvh * DH;
  auto issue_k = [&](int kb, int buf) {
#pragma unroll
    for (int t = 0; t < T; t++) {
      uint8_t* sK = lds + buf * kStage + t * 2 * kKB;
      const __bf16* kbase = (t ? qkv_lo : qkv) + kvo;
#pragma unroll
      for (int j = 0; j < kKLoads; j++) {
        const int kg = kb * kAttnKV + k_row[j];
        const __bf16* src =
            kbase + (size_t)(r0 + (kg < len ? kg : len - 1)) * p.ldqkv + k_chunk[j] * 8;
        lds_dma16(src, sK + (wave * kKLoads + j) * 1024);
      }
    }
  };
  // V DMA: the K slots with the V swizzle on 64-byte pieces (4 chunks)
  int v_chunk[kKLoads];
#pragma unroll
  for (int j = 0; j < kKLoads; j++) {
    const int off = (wave * kKLoads + j) * 1024 + lane * 16;
    v_chunk[j] = ((off % kRowB) >> 4) ^ (4 * attn_vswz<DH>(k_row[j]));
  }
  auto issue_v = [&](int kb, int buf) {
#pragma unroll
    for (int t = 0; t < T; t++) {
      uint8_t* sV = lds + buf * kStage + t * 2 * kKB + kKB;
      const __bf16* vbase = (t ? qkv_lo : qkv) + vvo;
#pragma unroll
      for (int j = 0; j < kKLoads; j++) {
        const int kg = kb * kAttnKV + k_row[j];
        lds_dma16(vbase + (size_t)(r0 + (kg < len ? kg : len - 1)) * p.ldqkv + v_chunk[j] * 8,
                  sV + (wave * kKLoads + j) * 1024);
      }
    }
  };
  // PV A fragments (lane (fr, g): dim 32t + fr of keys 16kc + 8(e/4) + 4g +
  // e%4, the key order of P^T's B fragment): lane s of 16-lane group G
  // addresses row 16kc + 4(G/2) + s/4 (+8 for elements 4..7), dims 32t +
  // 16(G%2) + 4(s%4) .. +3. The swizzle of those rows depends on s only;
  // 64t and the swizzled piece offset share bits 6 and up of a row's bytes,
  // below its row index, so base ^ 64t addresses dim tile t.
  int vt_off[DT];
  {
    const int s16 = lane & 15, vr = 4 * (lane >> 5) + (s16 >> 2);
    const int base = vr * kRowB + 64 * attn_vswz<DH>(vr) + 32 * ((lane >> 4) & 1) + 8 * (s16 & 3);
#pragma unroll
    for (int t = 0; t < DT; t++) vt_off[t] = base ^ (64 * t);
  }

  v16f o[DT];
#pragma unroll
  for (int t = 0; t < DT; t++)
#pragma unroll
    for (int e = 0; e < 16; e++) o[t][e] = 0.0f;
  float mrun = -INFINITY, lrun = 0.0f;
  const float cs = p.scale * 1.44269504088896341f;  // scores in log2 units
  int klo, khi;
  attn_key_range(p, qi, len, klo, khi);

  int kb_lo = 0, kb_hi = (len + kAttnKV - 1) / kAttnKV;
  const int qlast = min(q0 + kAttnQ, len) - 1;
  if (p.causal) kb_hi = min(kb_hi, qlast / kAttnKV + 1);
  if (p.window > 0) {
    kb_lo = max(0, q0 - p.window + 1) / kAttnKV;
    kb_hi = min(kb_hi, (qlast + p.window - 1) / kAttnKV + 1);
  }
  // every query sees every key of its text: the only mask is the text's end
  const bool text_mask = !p.causal && p.window <= 0;

  issue_k(kb_lo, 0);
  issue_v(kb_lo, 0);
  __syncthreads();  // waits for the DMA (vmcnt)

  for (int kb = kb_lo; kb < kb_hi; kb++) {
    const int buf = (kb - kb_lo) & 1;
    const bool next = kb + 1 < kb_hi;
    if (next) {
      issue_k(kb + 1, buf ^ 1);
      issue_v(kb + 1, buf ^ 1);
    }
    const uint8_t* sK = lds + buf * kStage;
    const uint8_t* sV = sK + kKB;
    const uint8_t* sKl = sK + 2 * kKB;  // T == 2: the lo planes
    const uint8_t* sVl = sKl + kKB;
    const int key0 = kb * kAttnKV;

    // A wave whose queries all lie past the text only helps stage blocks.
    if (q0 + wave * 32 < len) {
    // S^T for the two 32-key tiles, the two accumulation chains interleaved.
    v16f sc[2];
#pragma unroll
    for (int t2 = 0; t2 < 2; t2++)
#pragma unroll
      for (int e = 0; e < 16; e++) sc[t2][e] = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; s++)
#pragma unroll
      for (int t2 = 0; t2 < 2; t2++) {
        const int kr = t2 * 32 + fr;
        const int ko = kr * kRowB + (((2 * s + fg) ^ attn_kswz<DH>(kr)) << 4);
        const v8bf kf = *reinterpret_cast<const v8bf*>(sK + ko);
        sc[t2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[s], sc[t2], 0, 0, 0);
        if constexpr (T == 2) {  // hi·lo + lo·hi: the fp32-grade split
          const v8bf kl = *reinterpret_cast<const v8bf*>(sKl + ko);
          sc[t2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, ql[s], sc[t2], 0, 0, 0);
          sc[t2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kl, qf[s], sc[t2], 0, 0, 0);
        }
      }
    // Bidirectional attention masks only the keys past the text, the same
    // keys for every query: one more MFMA per tile adds -inf to their
    // scores (k-element 0 of a mask fragment times q-element 0 = 1; every
    // other product is 0 * 0) and +0 to the rest, which leaves those sums
    // as they were, in place of a compare and select per score.
    const bool key_tail = key0 + kAttnKV > len;
    if (text_mask && key_tail) {
      const v8bf q1 = {(__bf16)(fg == 0 ? 1.0f : 0.0f), (__bf16)0.0f, (__bf16)0.0f, (__bf16)0.0f,
                       (__bf16)0.0f, (__bf16)0.0f, (__bf16)0.0f, (__bf16)0.0f};
#pragma unroll
      for (int t2 = 0; t2 < 2; t2++) {
        const bool past = key0 + t2 * 32 + fr >= len;
        const v8bf km = {(__bf16)(fg == 0 && past ? -INFINITY : 0.0f), (__bf16)0.0f, (__bf16)0.0f,
                         (__bf16)0.0f, (__bf16)0.0f, (__bf16)0.0f, (__bf16)0.0f, (__bf16)0.0f};
        sc[t2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(km, q1, sc[t2], 0, 0, 0);
      }
    }

    // Scale, mask (only blocks that cross some query's visible range), online
    // softmax; the output is rescaled only when some query's reference max
    // moved, and never on the first block (the output is still zero).
    const bool masked = !text_mask && __any(key0 < klo || key0 + kAttnKV - 1 > khi);
    bool rescale;
    if (p.rel_bias) attn_rel_bias(p, sc, h, qi, key0, fg);
    const float alpha = attn_softmax_block(sc, key0, fg, klo, khi, masked,
                                           p.rel_bias ? 1.44269504088896341f : cs, mrun,
                                           lrun, rescale);
    if (rescale && kb != kb_lo) {
#pragma unroll
      for (int t = 0; t < DT; t++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[t][e] *= alpha;
    }

    // O^T += V^T · P^T over 4 chunks of 16 keys; lane half g, element e of
    // chunk kc is register sc[kc/2][(kc%2)*8 + e], key 16kc + 8(e/4) + 4g + e%4.
#pragma unroll
    for (int kc = 0; kc < 4; kc++) {
      v8bf ph, pl;
      if constexpr (T == 2) {
        attn_split8(sc[kc >> 1], (kc & 1) * 8, ph, pl);
      } else {
#pragma unroll
        for (int e = 0; e < 8; e++) ph[e] = (__bf16)sc[kc >> 1][(kc & 1) * 8 + e];
      }
#pragma unroll
      for (int t = 0; t < DT; t++) {
        const int vo = kc * 16 * kRowB + vt_off[t];
        const v8bf vf = attn_vt_frag(sV + vo, sV + vo + 8 * kRowB);
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, ph, o[t], 0, 0, 0);
        if constexpr (T == 2) {
          const v8bf vl = attn_vt_frag(sVl + vo, sVl + vo + 8 * kRowB);
          o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pl, o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vl, ph, o[t], 0, 0, 0);
        }
      }
    }
    }

    __syncthreads();  // next block landed (vmcnt) and this block's reads are done
  }

  const float ltot = lrun + __shfl_xor(lrun, 32, 64);
  const float inv = 1.0f / (qi < len ? ltot : 1.0f);
  // the loop's last barrier ordered every wave's reads of the key blocks
  attn_store_rows<DH>(p, o, inv, lds, wave, lane, r0, q0 + wave * 32, len, h);
}

// Head dim 256 on bf16 rows (EmbeddingGemma): eight waves of 16 queries on
// v_mfma_f32_16x16x32_bf16, two waves per SIMD. With 32 queries per wave
// (the kernel above) o, the Q fragments and the S tiles fill a wave's 256
// registers and one wave per SIMD waits on every LDS read; here o is 64
// registers, Q 32, S 16.
// 16x16x32 operand layouts (checked on the GPU): A lane l holds row l % 16,
// k = 8 (l / 16) .. +7; B lane l holds column l % 16, the same k; C lane l
// holds column l % 16, rows 4 (l / 16) .. +3.
// * S^T = K·Q^T per 16-key tile t: lane (query fr = l % 16, group fg = l /
//   16) holds keys 16t + 4fg + i. A query's 64 scores of a block sit in
//   the four lanes fr, fr+16, fr+32, fr+48 (two shuffles per statistic).
// * O^T += V^T·P^T per 32-key step kc: lane (fr, fg) feeds B element j with
//   its own scores, key 32kc + 4fg + j (j < 4) or 32kc + 16 + 4fg + j - 4.
//   V stays row-major in LDS (DMA-staged like K) and the V^T fragments come
//   from ds_read_b64_tr_b16, which within each 16-lane group gives lane i
//   element e = element i % 4 of what lane 4e + i / 4 addressed (checked on
//   the GPU). Lane s of group fg addresses key row 32kc + 4fg + s / 4 (then
//   16 rows further for elements 4..7), dims 16t + 4 (s % 4) .. +3, so lane
//   (fr, fg) receives dim 16t + fr of exactly the keys its B element j
//   holds. Rows go in pairs of 512 bytes (one 1 KiB DMA block) padded by 32
//   bytes: the 16 rows of one read then land two per 32-byte bank slot.
constexpr int kH256Waves = 8;


__global__ __launch_bounds__(64 * kH256Waves) void attention_h256_kernel(AttnArgs p) {
  constexpr int DH = 256, KS = DH / 32, NDT = DH / 16;
  constexpr int kRowB = DH * 2;               // bytes of one K or V row (512)
  constexpr int kKB = kAttnKV * kRowB;        // K block bytes (32 KiB)
  constexpr int kVPair = 2 * kRowB + 32;      // two V rows and their padding
  constexpr int kVB = kAttnKV / 2 * kVPair;   // V block bytes (33 KiB)
  constexpr int kStage = kKB + kVB;           // K + V
  constexpr int kKLoads = kKB / (kH256Waves * 1024);  // DMA instructions per wave (4)
  constexpr int kStride = DH + 4;             // output staging row (floats)
  constexpr int kOut = kH256Waves * 16 * kStride * 4;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * kStage > kOut ? 2 * kStage : kOut];
  const __bf16* qkv = static_cast<const __bf16*>(p.qkv);

  int b, h, qb;
  if (!attn_block(p, b, h, qb)) return;
  const int r0 = p.cu[b], len = p.cu[b + 1] - r0;
  const int q0 = qb * kAttnQ;
  if (q0 >= len) return;
  const int kvh = h / (p.heads / p.kv_heads);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, fg = lane >> 4;
  const int qw0 = q0 + wave * 16;
  const int qi = qw0 + fr;

  // Q fragments (B operand of S^T): k-step s, elements s*32 + 8fg .. +7
  v8bf qf[KS];
  {
    const size_t qo = (size_t)(r0 + (qi < len ? qi : len - 1)) * p.ldqkv + p.q_off + h * DH;
#pragma unroll
    for (int s = 0; s < KS; s++) qf[s] = *reinterpret_cast<const v8bf*>(qkv + qo + s * 32 + fg * 8);
  }

  // K DMA: 1 KiB blocks of the 64 x 512-byte block, chunk swizzled by row
  int k_row[kKLoads], k_chunk[kKLoads];
#pragma unroll
  for (int j = 0; j < kKLoads; j++) {
    const int off = (wave * kKLoads + j) * 1024 + lane * 16;
    k_row[j] = off / kRowB;
    k_chunk[j] = ((off % kRowB) >> 4) ^ attn_kswz<DH>(k_row[j]);
  }
  const __bf16* kbase = qkv + p.k_off + kvh * DH;
  const __bf16* vbase = qkv + p.v_off + kvh * DH;
  auto issue_k = [&](int kb, int buf) {
    uint8_t* sK = lds + buf * kStage;
#pragma unroll
    for (int j = 0; j < kKLoads; j++) {
      const int kg = kb * kAttnKV + k_row[j];
      lds_dma16(kbase + (size_t)(r0 + (kg < len ? kg : len - 1)) * p.ldqkv + k_chunk[j] * 8,
                sK + (wave * kKLoads + j) * 1024);
    }
  };
  // V DMA: 1 KiB block j holds rows 2j and 2j + 1 (lane l: row 2j + l / 32,
  // bytes 16 (l % 32)), blocks kVPair apart
  const int v_row = (wave * kKLoads) * 2 + (lane >> 5), v_col = (lane & 31) * 8;
  auto issue_v = [&](int kb, int buf) {
    uint8_t* sV = lds + buf * kStage + kKB;
#pragma unroll
    for (int j = 0; j < kKLoads; j++) {
      const int kg = kb * kAttnKV + v_row + 2 * j;
      lds_dma16(vbase + (size_t)(r0 + (kg < len ? kg : len - 1)) * p.ldqkv + v_col,
                sV + (wave * kKLoads + j) * kVPair);
    }
  };
  // this lane's transposed-read address in a V block (key row 4fg + fr / 4,
  // dims 4 (fr % 4) .. +3); step kc adds 16 row pairs, elements 4..7 eight
  // pairs, dim tile t 32 bytes
  const int vt_row = 4 * fg + (fr >> 2);
  const int vt_off = (vt_row >> 1) * kVPair + (vt_row & 1) * kRowB + 8 * (fr & 3);

  v4f o[NDT];
#pragma unroll
  for (int t = 0; t < NDT; t++) o[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  float mref = -INFINITY, lrun = 0.0f;
  const float cs = p.scale * 1.44269504088896341f;  // scores in log2 units
  int klo, khi;
  attn_key_range(p, qi, len, klo, khi);
  int kb_lo = 0, kb_hi = (len + kAttnKV - 1) / kAttnKV;
  const int qlast = min(q0 + kAttnQ, len) - 1;
  if (p.causal) kb_hi = min(kb_hi, qlast / kAttnKV + 1);
  if (p.window > 0) {
    kb_lo = max(0, q0 - p.window + 1) / kAttnKV;
    kb_hi = min(kb_hi, (qlast + p.window - 1) / kAttnKV + 1);
  }

  issue_k(kb_lo, 0);
  issue_v(kb_lo, 0);
  __syncthreads();

  for (int kb = kb_lo; kb < kb_hi; kb++) {
    const int buf = (kb - kb_lo) & 1;
    const bool next = kb + 1 < kb_hi;
    if (next) {
      issue_k(kb + 1, buf ^ 1);
      issue_v(kb + 1, buf ^ 1);
    }
    const uint8_t* sK = lds + buf * kStage;
    const uint8_t* sV = sK + kKB + vt_off;
    const int key0 = kb * kAttnKV;

    if (qw0 < len) {  // a wave whose queries all lie past the text only stages
      v4f sc[4];
#pragma unroll
      for (int t = 0; t < 4; t++) sc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < KS; s++)
#pragma unroll
        for (int t = 0; t < 4; t++) {
          const int kr = t * 16 + fr;
          const v8bf kf = *reinterpret_cast<const v8bf*>(
              sK + kr * kRowB + (((4 * s + fg) ^ attn_kswz<DH>(kr)) << 4));
          sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[s], sc[t], 0, 0, 0);
        }
      // keys outside this lane's query range (text end, causal, window): one
      // uniform branch around the range tests
      const bool masked = __any(key0 < klo || key0 + kAttnKV - 1 > khi);
      if (masked) {
        const unsigned span = (unsigned)(khi - klo);
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const unsigned off = (unsigned)(key0 + t * 16 + 4 * fg + i - klo);
            sc[t][i] = off > span ? -INFINITY : sc[t][i];
          }
      }
      // online softmax (the scheme of attn_softmax_block): reference max in
      // log2 units, moved only when a block's max exceeds it by more than 8
      float smax = -INFINITY;
#pragma unroll
      for (int t = 0; t < 4; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) smax = fmaxf(smax, sc[t][i]);
      smax = fmaxf(smax, __shfl_xor(smax, 16, 64));
      smax = fmaxf(smax, __shfl_xor(smax, 32, 64));
      const float mloc = smax * cs;
      const bool up = mloc > mref + 8.0f;
      const bool rescale = __any(up);
      float alpha = 1.0f;
      if (up) {
        alpha = __builtin_amdgcn_exp2f(mref - mloc);
        mref = mloc;
      }
      const float m = mref == -INFINITY ? 0.0f : mref;
      float psum = 0.0f;
#pragma unroll
      for (int t = 0; t < 4; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[t][i], cs, -m));
          sc[t][i] = pv;
          psum += pv;
        }
      lrun = lrun * alpha + psum;
      if (rescale && kb != kb_lo) {
#pragma unroll
        for (int t = 0; t < NDT; t++) o[t] *= alpha;
      }
      // O^T += V^T · P^T, two 32-key steps
#pragma unroll
      for (int kc = 0; kc < 2; kc++) {
        v8bf ph;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          ph[j] = (__bf16)sc[2 * kc][j];
          ph[4 + j] = (__bf16)sc[2 * kc + 1][j];
        }
#pragma unroll
        for (int t = 0; t < NDT; t++) {
          const uint8_t* v = sV + kc * 16 * kVPair + t * 32;
          const v8bf vf = attn_vt_frag(v, v + 8 * kVPair);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, ph, o[t], 0, 0, 0);
        }
      }
    }

    __syncthreads();  // next block landed (vmcnt) and this block's reads are done
  }

  // the row sum over the four lane groups of a query, then the rows leave
  // through LDS (the loop's last barrier ordered every read of the blocks)
  float ltot = lrun + __shfl_xor(lrun, 16, 64);
  ltot = ltot + __shfl_xor(ltot, 32, 64);
  const float inv = 1.0f / (qi < len ? ltot : 1.0f);
  float* st = reinterpret_cast<float*>(lds) + wave * 16 * kStride;
#pragma unroll
  for (int t = 0; t < NDT; t++)
    *reinterpret_cast<v4f*>(st + fr * kStride + t * 16 + 4 * fg) = o[t] * inv;
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's rows are in LDS
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int rr = 0; rr < 16; rr++) {
    const int q = qw0 + rr;
    if (q < len) {
      const v4f w = *reinterpret_cast<const v4f*>(st + rr * kStride + lane * 4);
      const size_t off = (size_t)(r0 + q) * p.ldctx + h * DH + lane * 4;
      if (p.ctx_hi) store_planes4(p.ctx_hi, p.ctx_lo, off, w);
      else *reinterpret_cast<v4f*>(p.ctx + off) = w;
    }
  }
}

template <int DH>
static hipError_t launch_attn_dh(const AttnArgs& a, int precision, hipStream_t s) {
  const int units = a.batch * a.kv_heads;
  const dim3 grid(8 * ceil_div(a.max_len, kAttnQ) * (a.heads / a.kv_heads) * ceil_div(units, 8));
  if (a.in_bf16 == 2) {  // hi/lo planes: the three-term products, pipelined
    if constexpr (DH <= 128) {
      if (precision != 3 || !a.qkv_lo) return hipErrorInvalidValue;
      timed_launch((attention_bf16_kernel<DH, 2>), grid, dim3(256), 0, s, a);
    } else {
      return hipErrorInvalidValue;
    }
  } else if (a.in_bf16) {  // bf16 input carries no low half: one-term products
    // head dim 256: the 16x16x32 kernel (two waves per SIMD; 324 against 372
    // µs at EmbeddingGemma's global layer, 186 against 219 at its window-512
    // layers), the 32x32 one where a relative-position bias is added
    if (DH == 256 && !a.rel_bias)
      timed_launch(attention_h256_kernel, grid, dim3(64 * kH256Waves), 0, s, a);
    else
      timed_launch((attention_bf16_kernel<DH, 1>), grid, dim3(256), 0, s, a);
  }
  else if (precision == 3)
    timed_launch((attention_kernel<DH, 3, float>), grid, dim3(256), 0, s, a);
  else
    timed_launch((attention_kernel<DH, 1, float>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& a, int precision, hipStream_t s) {
  if (a.batch <= 0 || a.max_len <= 0) return hipSuccess;
  if (a.kv_heads <= 0 || a.heads % a.kv_heads != 0) return hipErrorInvalidValue;
  switch (a.dh) {
    case 32: return launch_attn_dh<32>(a, precision, s);
    case 64: return launch_attn_dh<64>(a, precision, s);
    case 128: return launch_attn_dh<128>(a, precision, s);
    case 256: return launch_attn_dh<256>(a, precision, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rh
