// model.cpp — the device-resident encoder behind rh_model_*: the mirror of
// model.Load (internal/model/bert.go:307-524), encodeWorkers
// (bert.go:740-923), Forward/ForwardTokens (bert.go:649-731) and Embed's
// batch loop (rembed.go:287-411).
//
// Where the reference runs one unpadded forward per text, this runtime packs
// the batch's texts back to back into M = sum(len) rows: every linear is
// one GEMM over all texts, attention and pooling walk each text's own rows
// (cu offsets), so no pad token is ever computed or attended and each
// text's result equals its unpadded forward.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "context.h"

using namespace rh;

namespace {

struct HostTensor {
  std::vector<int64_t> shape;
  std::vector<float> data;
};

struct Layer {
  rh_weight* qkv = nullptr;  // fused [3H][H] (bert.go:479-485)
  rh_weight* o = nullptr;
  rh_weight* f1 = nullptr;
  rh_weight* f2 = nullptr;
  float *ln1_g = nullptr, *ln1_b = nullptr, *ln2_g = nullptr, *ln2_b = nullptr;
};

// One layer of the RoPE family on the device: Qwen3, Gemma3, nomic-bert,
// ModernBERT. q|k|v are fused into one weight and gate|up into one gated
// weight; norm weights are uploaded as the reference uses them (Gemma's with
// the unit offset folded in). nomic keeps norm1 in post_attn(_b) and norm2 in
// post_ffn(_b); ModernBERT keeps attn_norm in in_norm (null for layer 0, an
// identity in the reference) and mlp_norm in post_attn.
struct DecLayer {
  rh_weight* qkv = nullptr;  // [qdim + 2 kvdim][H], or null when q, k, v are separate
  rh_weight* o = nullptr;    // [H][qdim]
  rh_weight* gu = nullptr;   // gated [2I][H], or null when gate, up are separate
  rh_weight* down = nullptr; // [H][I]
  // The reference packs q, k, v, gate and up one matrix at a time
  // (qwen3.go:479-481,528-529; gemma3.go:297-299,363-364), so newDense can
  // leave them in different modes; a group whose modes differ stays as
  // separate weights (each [out][H]) and runs as separate GEMMs.
  rh_weight *q = nullptr, *k = nullptr, *v = nullptr, *gate = nullptr, *up = nullptr;
  float *in_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr, *post_attn = nullptr,
        *pre_ffn = nullptr, *post_ffn = nullptr;
  float *post_attn_b = nullptr, *post_ffn_b = nullptr;  // nomic's LayerNorm betas
  bool global = true;
};

template <class T>
hipError_t dalloc(T** p, size_t count) {
  return hipMalloc((void**)p, count * sizeof(T) + 16);
}

// A model's device weights: packed linears, norms, embedding tables, RoPE
// tables, the Dense head. Every rh_model handle over them (the one that
// finalized them and each made by rh_model_share) holds a reference, and
// the last one to go frees them. They are immutable once finalized, so
// handles on different streams read them concurrently.
struct WeightSet {
  rh_context* ctx = nullptr;  // the context they were packed on (a reference)
  std::vector<Layer> layers;
  std::vector<DecLayer> dlayers;
  std::vector<float*> bufs;

  WeightSet(rh_context* c, std::vector<Layer> l, std::vector<DecLayer> d,
            std::vector<float*> b)
      : ctx(c), layers(std::move(l)), dlayers(std::move(d)), bufs(std::move(b)) {
    ctx_retain(ctx);
  }
  WeightSet(const WeightSet&) = delete;
  WeightSet& operator=(const WeightSet&) = delete;
  // Each handle has synchronized its own streams before dropping its
  // reference, so no kernel still reads these.
  ~WeightSet() {
    (void)hipSetDevice(ctx->device);
    for (auto& L : layers) {
      for (rh_weight* w : {L.qkv, L.o, L.f1, L.f2}) {
        if (!w) continue;
        destroy_weight(w);
        ctx_release(ctx);  // never the last reference: this set holds one
      }
      for (float* p : {L.ln1_g, L.ln1_b, L.ln2_g, L.ln2_b})
        if (p) (void)hipFree(p);
    }
    for (auto& L : dlayers) {
      for (rh_weight* w : {L.qkv, L.o, L.gu, L.down, L.q, L.k, L.v, L.gate, L.up}) {
        if (!w) continue;
        destroy_weight(w);
        ctx_release(ctx);
      }
      for (float* p : {L.in_norm, L.q_norm, L.k_norm, L.post_attn, L.pre_ffn, L.post_ffn,
                       L.post_attn_b, L.post_ffn_b})
        if (p) (void)hipFree(p);
    }
    for (float* p : bufs)
      if (p) (void)hipFree(p);
    ctx_release(ctx);
  }
};

}  // namespace

struct rh_model {
  rh_context* ctx = nullptr;
  rh_model_config cfg{};
  int quant = 0;
  bool finalized = false;
  std::map<std::string, HostTensor> pending;
  std::mutex mu;

  float *word = nullptr, *pos = nullptr, *type0 = nullptr, *emb_g = nullptr,
        *emb_b = nullptr;
  // MPNet: the relative-position bias per head and relative position,
  // [heads][2 * max_seq - 1], entry (h, j - i + max_seq - 1)
  float* rel_bias = nullptr;
  std::vector<Layer> layers;
  // decoder family
  std::vector<DecLayer> dlayers;
  float *final_norm = nullptr;
  float *dense1 = nullptr, *dense2 = nullptr;  // Gemma Dense head, transposed [in][out]
  float *cos_g = nullptr, *sin_g = nullptr, *cos_l = nullptr, *sin_l = nullptr;
  float *normed = nullptr, *pooled = nullptr, *dense_hid = nullptr;
  int32_t* pos_d = nullptr;
  int attn_precision = 3;
  // RH_OPT_FUSED_FFN1: 0 split, 1 two passes, 2 one pass (default: 3.58-3.59
  // against 3.46-3.47 M tokens/s for split on the BERT-base int8 batch,
  // interleaved runs on one box)
  int fused_ffn1 = 2;
  // RH_OPT_EXACT (BERT family): LayerNorm's sums and attention in the
  // reference's own float32 order (fp32 q|k|v rows), so a full-int8 forward
  // is byte-identical to the reference's
  bool exact = false;
  // RH_OPT_FUSED_LN: off by default; measured slower on BERT-base int8 at
  // M = 10102 (2.947 vs 2.864 ms/step with two streams, 3.05 vs 2.97 with
  // one): the whole-row tiles give 158 workgroups for 256 CUs, one per CU,
  // and their main loop runs at ~80 % of the 128x256 tiles' rate per CU.
  bool fused_ln = false;
  bool producer_planes = true;  // RH_OPT_PRODUCER_PLANES
  int streams = 2;              // RH_OPT_STREAMS
  // RH_OPT_QK_EPILOGUE: on by default since the epilogue loads each band's
  // cos/sin pieces before its first store (Qwen3-0.6B W8 22.4 against
  // 23.1-23.4 ms/step, EmbeddingGemma 18.6 against 18.8); with a load per
  // row behind the previous row's store (vmcnt counts both) it had been
  // slower than the separate pass.
  bool qk_epilogue = true;
  // RH_OPT_FUSE_PROJECTIONS: decoder q|k|v and gate|up packed as one weight
  // each where newDense leaves the group in one mode (default), or always
  // as separate weights like the reference; set before finalize.
  bool fuse_projections = true;
  bool split_gu_any = false;  // some layer runs gate and up as separate GEMMs
  // extra streams (default priority) and the fork/join events of a forward
  // split into parts
  static constexpr int kMaxParts = 4;
  hipStream_t sx[kMaxParts] = {};
  hipEvent_t ev_fork = nullptr, ev_join[kMaxParts] = {};

  // workspace, sized for cap rows / cap_batch texts
  int cap = 0, cap_batch = 0;
  size_t cap_ids = 0;
  float *x = nullptr, *qkv = nullptr, *ctxb = nullptr, *y = nullptr, *hid = nullptr;
  float* hid2 = nullptr;  // [cap][I] up rows of a layer whose gate and up are separate
  __bf16* qkvh = nullptr;                 // bf16 QKV rows (bf16 attention)
  // bf16 hi/lo activation planes written by the producers of the
  // weight-only int8 / fp32 GEMMs: p0 [cap][ld0] holds a width-H or
  // width-qdim input (normed rows, attention output), p1 [cap][ld1] the
  // intermediate (the gated / GELU output feeding the down projection).
  __bf16 *p0h = nullptr, *p0l = nullptr, *p1h = nullptr, *p1l = nullptr;
  int ld0 = 0, ld1 = 0;
  uint8_t *qa = nullptr, *qa2 = nullptr;  // u8 activations: width H / width I
  float *rs = nullptr, *rs2 = nullptr, *absmax = nullptr;
  // the one-pass FFN1 (RH_OPT_FUSED_FFN1 2): per row one slot per column
  // tile [cap][kQsyncMaxTiles] (all ones when empty), and per part one
  // departure count per 128-row block (qsync_stride words after word 0,
  // the timeout flag); set when allocated and left so by every launch
  unsigned* qslots = nullptr;
  unsigned* qsync = nullptr;
  int qsync_stride = 0;
  int32_t* cu_d = nullptr;
  int32_t* ids_d = nullptr;
  float* out_d = nullptr;
  int* err_d = nullptr;
  int32_t* cu_pinned = nullptr;
  hipEvent_t cu_evt = nullptr;
  int cu_pinned_cap = 0;
  // pinned int32 staging rows of the host-buffer embed calls (ids narrowed
  // from the caller's int64); reused once the previous call has synced
  int32_t* ids_pinned = nullptr;
  size_t ids_pinned_cap = 0;
  std::vector<int32_t> cu_host;  // packed row offsets of the current call
  // Owner of the weights above once finalized, shared with every handle
  // made by rh_model_share; null while the model is being built.
  std::shared_ptr<WeightSet> weights;

  ~rh_model() { release(); }

  // The weight set of the pointers above, which it then owns.
  std::shared_ptr<WeightSet> own_weights() {
    return std::make_shared<WeightSet>(
        ctx, layers, dlayers,
        std::vector<float*>{word, pos, type0, emb_g, emb_b, final_norm, dense1, dense2, cos_g,
                            sin_g, cos_l, sin_l, rel_bias});
  }

  void release_ws() {
    for (void* p : {(void*)x, (void*)qkv, (void*)ctxb, (void*)y, (void*)hid, (void*)qa,
                    (void*)rs, (void*)cu_d, (void*)ids_d, (void*)out_d, (void*)qkvh,
                    (void*)qa2, (void*)rs2, (void*)absmax, (void*)normed, (void*)pooled,
                    (void*)dense_hid, (void*)p0h, (void*)p0l, (void*)p1h, (void*)p1l,
                    (void*)pos_d, (void*)hid2, (void*)qslots, (void*)qsync})
      if (p) (void)hipFree(p);
    x = qkv = ctxb = y = hid = rs = out_d = rs2 = absmax = normed = pooled = dense_hid = nullptr;
    qslots = qsync = nullptr;
    hid2 = nullptr;
    pos_d = nullptr;
    qa = qa2 = nullptr;
    qkvh = p0h = p0l = p1h = p1l = nullptr;
    cu_d = ids_d = nullptr;
    cap = cap_batch = cap_ids = 0;
  }
  void release() {
    if (ctx) {
      (void)hipSetDevice(ctx->device);
      (void)hipStreamSynchronize(ctx->stream);
    }
    for (hipStream_t& q : sx)
      if (q) {
        (void)hipStreamSynchronize(q);
        (void)hipStreamDestroy(q);
        q = nullptr;
      }
    if (ev_fork) (void)hipEventDestroy(ev_fork);
    ev_fork = nullptr;
    for (hipEvent_t& e : ev_join)
      if (e) {
        (void)hipEventDestroy(e);
        e = nullptr;
      }
    drop_graph();
    release_ws();
    // Drop this handle's reference to the weights; a model that never
    // finalized (or failed to) owns what it built so far and frees it here.
    try {
      if (ctx && !weights) weights = own_weights();
    } catch (...) {
    }  // out of host memory: the device weights leak rather than abort
    weights.reset();
    layers.clear();
    dlayers.clear();
    word = pos = type0 = emb_g = emb_b = rel_bias = nullptr;
    final_norm = dense1 = dense2 = cos_g = sin_g = cos_l = sin_l = nullptr;
    if (err_d) (void)hipFree(err_d);
    err_d = nullptr;
    if (cu_pinned) (void)hipHostFree(cu_pinned);
    cu_pinned = nullptr;
    if (ids_pinned) (void)hipHostFree(ids_pinned);
    ids_pinned = nullptr;
    ids_pinned_cap = 0;
    if (cu_evt) (void)hipEventDestroy(cu_evt);
    cu_evt = nullptr;
  }

  int H() const { return cfg.hidden; }
  int I() const { return cfg.intermediate; }
  // The RoPE family (Qwen3, Gemma3, nomic-bert, ModernBERT) runs
  // forward_dec; BERT / RoBERTa run forward.
  // BERT, DistilBERT and MPNet share the post-LN flow (encodeWorkers,
  // bert.go:740-923); the rest are the RoPE family
  bool rope_family() const {
    return cfg.arch != RH_ARCH_BERT && cfg.arch != RH_ARCH_DISTILBERT && cfg.arch != RH_ARCH_MPNET;
  }
  bool gemma() const { return cfg.arch == RH_ARCH_GEMMA3; }
  bool nomic() const { return cfg.arch == RH_ARCH_NOMIC; }
  bool modernbert() const { return cfg.arch == RH_ARCH_MODERNBERT; }
  // nomic and ModernBERT normalize with LayerNorm, the decoders with RMSNorm
  bool layer_norm() const { return nomic() || modernbert(); }
  int nq() const { return cfg.heads; }
  int nkv() const { return rope_family() && cfg.kv_heads > 0 ? cfg.kv_heads : cfg.heads; }
  int dh() const {
    return rope_family() && cfg.head_dim > 0 ? cfg.head_dim : cfg.hidden / cfg.heads;
  }
  int qdim() const { return nq() * dh(); }
  int kvdim() const { return nkv() * dh(); }
  int qkv_width() const { return rope_family() ? qdim() + 2 * kvdim() : 3 * cfg.hidden; }
  int ctx_width() const { return rope_family() ? qdim() : cfg.hidden; }
  int ldq_for(int k) const { return (int)round_up(k, 16); }
  // Does w take its input as producer-written planes? (w runs on planes and
  // K is a multiple of 64, so the producers' K columns fill the planes.)
  bool planes_in(const rh_weight* w) const {
    return w && producer_planes && p0h && linear_on_planes(ctx, w) && w->k % 64 == 0;
  }
  Planes plane(int which, const rh_weight* w) const {
    Planes p;
    if (!w) return p;  // a group run as separate weights takes fp32 rows
    p.hi = which ? p1h : p0h;
    p.lo = linear_a_terms(ctx, w) == 2 ? (which ? p1l : p0l) : nullptr;
    p.ld = which ? ld1 : ld0;
    return p;
  }
  float eps() const { return cfg.layer_norm_eps == 0.0f ? 1e-12f : cfg.layer_norm_eps; }
  // Can w, a projection onto the hidden width followed by the residual +
  // LayerNorm, finish those rows in its own epilogue? (A full-int8 weight
  // with its fragment image, a supported width, and a next GEMM that takes
  // u8 rows or nothing rather than bf16 planes.)
  bool fuse_ln(const rh_weight* w, bool consumer_planes) const {
    return fused_ln && !exact && w && w->mode == RH_MODE_A8W8 && w->d_frag && !w->glu &&
           w->n == cfg.hidden && gemm_i8_ln_supported(w->n, w->k) && !consumer_planes;
  }
  I8LnArgs ln_args(float* xp, const float* g, const float* b, uint8_t* qa_out, int ldq,
                   float* rs_out) const {
    I8LnArgs f{};
    f.x = xp;
    f.gamma = g;
    f.beta = b;
    f.eps = eps();
    f.qa = qa_out;
    f.ldq = ldq;
    f.row_scales = rs_out;
    return f;
  }
  int max_seq() const { return cfg.max_position - cfg.position_offset; }

  int ensure_ws(int rows, int batch, size_t ids_elems) {
    const int H = this->H(), I = this->I();
    if (rows > cap || batch > cap_batch || ids_elems > cap_ids) {
      RH_HIP(hipStreamSynchronize(ctx->stream));  // buffers may be in flight
      drop_graph();  // a recorded forward holds the old buffers' addresses
    }
    if (rows > cap) {
      int newcap = (int)round_up(rows, 256);
      for (void* p : {(void*)x, (void*)qkv, (void*)ctxb, (void*)y, (void*)hid, (void*)qa,
                      (void*)rs, (void*)qkvh, (void*)qa2, (void*)rs2, (void*)absmax,
                      (void*)normed, (void*)pos_d, (void*)p0h, (void*)p0l, (void*)p1h,
                      (void*)p1l, (void*)hid2, (void*)qslots, (void*)qsync})
        if (p) RH_HIP(hipFree(p));
      x = qkv = ctxb = y = hid = rs = rs2 = absmax = normed = hid2 = nullptr;
      qslots = qsync = nullptr;
      qa = qa2 = nullptr;
      qkvh = p0h = p0l = p1h = p1l = nullptr;
      pos_d = nullptr;
      const size_t r = newcap;
      RH_HIP(dalloc(&x, r * H));
      RH_HIP(dalloc(&qkv, r * qkv_width()));
      RH_HIP(dalloc(&qkvh, r * qkv_width()));
      RH_HIP(dalloc(&ctxb, r * ctx_width()));
      RH_HIP(dalloc(&y, r * H));
      RH_HIP(dalloc(&hid, r * I));
      if (split_gu_any) RH_HIP(dalloc(&hid2, r * I));
      RH_HIP(dalloc(&qa, r * ldq_for(std::max(H, ctx_width()))));
      RH_HIP(dalloc(&qa2, r * ldq_for(I)));
      if (rope_family()) {
        RH_HIP(dalloc(&normed, r * H));
        RH_HIP(dalloc(&pos_d, r));
      }
      RH_HIP(dalloc(&rs, r));
      RH_HIP(dalloc(&rs2, r));
      RH_HIP(dalloc(&absmax, r));
      RH_HIP(dalloc(&qslots, r * kQsyncMaxTiles));
      RH_HIP(hipMemset(qslots, 0xFF, r * kQsyncMaxTiles * sizeof(unsigned)));
      qsync_stride = (int)(r / 128) + 1;
      RH_HIP(dalloc(&qsync, 1 + (size_t)kMaxParts * qsync_stride));
      RH_HIP(hipMemset(qsync, 0, (1 + (size_t)kMaxParts * qsync_stride) * sizeof(unsigned)));
      if (quant != RH_QUANT_FULL) {
        ld0 = (int)round_up(std::max(H, ctx_width()), 64);
        ld1 = (int)round_up(I, 64);
        RH_HIP(dalloc(&p0h, r * ld0));
        RH_HIP(dalloc(&p0l, r * ld0));
        RH_HIP(dalloc(&p1h, r * ld1));
        RH_HIP(dalloc(&p1l, r * ld1));
      }
      cap = newcap;
    }
    if (batch > cap_batch) {
      if (cu_d) RH_HIP(hipFree(cu_d));
      if (out_d) RH_HIP(hipFree(out_d));
      if (pooled) RH_HIP(hipFree(pooled));
      if (dense_hid) RH_HIP(hipFree(dense_hid));
      dense_hid = nullptr;
      cu_d = nullptr;
      out_d = nullptr;
      pooled = nullptr;
      const int nb = (int)round_up(batch, 64);
      RH_HIP(dalloc(&cu_d, nb + 1));
      RH_HIP(dalloc(&out_d, (size_t)nb * H));
      RH_HIP(dalloc(&pooled, (size_t)nb * H));
      if (cfg.dense_hidden > 0) RH_HIP(dalloc(&dense_hid, (size_t)nb * cfg.dense_hidden));
      cap_batch = nb;
    }
    if (ids_elems > cap_ids) {
      if (ids_d) RH_HIP(hipFree(ids_d));
      ids_d = nullptr;
      const size_t n = round_up(ids_elems, 4096);
      RH_HIP(dalloc(&ids_d, n));
      cap_ids = n;
    }
    if (batch + 1 > cu_pinned_cap) {
      if (cu_pinned) {
        if (cu_evt) RH_HIP(hipEventSynchronize(cu_evt));
        RH_HIP(hipHostFree(cu_pinned));
      }
      cu_pinned = nullptr;
      const int n = (int)round_up(batch + 1, 256);
      RH_HIP(hipHostMalloc((void**)&cu_pinned, n * sizeof(int32_t)));
      cu_pinned_cap = n;
    }
    if (!cu_evt) RH_HIP(hipEventCreateWithFlags(&cu_evt, hipEventDisableTiming));
    if (!err_d) {
      RH_HIP(dalloc(&err_d, 1));
      RH_HIP(hipMemset(err_d, 0, sizeof(int)));
    }
    return RH_OK;
  }

  // Pinned staging for `elems` int32 ids (grow-only; the previous call has
  // synchronized its stream before returning, so the old buffer is idle).
  int ensure_ids_staging(size_t elems) {
    if (elems <= ids_pinned_cap) return RH_OK;
    if (ids_pinned) RH_HIP(hipHostFree(ids_pinned));
    ids_pinned = nullptr;
    ids_pinned_cap = 0;
    const size_t n = round_up(elems, 4096);
    RH_HIP(hipHostMalloc((void**)&ids_pinned, n * sizeof(int32_t)));
    ids_pinned_cap = n;
    return RH_OK;
  }

  // Validate lengths (bert.go:741-747) and build packed row offsets.
  int plan(const int32_t* lens, int batch, std::vector<int32_t>& cu, int* max_len) {
    cu.assign(batch + 1, 0);
    int mx = 0;
    for (int b = 0; b < batch; b++) {
      char buf[160];
      if (lens[b] <= 0) {
        snprintf(buf, sizeof buf, "text %d: empty token sequence", b);
        return fail(RH_ERR_SEQ, buf);
      }
      if (lens[b] > max_seq()) {
        snprintf(buf, sizeof buf,
                 "text %d: sequence length %d exceeds the model's maximum %d", b,
                 lens[b], max_seq());
        return fail(RH_ERR_SEQ, buf);
      }
      if ((long long)cu[b] + lens[b] > (long long)INT32_MAX)
        return fail(RH_ERR_INVALID, "total tokens of the batch exceed 2^31 - 1");
      cu[b + 1] = cu[b] + lens[b];
      mx = std::max(mx, (int)lens[b]);
    }
    *max_len = mx;
    return RH_OK;
  }

  // A forward runs over one part (all texts) or `streams` parts of whole
  // texts on as many streams: the parts' kernels share the GPU, so one
  // part's GEMMs (MFMA/LDS-bound) overlap another's row kernels
  // (VALU/HBM-bound). Every buffer is indexed by packed row (cu_d by text),
  // so a part only offsets its pointers; a part's results equal the
  // one-part forward's rows. Several parts need every linear to run without
  // the context's split workspace (full int8, or planes written by their
  // producers), which one buffer serves for all GEMMs of the context.
  struct Part {
    int row0, rows, b0, nb, max_len;
    hipStream_t s;
    int idx;  // 0..streams-1
  };
  bool uses_split_ws(const rh_weight* w, bool pin) const {
    return linear_on_planes(ctx, w) && !pin;
  }
  int plan_parts(const std::vector<int32_t>& cu, bool allowed, hipStream_t s,
                 std::vector<Part>& parts);
  int join_parts(const std::vector<Part>& parts, hipStream_t s);

  // The forward over rows already planned; ids_dev is [batch][stride].
  // RH_OPT_GRAPH: the BERT family's forward recorded once per batch shape
  // (row offsets, ids and output buffers, settings) as a HIP graph and
  // replayed; any change of shape, option or workspace records it again.
  bool use_graph = false;
  struct Graph {
    std::vector<int32_t> cu;
    const int32_t* ids = nullptr;
    int stride = 0, max_len = 0, generation = -1;
    bool pool = false;
    float* out = nullptr;
    hipGraphExec_t exec = nullptr;
  } graph;
  void drop_graph() {
    if (graph.exec) (void)hipGraphExecDestroy(graph.exec);
    graph = Graph{};
  }
  int ensure_streams();
  bool bert_no_ws() const;
  int forward_bert(const int32_t* ids_dev, int stride, const std::vector<int32_t>& cu,
                   int max_len, bool pool, float* out_dev);
  int forward(const int32_t* ids_dev, int stride, const std::vector<int32_t>& cu,
              int max_len, bool pool, float* out_dev);
  int forward_dec(const int32_t* ids_dev, int stride, const std::vector<int32_t>& cu,
                  int max_len, bool pool, float* out_dev);
};

static bool needs_q(const rh_weight* w) { return w->mode == RH_MODE_A8W8; }

// Part boundaries: the text whose start is closest to each k·M/n (whole
// texts, at least one per part); at least 2048 rows per part (smaller
// parts' GEMMs lose more than the overlap gains: MiniLM's 2260-row batch
// ran 8 % slower as two parts). Parts after
// the first run on extra streams that wait for everything enqueued on s.
int rh_model::plan_parts(const std::vector<int32_t>& cu, bool allowed, hipStream_t s,
                         std::vector<Part>& parts) {
  const int batch = (int)cu.size() - 1;
  const int M = cu[batch];
  int np = 1;
  if (streams > 1 && allowed) np = std::max(1, std::min({streams, batch, M / 2048}));
  std::vector<int> bounds{0};
  for (int k = 1; k < np; k++) {
    const long target = (long)M * k / np;
    int best = bounds.back() + 1;
    for (int b = best; b <= batch - (np - k); b++)
      if (std::labs(cu[b] - target) < std::labs(cu[best] - target)) best = b;
    bounds.push_back(best);
  }
  bounds.push_back(batch);
  parts.clear();
  if (np > 1) {
    if (!ev_fork) RH_HIP(hipEventCreateWithFlags(&ev_fork, hipEventDisableTiming));
    RH_HIP(hipEventRecord(ev_fork, s));
  }
  for (int k = 0; k < np; k++) {
    hipStream_t ps = s;
    if (k > 0) {
      if (!sx[k]) RH_HIP(hipStreamCreate(&sx[k]));
      if (!ev_join[k]) RH_HIP(hipEventCreateWithFlags(&ev_join[k], hipEventDisableTiming));
      RH_HIP(hipStreamWaitEvent(sx[k], ev_fork, 0));
      ps = sx[k];
    }
    Part p{cu[bounds[k]], cu[bounds[k + 1]] - cu[bounds[k]], bounds[k],
           bounds[k + 1] - bounds[k], 0, ps, k};
    for (int b = bounds[k]; b < bounds[k + 1]; b++) p.max_len = std::max(p.max_len, cu[b + 1] - cu[b]);
    parts.push_back(p);
  }
  return RH_OK;
}

// s waits for every part's stream.
int rh_model::join_parts(const std::vector<Part>& parts, hipStream_t s) {
  for (size_t k = 1; k < parts.size(); k++) {
    RH_HIP(hipEventRecord(ev_join[k], parts[k].s));
    RH_HIP(hipStreamWaitEvent(s, ev_join[k], 0));
  }
  return RH_OK;
}

// Streams and events the parts use, created before a recording (so nothing
// is created while the stream is captured).
int rh_model::ensure_streams() {
  if (!ev_fork) RH_HIP(hipEventCreateWithFlags(&ev_fork, hipEventDisableTiming));
  for (int k = 1; k < streams; k++) {
    if (!sx[k]) RH_HIP(hipStreamCreate(&sx[k]));
    if (!ev_join[k]) RH_HIP(hipEventCreateWithFlags(&ev_join[k], hipEventDisableTiming));
  }
  return RH_OK;
}

// No linear of the BERT-family forward falls back to the context's split
// workspace (full int8, or every input arrives as producer-written planes):
// the condition for parts on streams and for recording the forward.
bool rh_model::bert_no_ws() const {
  bool no_ws = true;
  for (const Layer& L : layers) {
    no_ws = no_ws && !uses_split_ws(L.qkv, planes_in(L.qkv)) &&
            !uses_split_ws(L.o, planes_in(L.o)) && !uses_split_ws(L.f1, planes_in(L.f1)) &&
            !uses_split_ws(L.f2, planes_in(L.f2) && linear_on_planes(ctx, L.f1));
  }
  return no_ws;
}

int rh_model::forward(const int32_t* ids_dev, int stride, const std::vector<int32_t>& cu,
                      int max_len, bool pool, float* out_dev) {
  if (rope_family()) return forward_dec(ids_dev, stride, cu, max_len, pool, out_dev);
  hipStream_t s = ctx->stream;
  const int batch = (int)cu.size() - 1;
  const int M = cu[batch];
  int st = ensure_ws(M, batch, 0);
  if (st) return st;
  // Row offsets: reuse the pinned buffer once its previous copy finished.
  RH_HIP(hipEventSynchronize(cu_evt));
  memcpy(cu_pinned, cu.data(), (batch + 1) * sizeof(int32_t));
  RH_HIP(hipMemcpyAsync(cu_d, cu_pinned, (batch + 1) * sizeof(int32_t),
                        hipMemcpyHostToDevice, s));
  RH_HIP(hipEventRecord(cu_evt, s));
  if (!use_graph || ctx->profiling || !bert_no_ws())
    return forward_bert(ids_dev, stride, cu, max_len, pool, out_dev);
  if (graph.exec && graph.cu == cu && graph.ids == ids_dev && graph.stride == stride &&
      graph.max_len == max_len && graph.pool == pool && graph.out == out_dev &&
      graph.generation == ctx->generation) {
    RH_HIP(hipGraphLaunch(graph.exec, s));
    return RH_OK;
  }
  drop_graph();
  if ((st = ensure_streams())) return st;
  // Record the forward's launches (every part's stream joins the capture
  // through the fork/join events), then replay the graph. The forward has
  // no memset, allocation or host synchronization once the workspace is
  // sized, so the recording holds only kernels and event edges.
  RH_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  st = forward_bert(ids_dev, stride, cu, max_len, pool, out_dev);
  hipGraph_t g = nullptr;
  const hipError_t ec = hipStreamEndCapture(s, &g);
  if (st || ec != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    return st ? st : hip_fail(ec, "forward capture", __FILE__, __LINE__);
  }
  hipGraphExec_t exec = nullptr;
  const hipError_t ei = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (ei != hipSuccess) return hip_fail(ei, "graph instantiate", __FILE__, __LINE__);
  graph.cu = cu;
  graph.ids = ids_dev;
  graph.stride = stride;
  graph.max_len = max_len;
  graph.pool = pool;
  graph.out = out_dev;
  graph.generation = ctx->generation;
  graph.exec = exec;
  RH_HIP(hipGraphLaunch(exec, s));
  return RH_OK;
}

int rh_model::forward_bert(const int32_t* ids_dev, int stride, const std::vector<int32_t>& cu,
                           int max_len, bool pool, float* out_dev) {
  hipStream_t s = ctx->stream;
  const int batch = (int)cu.size() - 1;
  const int M = cu[batch];
  const int H = this->H(), I = this->I();
  const int heads = cfg.heads, dh = H / heads;
  int st;

  // Embeddings + LayerNorm (+ u8 quantization when the first QKV is int8).
  const bool q0 = !layers.empty() && needs_q(layers[0].qkv);
  EmbedArgs ea{};
  ea.ids = ids_dev;
  ea.stride = stride;
  ea.cu = cu_d;
  ea.batch = batch;
  ea.word = word;
  ea.pos = pos;
  ea.type0 = type0;
  ea.gamma = emb_g;
  ea.beta = emb_b;
  ea.H = H;
  ea.vocab = cfg.vocab;
  ea.pos_off = cfg.position_offset;
  ea.eps = eps();
  ea.x = x;
  ea.qa = q0 ? qa : nullptr;
  ea.ldq = ldq_for(H);
  ea.row_scales = q0 ? rs : nullptr;
  ea.err_flag = err_d;
  ea.exact = exact;
  // the first QKV's planes, when it takes them
  const bool p0 = !layers.empty() && planes_in(layers[0].qkv);
  if (p0) {
    const Planes pq = plane(0, layers[0].qkv);
    ea.ph = pq.hi;
    ea.pl = pq.lo;
    ea.ldp = pq.ld;
  }
  RH_HIP(launch_embed_layernorm(ea, M, s));

  // Parts (see plan_parts): allowed when no linear falls back to the
  // context's split workspace.
  std::vector<Part> parts;
  if ((st = plan_parts(cu, bert_no_ws(), s, parts))) return st;
  auto part_attn_ops = [&](const Part& P) {
    double ops = 0;
    for (int b = P.b0; b < P.b0 + P.nb; b++) {
      const double L = cu[b + 1] - cu[b];
      ops += 4.0 * L * L * dh * heads;
    }
    return ops;
  };

  // p0 holds planes of x for the next QKV when its producer (the embedding
  // LayerNorm, then each layer's residual+LN) wrote them.
  bool x_planes = p0;
  auto layer = [&](size_t li, const Part& P) -> int {
    const Layer& L = layers[li];
    const hipStream_t ps = P.s;
    const int Mp = P.rows;
    const double MH = Mp;
    const size_t r0 = P.row0;
    float* xp = x + r0 * H;
    float* yp = y + r0 * H;
    float* hidp = hid + r0 * I;
    float* ctxp = ctxb + r0 * H;
    uint8_t* qap = qa + r0 * ldq_for(H);
    uint8_t* qa2p = qa2 + r0 * ldq_for(I);
    float* rsp = rs + r0;
    float* rs2p = rs2 + r0;
    auto at = [&](Planes p) {  // this part's rows of a planes buffer
      if (p.hi) p.hi += r0 * p.ld;
      if (p.lo) p.lo += r0 * p.ld;
      return p;
    };
    int st;
    // QKV projection. x was quantized into qa/rs by the producer if the
    // weight is full-int8. When attention runs on bf16 operands, a full-int8
    // QKV writes bf16 directly (attention would round the fp32 values to the
    // same bf16 on load), halving the write.
    // With fp32-grade attention it writes the rows' bf16 hi/lo split as two
    // planes (the same bytes as fp32 rows), which attention stages without a
    // conversion: hi in qkvh, lo in the fp32 q|k|v buffer's first half.
    // A weight-only int8 / fp32 q|k|v linear on bf16 planes writes the same
    // split through its planes epilogue.
    const bool qkv_bf16 = needs_q(L.qkv) && attn_precision == 1 && !exact;
    const bool qkv_planes = attn_precision == 3 && !exact && dh <= 128 &&
                            (needs_q(L.qkv) || linear_on_planes(ctx, L.qkv));
    __bf16* qkv_lo = reinterpret_cast<__bf16*>(qkv);
    if (qkv_bf16) {
      st = run_gemm_i8(ctx, L.qkv, qap, ldq_for(H), rsp, Mp, EPI_BF16, qkvh + r0 * 3 * H,
                       3 * H, ACT_NONE, L.qkv->d_bias, nullptr, nullptr, 2.0 * MH * H * 3 * H);
    } else if (qkv_planes && needs_q(L.qkv)) {
      st = run_gemm_i8(ctx, L.qkv, qap, ldq_for(H), rsp, Mp, EPI_PLANES, qkvh + r0 * 3 * H,
                       3 * H, ACT_NONE, L.qkv->d_bias, nullptr, nullptr, 2.0 * MH * H * 3 * H,
                       qkv_lo + r0 * 3 * H);
    } else if (qkv_planes) {
      const Planes pq = at(plane(0, L.qkv));
      const Planes pout{qkvh + r0 * 3 * H, qkv_lo + r0 * 3 * H, 3 * H};
      st = run_linear(ctx, L.qkv, xp, H, Mp, nullptr, 3 * H, ACT_NONE, L.qkv->d_bias, qap,
                      ldq_for(H), rsp, false, x_planes ? &pq : nullptr, &pout);
    } else {
      const Planes pq = at(plane(0, L.qkv));
      st = run_linear(ctx, L.qkv, xp, H, Mp, qkv + r0 * 3 * H, 3 * H, ACT_NONE, L.qkv->d_bias,
                      qap, ldq_for(H), rsp, false, x_planes ? &pq : nullptr);
    }
    if (st) return st;
    AttnArgs aa{};
    aa.qkv = qkv_bf16 || qkv_planes ? (const void*)qkvh : (const void*)qkv;  // absolute rows
    aa.qkv_lo = qkv_planes ? qkv_lo : nullptr;
    aa.in_bf16 = qkv_bf16 ? 1 : (qkv_planes ? 2 : 0);
    aa.ldqkv = 3 * H;
    aa.q_off = 0;
    aa.k_off = H;
    aa.v_off = 2 * H;
    aa.cu = cu_d + P.b0;
    aa.batch = P.nb;
    aa.max_len = P.max_len;
    aa.heads = heads;
    aa.kv_heads = heads;
    aa.dh = dh;
    aa.scale = (float)(1.0 / std::sqrt((double)dh));
    aa.rel_bias = rel_bias;
    aa.rel_center = max_seq() - 1;
    // the attention output goes straight to the output projection's planes
    // when it takes them (absolute rows, like the q|k|v rows)
    const bool po = planes_in(L.o);
    const Planes pov = plane(0, L.o);
    aa.ctx = po ? nullptr : ctxb;
    aa.ctx_hi = po ? pov.hi : nullptr;
    aa.ctx_lo = po ? pov.lo : nullptr;
    aa.ldctx = po ? pov.ld : H;
    int slot = -1;
    RH_HIP(ctx->prof_begin(3, part_attn_ops(P), 0.0, &slot));
    if (exact) RH_HIP(launch_attention_exact(aa, ps));
    else RH_HIP(launch_attention(aa, attn_precision, ps));
    RH_HIP(ctx->prof_end(slot));
    const Planes povp = at(pov);
    const bool qf1 = needs_q(L.f1);
    const bool pf1 = planes_in(L.f1);
    const Planes pf1v = at(plane(0, L.f1));
    if (fuse_ln(L.o, pf1) && !po) {
      // x = LayerNorm(x + O(ctx)) (+ FFN1's u8 rows) in the projection's
      // epilogue; the u8 rows may overwrite the projection's own input rows
      RH_HIP(launch_quantize_rows_u8(ctxp, H, Mp, H, qap, ldq_for(H), rsp, ps));
      st = run_gemm_i8_ln(ctx, L.o, qap, ldq_for(H), rsp, Mp,
                          ln_args(xp, L.ln1_g, L.ln1_b, qf1 ? qap : nullptr, ldq_for(H),
                                  qf1 ? rsp : nullptr),
                          2.0 * MH * H * H);
      if (st) return st;
    } else {
      st = run_linear(ctx, L.o, ctxp, H, Mp, yp, H, ACT_NONE, L.o->d_bias, qap, ldq_for(H),
                      rsp, needs_q(L.o) && !po, po ? &povp : nullptr);
      if (st) return st;
      RH_HIP(launch_add_layernorm(xp, yp, H, L.ln1_g, L.ln1_b, Mp, H, eps(),
                                  qf1 ? qap : nullptr, ldq_for(H), qf1 ? rsp : nullptr, ps,
                                  pf1 ? pf1v.hi : nullptr, pf1 ? pf1v.lo : nullptr, pf1v.ld,
                                  exact));
    }
    const bool last = li + 1 == layers.size();
    const bool qn = !last && needs_q(layers[li + 1].qkv);
    const bool xn_planes = !last && planes_in(layers[li + 1].qkv);
    const Planes pnv = last ? Planes{} : at(plane(0, layers[li + 1].qkv));
    // FFN2 finishes the layer (residual + LayerNorm + next QKV's u8 rows) in
    // its epilogue on the split full-int8 path
    const bool fused_ln2 = !(fused_ffn1 == 1 && qf1 && needs_q(L.f2)) && qf1 &&
                           needs_q(L.f2) && fuse_ln(L.f2, xn_planes);
    if (fused_ffn1 == 1 && qf1 && needs_q(L.f2)) {
      // FFN1 + GELU + QuantizeRowU8 without the fp32 intermediate: pass 1
      // finds each row's |max| of the GELU output, pass 2 recomputes the
      // identical values and writes the u8 bytes and row scales FFN2 reads.
      // Both passes see the same int32 accumulators, so the bytes equal
      // QuantizeRowU8 of the fp32 GELU row (bert.go:910-916).
      const double ops1 = 2.0 * MH * H * I;
      float* amx = absmax + r0;
      RH_HIP(launch_fill_zero(amx, Mp, ps));
      st = run_gemm_i8(ctx, L.f1, qap, ldq_for(H), rsp, Mp, EPI_ABSMAX, nullptr, 0, ACT_GELU,
                       L.f1->d_bias, amx, nullptr, ops1);
      if (st) return st;
      st = run_gemm_i8(ctx, L.f1, qap, ldq_for(H), rsp, Mp, EPI_QUANT, qa2p, ldq_for(I),
                       ACT_GELU, L.f1->d_bias, amx, rs2p, 0.0);
      if (st) return st;
      st = run_gemm_i8(ctx, L.f2, qa2p, ldq_for(I), rs2p, Mp, EPI_F32, yp, H, ACT_NONE,
                       L.f2->d_bias, nullptr, nullptr, 2.0 * MH * I * H);
      if (st) return st;
    } else if (qf1 && needs_q(L.f2)) {
      // FFN1 writes the fp32 pre-activation (dequant + bias); GELU moves into
      // FFN2's row quantizer, which has VALU to spare where the GEMM
      // epilogue does not. Same float32 operations in the same order as
      // GELU(dense(x)) then QuantizeRowU8 (bert.go:910-916).
      if (fused_ffn1 == 2 && I <= 256 * kQsyncMaxTiles) {
        // one pass: FFN1's workgroups exchange the GELU rows' |max| per row
        // block and write the u8 bytes and row scales (EPI_QSYNC), the same
        // bytes as the two kernels below
        st = run_gemm_i8(ctx, L.f1, qap, ldq_for(H), rsp, Mp, EPI_QSYNC, qa2p, ldq_for(I),
                         ACT_GELU, L.f1->d_bias, nullptr, rs2p, 2.0 * MH * H * I, nullptr,
                         qsync + 1 + (size_t)P.idx * qsync_stride,
                         qslots + r0 * kQsyncMaxTiles, kQsyncMaxTiles, qsync);
        if (st) return st;
      } else {
        st = run_linear(ctx, L.f1, xp, H, Mp, hidp, I, ACT_NONE, L.f1->d_bias, qap,
                        ldq_for(H), rsp, false);
        if (st) return st;
        RH_HIP(launch_quantize_rows_u8(hidp, I, Mp, I, qa2p, ldq_for(I), rs2p, ps, ACT_GELU));
      }
      if (fused_ln2) {
        st = run_gemm_i8_ln(ctx, L.f2, qa2p, ldq_for(I), rs2p, Mp,
                            ln_args(xp, L.ln2_g, L.ln2_b, qn ? qap : nullptr, ldq_for(H),
                                    qn ? rsp : nullptr),
                            2.0 * MH * I * H);
      } else {
        st = run_linear(ctx, L.f2, hidp, I, Mp, yp, H, ACT_NONE, L.f2->d_bias, qa2p,
                        ldq_for(I), rs2p, false);
      }
      if (st) return st;
    } else {
      // FFN1's GELU output goes to FFN2's planes when FFN2 takes them
      const bool pf2 = planes_in(L.f2) && linear_on_planes(ctx, L.f1);
      const Planes pf2v = at(plane(1, L.f2));
      st = run_linear(ctx, L.f1, xp, H, Mp, hidp, I, ACT_GELU, L.f1->d_bias, qap, ldq_for(H),
                      rsp, false, pf1 ? &pf1v : nullptr, pf2 ? &pf2v : nullptr);
      if (st) return st;
      st = run_linear(ctx, L.f2, hidp, I, Mp, yp, H, ACT_NONE, L.f2->d_bias, qa2p,
                      ldq_for(I), rs2p, needs_q(L.f2) && !pf2, pf2 ? &pf2v : nullptr);
      if (st) return st;
    }
    if (!fused_ln2) {
      RH_HIP(launch_add_layernorm(xp, yp, H, L.ln2_g, L.ln2_b, Mp, H, eps(),
                                  qn ? qap : nullptr, ldq_for(H), qn ? rsp : nullptr, ps,
                                  xn_planes ? pnv.hi : nullptr, xn_planes ? pnv.lo : nullptr,
                                  pnv.ld, exact));
    }
    return RH_OK;
  };
  // run_linear / run_gemm_i8 launch on ctx->stream: point it at each part's
  // stream while that part's work is enqueued (the context's mutex is held)
  const hipStream_t s_ctx = ctx->stream;
  for (size_t li = 0; li < layers.size(); li++) {
    for (const Part& P : parts) {
      ctx->stream = P.s;
      st = layer(li, P);
      if (st) break;
    }
    ctx->stream = s_ctx;
    if (st) break;
    x_planes = li + 1 < layers.size() && planes_in(layers[li + 1].qkv);
  }
  // join even after a failed launch: work already enqueued on the parts'
  // streams must be ordered before anything the caller does next on s
  // (buffer reuse, ensure_ws's sync-and-free)
  const int jst = join_parts(parts, s);
  if (st) return st;
  if ((st = jst)) return st;
  if (pool) {
    RH_HIP(launch_pool(x, H, cu_d, batch, cfg.pooling, cfg.normalize, out_dev, s));
  }
  return RH_OK;
}


// encodeQwen3 (qwen3.go:395-548) / encodeGemma3 (gemma3.go:206-384) /
// encodeNomic (nomic.go:113-250) / encodeModernBERT (modernbert.go:148-311)
// over the packed batch, then ForwardWorkers' pooling (bert.go:657-689).
// The four share one layer loop: fused q|k|v, (QK-norm +) RoPE, attention,
// output projection, a residual + norm, the gated MLP, a residual + norm.
// What differs is the norm (RMSNorm / LayerNorm), where it sits (pre-norm:
// the norm's output feeds the next GEMM and x keeps the sum; nomic's
// post-norm: x itself is normalized and feeds the next GEMM), the attention
// mask and scale, and the gate activation.
int rh_model::forward_dec(const int32_t* ids_dev, int stride, const std::vector<int32_t>& cu,
                          int max_len, bool pool, float* out_dev) {
  hipStream_t s = ctx->stream;
  const int batch = (int)cu.size() - 1;
  const int M = cu[batch];
  const int H = this->H(), I = this->I();
  const int qd = qdim(), kvd = kvdim(), qkvw = qkv_width();
  int st = ensure_ws(M, batch, 0);
  if (st) return st;
  RH_HIP(hipEventSynchronize(cu_evt));
  memcpy(cu_pinned, cu.data(), (batch + 1) * sizeof(int32_t));
  RH_HIP(hipMemcpyAsync(cu_d, cu_pinned, (batch + 1) * sizeof(int32_t),
                        hipMemcpyHostToDevice, s));
  RH_HIP(hipEventRecord(cu_evt, s));

  const float emb_scale = gemma() ? (float)std::sqrt((double)H) : 1.0f;
  // nomic adds the segment-0 row (type0 is null for the others)
  RH_HIP(launch_embed_gather(ids_dev, stride, cu_d, batch, word, type0, H, cfg.vocab,
                             emb_scale, x, pos_d, err_d, M, s));
  const float e = eps();
  const bool ln = layer_norm(), post = nomic();
  const int ldqH = ldq_for(std::max(H, qd)), ldqI = ldq_for(I);
  // this part's rows of a planes buffer
  auto at = [](Planes p, size_t r0) {
    if (p.hi) p.hi += r0 * p.ld;
    if (p.lo) p.lo += r0 * p.ld;
    return p;
  };
  // The norms write what the next GEMM reads: its bf16 planes or its u8
  // rows (RmsArgs), and fp32 rows: x itself when in_place (nomic's post-norm
  // blocks, the embedding norm of nomic and ModernBERT, the final norm),
  // else `normed` unless the planes replace them; rows [r0, r0 + m).
  auto norm_to = [&](size_t r0, int m, hipStream_t ps, const float* yy, const float* post_g,
                     const float* pre, const float* pre_b, const rh_weight* next,
                     bool in_place) {
    RmsArgs ra{};
    ra.x = x + r0 * H;
    ra.y = yy ? yy + r0 * H : nullptr;
    ra.post_g = post_g;
    ra.pre_g = pre;
    ra.layer_norm = ln ? 1 : 0;
    ra.ln_b = pre_b;
    ra.m = m;
    ra.H = H;
    ra.eps = e;
    const bool pl = planes_in(next);
    if (in_place) ra.out = ra.x;
    else if (!pl) ra.out = normed + r0 * H;
    if (pl) {
      const Planes p = at(plane(0, next), r0);
      ra.ph = p.hi;
      ra.pl = p.lo;
      ra.ldp = p.ld;
    }
    if (next && needs_q(next)) {
      ra.qa = qa + r0 * ldqH;
      ra.ldq = ldqH;
      ra.row_scales = rs + r0;
    }
    return launch_rms_residual(ra, ps);
  };
  if (ln) {  // LayerNorm(x) in place: the embedding norm (nomic.go:176, modernbert.go:211)
    RH_HIP(norm_to(0, M, s, nullptr, nullptr, emb_g, emb_b, dlayers[0].qkv, true));
  } else {
    RH_HIP(norm_to(0, M, s, nullptr, nullptr, dlayers[0].in_norm, nullptr, dlayers[0].qkv,
                   false));
  }

  // Parts (see plan_parts): allowed when no linear falls back to the
  // context's split workspace.
  bool no_ws = true;
  auto ws = [&](const rh_weight* w, bool pin) { return w && uses_split_ws(w, pin); };
  for (const DecLayer& L : dlayers) {
    // separate q/k/v/gate/up weights take fp32 rows (no producer planes)
    no_ws = no_ws && !ws(L.qkv, planes_in(L.qkv)) && !ws(L.q, false) && !ws(L.k, false) &&
            !ws(L.v, false) && !ws(L.o, planes_in(L.o)) && !ws(L.gu, planes_in(L.gu)) &&
            !ws(L.gate, false) && !ws(L.up, false) &&
            !ws(L.down, L.gu && planes_in(L.down) && linear_on_planes(ctx, L.gu));
  }
  std::vector<Part> parts;
  if ((st = plan_parts(cu, no_ws, s, parts))) return st;
  const int glu = gemma() ? ACT_GEGLU : modernbert() ? ACT_GEGLU_ERF : ACT_SWIGLU;
  auto layer = [&](size_t li, const Part& P) -> int {
    const DecLayer& L = dlayers[li];
    const hipStream_t ps = P.s;
    const int Mp = P.rows;
    const size_t r0 = P.row0;
    float* normedp = normed + r0 * H;
    float* qkvp = qkv + r0 * qkvw;
    float* yp = y + r0 * H;
    float* hidp = hid + r0 * I;
    uint8_t* qap = qa + r0 * ldqH;
    uint8_t* qa2p = qa2 + r0 * ldqI;
    float* rsp = rs + r0;
    float* rs2p = rs2 + r0;
    float* xp = x + r0 * H;
    // the fp32 rows the projections read: x itself after nomic's post-norms
    // and for ModernBERT's layer 0 (its attention norm is an identity,
    // modernbert.go:229-236), else the pre-norm's output
    const float* attn_in = post || (modernbert() && li == 0) ? xp : normedp;
    const float* mlp_in = post ? xp : normedp;
    int st;
    // attention block: fused q|k|v, QK-norm + RoPE, GQA attention, o_proj
    const Planes pq = at(plane(0, L.qkv), r0);
    const bool local = (gemma() || modernbert()) && !L.global;
    // bf16 attention reads bf16 q|k|v rows: written by the q|k|v GEMM's
    // QK-norm + RoPE epilogue where that applies, else by the separate pass
    const bool hb = attn_precision == 1;
    bool fused_qk = false;
    if (qk_epilogue && hb && L.qkv && L.q_norm && planes_in(L.qkv)) {
      const QkEpilogue q{L.q_norm, L.k_norm, local ? cos_l : cos_g, local ? sin_l : sin_g,
                         pos_d + r0, nq(), nkv(), dh(), e};
      st = run_linear_qk(ctx, L.qkv, pq, Mp, q, qkvh + r0 * qkvw, qkvw, &fused_qk);
      if (st) return st;
    }
    if (!fused_qk && L.qkv) {
      st = run_linear(ctx, L.qkv, attn_in, H, Mp, qkvp, qkvw, ACT_NONE, nullptr, qap, ldqH,
                      rsp, false, planes_in(L.qkv) ? &pq : nullptr);
      if (st) return st;
    } else if (!fused_qk) {
      // q, k, v in different modes: three GEMMs over the fp32 normed rows,
      // each writing its columns of the q|k|v rows
      const rh_weight* sep[3] = {L.q, L.k, L.v};
      const int col[3] = {0, qd, qd + kvd};
      for (int j = 0; j < 3; j++) {
        st = run_linear(ctx, sep[j], attn_in, H, Mp, qkvp + col[j], qkvw, ACT_NONE, nullptr,
                        qap, ldqH, rsp, needs_q(sep[j]));
        if (st) return st;
      }
    }
    if (!fused_qk) {
      RH_HIP(launch_qk_norm_rope(qkvp, qkvw, Mp, nq(), nkv(), dh(), L.q_norm, L.k_norm, e,
                                 local ? cos_l : cos_g, local ? sin_l : sin_g, pos_d + r0,
                                 hb ? qkvh + r0 * qkvw : nullptr, ps));
    }
    AttnArgs aa{};
    aa.qkv = hb ? (const void*)qkvh : (const void*)qkv;  // rows are absolute (cu)
    aa.in_bf16 = hb ? 1 : 0;
    aa.ldqkv = qkvw;
    aa.q_off = 0;
    aa.k_off = qd;
    aa.v_off = qd + kvd;
    aa.cu = cu_d + P.b0;
    aa.batch = P.nb;
    aa.max_len = P.max_len;
    aa.heads = nq();
    aa.kv_heads = nkv();
    aa.dh = dh();
    aa.scale = gemma() ? (float)(1.0 / std::sqrt((double)cfg.query_pre_attn_scalar))
                       : (float)(1.0 / std::sqrt((double)dh()));
    // the attention output goes straight to o_proj's planes when it takes
    // them (absolute rows, like the q|k|v rows)
    const bool po = planes_in(L.o);
    const Planes pov = plane(0, L.o);
    aa.ctx = po ? nullptr : ctxb;
    aa.ctx_hi = po ? pov.hi : nullptr;
    aa.ctx_lo = po ? pov.lo : nullptr;
    aa.ldctx = po ? pov.ld : qd;
    aa.causal = cfg.arch == RH_ARCH_QWEN3 ? 1 : 0;
    // the kernel keeps keys with |i - j| < window: Gemma's sliding_window as
    // is (gemma3.go:331-351), ModernBERT's |i - j| <= local_attention / 2
    // (modernbert.go:156,264-273) as local_attention / 2 + 1
    aa.window = !local ? 0 : modernbert() ? cfg.sliding_window / 2 + 1 : cfg.sliding_window;
    double attn_ops = 0;
    for (int b = P.b0; b < P.b0 + P.nb; b++) {
      const double Lb = cu[b + 1] - cu[b];
      attn_ops += 4.0 * Lb * Lb * dh() * nq() * (cfg.arch == RH_ARCH_QWEN3 ? 0.5 : 1.0);
    }
    int slot = -1;
    RH_HIP(ctx->prof_begin(3, attn_ops, 0.0, &slot));
    RH_HIP(launch_attention(aa, attn_precision, ps));
    RH_HIP(ctx->prof_end(slot));
    const Planes povp = at(pov, r0);
    st = run_linear(ctx, L.o, ctxb + r0 * qd, qd, Mp, yp, H, ACT_NONE, nullptr, qap, ldqH, rsp,
                    needs_q(L.o) && !po, po ? &povp : nullptr);
    if (st) return st;
    // x += [RMSNorm(attn, post_attn)]; normed = norm(x, pre-MLP norm), or
    // nomic's x = LayerNorm(x + attn, norm1) (nomic.go:226-227)
    RH_HIP(norm_to(r0, Mp, ps, y, gemma() ? L.post_attn : nullptr,
                   gemma() ? L.pre_ffn : L.post_attn, L.post_attn_b, L.gu, post));
    // gated MLP: one GEMM over gate|up writes act(gate) * up (as the down
    // projection's planes when it takes them), then down
    if (L.gu) {
      const Planes pg = at(plane(0, L.gu), r0), pd = at(plane(1, L.down), r0);
      const bool pdown = planes_in(L.down) && linear_on_planes(ctx, L.gu);
      st = run_linear(ctx, L.gu, mlp_in, H, Mp, hidp, I, glu, nullptr, qap, ldqH, rsp, false,
                      planes_in(L.gu) ? &pg : nullptr, pdown ? &pd : nullptr);
      if (st) return st;
      st = run_linear(ctx, L.down, hidp, I, Mp, yp, H, ACT_NONE, nullptr, qa2p, ldqI, rs2p,
                      needs_q(L.down), pdown ? &pd : nullptr);
      if (st) return st;
    } else {
      // gate and up in different modes: two GEMMs, the glue, then down
      float* hid2p = hid2 + r0 * I;
      st = run_linear(ctx, L.gate, mlp_in, H, Mp, hidp, I, ACT_NONE, nullptr, qap, ldqH, rsp,
                      needs_q(L.gate));
      if (st) return st;
      st = run_linear(ctx, L.up, mlp_in, H, Mp, hid2p, I, ACT_NONE, nullptr, qap, ldqH, rsp,
                      needs_q(L.up));
      if (st) return st;
      RH_HIP(launch_glu_rows(hidp, hid2p, hidp, (size_t)Mp * I, glu, ps));
      st = run_linear(ctx, L.down, hidp, I, Mp, yp, H, ACT_NONE, nullptr, qa2p, ldqI, rs2p,
                      needs_q(L.down));
      if (st) return st;
    }
    // x += [RMSNorm(mlp, post_ffn)]; then the next layer's input norm, or the
    // final norm in place (qwen3.go:543, gemma3.go:379, modernbert.go:307);
    // nomic: x = LayerNorm(x + mlp, norm2), its last one the final norm
    // (nomic.go:244-245)
    const bool last = li + 1 == dlayers.size();
    const rh_weight* next = last ? nullptr : dlayers[li + 1].qkv;
    if (post) {
      RH_HIP(norm_to(r0, Mp, ps, y, nullptr, L.post_ffn, L.post_ffn_b, next, true));
    } else {
      RH_HIP(norm_to(r0, Mp, ps, y, gemma() ? L.post_ffn : nullptr,
                     last ? final_norm : dlayers[li + 1].in_norm, nullptr, next, last));
    }
    return RH_OK;
  };
  // run_linear launches on ctx->stream: point it at each part's stream
  // while that part's work is enqueued (the context's mutex is held)
  const hipStream_t s_ctx = ctx->stream;
  for (size_t li = 0; li < dlayers.size(); li++) {
    for (const Part& P : parts) {
      ctx->stream = P.s;
      st = layer(li, P);
      if (st) break;
    }
    ctx->stream = s_ctx;
    if (st) break;
  }
  // join even after a failed launch (see the encoder's forward)
  const int jst = join_parts(parts, s);
  if (st) return st;
  if ((st = jst)) return st;
  if (pool) {
    if (gemma() && dense1 && dense2) {
      RH_HIP(launch_pool(x, H, cu_d, batch, cfg.pooling, 0, pooled, s));
      RH_HIP(launch_dense_head(pooled, batch, H, cfg.dense_hidden, dense1, dense2, cfg.normalize,
                               dense_hid, out_dev, s));
    } else {
      RH_HIP(launch_pool(x, H, cu_d, batch, cfg.pooling, cfg.normalize, out_dev, s));
    }
  }
  return RH_OK;
}

// ---- tensor bookkeeping ----------------------------------------------------------

static const char* kPrefixes[] = {"", "bert.", "roberta.", "mpnet.", "distilbert."};

static int find_tensor(rh_model* m, const std::string& prefix, const std::string& name,
                       std::initializer_list<int64_t> shape, const HostTensor** out) {
  auto it = m->pending.find(prefix + name);
  char buf[256];
  if (it == m->pending.end()) {
    snprintf(buf, sizeof buf, "missing tensor \"%s\"", (prefix + name).c_str());
    return fail(RH_ERR_MISSING, buf);
  }
  const HostTensor& t = it->second;
  bool ok = t.shape.size() == shape.size();
  size_t i = 0;
  for (int64_t d : shape) {
    if (!ok) break;
    if (d >= 0 && t.shape[i] != d) ok = false;
    i++;
  }
  if (!ok) {
    snprintf(buf, sizeof buf, "tensor \"%s\" has the wrong shape", (prefix + name).c_str());
    return fail(RH_ERR_MISSING, buf);
  }
  *out = &t;
  return RH_OK;
}

static int upload(const float* src, size_t n, float** dst) {
  RH_HIP(hipMalloc((void**)dst, n * sizeof(float)));
  RH_HIP(hipMemcpy(*dst, src, n * sizeof(float), hipMemcpyHostToDevice));
  return RH_OK;
}

// A packer's refusal (bad shape, non-finite weight) sends newDense to the
// next mode; anything else (device allocation, HIP, host memory) is the
// caller's error and ends the load.
static bool pack_refused(int st) { return st == RH_ERR_SHAPE || st == RH_ERR_NONFINITE; }

// newDense (bert.go:263-278): requested mode, then the fallback chain
// A8W8 -> W8 -> F32 when the packer refuses the matrix.
static int new_dense(rh_model* m, const float* raw, const float* bias, int in, int out,
                     rh_weight** w) {
  int st;
  if (m->quant == RH_QUANT_FULL) {
    st = pack_weight(m->ctx, RH_MODE_A8W8, raw, bias, in, out, w);
    if (!pack_refused(st)) return st;
  }
  if (m->quant >= RH_QUANT_WEIGHTS) {
    st = pack_weight(m->ctx, RH_MODE_W8, raw, bias, in, out, w);
    if (!pack_refused(st)) return st;
  }
  // PackB, then the unpacked weights (bert.go:274-277)
  return pack_weight(m->ctx, RH_MODE_F32, raw, bias, in, out, w, true);
}

// The mode newDense ends at for one matrix: the requested one unless its
// packer refuses the matrix, then the next (bert.go:263-278).
static int dense_mode(const rh_model* m, const float* raw, int in, int out) {
  if (m->quant == RH_QUANT_FULL && pack_check(RH_MODE_A8W8, raw, in, out) == RH_OK)
    return RH_MODE_A8W8;
  if (m->quant >= RH_QUANT_WEIGHTS && pack_check(RH_MODE_W8, raw, in, out) == RH_OK)
    return RH_MODE_W8;
  return RH_MODE_F32;
}

// relPosBucket (bert.go:123-150), HF's relative_position_bucket with
// max_distance 128: n = -(j - i); the sign picks the table half; |n| below
// half/2 keeps its own bucket, larger distances share log-spaced buckets
// (float64 log), clamped to the half's last.
static int rel_pos_bucket(int rel, int buckets) {
  int n = -rel, ret = 0;
  const int half = buckets / 2, exact = half / 2;
  if (n < 0) {
    ret = half;
    n = -n;
  }
  if (n < exact) return ret + n;
  const int v = exact + (int)(std::log((double)n / exact) / std::log(128.0 / exact) *
                              (double)(half - exact));
  return ret + std::min(v, half - 1);
}

// Load (bert.go:307-524) for BERT / RoBERTa, DistilBERT and MPNet: the same
// post-LN layers under each one's tensor names (bert.go:399-470); only BERT
// and RoBERTa have a token-type table (row 0 used); MPNet adds one shared
// [buckets][heads] relative-position bias table (bert.go:511-519), expanded
// here once into the per-head table over every relative position a text can
// have (the reference rebuilds its [heads][2 seq - 1] slice per forward,
// bert.go:816-830).
static int finalize_bert(rh_model* m) {
  const int H = m->cfg.hidden, I = m->cfg.intermediate;
  const bool distil = m->cfg.arch == RH_ARCH_DISTILBERT, mpnet = m->cfg.arch == RH_ARCH_MPNET;
  std::string prefix;
  for (const char* p : kPrefixes)
    if (m->pending.count(std::string(p) + "embeddings.word_embeddings.weight")) prefix = p;
  const HostTensor *we, *pe, *tt = nullptr, *eg, *eb;
  int st;
  if ((st = find_tensor(m, prefix, "embeddings.word_embeddings.weight", {m->cfg.vocab, H}, &we)))
    return st;
  if ((st = find_tensor(m, prefix, "embeddings.position_embeddings.weight",
                        {m->cfg.max_position, H}, &pe)))
    return st;
  if (!distil && !mpnet) {
    if ((st = find_tensor(m, prefix, "embeddings.token_type_embeddings.weight", {-1, H}, &tt)))
      return st;
    if (tt->shape[0] < 1) return fail(RH_ERR_MISSING, "token_type_embeddings has no rows");
  }
  if ((st = find_tensor(m, prefix, "embeddings.LayerNorm.weight", {H}, &eg))) return st;
  if ((st = find_tensor(m, prefix, "embeddings.LayerNorm.bias", {H}, &eb))) return st;
  if ((st = upload(we->data.data(), we->data.size(), &m->word))) return st;
  if ((st = upload(pe->data.data(), pe->data.size(), &m->pos))) return st;
  if (tt && (st = upload(tt->data.data(), H, &m->type0))) return st;
  if ((st = upload(eg->data.data(), H, &m->emb_g))) return st;
  if ((st = upload(eb->data.data(), H, &m->emb_b))) return st;
  if (mpnet) {
    const int nb = m->cfg.rel_buckets, heads = m->cfg.heads, L = m->max_seq();
    const HostTensor* rb;
    if ((st = find_tensor(m, prefix, "encoder.relative_attention_bias.weight", {nb, heads}, &rb)))
      return st;
    const int nd = 2 * L - 1;
    std::vector<float> tab((size_t)heads * nd);
    for (int d = -(L - 1); d <= L - 1; d++) {
      const int b = rel_pos_bucket(d, nb);
      for (int h = 0; h < heads; h++) tab[(size_t)h * nd + d + L - 1] = rb->data[(size_t)b * heads + h];
    }
    if ((st = upload(tab.data(), tab.size(), &m->rel_bias))) return st;
  }

  // tensor names per layer: BERT / RoBERTa, DistilBERT, MPNet
  struct Names {
    const char *q, *qb, *k, *kb, *v, *vb, *o, *ob, *g1, *b1, *f1, *f1b, *f2, *f2b, *g2, *b2;
  };
  static const Names kBert = {"attention.self.query.weight", "attention.self.query.bias",
                              "attention.self.key.weight", "attention.self.key.bias",
                              "attention.self.value.weight", "attention.self.value.bias",
                              "attention.output.dense.weight", "attention.output.dense.bias",
                              "attention.output.LayerNorm.weight", "attention.output.LayerNorm.bias",
                              "intermediate.dense.weight", "intermediate.dense.bias",
                              "output.dense.weight", "output.dense.bias",
                              "output.LayerNorm.weight", "output.LayerNorm.bias"};
  static const Names kDistil = {"attention.q_lin.weight", "attention.q_lin.bias",
                                "attention.k_lin.weight", "attention.k_lin.bias",
                                "attention.v_lin.weight", "attention.v_lin.bias",
                                "attention.out_lin.weight", "attention.out_lin.bias",
                                "sa_layer_norm.weight", "sa_layer_norm.bias",
                                "ffn.lin1.weight", "ffn.lin1.bias", "ffn.lin2.weight",
                                "ffn.lin2.bias", "output_layer_norm.weight",
                                "output_layer_norm.bias"};
  static const Names kMpnet = {"attention.attn.q.weight", "attention.attn.q.bias",
                               "attention.attn.k.weight", "attention.attn.k.bias",
                               "attention.attn.v.weight", "attention.attn.v.bias",
                               "attention.attn.o.weight", "attention.attn.o.bias",
                               "attention.LayerNorm.weight", "attention.LayerNorm.bias",
                               "intermediate.dense.weight", "intermediate.dense.bias",
                               "output.dense.weight", "output.dense.bias",
                               "output.LayerNorm.weight", "output.LayerNorm.bias"};
  const Names& nm = distil ? kDistil : (mpnet ? kMpnet : kBert);

  m->layers.resize(m->cfg.layers);
  for (int l = 0; l < m->cfg.layers; l++) {
    char p[64];
    snprintf(p, sizeof p, distil ? "transformer.layer.%d." : "encoder.layer.%d.", l);
    const std::string lp = p;
    const HostTensor *qw, *qb, *kw, *kb, *vw, *vb, *ow, *ob, *g1, *b1, *f1w, *f1b, *f2w,
        *f2b, *g2, *b2;
    struct Need {
      const char* name;
      std::initializer_list<int64_t> shape;
      const HostTensor** dst;
    };
    const Need needs[] = {
        {nm.q, {H, H}, &qw},   {nm.qb, {H}, &qb},   {nm.k, {H, H}, &kw},   {nm.kb, {H}, &kb},
        {nm.v, {H, H}, &vw},   {nm.vb, {H}, &vb},   {nm.o, {H, H}, &ow},   {nm.ob, {H}, &ob},
        {nm.g1, {H}, &g1},     {nm.b1, {H}, &b1},   {nm.f1, {I, H}, &f1w}, {nm.f1b, {I}, &f1b},
        {nm.f2, {H, I}, &f2w}, {nm.f2b, {H}, &f2b}, {nm.g2, {H}, &g2},     {nm.b2, {H}, &b2},
    };
    for (const Need& n : needs)
      if ((st = find_tensor(m, prefix, lp + n.name, n.shape, n.dst))) return st;
    // Fuse Q|K|V rows into [3H][H] and the biases into [3H] (bert.go:479-485).
    std::vector<float> qkvw((size_t)3 * H * H), qkvb((size_t)3 * H);
    memcpy(qkvw.data(), qw->data.data(), sizeof(float) * H * H);
    memcpy(qkvw.data() + (size_t)H * H, kw->data.data(), sizeof(float) * H * H);
    memcpy(qkvw.data() + (size_t)2 * H * H, vw->data.data(), sizeof(float) * H * H);
    memcpy(qkvb.data(), qb->data.data(), sizeof(float) * H);
    memcpy(qkvb.data() + H, kb->data.data(), sizeof(float) * H);
    memcpy(qkvb.data() + 2 * H, vb->data.data(), sizeof(float) * H);
    Layer& L = m->layers[l];
    if ((st = new_dense(m, qkvw.data(), qkvb.data(), H, 3 * H, &L.qkv))) return st;
    if ((st = new_dense(m, ow->data.data(), ob->data.data(), H, H, &L.o))) return st;
    if ((st = new_dense(m, f1w->data.data(), f1b->data.data(), H, I, &L.f1))) return st;
    if ((st = new_dense(m, f2w->data.data(), f2b->data.data(), I, H, &L.f2))) return st;
    if ((st = upload(g1->data.data(), H, &L.ln1_g))) return st;
    if ((st = upload(b1->data.data(), H, &L.ln1_b))) return st;
    if ((st = upload(g2->data.data(), H, &L.ln2_g))) return st;
    if ((st = upload(b2->data.data(), H, &L.ln2_b))) return st;
  }
  return RH_OK;
}


// newDense for the gate and up projections (qwen3.go:528-529,
// gemma3.go:363-364): each matrix goes through the chain on its own. When both
// end in the same mode they are packed as one gated weight (the GEMM's
// epilogue then writes act(gate) * up), else as two weights.
static int new_dense_gated(rh_model* m, const float* gate, const float* up, int in, int i,
                           DecLayer& L) {
  const int mg = dense_mode(m, gate, in, i), mu = dense_mode(m, up, in, i);
  if (m->fuse_projections && mg == mu) {
    int st = pack_weight_gated(m->ctx, mg, gate, up, in, i, &L.gu, true);
    if (st == RH_OK || !pack_refused(st)) return st;
  }
  m->split_gu_any = true;
  int st = new_dense(m, gate, nullptr, in, i, &L.gate);
  if (st) return st;
  return new_dense(m, up, nullptr, in, i, &L.up);
}

// newDense for q, k and v (qwen3.go:479-481, gemma3.go:297-299): one fused
// [qdim + 2 kvdim][H] weight when all three end in the same mode, else three.
static int new_dense_qkv(rh_model* m, const float* qw, const float* kw, const float* vw, int H,
                         int qd, int kvd, DecLayer& L) {
  const int mq = dense_mode(m, qw, H, qd), mk = dense_mode(m, kw, H, kvd),
            mv = dense_mode(m, vw, H, kvd);
  if (m->fuse_projections && mq == mk && mk == mv) {
    // rows fused: each output column is the same dot product as in the
    // reference's three separate applyDense calls
    std::vector<float> qkvw((size_t)(qd + 2 * kvd) * H);
    memcpy(qkvw.data(), qw, sizeof(float) * (size_t)qd * H);
    memcpy(qkvw.data() + (size_t)qd * H, kw, sizeof(float) * (size_t)kvd * H);
    memcpy(qkvw.data() + (size_t)(qd + kvd) * H, vw, sizeof(float) * (size_t)kvd * H);
    int st = pack_weight(m->ctx, mq, qkvw.data(), nullptr, H, qd + 2 * kvd, &L.qkv, true);
    if (st == RH_OK || !pack_refused(st)) return st;
  }
  int st = new_dense(m, qw, nullptr, H, qd, &L.q);
  if (st) return st;
  if ((st = new_dense(m, kw, nullptr, H, kvd, &L.k))) return st;
  return new_dense(m, vw, nullptr, H, kvd, &L.v);
}

// Upload a norm weight, adding Gemma's unit offset (gemma3.go:40-50).
static int upload_norm(const HostTensor* t, int n, bool unit_offset, float** dst) {
  std::vector<float> v(t->data.begin(), t->data.begin() + n);
  if (unit_offset)
    for (float& x : v) x = x + 1.0f;
  return upload(v.data(), n, dst);
}

// ropeTable (modernbert.go:112-122) for positions [0, seq): float64 trig
// rounded to float32, [seq][dh/2], uploaded once at load.
static int upload_rope(int seq, int dh, double theta, float** cos_d, float** sin_d) {
  const int half = dh / 2;
  std::vector<float> c((size_t)seq * half), sn((size_t)seq * half);
  for (int d = 0; d < half; d++) {
    const double inv_freq = std::pow(theta, -2.0 * (double)d / (double)dh);
    for (int p = 0; p < seq; p++) {
      const double ang = (double)p * inv_freq;
      c[(size_t)p * half + d] = (float)std::cos(ang);
      sn[(size_t)p * half + d] = (float)std::sin(ang);
    }
  }
  int st = upload(c.data(), c.size(), cos_d);
  if (st) return st;
  return upload(sn.data(), sn.size(), sin_d);
}

// loadQwen3 (qwen3.go:37-135) / loadGemma3 (gemma3.go:57-158).
static int finalize_decoder(rh_model* m) {
  const bool gemma = m->gemma();
  const int H = m->cfg.hidden, I = m->cfg.intermediate, dh = m->dh();
  const int qd = m->qdim(), kvd = m->kvdim();
  std::string prefix;
  if (m->pending.count("model.embed_tokens.weight")) prefix = "model.";
  const HostTensor *emb, *fn;
  int st;
  if ((st = find_tensor(m, prefix, "embed_tokens.weight", {m->cfg.vocab, H}, &emb))) return st;
  if ((st = find_tensor(m, prefix, "norm.weight", {H}, &fn))) return st;
  if ((st = upload(emb->data.data(), emb->data.size(), &m->word))) return st;
  if ((st = upload_norm(fn, H, gemma, &m->final_norm))) return st;
  const int seq_cap = m->max_seq();
  if ((st = upload_rope(seq_cap, dh, m->cfg.rope_theta, &m->cos_g, &m->sin_g))) return st;
  if (gemma &&
      (st = upload_rope(seq_cap, dh, m->cfg.rope_local_theta, &m->cos_l, &m->sin_l)))
    return st;
  if (gemma && m->cfg.dense_hidden > 0) {
    const HostTensor *d1, *d2;
    if ((st = find_tensor(m, "", "2_Dense.linear.weight", {m->cfg.dense_hidden, H}, &d1)))
      return st;
    if ((st = find_tensor(m, "", "3_Dense.linear.weight", {H, m->cfg.dense_hidden}, &d2)))
      return st;
    // kept transposed ([in][out]) for the per-output Dense kernels
    const int D = m->cfg.dense_hidden;
    std::vector<float> t1((size_t)H * D), t2((size_t)D * H);
    for (int o = 0; o < D; o++)
      for (int i = 0; i < H; i++) t1[(size_t)i * D + o] = d1->data[(size_t)o * H + i];
    for (int o = 0; o < H; o++)
      for (int i = 0; i < D; i++) t2[(size_t)i * H + o] = d2->data[(size_t)o * D + i];
    if ((st = upload(t1.data(), t1.size(), &m->dense1))) return st;
    if ((st = upload(t2.data(), t2.size(), &m->dense2))) return st;
  }
  m->dlayers.resize(m->cfg.layers);
  for (int l = 0; l < m->cfg.layers; l++) {
    char buf[64];
    snprintf(buf, sizeof buf, "layers.%d.", l);
    const std::string lp = buf;
    const HostTensor *in_n, *qw, *kw, *vw, *ow, *qn, *kn, *pa, *gw, *uw, *dw;
    const HostTensor *pf = nullptr, *po = nullptr;
    struct Need {
      const char* name;
      std::initializer_list<int64_t> shape;
      const HostTensor** dst;
    };
    const Need needs[] = {
        {"input_layernorm.weight", {H}, &in_n},
        {"self_attn.q_proj.weight", {qd, H}, &qw},
        {"self_attn.k_proj.weight", {kvd, H}, &kw},
        {"self_attn.v_proj.weight", {kvd, H}, &vw},
        {"self_attn.o_proj.weight", {H, qd}, &ow},
        {"self_attn.q_norm.weight", {dh}, &qn},
        {"self_attn.k_norm.weight", {dh}, &kn},
        {"post_attention_layernorm.weight", {H}, &pa},
        {"mlp.gate_proj.weight", {I, H}, &gw},
        {"mlp.up_proj.weight", {I, H}, &uw},
        {"mlp.down_proj.weight", {H, I}, &dw},
    };
    for (const Need& n : needs)
      if ((st = find_tensor(m, prefix, lp + n.name, n.shape, n.dst))) return st;
    if (gemma) {
      if ((st = find_tensor(m, prefix, lp + "pre_feedforward_layernorm.weight", {H}, &pf)))
        return st;
      if ((st = find_tensor(m, prefix, lp + "post_feedforward_layernorm.weight", {H}, &po)))
        return st;
    }
    DecLayer& L = m->dlayers[l];
    L.global = !gemma || (l + 1) % m->cfg.sliding_pattern == 0;  // gemma3.go:87
    if ((st = new_dense_qkv(m, qw->data.data(), kw->data.data(), vw->data.data(), H, qd, kvd,
                            L)))
      return st;
    if ((st = new_dense(m, ow->data.data(), nullptr, qd, H, &L.o))) return st;
    if ((st = new_dense_gated(m, gw->data.data(), uw->data.data(), H, I, L))) return st;
    if ((st = new_dense(m, dw->data.data(), nullptr, I, H, &L.down))) return st;
    if ((st = upload_norm(in_n, H, gemma, &L.in_norm))) return st;
    if ((st = upload_norm(qn, dh, gemma, &L.q_norm))) return st;
    if ((st = upload_norm(kn, dh, gemma, &L.k_norm))) return st;
    if ((st = upload_norm(pa, H, gemma, &L.post_attn))) return st;
    if (gemma) {
      if ((st = upload_norm(pf, H, true, &L.pre_ffn))) return st;
      if ((st = upload_norm(po, H, true, &L.post_ffn))) return st;
    }
  }
  return RH_OK;
}

// loadNomic (nomic.go:33-110) / loadModernBERT (modernbert.go:34-104): the
// bias-free RoPE encoders, tensor names without a prefix. Each projection
// goes through newDense on its own, as there: nomic's fc12 (silu-gated) and
// fc11 form the gated pair (gate = fc12, up = fc11, nomic.go:232-242);
// ModernBERT's Wi [2I][H] is one matrix whose halves are gate = Wi[:I] and
// up = Wi[I:] (modernbert.go:292-301), so both halves take the one mode
// newDense gives the whole matrix.
static int finalize_renc(rh_model* m) {
  const bool mb = m->modernbert();
  const int H = m->cfg.hidden, I = m->cfg.intermediate, dh = m->dh();
  const HostTensor *we, *tt = nullptr, *eg, *eb = nullptr, *fn = nullptr;
  int st;
  if (mb) {
    if ((st = find_tensor(m, "", "embeddings.tok_embeddings.weight", {m->cfg.vocab, H}, &we)))
      return st;
    if ((st = find_tensor(m, "", "embeddings.norm.weight", {H}, &eg))) return st;
    if ((st = find_tensor(m, "", "final_norm.weight", {H}, &fn))) return st;
  } else {
    if ((st = find_tensor(m, "", "embeddings.word_embeddings.weight", {m->cfg.vocab, H}, &we)))
      return st;
    if ((st = find_tensor(m, "", "embeddings.token_type_embeddings.weight", {2, H}, &tt)))
      return st;
    if ((st = find_tensor(m, "", "emb_ln.weight", {H}, &eg))) return st;
    if ((st = find_tensor(m, "", "emb_ln.bias", {H}, &eb))) return st;
  }
  if ((st = upload(we->data.data(), we->data.size(), &m->word))) return st;
  if ((st = upload(eg->data.data(), H, &m->emb_g))) return st;
  if (eb && (st = upload(eb->data.data(), H, &m->emb_b))) return st;
  if (tt && (st = upload(tt->data.data(), H, &m->type0))) return st;  // row 0
  if (fn && (st = upload(fn->data.data(), H, &m->final_norm))) return st;
  const int seq_cap = m->max_seq();
  if ((st = upload_rope(seq_cap, dh, m->cfg.rope_theta, &m->cos_g, &m->sin_g))) return st;
  if (mb && (st = upload_rope(seq_cap, dh, m->cfg.rope_local_theta, &m->cos_l, &m->sin_l)))
    return st;
  m->dlayers.resize(m->cfg.layers);
  for (int l = 0; l < m->cfg.layers; l++) {
    DecLayer& L = m->dlayers[l];
    char buf[64];
    if (mb) {
      snprintf(buf, sizeof buf, "layers.%d.", l);
      const std::string lp = buf;
      const HostTensor *an = nullptr, *qkv, *wo, *mn, *wi, *wmo;
      // layer 0's attention norm is an identity with no tensor (modernbert.go:74-81)
      if (l != 0 && (st = find_tensor(m, "", lp + "attn_norm.weight", {H}, &an))) return st;
      if ((st = find_tensor(m, "", lp + "attn.Wqkv.weight", {3 * H, H}, &qkv))) return st;
      if ((st = find_tensor(m, "", lp + "attn.Wo.weight", {H, H}, &wo))) return st;
      if ((st = find_tensor(m, "", lp + "mlp_norm.weight", {H}, &mn))) return st;
      if ((st = find_tensor(m, "", lp + "mlp.Wi.weight", {2 * I, H}, &wi))) return st;
      if ((st = find_tensor(m, "", lp + "mlp.Wo.weight", {H, I}, &wmo))) return st;
      L.global = l % m->cfg.sliding_pattern == 0;  // modernbert.go:73
      if ((st = new_dense(m, qkv->data.data(), nullptr, H, 3 * H, &L.qkv))) return st;
      if ((st = new_dense(m, wo->data.data(), nullptr, H, H, &L.o))) return st;
      const float* gate = wi->data.data();
      const float* up = gate + (size_t)I * H;
      const int mode = dense_mode(m, gate, H, 2 * I);
      if (m->fuse_projections) {
        if ((st = pack_weight_gated(m->ctx, mode, gate, up, H, I, &L.gu, true))) return st;
      } else {
        m->split_gu_any = true;
        if ((st = pack_weight(m->ctx, mode, gate, nullptr, H, I, &L.gate, true))) return st;
        if ((st = pack_weight(m->ctx, mode, up, nullptr, H, I, &L.up, true))) return st;
      }
      if ((st = new_dense(m, wmo->data.data(), nullptr, I, H, &L.down))) return st;
      if (an && (st = upload(an->data.data(), H, &L.in_norm))) return st;
      if ((st = upload(mn->data.data(), H, &L.post_attn))) return st;
    } else {
      snprintf(buf, sizeof buf, "encoder.layers.%d.", l);
      const std::string lp = buf;
      const HostTensor *qkv, *wo, *n1g, *n1b, *f11, *f12, *f2, *n2g, *n2b;
      struct Need {
        const char* name;
        std::initializer_list<int64_t> shape;
        const HostTensor** dst;
      };
      const Need needs[] = {
          {"attn.Wqkv.weight", {3 * H, H}, &qkv}, {"attn.out_proj.weight", {H, H}, &wo},
          {"norm1.weight", {H}, &n1g},           {"norm1.bias", {H}, &n1b},
          {"mlp.fc11.weight", {I, H}, &f11},     {"mlp.fc12.weight", {I, H}, &f12},
          {"mlp.fc2.weight", {H, I}, &f2},       {"norm2.weight", {H}, &n2g},
          {"norm2.bias", {H}, &n2b},
      };
      for (const Need& n : needs)
        if ((st = find_tensor(m, "", lp + n.name, n.shape, n.dst))) return st;
      if ((st = new_dense(m, qkv->data.data(), nullptr, H, 3 * H, &L.qkv))) return st;
      if ((st = new_dense(m, wo->data.data(), nullptr, H, H, &L.o))) return st;
      if ((st = new_dense_gated(m, f12->data.data(), f11->data.data(), H, I, L))) return st;
      if ((st = new_dense(m, f2->data.data(), nullptr, I, H, &L.down))) return st;
      if ((st = upload(n1g->data.data(), H, &L.post_attn))) return st;
      if ((st = upload(n1b->data.data(), H, &L.post_attn_b))) return st;
      if ((st = upload(n2g->data.data(), H, &L.post_ffn))) return st;
      if ((st = upload(n2b->data.data(), H, &L.post_ffn_b))) return st;
    }
  }
  return RH_OK;
}

// ---- C ABI ------------------------------------------------------------------------

#define MODEL_GUARD(m)                                                   \
  if (!(m)) return fail(RH_ERR_INVALID, "null model");                  \
  std::lock_guard<std::mutex> mlk_((m)->mu);                            \
  std::lock_guard<std::mutex> clk_((m)->ctx->mu);                       \
  RH_HIP(hipSetDevice((m)->ctx->device))

extern "C" {

int rh_model_create(rh_context* ctx, const rh_model_config* cfg, int quant, rh_model** out) {
  return api_call([&]() -> int {
    if (!ctx || !cfg || !out) return fail(RH_ERR_INVALID, "null argument");
    if (cfg->arch < RH_ARCH_BERT || cfg->arch > RH_ARCH_MPNET)
      return fail(RH_ERR_INVALID, "unsupported arch");
    const bool bert_family = cfg->arch == RH_ARCH_BERT || cfg->arch == RH_ARCH_DISTILBERT ||
                             cfg->arch == RH_ARCH_MPNET;
    if (cfg->hidden <= 0 || cfg->heads <= 0) return fail(RH_ERR_INVALID, "bad hidden/heads");
    if (cfg->intermediate <= 0 || cfg->layers <= 0 || cfg->vocab <= 0 || cfg->max_position <= 0)
      return fail(RH_ERR_INVALID, "bad config sizes");
    if (cfg->hidden % 64 != 0 || cfg->hidden > 4096)
      return fail(RH_ERR_INVALID, "hidden must be a multiple of 64 and <= 4096");
    if (quant < RH_QUANT_NONE || quant > RH_QUANT_FULL) return fail(RH_ERR_INVALID, "bad quant");
    if (bert_family) {
      // MPNet's bucketing is HF's at 32 buckets (config.go:219-221); the
      // others have no relative-position bias
      if ((cfg->arch == RH_ARCH_MPNET) != (cfg->rel_buckets != 0) ||
          (cfg->rel_buckets != 0 && cfg->rel_buckets != 32))
        return fail(RH_ERR_INVALID, "relative-position buckets: 32 for MPNet, 0 otherwise");
      if (cfg->position_offset < 0 || cfg->position_offset >= cfg->max_position)
        return fail(RH_ERR_INVALID, "bad position offset");
      if (cfg->intermediate % 4 != 0)
        return fail(RH_ERR_INVALID, "intermediate must divide by 4");
      if (cfg->hidden % cfg->heads != 0 || cfg->hidden > 2048)
        return fail(RH_ERR_INVALID, "hidden must divide by heads and be <= 2048");
      const int dh = cfg->hidden / cfg->heads;
      if (dh != 32 && dh != 64 && dh != 128)
        return fail(RH_ERR_INVALID, "head dim must be 32, 64 or 128");
    } else if (cfg->arch == RH_ARCH_NOMIC || cfg->arch == RH_ARCH_MODERNBERT) {
      // config.go:130-148,163-175
      const int dh = cfg->head_dim > 0 ? cfg->head_dim : cfg->hidden / cfg->heads;
      if (cfg->kv_heads != 0 && cfg->kv_heads != cfg->heads)
        return fail(RH_ERR_INVALID, "nomic / ModernBERT attention has no kv head groups");
      if (dh * cfg->heads != cfg->hidden)
        return fail(RH_ERR_INVALID, "head_dim * heads must equal hidden");
      if (dh != 32 && dh != 64 && dh != 128 && dh != 256)
        return fail(RH_ERR_INVALID, "head dim must be 32, 64, 128 or 256");
      if (cfg->intermediate % 16 != 0)
        return fail(RH_ERR_INVALID, "intermediate must divide by 16");
      if (cfg->rope_theta <= 0) return fail(RH_ERR_INVALID, "rope_theta must be positive");
      if (cfg->arch == RH_ARCH_MODERNBERT &&
          (cfg->rope_local_theta <= 0 || cfg->sliding_pattern < 1 || cfg->sliding_window < 2 ||
           cfg->sliding_window % 2 != 0))
        return fail(RH_ERR_INVALID,
                    "ModernBERT needs local theta, global_attn_every_n_layers >= 1 and an even "
                    "local_attention >= 2");
    } else {
      const int nkv = cfg->kv_heads > 0 ? cfg->kv_heads : cfg->heads;
      const int dh = cfg->head_dim > 0 ? cfg->head_dim : cfg->hidden / cfg->heads;
      if (cfg->heads % nkv != 0) return fail(RH_ERR_INVALID, "heads must be a multiple of kv_heads");
      if (dh != 64 && dh != 128 && dh != 256)
        return fail(RH_ERR_INVALID, "head dim must be 64, 128 or 256");
      if (cfg->intermediate % 8 != 0) return fail(RH_ERR_INVALID, "intermediate must divide by 8");
      if (cfg->rope_theta <= 0) return fail(RH_ERR_INVALID, "rope_theta must be positive");
      if (cfg->arch == RH_ARCH_GEMMA3) {
        if (cfg->rope_local_theta <= 0 || cfg->sliding_pattern <= 0 || cfg->sliding_window <= 0 ||
            cfg->query_pre_attn_scalar <= 0)
          return fail(RH_ERR_INVALID, "gemma needs local theta, window, pattern, attn scalar");
        if (cfg->dense_hidden < 0 || cfg->dense_hidden > 16384)
          return fail(RH_ERR_INVALID, "bad dense_hidden");
      }
    }
    auto* m = new rh_model();
    m->ctx = ctx;
    ctx_retain(ctx);
    m->cfg = *cfg;
    m->quant = quant;
    // fp32-grade attention (the reference's attention is float32) for the
    // BERT family in every mode; the RoPE family's quantized modes keep bf16
    // operands (their dh-256 fp32-grade kernel is the unpipelined one)
    m->attn_precision = quant == RH_QUANT_NONE || bert_family ? 3 : 1;
    *out = m;
    return RH_OK;
  });
}

int rh_model_set_option(rh_model* m, int option, int value) {
  return api_call([&]() -> int {
    if (!m) return fail(RH_ERR_INVALID, "null model");
    std::lock_guard<std::mutex> lk(m->mu);
    m->drop_graph();  // a recorded forward follows the settings it was recorded under
    if (option == RH_OPT_GRAPH) {
      if (value != 0 && value != 1) return fail(RH_ERR_INVALID, "graph must be 0 or 1");
      m->use_graph = value != 0;
      return RH_OK;
    }
    if (option == RH_OPT_ATTN_PRECISION) {
      if (value != 1 && value != 3) return fail(RH_ERR_INVALID, "attn precision must be 1 or 3");
      m->attn_precision = value;
      return RH_OK;
    }
    if (option == RH_OPT_FUSED_FFN1) {
      if (value < 0 || value > 2) return fail(RH_ERR_INVALID, "fused FFN1 must be 0, 1 or 2");
      m->fused_ffn1 = value;
      return RH_OK;
    }
    if (option == RH_OPT_EXACT) {
      if (value != 0 && value != 1) return fail(RH_ERR_INVALID, "exact must be 0 or 1");
      if (value && m->rope_family())
        return fail(RH_ERR_INVALID, "the exact forward is for the BERT family");
      m->exact = value != 0;
      return RH_OK;
    }
    if (option == RH_OPT_FUSED_LN) {
      if (value != 0 && value != 1) return fail(RH_ERR_INVALID, "fused LN must be 0 or 1");
      m->fused_ln = value != 0;
      return RH_OK;
    }
    if (option == RH_OPT_PRODUCER_PLANES) {
      if (value != 0 && value != 1) return fail(RH_ERR_INVALID, "producer planes must be 0 or 1");
      m->producer_planes = value != 0;
      return RH_OK;
    }
    if (option == RH_OPT_QK_EPILOGUE) {
      if (value != 0 && value != 1) return fail(RH_ERR_INVALID, "qk epilogue must be 0 or 1");
      m->qk_epilogue = value != 0;
      return RH_OK;
    }
    if (option == RH_OPT_FUSE_PROJECTIONS) {
    if (value != 0 && value != 1) return fail(RH_ERR_INVALID, "fuse projections must be 0 or 1");
    if (m->finalized) return fail(RH_ERR_INVALID, "fuse projections is set before finalize");
    m->fuse_projections = value != 0;
    return RH_OK;
  }
  if (option == RH_OPT_STREAMS) {
      if (value < 1 || value > rh_model::kMaxParts)
        return fail(RH_ERR_INVALID, "streams must be 1 to 4");
      m->streams = value;
      return RH_OK;
    }
    return fail(RH_ERR_INVALID, "unknown option");
  });
}

int rh_model_set_tensor(rh_model* m, const char* name, const float* host,
                        const int64_t* shape, int ndim) {
  return api_call([&]() -> int {
    if (!m || !name || !host || (ndim > 0 && !shape) || ndim < 0 || ndim > 4)
      return fail(RH_ERR_INVALID, "bad argument");
    std::lock_guard<std::mutex> lk(m->mu);
    if (m->finalized) return fail(RH_ERR_INVALID, "model already finalized");
    HostTensor t;
    size_t n = 1;
    for (int i = 0; i < ndim; i++) {
      if (shape[i] < 0) return fail(RH_ERR_INVALID, "negative dim");
      t.shape.push_back(shape[i]);
      n *= (size_t)shape[i];
    }
    t.data.assign(host, host + n);
    m->pending[name] = std::move(t);
    return RH_OK;
  });
}

int rh_model_finalize(rh_model* m) {
  return api_call([&]() -> int {
    MODEL_GUARD(m);
    if (m->finalized) return fail(RH_ERR_INVALID, "model already finalized");
    // A failed finalize (a status or an exception) releases every device
    // object made so far, so the model is left empty rather than half built.
    int st;
    try {
      st = m->nomic() || m->modernbert() ? finalize_renc(m)
           : m->rope_family()            ? finalize_decoder(m)
                                         : finalize_bert(m);
    } catch (...) {
      m->release();
      throw;
    }
    if (st) {
      char msg[512];
      snprintf(msg, sizeof msg, "%s", rh_last_error());
      m->release();
      set_error(msg);
      return st;
    }
    m->weights = m->own_weights();
    m->pending.clear();
    m->finalized = true;
    return RH_OK;
  });
}

int rh_model_share(rh_model* src, rh_context* ctx, rh_model** out) {
  return api_call([&]() -> int {
    if (!src || !ctx || !out) return fail(RH_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lk(src->mu);
    if (!src->finalized || !src->weights) return fail(RH_ERR_INVALID, "model not finalized");
    if (ctx->device != src->ctx->device)
      return fail(RH_ERR_INVALID, "the context is on another device than the model's weights");
    std::unique_ptr<rh_model> m(new rh_model());
    m->cfg = src->cfg;
    m->quant = src->quant;
    m->layers = src->layers;
    m->dlayers = src->dlayers;
    m->word = src->word;
    m->pos = src->pos;
    m->type0 = src->type0;
    m->emb_g = src->emb_g;
    m->emb_b = src->emb_b;
    m->final_norm = src->final_norm;
    m->dense1 = src->dense1;
    m->dense2 = src->dense2;
    m->cos_g = src->cos_g;
    m->sin_g = src->sin_g;
    m->cos_l = src->cos_l;
    m->sin_l = src->sin_l;
    m->attn_precision = src->attn_precision;
    m->fused_ffn1 = src->fused_ffn1;
    m->exact = src->exact;
    m->use_graph = src->use_graph;
    m->fused_ln = src->fused_ln;
    m->producer_planes = src->producer_planes;
    m->streams = src->streams;
    m->qk_epilogue = src->qk_epilogue;
    m->fuse_projections = src->fuse_projections;
    m->split_gu_any = src->split_gu_any;
    m->weights = src->weights;
    m->finalized = true;
    m->ctx = ctx;
    ctx_retain(ctx);
    *out = m.release();
    return RH_OK;
  });
}

void rh_model_destroy(rh_model* m) {
  api_void([&] {
    if (!m) return;
    rh_context* ctx = m->ctx;
    {
      std::lock_guard<std::mutex> lk(ctx->mu);
      m->release();
    }
    m->ctx = nullptr;
    delete m;
    ctx_release(ctx);
  });
}

// Does every per-layer weight satisfy pred? (Walks the handles in place:
// the introspection calls allocate nothing.)
static bool all_weights(const rh_model* m, bool (*pred)(const rh_weight*)) {
  for (const Layer& L : m->layers)
    for (const rh_weight* w : {L.qkv, L.o, L.f1, L.f2})
      if (!pred(w)) return false;
  for (const DecLayer& L : m->dlayers)
    for (const rh_weight* w : {L.qkv, L.o, L.gu, L.down, L.q, L.k, L.v, L.gate, L.up})
      if (w && !pred(w)) return false;
  return true;
}

int rh_model_quantized(const rh_model* m) {
  if (!m || !m->finalized) return 0;
  return all_weights(m, [](const rh_weight* w) { return w->mode != RH_MODE_F32; }) ? 1 : 0;
}

int rh_model_quantized_activations(const rh_model* m) {
  if (!m || !m->finalized) return 0;
  return all_weights(m, [](const rh_weight* w) { return w->mode == RH_MODE_A8W8; }) ? 1 : 0;
}

// The host-buffer forward of Embed / EmbedTokens. ids are int64 as the
// reference passes them (bert.go:649, rembed.go:416); each one is checked
// against the vocabulary (bert.go:797-800) while it is narrowed into the
// model's pinned int32 staging rows, which go to HBM in one copy.
static int embed_common(rh_model* m, const int64_t* ids, const int32_t* lens, int batch,
                        int stride, float* out, bool pool) {
  if (!ids || !lens || !out || batch < 0 || stride < 1)
    return fail(RH_ERR_INVALID, "bad argument");
  if (!m->finalized) return fail(RH_ERR_INVALID, "model not finalized");
  if (batch == 0) return RH_OK;
  const size_t elems = (size_t)batch * (size_t)stride;
  if (elems > (size_t)INT32_MAX)
    return fail(RH_ERR_INVALID, "batch * stride exceeds 2^31 - 1 token slots");
  for (int b = 0; b < batch; b++)
    if (lens[b] > stride) return fail(RH_ERR_INVALID, "length exceeds row stride");
  std::vector<int32_t>& cu = m->cu_host;
  int max_len = 0;
  int st = m->plan(lens, batch, cu, &max_len);
  if (st) return st;
  const int M = cu[batch], H = m->cfg.hidden;
  if ((st = m->ensure_ws(M, batch, elems))) return st;
  if ((st = m->ensure_ids_staging(elems))) return st;
  int32_t* stage = m->ids_pinned;
  for (int b = 0; b < batch; b++) {
    const int64_t* row = ids + (size_t)b * stride;
    int32_t* srow = stage + (size_t)b * stride;
    for (int t = 0; t < lens[b]; t++) {
      const int64_t id = row[t];
      if (id < 0 || id >= m->cfg.vocab) {
        char buf[160];
        snprintf(buf, sizeof buf, "text %d: token id %lld out of vocab range %d", b,
                 (long long)id, m->cfg.vocab);
        return fail(RH_ERR_VOCAB, buf);
      }
      srow[t] = (int32_t)id;
    }
    for (int t = lens[b]; t < stride; t++) srow[t] = 0;  // never read
  }
  hipStream_t s = m->ctx->stream;
  RH_HIP(hipMemcpyAsync(m->ids_d, stage, elems * sizeof(int32_t), hipMemcpyHostToDevice, s));
  // the staging rows are reused by the next call only after this one's sync
  st = m->forward(m->ids_d, stride, cu, max_len, pool, m->out_d);
  if (st) {
    (void)hipStreamSynchronize(s);
    return st;
  }
  if (pool)
    RH_HIP(hipMemcpyAsync(out, m->out_d, (size_t)batch * H * sizeof(float),
                          hipMemcpyDeviceToHost, s));
  else
    RH_HIP(hipMemcpyAsync(out, m->x, (size_t)M * H * sizeof(float), hipMemcpyDeviceToHost,
                          s));
  // a one-pass FFN1 row wait that timed out left bytes that may be wrong
  unsigned late = 0;
  const bool onepass = m->qsync && m->fused_ffn1 == 2;
  if (onepass) RH_HIP(hipMemcpyAsync(&late, m->qsync, sizeof(unsigned), hipMemcpyDeviceToHost, s));
  RH_HIP(hipStreamSynchronize(s));
  if (late) {
    RH_HIP(hipMemset(m->qsync, 0, sizeof(unsigned)));
    return fail(RH_ERR_HIP, "one-pass FFN1: a row's wait for its row maxima timed out");
  }
  return RH_OK;
}

int rh_model_embed(rh_model* m, const int64_t* ids, const int32_t* lens, int batch,
                   int stride, float* out) {
  return api_call([&]() -> int {
    MODEL_GUARD(m);
    return embed_common(m, ids, lens, batch, stride, out, true);
  });
}

int rh_model_embed_tokens(rh_model* m, const int64_t* ids, const int32_t* lens, int batch,
                          int stride, float* out) {
  return api_call([&]() -> int {
    MODEL_GUARD(m);
    return embed_common(m, ids, lens, batch, stride, out, false);
  });
}

int rh_model_embed_device(rh_model* m, const int32_t* ids_dev, const int32_t* lens,
                          int batch, int stride, float* out_dev) {
  return api_call([&]() -> int {
    MODEL_GUARD(m);
    if (!ids_dev || !lens || !out_dev || batch < 0 || stride < 1)
      return fail(RH_ERR_INVALID, "bad argument");
    if (!m->finalized) return fail(RH_ERR_INVALID, "model not finalized");
    if (batch == 0) return RH_OK;
    if ((size_t)batch * (size_t)stride > (size_t)INT32_MAX)
      return fail(RH_ERR_INVALID, "batch * stride exceeds 2^31 - 1 token slots");
    for (int b = 0; b < batch; b++)
      if (lens[b] > stride) return fail(RH_ERR_INVALID, "length exceeds row stride");
    int max_len = 0;
    int st = m->plan(lens, batch, m->cu_host, &max_len);
    if (st) return st;
    return m->forward(ids_dev, stride, m->cu_host, max_len, true, out_dev);
  });
}

int rh_model_check(rh_model* m) {
  return api_call([&]() -> int {
    MODEL_GUARD(m);
    RH_HIP(hipStreamSynchronize(m->ctx->stream));
    if (m->qsync) {
      unsigned late = 0;
      RH_HIP(hipMemcpy(&late, m->qsync, sizeof(unsigned), hipMemcpyDeviceToHost));
      if (late) {
        RH_HIP(hipMemset(m->qsync, 0, sizeof(unsigned)));
        return fail(RH_ERR_HIP, "one-pass FFN1: a row's wait for its row maxima timed out");
      }
    }
    if (!m->err_d) return RH_OK;
    int flag = 0;
    RH_HIP(hipMemcpy(&flag, m->err_d, sizeof(int), hipMemcpyDeviceToHost));
    if (flag) {
      RH_HIP(hipMemset(m->err_d, 0, sizeof(int)));
      return fail(RH_ERR_VOCAB, "a token id was out of vocab range (clamped on device)");
    }
    return RH_OK;
  });
}

}  // extern "C"
