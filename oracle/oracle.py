"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the parity reference. The product never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    sig = {
        "or_pack_b8": (I, [P, I, I, P, P]),
        "or_pack_b8_vnni": (I, [P, I, I, P, P, P]),
        "or_quantize_row_u8": (F, [P, I, P, I]),
        "or_matmul_f32": (None, [P, P, P, I, I, I]),
        "or_matmul_w8": (None, [P, P, P, P, I, I, I]),
        "or_gemm_u8s8_i32": (None, [P, P, I, P, I, I, I]),
        "or_matmul_vnni": (None, [P, P, P, P, P, I, I, I, P, P, P]),
        "or_expf32": (F, [F]),
        "or_erff32": (F, [F]),
        "or_add_bias": (None, [P, P, I, I]),
        "or_add": (None, [P, P, I]),
        "or_softmax": (None, [P, I, I]),
        "or_layernorm": (None, [P, P, P, I, I, F]),
        "or_rmsnorm": (None, [P, P, I, I, F]),
        "or_gelu": (None, [P, I]),
        "or_gelu_ref": (None, [P, I]),
        "or_gelu_avx2_lane": (F, [F]),
        "or_gelu_tanh": (None, [P, I]),
        "or_silu": (None, [P, I]),
        "or_l2normalize": (None, [P, I]),
        "or_dot4": (None, [P, P, P, P, P, P, I]),
        "or_matmul_serial": (None, [P, P, P, I, I, I]),
        "or_bert_create": (P, [P, I, P, P, P, P, P, P]),
        "or_bert_set_rel_bias": (None, [P, P]),
        "or_rel_pos_bucket": (I, [I, I]),
        "or_bert_free": (None, [P]),
        "or_bert_encode": (I, [P, P, I, P]),
        "or_bert_encode_layers": (I, [P, P, I, P, I]),
        "or_bert_forward": (I, [P, P, I, P]),
        "or_bert_embed_batch": (I, [P, P, P, I, I, P, I]),
        "or_bert_embed_batch_timed": (I, [P, P, P, I, I, P, I, P]),
        "or_vnni_kind": (I, []),
        "or_pack_vnni_panels": (None, [P, I, I, P]),
        "or_gemm_u8s8_panels": (None, [P, P, I, P, I, I, I]),
        "or_vnni_panel_kind": (I, []),
        "or_set_gemm_impl": (None, [I]),
        "or_dec_create": (P, [P, I, P, P, P, P, P]),
        "or_dec_free": (None, [P]),
        "or_dec_quantized_kind": (I, [P]),
        "or_dec_encode": (I, [P, P, I, P]),
        "or_dec_forward": (I, [P, P, I, P]),
        "or_dec_embed_batch": (I, [P, P, P, I, I, P, I]),
        "or_dec_embed_batch_timed": (I, [P, P, P, I, I, P, I, P]),
        "or_renc_create": (P, [P, I, P, P, P, P, P, P]),
        "or_renc_free": (None, [P]),
        "or_renc_quantized_kind": (I, [P]),
        "or_renc_encode": (I, [P, P, I, P]),
        "or_renc_forward": (I, [P, P, I, P]),
        "or_renc_embed_batch_timed": (I, [P, P, P, I, I, P, I, P]),
        "or_rope_table": (None, [P, P, I, I, ctypes.c_double]),
        "or_apply_rope": (None, [P, I, I, P, P]),
        "or_flash_causal_head": (None, [P, P, P, P, I, I, F]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _p(a):
    return a.ctypes.data


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- tensor-level wrappers ------------------------------------------------------

def pack_b8(bT, k, n):
    q = np.empty((n, k), np.int8)
    sc = np.empty(n, np.float32)
    bT = f32(bT)
    st = lib.or_pack_b8(_p(bT), k, n, _p(q), _p(sc))
    return st, q, sc


def pack_b8_vnni(bT, k, n):
    q = np.empty((n, k), np.int8)
    sc = np.empty(n, np.float32)
    cs = np.empty(n, np.int32)
    bT = f32(bT)
    st = lib.or_pack_b8_vnni(_p(bT), k, n, _p(q), _p(cs), _p(sc))
    return st, q, sc, cs


def pack_vnni_panels(q):
    """PackB8VNNI's panel layout of int8 q [n][k] (pack_vnni.go:44-72)."""
    q = np.ascontiguousarray(q, np.int8)
    n, k = q.shape
    kg = (k + 3) // 4
    pb = np.empty((n // 16) * kg * 64, np.int8)
    lib.or_pack_vnni_panels(_p(q), k, n, _p(pb))
    return pb


def gemm_u8s8_panels(qa, pb, k, n):
    """The 4x16 VPDPBUSD tiles of the reference over qa rows [m][lda]."""
    qa = np.ascontiguousarray(qa, np.uint8)
    m, lda = qa.shape
    acc = np.empty((m, n), np.int32)
    lib.or_gemm_u8s8_panels(_p(acc), _p(qa), lda, _p(pb), m, k, n)
    return acc


def quantize_row_u8(a, dstlen=None):
    a = f32(a)
    k = a.shape[0]
    dst = np.empty(dstlen or k, np.uint8)
    s = lib.or_quantize_row_u8(_p(dst), dst.shape[0], _p(a), k)
    return dst, np.float32(s)


def matmul_f32(a, bT):
    a, bT = f32(a), f32(bT)
    m, k = a.shape
    n = bT.shape[0]
    out = np.empty((m, n), np.float32)
    lib.or_matmul_f32(_p(out), _p(a), _p(bT), m, k, n)
    return out


def matmul_w8(a, q, scales):
    a = f32(a)
    m, k = a.shape
    n = q.shape[0]
    out = np.empty((m, n), np.float32)
    q = np.ascontiguousarray(q, np.int8)
    scales = f32(scales)
    lib.or_matmul_w8(_p(out), _p(a), _p(q), _p(scales), m, k, n)
    return out


def gemm_u8s8_i32(qa, q):
    qa = np.ascontiguousarray(qa, np.uint8)
    q = np.ascontiguousarray(q, np.int8)
    m, lda = qa.shape
    n, k = q.shape
    acc = np.empty((m, n), np.int32)
    lib.or_gemm_u8s8_i32(_p(acc), _p(qa), lda, _p(q), m, k, n)
    return acc


def matmul_vnni(a, q, colsum, scales):
    """Returns (dst, qa, row_scales, acc)."""
    a = f32(a)
    m, k = a.shape
    n = q.shape[0]
    out = np.empty((m, n), np.float32)
    qa = np.empty((m, k), np.uint8)
    rs = np.empty(m, np.float32)
    acc = np.empty((m, n), np.int32)
    q = np.ascontiguousarray(q, np.int8)
    colsum = np.ascontiguousarray(colsum, np.int32)
    scales = f32(scales)
    lib.or_matmul_vnni(_p(out), _p(a), _p(q), _p(colsum), _p(scales),
                       m, k, n, _p(qa), _p(rs), _p(acc))
    return out, qa, rs, acc


def rowwise(fn, x, *args):
    x = f32(x).copy()
    fn(_p(x), *args)
    return x


def gelu(x):
    """geluScalar (internal/tensor/tensor.go:508-538)."""
    x = f32(x).copy()
    lib.or_gelu(_p(x), x.size)
    return x


def gelu_ref(x):
    """GELU as rembed runs it on amd64: geluAVX2 over whole 8-lane groups of
    the array, geluScalar for the tail (internal/tensor/gelu_amd64.go:16-26)."""
    x = f32(x).copy()
    lib.or_gelu_ref(_p(x), x.size)
    return x


def silu(x):
    """SiLU (internal/tensor/tensor.go:477-481)."""
    x = f32(x).copy()
    lib.or_silu(_p(x), x.size)
    return x


def gelu_tanh(x):
    """GELUTanh (internal/tensor/tensor.go:490-497)."""
    x = f32(x).copy()
    lib.or_gelu_tanh(_p(x), x.size)
    return x


def rmsnorm(x, g, eps):
    """RMSNorm (internal/tensor/tensor.go:459-471) over the rows of x."""
    x = f32(x).copy()
    m, n = x.shape
    lib.or_rmsnorm(_p(x), _p(f32(g)), m, n, eps)
    return x


def layernorm(x, g, b, eps):
    x = f32(x).copy()
    m, n = x.shape
    g, b = f32(g), f32(b)
    lib.or_layernorm(_p(x), _p(g), _p(b), m, n, eps)
    return x


def matmul_serial(a, bT):
    """MatMulSerial (tensor.go:284-330): dot4 over column quads, in-order
    scalar sums for the n % 4 remainder columns."""
    a, bT = f32(a), f32(bT)
    m, k = a.shape
    n = bT.shape[0]
    out = np.empty((m, n), np.float32)
    lib.or_matmul_serial(_p(out), _p(a), _p(bT), m, k, n)
    return out


def softmax(x):
    """Softmax (tensor.go:389-428) over the rows of x."""
    x = f32(x).copy()
    m, n = x.shape
    lib.or_softmax(_p(x), m, n)
    return x


def attention_ref(qkv, lens, heads, dh, scale, q_off, k_off, v_off):
    """bert.go:853-902 per text and head: scores = MatMulSerial(Qh, Kh),
    scores *= scale (float32), Softmax, ctx = MatMulSerial(P, Vhᵀ)."""
    qkv = f32(qkv)
    out = np.zeros((qkv.shape[0], heads * dh), np.float32)
    r0 = 0
    for L in lens:
        rows = slice(r0, r0 + L)
        for h in range(heads):
            q = qkv[rows, q_off + h * dh:q_off + (h + 1) * dh]
            k = qkv[rows, k_off + h * dh:k_off + (h + 1) * dh]
            v = qkv[rows, v_off + h * dh:v_off + (h + 1) * dh]
            sc = matmul_serial(q, k) * np.float32(scale)
            out[rows, h * dh:(h + 1) * dh] = matmul_serial(softmax(sc), np.ascontiguousarray(v.T))
        r0 += L
    return out


# ---- BERT model ------------------------------------------------------------------

class BertConfig(ctypes.Structure):
    _fields_ = [("vocab", ctypes.c_int), ("hidden", ctypes.c_int),
                ("layers", ctypes.c_int), ("heads", ctypes.c_int),
                ("inter", ctypes.c_int), ("max_pos", ctypes.c_int),
                ("type_vocab", ctypes.c_int), ("eps", ctypes.c_float),
                ("pooling", ctypes.c_int), ("normalize", ctypes.c_int),
                ("pos_off", ctypes.c_int), ("rel_buckets", ctypes.c_int)]


def rel_pos_bucket(rel, num_buckets=32):
    """relPosBucket (bert.go:123-150), the oracle's restatement."""
    return lib.or_rel_pos_bucket(rel, num_buckets)


LAYER_ORDER = [
    "attention.self.query.weight", "attention.self.query.bias",
    "attention.self.key.weight", "attention.self.key.bias",
    "attention.self.value.weight", "attention.self.value.bias",
    "attention.output.dense.weight", "attention.output.dense.bias",
    "attention.output.LayerNorm.weight", "attention.output.LayerNorm.bias",
    "intermediate.dense.weight", "intermediate.dense.bias",
    "output.dense.weight", "output.dense.bias",
    "output.LayerNorm.weight", "output.LayerNorm.bias",
]


class BertOracle:
    """The reference's per-text unpadded BERT forward on the CPU."""

    def __init__(self, shape, tensors, quant):
        """BERT/RoBERTa, DistilBERT (transformer.layer.N names, no token-type
        table) or MPNet (attention.attn names, relative-position bias), by
        shape.arch (bert.go:378-522)."""
        from rembed_amd.synthetic import layer_names
        self._keep = {k: f32(v) for k, v in tensors.items()}
        t = self._keep
        arch = getattr(shape, "arch", 0)
        rel = getattr(shape, "rel_buckets", 0)
        cfg = BertConfig(shape.vocab, shape.hidden, shape.layers, shape.heads,
                         shape.intermediate, shape.max_position, shape.type_vocab,
                         shape.eps, shape.pooling, shape.normalize,
                         getattr(shape, "position_offset", 0), rel)
        self.shape = shape
        layer_ptrs = [t[n].ctypes.data for l in range(shape.layers)
                      for n in layer_names(arch, l)]
        self._arr = (ctypes.c_void_p * len(layer_ptrs))(*layer_ptrs)
        tt = t.get("embeddings.token_type_embeddings.weight")
        self.h = lib.or_bert_create(
            ctypes.byref(cfg), quant,
            _p(t["embeddings.word_embeddings.weight"]),
            _p(t["embeddings.position_embeddings.weight"]),
            None if tt is None else _p(tt),
            _p(t["embeddings.LayerNorm.weight"]), _p(t["embeddings.LayerNorm.bias"]),
            ctypes.cast(self._arr, ctypes.c_void_p))
        if not self.h:
            raise RuntimeError("oracle: bad BERT config")
        if rel:
            lib.or_bert_set_rel_bias(self.h, _p(t["encoder.relative_attention_bias.weight"]))

    def close(self):
        if self.h:
            lib.or_bert_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def encode(self, ids, layers=None):
        """Final hidden states [len][H]; with `layers`, the hidden states
        after that many layers."""
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty((ids.shape[0], self.shape.hidden), np.float32)
        n = self.shape.layers if layers is None else layers
        st = lib.or_bert_encode_layers(self.h, _p(ids), ids.shape[0], _p(out), n)
        if st:
            raise RuntimeError(f"oracle encode status {st}")
        return out

    def forward(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty(self.shape.hidden, np.float32)
        st = lib.or_bert_forward(self.h, _p(ids), ids.shape[0], _p(out))
        if st:
            raise RuntimeError(f"oracle forward status {st}")
        return out

    def embed_batch(self, ids, lens, threads=1, secs=None):
        """One forward per text across `threads`; `secs` (float64 [batch])
        receives each text's forward time."""
        ids = np.ascontiguousarray(ids, np.int32)
        lens = np.ascontiguousarray(lens, np.int32)
        out = np.empty((ids.shape[0], self.shape.hidden), np.float32)
        st = lib.or_bert_embed_batch_timed(self.h, _p(ids), _p(lens), ids.shape[0],
                                           ids.shape[1], _p(out), threads,
                                           None if secs is None else _p(secs))
        if st:
            raise RuntimeError(f"oracle embed status {st}")
        return out


# ---- decoder-family embedders (Qwen3, EmbeddingGemma) ------------------------------

ARCH_QWEN3, ARCH_GEMMA3 = 1, 2


class DecConfig(ctypes.Structure):
    _fields_ = [("arch", ctypes.c_int), ("vocab", ctypes.c_int), ("hidden", ctypes.c_int),
                ("layers", ctypes.c_int), ("heads", ctypes.c_int), ("kv_heads", ctypes.c_int),
                ("head_dim", ctypes.c_int), ("inter", ctypes.c_int), ("eps", ctypes.c_float),
                ("rope_theta", ctypes.c_double), ("rope_local_theta", ctypes.c_double),
                ("sliding_window", ctypes.c_int), ("sliding_pattern", ctypes.c_int),
                ("query_pre_attn_scalar", ctypes.c_int), ("dense_hidden", ctypes.c_int),
                ("pooling", ctypes.c_int), ("normalize", ctypes.c_int), ("max_seq", ctypes.c_int)]


QWEN3_LAYER_ORDER = [
    "input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight",
    "self_attn.v_proj.weight", "self_attn.o_proj.weight", "self_attn.q_norm.weight",
    "self_attn.k_norm.weight", "post_attention_layernorm.weight", "mlp.gate_proj.weight",
    "mlp.up_proj.weight", "mlp.down_proj.weight",
]
GEMMA3_LAYER_ORDER = QWEN3_LAYER_ORDER[:8] + [
    "pre_feedforward_layernorm.weight", "post_feedforward_layernorm.weight",
    "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight",
]


class DecoderOracle:
    """The reference's per-text unpadded Qwen3 / EmbeddingGemma forward on the
    CPU (internal/model/qwen3.go, gemma3.go). `shape` is a
    rembed_amd.synthetic.DecoderShape; tensors use HF names (Gemma's Dense
    head as "2_Dense.linear.weight" / "3_Dense.linear.weight")."""

    def __init__(self, shape, tensors, quant):
        self._keep = {k: f32(v) for k, v in tensors.items()}
        t = self._keep
        gemma = shape.arch == ARCH_GEMMA3
        cfg = DecConfig(shape.arch, shape.vocab, shape.hidden, shape.layers, shape.heads,
                        shape.kv_heads, shape.head_dim, shape.intermediate, shape.eps,
                        shape.rope_theta, shape.rope_local_theta, shape.sliding_window,
                        shape.sliding_pattern, shape.query_pre_attn_scalar,
                        shape.dense_hidden, shape.pooling, shape.normalize, shape.max_seq)
        self.shape = shape
        order = GEMMA3_LAYER_ORDER if gemma else QWEN3_LAYER_ORDER
        ptrs = [t[f"layers.{l}.{n}"].ctypes.data for l in range(shape.layers) for n in order]
        self._arr = (ctypes.c_void_p * len(ptrs))(*ptrs)
        d1 = t.get("2_Dense.linear.weight")
        d2 = t.get("3_Dense.linear.weight")
        self.h = lib.or_dec_create(
            ctypes.byref(cfg), quant, _p(t["embed_tokens.weight"]), _p(t["norm.weight"]),
            ctypes.cast(self._arr, ctypes.c_void_p),
            _p(d1) if d1 is not None else None, _p(d2) if d2 is not None else None)
        if not self.h:
            raise RuntimeError("oracle: bad decoder config")

    def close(self):
        if self.h:
            lib.or_dec_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def quantized_kind(self):
        return lib.or_dec_quantized_kind(self.h)

    def encode(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty((ids.shape[0], self.shape.hidden), np.float32)
        st = lib.or_dec_encode(self.h, _p(ids), ids.shape[0], _p(out))
        if st:
            raise RuntimeError(f"oracle encode status {st}")
        return out

    def forward(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty(self.shape.hidden, np.float32)
        st = lib.or_dec_forward(self.h, _p(ids), ids.shape[0], _p(out))
        if st:
            raise RuntimeError(f"oracle forward status {st}")
        return out

    def embed_batch(self, ids, lens, threads=1, secs=None):
        """One forward per text across `threads`; `secs` (float64 [batch])
        receives each text's forward time."""
        ids = np.ascontiguousarray(ids, np.int32)
        lens = np.ascontiguousarray(lens, np.int32)
        out = np.empty((ids.shape[0], self.shape.hidden), np.float32)
        st = lib.or_dec_embed_batch_timed(self.h, _p(ids), _p(lens), ids.shape[0],
                                          ids.shape[1], _p(out), threads,
                                          None if secs is None else _p(secs))
        if st:
            raise RuntimeError(f"oracle embed status {st}")
        return out


# ---- bias-free RoPE encoders (nomic-embed, ModernBERT) ------------------------------

ARCH_NOMIC, ARCH_MODERNBERT = 3, 4


class RencConfig(ctypes.Structure):
    _fields_ = [("arch", ctypes.c_int), ("vocab", ctypes.c_int), ("hidden", ctypes.c_int),
                ("layers", ctypes.c_int), ("heads", ctypes.c_int), ("inter", ctypes.c_int),
                ("eps", ctypes.c_float), ("rope_theta", ctypes.c_double),
                ("rope_local_theta", ctypes.c_double), ("local_attention", ctypes.c_int),
                ("global_every", ctypes.c_int), ("pooling", ctypes.c_int),
                ("normalize", ctypes.c_int), ("max_seq", ctypes.c_int)]


NOMIC_LAYER_ORDER = [
    "attn.Wqkv.weight", "attn.out_proj.weight", "norm1.weight", "norm1.bias",
    "mlp.fc11.weight", "mlp.fc12.weight", "mlp.fc2.weight", "norm2.weight", "norm2.bias",
]
MODERNBERT_LAYER_ORDER = [
    "attn_norm.weight", "attn.Wqkv.weight", "attn.Wo.weight", "mlp_norm.weight",
    "mlp.Wi.weight", "mlp.Wo.weight",
]


class RopeEncoderOracle:
    """The reference's per-text unpadded nomic-embed / ModernBERT forward on
    the CPU (internal/model/nomic.go, modernbert.go). `shape` is a
    rembed_amd.synthetic.RopeEncoderShape; tensors use HF names."""

    def __init__(self, shape, tensors, quant):
        self._keep = {k: f32(v) for k, v in tensors.items()}
        t = self._keep
        mb = shape.arch == ARCH_MODERNBERT
        cfg = RencConfig(shape.arch, shape.vocab, shape.hidden, shape.layers, shape.heads,
                         shape.intermediate, shape.eps, shape.rope_theta,
                         shape.rope_local_theta, shape.local_attention, shape.global_every,
                         shape.pooling, shape.normalize, shape.max_seq)
        self.shape = shape
        if mb:
            ptrs = [t[f"layers.{l}.{n}"].ctypes.data if f"layers.{l}.{n}" in t else None
                    for l in range(shape.layers) for n in MODERNBERT_LAYER_ORDER]
            model = (t["embeddings.tok_embeddings.weight"], None, t["embeddings.norm.weight"],
                     None, t["final_norm.weight"])
        else:
            ptrs = [t[f"encoder.layers.{l}.{n}"].ctypes.data
                    for l in range(shape.layers) for n in NOMIC_LAYER_ORDER]
            model = (t["embeddings.word_embeddings.weight"],
                     t["embeddings.token_type_embeddings.weight"], t["emb_ln.weight"],
                     t["emb_ln.bias"], None)
        self._arr = (ctypes.c_void_p * len(ptrs))(*ptrs)
        self.h = lib.or_renc_create(ctypes.byref(cfg), quant,
                                    *[None if a is None else _p(a) for a in model],
                                    ctypes.cast(self._arr, ctypes.c_void_p))
        if not self.h:
            raise RuntimeError("oracle: bad RoPE encoder config")

    def close(self):
        if self.h:
            lib.or_renc_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def quantized_kind(self):
        return lib.or_renc_quantized_kind(self.h)

    def encode(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty((ids.shape[0], self.shape.hidden), np.float32)
        st = lib.or_renc_encode(self.h, _p(ids), ids.shape[0], _p(out))
        if st:
            raise RuntimeError(f"oracle encode status {st}")
        return out

    def forward(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty(self.shape.hidden, np.float32)
        st = lib.or_renc_forward(self.h, _p(ids), ids.shape[0], _p(out))
        if st:
            raise RuntimeError(f"oracle forward status {st}")
        return out

    def embed_batch(self, ids, lens, threads=1, secs=None):
        """One forward per text across `threads`; `secs` (float64 [batch])
        receives each text's forward time."""
        ids = np.ascontiguousarray(ids, np.int32)
        lens = np.ascontiguousarray(lens, np.int32)
        out = np.empty((ids.shape[0], self.shape.hidden), np.float32)
        st = lib.or_renc_embed_batch_timed(self.h, _p(ids), _p(lens), ids.shape[0],
                                           ids.shape[1], _p(out), threads,
                                           None if secs is None else _p(secs))
        if st:
            raise RuntimeError(f"oracle embed status {st}")
        return out


def rope_table(seq, dh, theta):
    c = np.empty((seq, dh // 2), np.float32)
    s = np.empty((seq, dh // 2), np.float32)
    lib.or_rope_table(_p(c), _p(s), seq, dh, float(theta))
    return c, s


def apply_rope(x, cos_t, sin_t):
    x = f32(x).copy()
    seq, dh = x.shape
    lib.or_apply_rope(_p(x), seq, dh, _p(f32(cos_t)), _p(f32(sin_t)))
    return x


def flash_causal_head(qh, kh, vh, scale):
    qh, kh, vh = f32(qh), f32(kh), f32(vh)
    seq, dh = qh.shape
    out = np.empty((seq, dh), np.float32)
    lib.or_flash_causal_head(_p(qh), _p(kh), _p(vh), _p(out), seq, dh, scale)
    return out
