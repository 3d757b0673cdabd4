"""ctypes binding of librembed_hip.so (the C ABI in include/rembed_hip.h).

The shared library is the product; this module only declares its
signatures and turns non-zero status codes into exceptions. There is no
fallback: if the library is missing or fails to load, importing the binding
raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("REMBED_HIP_LIB", os.path.join(HERE, "librembed_hip.so"))

RH_OK = 0
RH_ERR_NO_DEVICE = 1
RH_ERR_INVALID = 2
RH_ERR_SHAPE = 3
RH_ERR_NONFINITE = 4
RH_ERR_HIP = 5
RH_ERR_OOM = 6
RH_ERR_VOCAB = 7
RH_ERR_SEQ = 8
RH_ERR_MISSING = 9

RH_MODE_F32, RH_MODE_W8, RH_MODE_A8W8 = 0, 1, 2
RH_QUANT_NONE, RH_QUANT_WEIGHTS, RH_QUANT_FULL = 0, 1, 2
RH_POOL_MEAN, RH_POOL_CLS, RH_POOL_LAST = 0, 1, 2
RH_ACT_NONE, RH_ACT_GELU, RH_ACT_SWIGLU, RH_ACT_GEGLU = 0, 1, 2, 3
RH_ACT_GEGLU_ERF = 4
RH_ARCH_BERT, RH_ARCH_QWEN3, RH_ARCH_GEMMA3, RH_ARCH_NOMIC, RH_ARCH_MODERNBERT = 0, 1, 2, 3, 4
RH_ARCH_DISTILBERT, RH_ARCH_MPNET = 5, 6
RH_OPT_ATTN_PRECISION = 1
RH_OPT_FUSED_FFN1 = 2
RH_OPT_PRODUCER_PLANES = 3
RH_OPT_STREAMS = 4
RH_OPT_QK_EPILOGUE = 5
RH_OPT_FUSE_PROJECTIONS = 6
RH_OPT_FUSED_LN = 7
RH_OPT_EXACT = 8
RH_OPT_GRAPH = 9
RH_CTX_F32_ALGO, RH_CTX_W8_TERMS, RH_CTX_I8_TILE, RH_CTX_BF_ALGO, RH_CTX_BF_TILE = 1, 2, 3, 4, 5
RH_CTX_TILE_GROUP = 6
RH_NOALLOC_SCRATCH_BYTES = 64 * 1024 * 1024

# Symbols the header declares (checked by the CPU test suite).
EXPORTS = [
    "rh_last_error", "rh_version", "rh_device_count", "rh_context_create",
    "rh_context_destroy", "rh_context_sync", "rh_context_stream",
    "rh_context_set_option", "rh_malloc", "rh_free", "rh_memcpy_h2d",
    "rh_memcpy_d2h", "rh_profile_enable", "rh_profile_read", "rh_pack_weight",
    "rh_pack_weight_gated", "rh_attention", "rh_attention_planes",
    "rh_weight_destroy", "rh_weight_info", "rh_weight_export",
    "rh_quantize_rows_u8", "rh_gelu_quantize_rows_u8", "rh_matmul", "rh_matmul_packed", "rh_matmul_packed8",
    "rh_matmul_packed_vnni", "rh_gemm_u8s8_i32", "rh_linear", "rh_linear_u8",
    "rh_linear_noalloc", "rh_gelu",
    "rh_layernorm", "rh_model_create", "rh_model_set_tensor",
    "rh_model_finalize", "rh_model_share", "rh_model_destroy", "rh_model_set_option",
    "rh_model_quantized", "rh_model_quantized_activations", "rh_model_embed",
    "rh_model_embed_tokens", "rh_model_embed_device", "rh_model_check",
    "rh_tokenizer_wordpiece_load", "rh_tokenizer_bpe_load", "rh_tokenizer_bpe_load_json",
    "rh_tokenizer_sentencepiece_load", "rh_tokenizer_sentencepiece_normalize",
    "rh_tokenizer_gemma_load",
    "rh_tokenizer_vocab_size", "rh_tokenizer_encode",
    "rh_tokenizer_encode_batch", "rh_tokenizer_destroy",
]


class RembedError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class ModelConfig(ctypes.Structure):
    _fields_ = [
        ("arch", ctypes.c_int), ("hidden", ctypes.c_int), ("layers", ctypes.c_int),
        ("heads", ctypes.c_int), ("intermediate", ctypes.c_int),
        ("vocab", ctypes.c_int), ("max_position", ctypes.c_int),
        ("position_offset", ctypes.c_int), ("type_vocab", ctypes.c_int),
        ("layer_norm_eps", ctypes.c_float), ("pooling", ctypes.c_int),
        ("normalize", ctypes.c_int),
        ("kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
        ("rope_theta", ctypes.c_double), ("rope_local_theta", ctypes.c_double),
        ("sliding_window", ctypes.c_int), ("sliding_pattern", ctypes.c_int),
        ("query_pre_attn_scalar", ctypes.c_int), ("dense_hidden", ctypes.c_int),
        ("rel_buckets", ctypes.c_int), ("reserved", ctypes.c_int * 7),
    ]


class ProfileStat(ctypes.Structure):
    _fields_ = [("launches", ctypes.c_int64), ("total_ms", ctypes.c_double),
                ("total_ops", ctypes.c_double), ("total_bytes", ctypes.c_double)]


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `python -m rembed_amd.build` "
            "(the HIP path has no fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    P = ctypes.c_void_p
    I = ctypes.c_int
    F = ctypes.c_float
    S = ctypes.c_size_t
    sig = {
        "rh_last_error": (ctypes.c_char_p, []),
        "rh_version": (I, []),
        "rh_device_count": (I, [ctypes.POINTER(I)]),
        "rh_context_create": (I, [I, ctypes.POINTER(P)]),
        "rh_context_destroy": (None, [P]),
        "rh_context_sync": (I, [P]),
        "rh_context_stream": (P, [P]),
        "rh_context_set_option": (I, [P, I, I]),
        "rh_malloc": (I, [P, S, ctypes.POINTER(P)]),
        "rh_free": (I, [P, P]),
        "rh_memcpy_h2d": (I, [P, P, P, S]),
        "rh_memcpy_d2h": (I, [P, P, P, S]),
        "rh_profile_enable": (I, [P, I]),
        "rh_profile_read": (I, [P, I, ctypes.POINTER(ProfileStat)]),
        "rh_pack_weight": (I, [P, I, P, P, I, I, ctypes.POINTER(P)]),
        "rh_pack_weight_gated": (I, [P, I, P, P, I, I, ctypes.POINTER(P)]),
        "rh_attention_planes": (I, [P, P, P, I, I, I, I, P, I, I, I, I, I, ctypes.c_float, I, I,
                                    P, I]),
        "rh_attention": (I, [P, P, I, I, I, I, I, P, I, I, I, I, I, ctypes.c_float, I, I, I, P,
                             I]),
        "rh_weight_destroy": (None, [P]),
        "rh_weight_info": (I, [P, ctypes.POINTER(I), ctypes.POINTER(I), ctypes.POINTER(I)]),
        "rh_weight_export": (I, [P, P, P, P]),
        "rh_quantize_rows_u8": (I, [P, P, I, I, P, I, P]),
        "rh_gelu_quantize_rows_u8": (I, [P, P, I, I, P, I, P]),
        "rh_matmul": (I, [P, P, P, P, I, I, I]),
        "rh_matmul_packed": (I, [P, P, P, P, I]),
        "rh_matmul_packed8": (I, [P, P, P, P, I]),
        "rh_matmul_packed_vnni": (I, [P, P, P, P, I, P, I, P]),
        "rh_gemm_u8s8_i32": (I, [P, P, P, I, P, I]),
        "rh_linear": (I, [P, P, P, P, I, I, P, I, P]),
        "rh_linear_u8": (I, [P, P, I, P, P, I, I, P, I, P, P]),
        "rh_linear_noalloc": (I, [P, P, P, P, I, I]),
        "rh_gelu": (I, [P, P, S]),
        "rh_layernorm": (I, [P, P, P, P, I, I, F]),
        "rh_model_create": (I, [P, ctypes.POINTER(ModelConfig), I, ctypes.POINTER(P)]),
        "rh_model_set_tensor": (I, [P, ctypes.c_char_p, P, P, I]),
        "rh_model_finalize": (I, [P]),
        "rh_model_share": (I, [P, P, ctypes.POINTER(P)]),
        "rh_model_destroy": (None, [P]),
        "rh_model_set_option": (I, [P, I, I]),
        "rh_model_quantized": (I, [P]),
        "rh_model_quantized_activations": (I, [P]),
        "rh_model_embed": (I, [P, P, P, I, I, P]),
        "rh_model_embed_tokens": (I, [P, P, P, I, I, P]),
        "rh_model_embed_device": (I, [P, P, P, I, I, P]),
        "rh_model_check": (I, [P]),
        "rh_tokenizer_wordpiece_load": (I, [ctypes.c_char_p, I, ctypes.c_char_p,
                                            ctypes.c_char_p, ctypes.c_char_p,
                                            ctypes.POINTER(P)]),
        "rh_tokenizer_bpe_load": (I, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p,
                                      ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(P)]),
        "rh_tokenizer_bpe_load_json": (I, [ctypes.c_char_p, I, ctypes.c_char_p,
                                           ctypes.c_char_p, ctypes.c_char_p,
                                           ctypes.POINTER(P)]),
        "rh_tokenizer_sentencepiece_load": (I, [ctypes.c_char_p, ctypes.POINTER(P)]),
        "rh_tokenizer_gemma_load": (I, [ctypes.c_char_p, ctypes.POINTER(P)]),
        "rh_tokenizer_sentencepiece_normalize": (I, [P, ctypes.c_char_p, S, P, S,
                                                     ctypes.POINTER(S)]),
        "rh_tokenizer_vocab_size": (ctypes.c_int64, [P]),
        "rh_tokenizer_encode": (I, [P, ctypes.c_char_p, S, I, P, I, ctypes.POINTER(I)]),
        "rh_tokenizer_encode_batch": (I, [P, P, P, I, I, ctypes.c_int64, P, P]),
        "rh_tokenizer_destroy": (None, [P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def hip_runtime():
    """The HIP runtime instance this library is linked against, for host
    calls beside it (events on its stream, memory queries). Opened by its
    soname, so the dynamic loader returns the copy already mapped for the
    library; a lookup by file name could map a second runtime (another
    package may ship a libamdhip64.so of its own) that shares no state with
    the library's streams or devices."""
    return ctypes.CDLL("libamdhip64.so.7")


def check(code):
    """Raise RembedError for a non-zero status."""
    if code != RH_OK:
        raise RembedError(code, lib.rh_last_error().decode(errors="replace"))
    return code
