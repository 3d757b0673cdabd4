"""Python mirror of rembed's encoder API over the C ABI.

Model follows internal/model (Load, Forward/ForwardTokens, Quantized,
QuantizedActivations); embed()/embed_tokens() take token ids the way
Embedder.Embed/EmbedTokens feed them (rembed.go:287-411), batched.
"""
import ctypes
import os
import sys

import numpy as np

from . import _lib
from ._lib import check, lib

QUANT_NONE = _lib.RH_QUANT_NONE       # default fp32
QUANT_WEIGHTS = _lib.RH_QUANT_WEIGHTS  # WithInt8 (rembed.go:67-69)
QUANT_FULL = _lib.RH_QUANT_FULL        # WithInt8Activations (rembed.go:79-81)
ARCH_BERT, ARCH_QWEN3, ARCH_GEMMA3 = _lib.RH_ARCH_BERT, _lib.RH_ARCH_QWEN3, _lib.RH_ARCH_GEMMA3
ARCH_NOMIC, ARCH_MODERNBERT = _lib.RH_ARCH_NOMIC, _lib.RH_ARCH_MODERNBERT
ARCH_DISTILBERT, ARCH_MPNET = _lib.RH_ARCH_DISTILBERT, _lib.RH_ARCH_MPNET


def make_config(shape):
    """rh_model_config from a synthetic.BertShape, DecoderShape or
    RopeEncoderShape."""
    c = _lib.ModelConfig()
    c.arch = getattr(shape, "arch", _lib.RH_ARCH_BERT)
    c.hidden = shape.hidden
    c.layers = shape.layers
    c.heads = shape.heads
    c.intermediate = shape.intermediate
    c.vocab = shape.vocab
    c.layer_norm_eps = shape.eps
    c.pooling = shape.pooling
    c.normalize = shape.normalize
    if c.arch in (_lib.RH_ARCH_BERT, _lib.RH_ARCH_DISTILBERT, _lib.RH_ARCH_MPNET):
        c.max_position = shape.max_position
        c.position_offset = getattr(shape, "position_offset", 0)
        c.type_vocab = shape.type_vocab
        c.rel_buckets = getattr(shape, "rel_buckets", 0)
    elif c.arch in (_lib.RH_ARCH_NOMIC, _lib.RH_ARCH_MODERNBERT):  # config.go:44-53,163-175
        c.max_position = shape.max_seq
        c.head_dim = shape.head_dim
        c.rope_theta = shape.rope_theta
        c.rope_local_theta = shape.rope_local_theta
        c.sliding_window = shape.local_attention
        c.sliding_pattern = shape.global_every
        c.type_vocab = 2 if c.arch == _lib.RH_ARCH_NOMIC else 0
    else:  # Qwen3 / Gemma3 (config.go:56-77)
        c.max_position = shape.max_seq
        c.kv_heads = shape.kv_heads
        c.head_dim = shape.head_dim
        c.rope_theta = shape.rope_theta
        c.rope_local_theta = shape.rope_local_theta
        c.sliding_window = shape.sliding_window
        c.sliding_pattern = shape.sliding_pattern
        c.query_pre_attn_scalar = shape.query_pre_attn_scalar
        c.dense_hidden = shape.dense_hidden
    return c


class Model:
    """A loaded encoder resident in HBM (rh_model)."""

    def __init__(self, ctx, shape, tensors, quant=QUANT_NONE, fuse_projections=True):
        self.ctx = ctx
        self.shape = shape
        cfg = make_config(shape)
        h = ctypes.c_void_p()
        check(lib.rh_model_create(ctx.h, ctypes.byref(cfg), quant, ctypes.byref(h)))
        self.h = h
        try:
            if not fuse_projections:
                self.set_fuse_projections(False)
            for name, arr in tensors.items():
                arr = np.ascontiguousarray(arr, dtype=np.float32)
                dims = (ctypes.c_int64 * arr.ndim)(*arr.shape)
                check(lib.rh_model_set_tensor(h, name.encode(), arr.ctypes.data,
                                              dims, arr.ndim))
            check(lib.rh_model_finalize(h))
        except Exception:
            self.close()
            raise

    @classmethod
    def from_safetensors(cls, ctx, shape, path, quant=QUANT_NONE, **kw):
        """model.Load (bert.go:307-524) over `path`: a model directory
        (model.safetensors, or the shards its model.safetensors.index.json
        names, safetensors.go:54-121; for Gemma also 2_Dense/ and 3_Dense/,
        gemma3.go:144-172) or one .safetensors file. Every tensor is widened
        to float32 and handed over by name; the library fuses projections and
        packs on finalize."""
        from . import checkpoint
        if os.path.isdir(path):
            dense = getattr(shape, "dense_hidden", 0)
            t = checkpoint.load_model_dir(path, dense, shape.hidden)
        else:
            t = checkpoint.load_any(path)
        return cls(ctx, shape, t, quant, **kw)

    def share(self, ctx):
        """Another Model over these weights, bound to `ctx` (same device):
        the weights stay in HBM once and the two run concurrently on their
        own streams (rh_model_share). Close them in any order."""
        h = ctypes.c_void_p()
        check(lib.rh_model_share(self.h, ctx.h, ctypes.byref(h)))
        other = Model.__new__(Model)
        other.ctx, other.shape, other.h = ctx, self.shape, h
        return other

    def close(self):
        if getattr(self, "h", None):
            lib.rh_model_destroy(self.h)
            self.h = None

    def __del__(self):
        if sys.is_finalizing():
            return  # the HIP runtime may already be torn down
        try:
            self.close()
        except Exception:
            pass

    def set_attention_precision(self, prec):
        check(lib.rh_model_set_option(self.h, _lib.RH_OPT_ATTN_PRECISION, prec))

    def set_exact(self, on=True):
        """RH_OPT_EXACT (BERT family): LayerNorm's sums and attention in the
        reference's own float32 order, so a full-int8 forward is
        byte-identical to the reference's (False: the default kernels)."""
        check(lib.rh_model_set_option(self.h, _lib.RH_OPT_EXACT, 1 if on else 0))

    def set_graph(self, on=True):
        """RH_OPT_GRAPH (BERT family): record a forward once per batch shape
        as a HIP graph and replay it (identical results)."""
        check(lib.rh_model_set_option(self.h, _lib.RH_OPT_GRAPH, 1 if on else 0))

    def set_fused_ln(self, on=True):
        """RH_OPT_FUSED_LN: full-int8 O / FFN2 projections finish the
        residual add + LayerNorm in their epilogue (identical results)."""
        check(lib.rh_model_set_option(self.h, _lib.RH_OPT_FUSED_LN, 1 if on else 0))

    def set_fused_ffn1(self, mode):
        """RH_OPT_FUSED_FFN1 (full int8): 0 / False = fp32 FFN1 rows, then
        GELU + QuantizeRowU8 as a separate pass; 1 / True = two GEMM passes
        (row |max|, then the u8 bytes); 2 = one pass whose workgroups meet
        per row block on the row |max|. Identical bytes in every mode."""
        mode = int(mode)
        check(lib.rh_model_set_option(self.h, _lib.RH_OPT_FUSED_FFN1, mode))

    def set_producer_planes(self, on=True):
        """Weight-only int8 / fp32 GEMM inputs written as bf16 planes by their
        producers (True, default) or split by each GEMM (False); same values."""
        check(lib.rh_model_set_option(self.h, _lib.RH_OPT_PRODUCER_PLANES, 1 if on else 0))

    def set_streams(self, n):
        """n = 1..4 (default 2): a batch runs as up to n parts of whole texts
        (>= 2048 tokens each) on as many streams when no GEMM needs the
        context's split workspace; 1: one stream. Same results."""
        check(lib.rh_model_set_option(self.h, _lib.RH_OPT_STREAMS, n))

    def set_fuse_projections(self, on=True):
        """Decoders, before finalize: q|k|v and gate|up packed as one weight
        each where their modes agree (True, default), or as separate weights
        like the reference (False); same results."""
        check(lib.rh_model_set_option(self.h, _lib.RH_OPT_FUSE_PROJECTIONS, 1 if on else 0))

    def set_qk_epilogue(self, on=True):
        """Decoders: QK-norm + RoPE in the q|k|v GEMM's epilogue (True,
        where the shape allows) or a separate pass (False, the default:
        measured faster); same results."""
        check(lib.rh_model_set_option(self.h, _lib.RH_OPT_QK_EPILOGUE, 1 if on else 0))

    def quantized(self):
        return bool(lib.rh_model_quantized(self.h))

    def quantized_activations(self):
        return bool(lib.rh_model_quantized_activations(self.h))

    @staticmethod
    def _pack(ids, lens):
        """int64 id rows [batch][stride] and int32 lengths, as the C ABI takes
        them (the reference's ids are []int64, bert.go:649)."""
        if lens is None:  # list of sequences
            seqs = [np.asarray(s, np.int64) for s in ids]
            lens = np.array([len(s) for s in seqs], np.int32)
            stride = max(1, int(lens.max())) if len(seqs) else 1
            arr = np.zeros((len(seqs), stride), np.int64)
            for i, s in enumerate(seqs):
                arr[i, : len(s)] = s
            return arr, lens
        ids = np.ascontiguousarray(ids, np.int64)
        lens = np.ascontiguousarray(lens, np.int32)
        if ids.ndim != 2:
            raise ValueError(f"ids must be [batch][stride], got shape {ids.shape}")
        if lens.ndim != 1 or lens.shape[0] != ids.shape[0]:
            raise ValueError(f"lens must hold one length per row of ids "
                             f"({ids.shape[0]}), got shape {lens.shape}")
        return ids, lens

    def embed(self, ids, lens=None):
        """Pooled (and L2-normalized per config) vectors, [batch][H]."""
        ids, lens = self._pack(ids, lens)
        out = np.empty((ids.shape[0], self.shape.hidden), np.float32)
        check(lib.rh_model_embed(self.h, ids.ctypes.data, lens.ctypes.data,
                                 ids.shape[0], ids.shape[1], out.ctypes.data))
        return out

    def embed_tokens(self, ids, lens=None):
        """Per-token final hidden states, one [len][H] array per text."""
        ids, lens = self._pack(ids, lens)
        tot = int(lens.sum())
        out = np.empty((tot, self.shape.hidden), np.float32)
        check(lib.rh_model_embed_tokens(self.h, ids.ctypes.data, lens.ctypes.data,
                                        ids.shape[0], ids.shape[1], out.ctypes.data))
        offs = np.concatenate([[0], np.cumsum(lens)])
        return [out[offs[i]: offs[i + 1]] for i in range(len(lens))]

    def embed_device(self, ids_dev, lens, batch, stride, out_dev):
        """Enqueue a forward over HBM-resident ids; no host sync."""
        lens = np.ascontiguousarray(lens, np.int32)
        check(lib.rh_model_embed_device(self.h, ids_dev.ptr, lens.ctypes.data, batch,
                                        stride, out_dev.ptr))

    def check(self):
        """rh_model_check: waits for the model's work and reports a device-side
        error (an out-of-range token id, a one-pass FFN1 wait that timed out)."""
        check(lib.rh_model_check(self.h))
