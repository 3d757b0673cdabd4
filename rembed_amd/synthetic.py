"""Deterministic synthetic BERT-family weights and token batches.

There are no checkpoints or datasets offline, so the benchmark and the parity
tests use random-init weights of the real architectures and random token ids:

* linear weights, biases and embedding tables ~ N(0, 0.02) in float32;
* LayerNorm gammas 1 + N(0, 0.02) and betas N(0, 0.02) (drawing gammas
  from N(0, 0.02) itself would shrink every post-LN activation ~50x and make
  the fp32 and int8 checks nearly vacuous);
* token ids uniform in [id_lo, vocab), lengths uniform in [len_lo, len_hi].

Tensor names are Hugging Face BertModel names (what rembed's loader reads,
internal/model/bert.go:378-460).
"""
from dataclasses import dataclass

import numpy as np


ARCH_BERT, ARCH_DISTILBERT, ARCH_MPNET = 0, 5, 6  # RH_ARCH_* of the BERT family


@dataclass(frozen=True)
class BertShape:
    name: str
    layers: int
    hidden: int
    heads: int
    intermediate: int
    vocab: int = 30522
    max_position: int = 512
    type_vocab: int = 2
    eps: float = 1e-12
    pooling: int = 0      # 0 mean, 1 cls, 2 last
    normalize: int = 1
    arch: int = ARCH_BERT  # BERT / RoBERTa, DistilBERT or MPNet names and attention
    position_offset: int = 0  # Config.PositionOffset (config.go:84-89)
    rel_buckets: int = 0  # MPNet's relative-position bias buckets


MINILM_L6 = BertShape("minilm-l6", 6, 384, 12, 1536, pooling=0)
BERT_BASE = BertShape("bert-base", 12, 768, 12, 3072, pooling=1)
# multi-qa-distilbert-cos-v1 / all-mpnet-base-v2 shapes (the reference's
# testdata goldens for the two architectures); DistilBERT has no token-type
# table, MPNet neither, and MPNet's position rows start past pad_token_id = 1
# (config.go:84-89) with 32 relative-position buckets (config.go:219-224).
DISTILBERT_BASE = BertShape("distilbert-base", 6, 768, 12, 3072, type_vocab=0, pooling=1,
                            arch=ARCH_DISTILBERT)
MPNET_BASE = BertShape("mpnet-base", 12, 768, 12, 3072, vocab=30527, max_position=514,
                       type_vocab=0, eps=1e-5, pooling=0, arch=ARCH_MPNET, position_offset=2,
                       rel_buckets=32)


def layer_names(arch, l):
    """The 16 per-layer tensor names, in the order q_w q_b k_w k_b v_w v_b
    o_w o_b ln1_g ln1_b f1_w f1_b f2_w f2_b ln2_g ln2_b (bert.go:399-470)."""
    if arch == ARCH_DISTILBERT:
        p = f"transformer.layer.{l}."
        attn = [p + f"attention.{n}_lin.{w}" for n in ("q", "k", "v", "out") for w in ("weight", "bias")]
        return attn + [p + "sa_layer_norm.weight", p + "sa_layer_norm.bias",
                       p + "ffn.lin1.weight", p + "ffn.lin1.bias",
                       p + "ffn.lin2.weight", p + "ffn.lin2.bias",
                       p + "output_layer_norm.weight", p + "output_layer_norm.bias"]
    p = f"encoder.layer.{l}."
    if arch == ARCH_MPNET:
        attn = [p + f"attention.attn.{n}.{w}" for n in ("q", "k", "v", "o") for w in ("weight", "bias")]
        ln1 = [p + "attention.LayerNorm.weight", p + "attention.LayerNorm.bias"]
    else:
        attn = [p + f"attention.self.{n}.{w}" for n in ("query", "key", "value")
                for w in ("weight", "bias")]
        attn += [p + "attention.output.dense.weight", p + "attention.output.dense.bias"]
        ln1 = [p + "attention.output.LayerNorm.weight", p + "attention.output.LayerNorm.bias"]
    return attn + ln1 + [p + "intermediate.dense.weight", p + "intermediate.dense.bias",
                         p + "output.dense.weight", p + "output.dense.bias",
                         p + "output.LayerNorm.weight", p + "output.LayerNorm.bias"]


def bert_tensors(shape: BertShape, seed: int = 0x5EED0001):
    """HF-named float32 tensors for a BERT-family encoder."""
    rng = np.random.Generator(np.random.PCG64(seed))
    H, I = shape.hidden, shape.intermediate

    def normal(*dims):
        return (rng.standard_normal(dims, dtype=np.float32) * np.float32(0.02))

    def gamma(n):
        return (np.float32(1.0) + normal(n)).astype(np.float32)

    t = {
        "embeddings.word_embeddings.weight": normal(shape.vocab, H),
        "embeddings.position_embeddings.weight": normal(shape.max_position, H),
    }
    if shape.type_vocab:
        t["embeddings.token_type_embeddings.weight"] = normal(shape.type_vocab, H)
    t["embeddings.LayerNorm.weight"] = gamma(H)
    t["embeddings.LayerNorm.bias"] = normal(H)
    for l in range(shape.layers):
        names = layer_names(shape.arch, l)
        dims = [(H, H), (H,)] * 4 + [None, None, (I, H), (I,), (H, I), (H,), None, None]
        for nm, d in zip(names, dims):
            t[nm] = gamma(H) if d is None and nm.endswith("weight") else (
                normal(H) if d is None else normal(*d))
    if shape.rel_buckets:
        # MPNet's bias table, scaled like a trained one (O(1) logits) so it
        # moves the softmax
        t["encoder.relative_attention_bias.weight"] = normal(shape.rel_buckets, shape.heads) * 25
    return t


def token_batch(batch, stride, len_lo, len_hi, vocab=30522, id_lo=1000,
                seed=0x5EED0002):
    """Padded ids [batch][stride] (int32, pad = 0) and lengths [batch]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    lens = rng.integers(len_lo, len_hi + 1, size=batch).astype(np.int32)
    ids = np.zeros((batch, stride), np.int32)
    for b in range(batch):
        ids[b, : lens[b]] = rng.integers(id_lo, vocab, size=lens[b])
    return ids, lens



# ---- decoder-family embedders (Qwen3, EmbeddingGemma) ------------------------------

ARCH_QWEN3, ARCH_GEMMA3 = 1, 2


@dataclass(frozen=True)
class DecoderShape:
    """Config of a Qwen3 / EmbeddingGemma embedder (internal/model/config.go:56-77)."""
    name: str
    arch: int
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    eps: float = 1e-6
    rope_theta: float = 1e6           # Qwen3 RopeTheta / Gemma GlobalRopeTheta
    rope_local_theta: float = 1e4     # Gemma LocalRopeTheta
    sliding_window: int = 0           # Gemma effective window: |i-j| < w
    sliding_pattern: int = 1          # Gemma: layer l global iff (l+1) % pattern == 0
    query_pre_attn_scalar: int = 0    # Gemma attention scale 1/sqrt(scalar)
    dense_hidden: int = 0             # Gemma Dense head width
    pooling: int = 2                  # 0 mean, 1 cls, 2 last token
    normalize: int = 1
    max_seq: int = 32768


# Qwen3-Embedding-0.6B-shaped: 28 layers, hidden 1024, 16 Q / 8 KV heads of 128,
# SwiGLU 3072, RoPE theta 1e6, last-token pooling.
QWEN3_0_6B = DecoderShape("qwen3-0.6b", ARCH_QWEN3, 28, 1024, 16, 8, 128, 3072, 151669)
# EmbeddingGemma-300m-shaped: 24 layers, hidden 768, 3 Q / 1 KV heads of 256,
# GeGLU 1152, alternating sliding-window-512 (effective 257) / global layers,
# mean pooling + Dense 768 -> 3072 -> 768.
GEMMA3_300M = DecoderShape("embeddinggemma-300m", ARCH_GEMMA3, 24, 768, 3, 1, 256, 1152,
                           262144, rope_theta=1e6, rope_local_theta=1e4,
                           sliding_window=257, sliding_pattern=6,
                           query_pre_attn_scalar=256, dense_hidden=3072, pooling=0)


def decoder_tensors(shape: DecoderShape, seed: int = 0x5EED0001, bf16: bool = False):
    """HF-named float32 tensors for a Qwen3 / Gemma3 backbone: projections and
    the embedding table N(0, 0.02) (rounded through bf16 when `bf16`, as a
    BF16 checkpoint widens, internal/safetensors/safetensors.go:199-203);
    Qwen3 RMSNorm weights 1 + N(0, 0.02); Gemma norm weights N(0, 0.02)
    (the checkpoint form, unit offset added at load)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    H, I, dh = shape.hidden, shape.intermediate, shape.head_dim
    qdim, kvdim = shape.heads * dh, shape.kv_heads * dh
    gemma = shape.arch == ARCH_GEMMA3

    def normal(*dims):
        w = rng.standard_normal(dims, dtype=np.float32) * np.float32(0.02)
        if bf16:
            w = (w.view(np.uint32) + np.uint32(0x7FFF) + ((w.view(np.uint32) >> 16) & 1)
                 ) & np.uint32(0xFFFF0000)
            w = w.view(np.float32)
        return w.astype(np.float32)

    def norm(n):
        w = rng.standard_normal(n, dtype=np.float32) * np.float32(0.02)
        return (w if gemma else np.float32(1.0) + w).astype(np.float32)

    t = {"embed_tokens.weight": normal(shape.vocab, H), "norm.weight": norm(H)}
    for l in range(shape.layers):
        p = f"layers.{l}."
        t[p + "input_layernorm.weight"] = norm(H)
        t[p + "self_attn.q_proj.weight"] = normal(qdim, H)
        t[p + "self_attn.k_proj.weight"] = normal(kvdim, H)
        t[p + "self_attn.v_proj.weight"] = normal(kvdim, H)
        t[p + "self_attn.o_proj.weight"] = normal(H, qdim)
        t[p + "self_attn.q_norm.weight"] = norm(dh)
        t[p + "self_attn.k_norm.weight"] = norm(dh)
        t[p + "post_attention_layernorm.weight"] = norm(H)
        if gemma:
            t[p + "pre_feedforward_layernorm.weight"] = norm(H)
            t[p + "post_feedforward_layernorm.weight"] = norm(H)
        t[p + "mlp.gate_proj.weight"] = normal(I, H)
        t[p + "mlp.up_proj.weight"] = normal(I, H)
        t[p + "mlp.down_proj.weight"] = normal(H, I)
    if gemma and shape.dense_hidden:
        t["2_Dense.linear.weight"] = normal(shape.dense_hidden, H)
        t["3_Dense.linear.weight"] = normal(H, shape.dense_hidden)
    return t


# ---- bias-free RoPE encoders (nomic-embed, ModernBERT) ----------------------------

ARCH_NOMIC, ARCH_MODERNBERT = 3, 4


@dataclass(frozen=True)
class RopeEncoderShape:
    """Config of a nomic-embed / ModernBERT encoder (internal/model/config.go:44-53,
    130-148,163-175); head_dim = hidden / heads."""
    name: str
    arch: int
    layers: int
    hidden: int
    heads: int
    intermediate: int
    vocab: int
    eps: float = 1e-12
    rope_theta: float = 1000.0     # nomic RopeTheta / ModernBERT GlobalRopeTheta
    rope_local_theta: float = 0.0  # ModernBERT LocalRopeTheta
    local_attention: int = 0       # ModernBERT: local layers keep |i-j| <= local_attention/2
    global_every: int = 1          # ModernBERT: layer l is global iff l % global_every == 0
    pooling: int = 0               # 0 mean, 1 cls, 2 last token
    normalize: int = 1
    max_seq: int = 8192

    @property
    def head_dim(self):
        return self.hidden // self.heads


# nomic-embed-text-v1.5-shaped: 12 layers, hidden 768, 12 heads of 64, SwiGLU
# 3072, RoPE base 1000, mean pooling.
NOMIC_V15 = RopeEncoderShape("nomic-embed-text-v1.5", ARCH_NOMIC, 12, 768, 12, 3072, 30528,
                             eps=1e-12, rope_theta=1000.0)
# modernbert-embed-base-shaped: 22 layers, hidden 768, 12 heads of 64, GeGLU
# 1152, every third layer global (theta 160000), the others local within ±64
# tokens (theta 10000), mean pooling.
MODERNBERT_BASE = RopeEncoderShape("modernbert-embed-base", ARCH_MODERNBERT, 22, 768, 12, 1152,
                                   50368, eps=1e-5, rope_theta=160000.0,
                                   rope_local_theta=10000.0, local_attention=128,
                                   global_every=3)


def rope_encoder_tensors(shape: RopeEncoderShape, seed: int = 0x5EED0001, std: float = 0.02):
    """HF-named float32 tensors of a nomic-embed (internal/model/nomic.go:33-110)
    or ModernBERT (internal/model/modernbert.go:34-104) encoder: projections
    and embedding tables N(0, std), LayerNorm gammas 1 + N(0, std), nomic's
    betas N(0, std); ModernBERT's layer 0 has no attention norm. (A larger
    std on a small hidden size makes every sublayer move the output, for
    tests that must see each one.)"""
    rng = np.random.Generator(np.random.PCG64(seed))
    H, I = shape.hidden, shape.intermediate

    def normal(*dims):
        return rng.standard_normal(dims, dtype=np.float32) * np.float32(std)

    def gamma(n):
        return (np.float32(1.0) + normal(n)).astype(np.float32)

    if shape.arch == ARCH_NOMIC:
        t = {
            "embeddings.word_embeddings.weight": normal(shape.vocab, H),
            "embeddings.token_type_embeddings.weight": normal(2, H),
            "emb_ln.weight": gamma(H),
            "emb_ln.bias": normal(H),
        }
        for l in range(shape.layers):
            p = f"encoder.layers.{l}."
            t[p + "attn.Wqkv.weight"] = normal(3 * H, H)
            t[p + "attn.out_proj.weight"] = normal(H, H)
            t[p + "norm1.weight"] = gamma(H)
            t[p + "norm1.bias"] = normal(H)
            t[p + "mlp.fc11.weight"] = normal(I, H)
            t[p + "mlp.fc12.weight"] = normal(I, H)
            t[p + "mlp.fc2.weight"] = normal(H, I)
            t[p + "norm2.weight"] = gamma(H)
            t[p + "norm2.bias"] = normal(H)
        return t
    t = {
        "embeddings.tok_embeddings.weight": normal(shape.vocab, H),
        "embeddings.norm.weight": gamma(H),
        "final_norm.weight": gamma(H),
    }
    for l in range(shape.layers):
        p = f"layers.{l}."
        if l:
            t[p + "attn_norm.weight"] = gamma(H)
        t[p + "attn.Wqkv.weight"] = normal(3 * H, H)
        t[p + "attn.Wo.weight"] = normal(H, H)
        t[p + "mlp_norm.weight"] = gamma(H)
        t[p + "mlp.Wi.weight"] = normal(2 * I, H)
        t[p + "mlp.Wo.weight"] = normal(H, I)
    return t
