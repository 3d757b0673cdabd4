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


MINILM_L6 = BertShape("minilm-l6", 6, 384, 12, 1536, pooling=0)
BERT_BASE = BertShape("bert-base", 12, 768, 12, 3072, pooling=1)


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
        "embeddings.token_type_embeddings.weight": normal(shape.type_vocab, H),
        "embeddings.LayerNorm.weight": gamma(H),
        "embeddings.LayerNorm.bias": normal(H),
    }
    for l in range(shape.layers):
        p = f"encoder.layer.{l}."
        for nm in ("query", "key", "value"):
            t[p + f"attention.self.{nm}.weight"] = normal(H, H)
            t[p + f"attention.self.{nm}.bias"] = normal(H)
        t[p + "attention.output.dense.weight"] = normal(H, H)
        t[p + "attention.output.dense.bias"] = normal(H)
        t[p + "attention.output.LayerNorm.weight"] = gamma(H)
        t[p + "attention.output.LayerNorm.bias"] = normal(H)
        t[p + "intermediate.dense.weight"] = normal(I, H)
        t[p + "intermediate.dense.bias"] = normal(I)
        t[p + "output.dense.weight"] = normal(H, I)
        t[p + "output.dense.bias"] = normal(H)
        t[p + "output.LayerNorm.weight"] = gamma(H)
        t[p + "output.LayerNorm.bias"] = normal(H)
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

