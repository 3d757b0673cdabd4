"""Text to embeddings on the GPU: the WordPiece tokenizer's batch ids
(rh_tokenizer_encode_batch) fed straight to rh_model_embed, against the
oracle run on the same ids — the Embed path of the reference from text
(rembed.go:287-332: tokenize, then Forward). The vocabulary is synthetic
(no real vocab files offline), built from the reference's golden texts, and
the model is MiniLM-shaped with that vocabulary size."""
import dataclasses
import json
import os

import numpy as np
import pytest

from oracle import oracle as O
from rembed_amd.model import QUANT_NONE, QUANT_WEIGHTS, Model
from rembed_amd.synthetic import MINILM_L6, bert_tensors
from rembed_amd.tokenizer import WordPieceTokenizer

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("quant", [QUANT_NONE, QUANT_WEIGHTS], ids=["fp32", "w8"])
def test_text_to_embeddings(gpu_ctx, tmp_path, quant):
    from test_tokenizer import TEXTS, synthetic_vocab
    vocab = synthetic_vocab(TEXTS, True)
    path = tmp_path / "vocab.txt"
    path.write_bytes("\n".join(vocab).encode("utf-8"))
    tok = WordPieceTokenizer(str(path))
    ids, lens = tok.encode_batch(TEXTS, max_len=128)
    print(f"{len(TEXTS)} texts, {int(lens.sum())} tokens, vocab {len(vocab)}", flush=True)
    shape = dataclasses.replace(MINILM_L6, vocab=len(vocab), layers=2)
    t = bert_tensors(shape, seed=0x5EED0031)
    got = Model(gpu_ctx, shape, t, quant).embed(ids, lens)
    want = O.BertOracle(shape, t, quant).embed_batch(ids.astype(np.int32), lens, threads=8)
    if quant == QUANT_NONE:
        assert np.abs(got - want).max() <= 1e-4
    else:
        c = np.sum(got.astype(np.float64) * want, axis=1)
        assert c.min() >= 0.9999
