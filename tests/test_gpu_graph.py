"""The BERT-family forward recorded as a HIP graph (RH_OPT_GRAPH) against the
launch-by-launch forward: bit-identical vectors and hidden states on every
replay, with eager forwards of other shapes and host synchronizations
between the replays; a new shape, a changed model option or a changed
context option records the graph again; one and two streams; full int8
(BERT-base shape) and weight-only int8 (MiniLM shape).
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("which,quant,streams", [
    ("minilm", 1, 1), ("minilm", 1, 2), ("minilm", 2, 2), ("bert-base", 2, 2)])
def test_graph_replays_match_eager(gpu_ctx, which, quant, streams):
    from rembed_amd import _lib
    from rembed_amd import synthetic as S
    from rembed_amd.model import Model
    shape = S.MINILM_L6 if which == "minilm" else S.BERT_BASE
    t = S.bert_tensors(shape, seed=0x5EED0001)
    ids, lens = S.token_batch(48, 128, 16, 128, seed=0x5EED0002)
    ids2, lens2 = S.token_batch(17, 128, 5, 128, seed=0x5EED0003)
    say(f"graph {which} quant={quant} streams={streams} tokens={int(lens.sum())}")
    m = Model(gpu_ctx, shape, t, quant)
    m.set_streams(streams)
    want = m.embed(ids, lens)
    want2 = m.embed(ids2, lens2)
    want_tok = m.embed_tokens(ids, lens)
    m.set_graph(True)
    for rep in range(4):
        got = m.embed(ids, lens)  # first: recorded; then replayed
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rep
        if rep == 1:  # another shape in between: recorded anew, then back
            assert np.array_equal(m.embed(ids2, lens2), want2)
        if rep == 2:
            toks = m.embed_tokens(ids, lens)
            for a, b in zip(toks, want_tok):
                assert np.array_equal(a, b)
    # device-resident ids and output, replayed several times in a row
    ids_d = gpu_ctx.upload(ids)
    out_d = gpu_ctx.alloc(len(lens) * shape.hidden * 4)
    for _ in range(3):
        m.embed_device(ids_d, lens, len(lens), ids.shape[1], out_d)
    gpu_ctx.sync()
    got = out_d.download(np.float32, (len(lens), shape.hidden))
    assert np.array_equal(got, want)
    # a model option and a context option change: recorded again, same bits
    m.set_attention_precision(1)
    m.set_attention_precision(3)
    assert np.array_equal(m.embed(ids, lens), want)
    gpu_ctx.set_option(_lib.RH_CTX_TILE_GROUP, 4)
    assert np.array_equal(m.embed(ids, lens), want)
    m.close()
