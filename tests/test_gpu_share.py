"""One weight set, several contexts (rh_model_share).

The reference's Model and Embedder are safe for concurrent use with the
weights held once (internal/model/bert.go:52-56, rembed.go:36-41). A device
model is bound to one context and stream; rh_model_share gives another
handle on the same HBM weights with its own context, stream and workspace.
These tests check, on the GPU:

* a shared handle embeds bit for bit as the model it shares (BERT fp32 and
  full int8, Qwen3 weight-only int8), also after the original handle and its
  context are destroyed;
* handles on two contexts called from two threads at once give the
  single-threaded bytes on every call;
* sharing allocates no second copy of the weights;
* options are per handle; an unfinalized model cannot be shared.
"""
import dataclasses
import threading

import numpy as np
import pytest

from rembed_amd import _lib
from rembed_amd.model import QUANT_FULL, QUANT_NONE, QUANT_WEIGHTS, Model
from rembed_amd.synthetic import (QWEN3_0_6B, BertShape, bert_tensors, decoder_tensors,
                                  token_batch)
from rembed_amd.tensor import Context

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def bert_case():
    shape = BertShape("share-bert", layers=2, hidden=384, heads=6, intermediate=1536,
                      vocab=4000, max_position=256, pooling=0)
    ids, lens = token_batch(24, 128, 8, 128, vocab=shape.vocab, seed=41)
    return shape, bert_tensors(shape, seed=42), ids, lens


def qwen3_case():
    shape = dataclasses.replace(QWEN3_0_6B, name="share-qwen3", layers=2, vocab=3000,
                                max_seq=512)
    ids, lens = token_batch(8, 256, 8, 256, vocab=shape.vocab, id_lo=0, seed=43)
    return shape, decoder_tensors(shape, seed=44, bf16=True), ids, lens


CASES = [("bert", QUANT_NONE), ("bert", QUANT_FULL), ("qwen3", QUANT_WEIGHTS)]


@pytest.mark.parametrize("arch,quant", CASES, ids=["bert-fp32", "bert-a8w8", "qwen3-w8"])
def test_shared_handle_is_identical_and_outlives_the_first(arch, quant):
    shape, t, ids, lens = bert_case() if arch == "bert" else qwen3_case()
    say(f"{arch} quant={quant} lens {lens.tolist()}")
    c1, c2 = Context(0), Context(0)
    m1 = Model(c1, shape, t, quant)
    want = m1.embed(ids, lens)
    m2 = m1.share(c2)
    assert m2.quantized() == m1.quantized()
    assert m2.quantized_activations() == m1.quantized_activations()
    assert np.array_equal(m2.embed(ids, lens), want)
    tok1 = m1.embed_tokens(ids[:3], lens[:3])
    m1.close()
    c1.close()
    got = m2.embed(ids, lens)
    assert np.array_equal(got, want)
    for a, b in zip(m2.embed_tokens(ids[:3], lens[:3]), tok1):
        assert np.array_equal(a, b)
    m2.close()
    c2.close()


def test_two_threads_two_contexts_one_weight_set():
    shape, t, ids, lens = bert_case()
    ctxs = [Context(0), Context(0)]
    base = Model(ctxs[0], shape, t, QUANT_FULL)
    handles = [base, base.share(ctxs[1])]
    halves = [(ids[:12], lens[:12]), (ids[12:], lens[12:])]
    want = [base.embed(*h) for h in halves]
    errors, start = [], threading.Barrier(2)

    def worker(k):
        try:
            start.wait()
            for it in range(20):
                got = handles[k].embed(*halves[k])
                if not np.array_equal(got, want[k]):
                    errors.append(f"handle {k} call {it} differs")
                    return
        except Exception as e:  # reported below
            errors.append(f"handle {k}: {e!r}")

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads)
    say(f"  errors {errors}")
    assert not errors
    for h in handles[::-1]:
        h.close()
    for c in ctxs:
        c.close()


def free_bytes():
    """hipMemGetInfo's free bytes on the current device (the library's
    contexts have set device 0)."""
    import ctypes
    hip = _lib.hip_runtime()
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipDeviceSynchronize() == 0
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_share_holds_one_copy_of_the_weights():
    shape = dataclasses.replace(QWEN3_0_6B, name="share-mem", layers=4, vocab=20000,
                                max_seq=512)
    t = decoder_tensors(shape, seed=45, bf16=True)
    c1, c2 = Context(0), Context(0)
    free0 = free_bytes()
    m1 = Model(c1, shape, t, QUANT_NONE)
    free1 = free_bytes()
    m2 = m1.share(c2)
    free2 = free_bytes()
    weights = free0 - free1
    say(f"  weights {weights / 2**20:.1f} MiB, share {(free1 - free2) / 2**20:.1f} MiB")
    assert weights > 100 * 2**20
    assert free1 - free2 < weights // 20
    m2.close()
    m1.close()
    c2.close()
    c1.close()


def test_options_are_per_handle_and_unfinalized_models_refused():
    shape, t, ids, lens = bert_case()
    c1, c2 = Context(0), Context(0)
    m1 = Model(c1, shape, t, QUANT_NONE)
    m2 = m1.share(c2)
    m2.set_attention_precision(1)  # bf16 attention on the second handle only
    a, b = m1.embed(ids, lens), m2.embed(ids, lens)
    m3 = Model(c1, shape, t, QUANT_NONE)
    m3.set_attention_precision(1)
    assert np.array_equal(b, m3.embed(ids, lens))
    assert not np.array_equal(a, b)
    with pytest.raises(_lib.RembedError):
        m2.set_fuse_projections(False)
    import ctypes
    from rembed_amd.model import make_config
    h, out = ctypes.c_void_p(), ctypes.c_void_p()
    cfg = make_config(shape)
    assert _lib.lib.rh_model_create(c1.h, ctypes.byref(cfg), 0, ctypes.byref(h)) == 0
    assert _lib.lib.rh_model_share(h, c2.h, ctypes.byref(out)) == _lib.RH_ERR_INVALID
    assert "not finalized" in _lib.lib.rh_last_error().decode()
    _lib.lib.rh_model_destroy(h)
    for m in (m3, m2, m1):
        m.close()
    c2.close()
    c1.close()
