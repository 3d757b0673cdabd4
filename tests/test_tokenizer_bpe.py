"""The byte-level BPE tokenizer behind rh_tokenizer_bpe_load* (host code, no
GPU): RoBERTa / GPT-2 (vocab.json + merges.txt), ModernBERT and Qwen3
(tokenizer.json), after tokenizer/bpe/bpe.go.

The reference's own BPE tests need the real vocabularies (absent offline;
they skip there too), so the tokenizer is checked against HF `tokenizers`
— the implementation the reference's fixtures were made with — on the
135 input texts of the reference's golden files
(tests/golden/tokenizer_texts.json) plus pre-tokenizer stress strings,
with a byte-level BPE trained on those texts:
* RoBERTa: ByteLevelBPETokenizer over the same vocab.json / merges.txt;
* ModernBERT: a tokenizer.json with an NFC normalizer, the GPT-2 ByteLevel
  pre-tokenizer, specials, [MASK] with lstrip, and whitespace-run added
  tokens (2-24 spaces);
* Qwen3: a tokenizer.json with an NFC normalizer and the Qwen Split regex
  ahead of a regex-free ByteLevel step.
The merge loop is also checked against a round-based restatement of GPT-2's
algorithm (bpe_test.go:241-274), and the framing, truncation and refusal
rules of bpe.go directly.
"""
import json
import os
import random
import time

import pytest

from rembed_amd import _lib
from rembed_amd.tokenizer import BpeTokenizer

tokenizers = pytest.importorskip("tokenizers")
from tokenizers import AddedToken, Regex, Tokenizer, models, normalizers, pre_tokenizers  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
TEXTS = json.load(open(os.path.join(HERE, "golden", "tokenizer_texts.json"),
                       encoding="utf-8"))["texts"]
# pre-tokenizer branches: contractions (and case), space joining, whitespace
# backtracking, newline runs, digits, punctuation runs, long s, mixed scripts
STRESS = [
    "it's IT'S it'S 'll 're've", "don'tſ 'ſ 'S", "a  b   c\t\td \n\n e\r\n f",
    "x \n\ny", "  leading", "trailing  ", " ", "", "123456 7,890.12", "!!!'s ?!?",
    "hello world x", "naïve café", "café", "日本語のテキスト 123",
    "emoji 🚀🚀 ok", "tab\tsep", "[MASK] x [MASK]", "a   [MASK]   b", "[CLS] [SEP]",
    "<|endoftext|> tail", "line\r\n\r\n  next", "x" * 300, "ab" * 120 + " z",
]
SPECIALS = ["<s>", "<pad>", "</s>", "<unk>"]
QWEN_PATTERN = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}|"
                r" ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+")


@pytest.fixture(scope="module")
def trained(tmp_path_factory):
    """A byte-level BPE (vocab.json, merges.txt) trained on the texts."""
    d = tmp_path_factory.mktemp("bpe")
    hf = tokenizers.ByteLevelBPETokenizer()
    hf.train_from_iterator(TEXTS + STRESS, vocab_size=1500, min_frequency=1,
                           special_tokens=SPECIALS, show_progress=False)
    hf.save_model(str(d))
    return str(d / "vocab.json"), str(d / "merges.txt")


def all_texts():
    return TEXTS + STRESS


def test_roberta_matches_hf(trained):
    vocab, merges = trained
    ours = BpeTokenizer.from_files(vocab, merges)
    hf = tokenizers.ByteLevelBPETokenizer(vocab, merges)
    v = json.load(open(vocab, encoding="utf-8"))
    cls, sep = v["<s>"], v["</s>"]
    bad = []
    for text in all_texts():
        got = ours.encode(text, 100000)[0]
        want = [cls] + hf.encode(text).ids + [sep]
        if got != want:
            bad.append((text, got, want))
    assert not bad, bad[:2]
    assert ours.vocab_size() == len(v)


def _tokenizer_json(trained, d, name, pre, added):
    vocab, merges = trained
    tok = Tokenizer(models.BPE.from_file(vocab, merges))
    tok.normalizer = normalizers.NFC()
    tok.pre_tokenizer = pre
    tok.add_special_tokens(added)
    path = os.path.join(d, name)
    tok.save(path)
    return path, tok


def test_modernbert_matches_hf(trained, tmp_path):
    added = [AddedToken("[CLS]", special=True), AddedToken("[SEP]", special=True),
             AddedToken("[UNK]", special=True), AddedToken("[PAD]", special=True),
             AddedToken("[MASK]", lstrip=True, special=True)]
    path, hf = _tokenizer_json(trained, str(tmp_path), "mb.json",
                               pre_tokenizers.ByteLevel(add_prefix_space=False), added)
    # whitespace runs as ordinary (normalized) added tokens, as ModernBERT
    # declares them: HF matches them after the specials, so an lstrip [MASK]
    # takes a whitespace run before it (bpe.go:52-58)
    hf.add_tokens([AddedToken(" " * k) for k in range(2, 25)])
    hf.save(path)
    ours = BpeTokenizer.from_tokenizer_json(path)
    j = json.load(open(path, encoding="utf-8"))
    ids = {a["content"]: a["id"] for a in j["added_tokens"]}
    bad = []
    for text in all_texts():
        got = ours.encode(text, 100000)[0]
        want = [ids["[CLS]"]] + hf.encode(text, add_special_tokens=False).ids + [ids["[SEP]"]]
        if got != want:
            bad.append((text, got, want))
    assert not bad, bad[:2]


def test_qwen_matches_hf(trained, tmp_path):
    pre = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(QWEN_PATTERN), behavior="isolated", invert=False),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    path, hf = _tokenizer_json(trained, str(tmp_path), "qwen.json", pre,
                               [AddedToken("<|endoftext|>", special=True)])
    ours = BpeTokenizer.qwen(path)
    eos = [a["id"] for a in json.load(open(path, encoding="utf-8"))["added_tokens"]
           if a["content"] == "<|endoftext|>"][0]
    bad = []
    for text in all_texts():
        got = ours.encode(text, 100000)[0]
        want = hf.encode(text, add_special_tokens=False).ids + [eos]
        if got != want:
            bad.append((text, got, want))
    assert not bad, bad[:2]


def bpe_rounds(word, ranks):
    """GPT-2's round-based merge (bpe_test.go:241-274): merge every
    occurrence of the lowest-ranked adjacent pair, left to right, repeat."""
    w = list(word)
    while len(w) > 1:
        best = min(((ranks[(a, b)], (a, b)) for a, b in zip(w, w[1:]) if (a, b) in ranks),
                   default=None)
        if best is None:
            break
        a, b = best[1]
        out, i = [], 0
        while i < len(w):
            if i + 1 < len(w) and w[i] == a and w[i + 1] == b:
                out.append(a + b)
                i += 2
            else:
                out.append(w[i])
                i += 1
        w = out
    return w


def test_merge_order_matches_round_based(trained):
    vocab_path, merges_path = trained
    vocab = json.load(open(vocab_path, encoding="utf-8"))
    ranks = {}
    for line in open(merges_path, encoding="utf-8").read().split("\n"):
        if line and not line.startswith("#version"):
            a, b = line.split(" ")
            ranks[(a, b)] = len(ranks)
    ours = BpeTokenizer.from_files(vocab_path, merges_path)
    pre = pre_tokenizers.ByteLevel(add_prefix_space=False)
    rng = random.Random(11)
    alphabet = "abcdefghijklmnopqrstuvwxyzABC0123456789 .,!?'-éü你🚀"
    words = ["".join(rng.choice(alphabet) for _ in range(rng.randint(1, 24)))
             for _ in range(400)]
    words += [c * n for c in "aes0" for n in (2, 3, 7, 64, 257)] + TEXTS
    for w in words:
        want = [vocab[s] for p, _ in pre.pre_tokenize_str(w) for s in bpe_rounds(p, ranks)]
        assert ours.encode(w, 100000)[0][1:-1] == want, w


def test_framing_and_truncation(trained, tmp_path):
    vocab, merges = trained
    v = json.load(open(vocab, encoding="utf-8"))
    ours = BpeTokenizer.from_files(vocab, merges)
    for max_len in (0, 1, 2):  # the framing survives any ceiling
        assert ours.encode("hello world", max_len)[0] == [v["<s>"], v["</s>"]]
    ids = ours.encode("supercalifragilisticexpialidocious " * 200, 16)[0]
    assert len(ids) == 16 and ids[0] == v["<s>"] and ids[-1] == v["</s>"]
    batch, lens = ours.encode_batch(["hello world", "", "x " * 100], max_len=8, pad_id=-1)
    assert batch.shape == (3, 8) and lens.tolist()[1] == 2 and lens.tolist()[2] == 8
    for b, t in enumerate(["hello world", "", "x " * 100]):
        assert batch[b, :lens[b]].tolist() == ours.encode(t, 8)[0]
        assert (batch[b, lens[b]:] == -1).all()
    pre = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(QWEN_PATTERN), behavior="isolated"),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    path, _ = _tokenizer_json(trained, str(tmp_path), "q.json", pre,
                              [AddedToken("<|endoftext|>", special=True)])
    q = BpeTokenizer.qwen(path)
    assert len(q.encode("hello world", 0)[0]) == 1  # the eos alone
    assert len(q.encode("hello world " * 50, 5)[0]) == 5


def test_long_word_is_not_quadratic(trained):
    ours = BpeTokenizer.from_files(*trained)
    t0 = time.perf_counter()
    ids = ours.encode("abcdefghij" * 5000, 512)[0]
    assert time.perf_counter() - t0 < 2.0
    assert len(ids) == 512


def test_refusals(trained, tmp_path):
    vocab, merges = trained
    with pytest.raises(_lib.RembedError) as e:
        BpeTokenizer.from_files(vocab, merges, cls_tok="<missing>")
    assert e.value.code == _lib.RH_ERR_INVALID
    bad = tmp_path / "merges_bad.txt"
    bad.write_text("#version: 0.2\nab\n")
    with pytest.raises(_lib.RembedError):
        BpeTokenizer.from_files(vocab, str(bad))
    empty = tmp_path / "merges_empty.txt"
    empty.write_text("#version: 0.2\n\n")
    with pytest.raises(_lib.RembedError):
        BpeTokenizer.from_files(vocab, str(empty))
    notbpe = tmp_path / "wp.json"
    notbpe.write_text(json.dumps({"model": {"type": "WordPiece", "vocab": {"a": 0}}}))
    with pytest.raises(_lib.RembedError):
        BpeTokenizer.from_tokenizer_json(str(notbpe))
    broken = tmp_path / "broken.json"
    broken.write_text('{"model": {"type": "BPE", "vocab": {"a": 0}, "merges": [')
    with pytest.raises(_lib.RembedError):
        BpeTokenizer.from_tokenizer_json(str(broken))
