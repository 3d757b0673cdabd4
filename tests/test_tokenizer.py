"""The WordPiece tokenizer behind rh_tokenizer_* (host code, no GPU).

* Every vocabulary, text and expected id list of the reference's own tests
  (tokenizer/tokenizer_test.go), kept as data in
  tests/golden/wordpiece_cases.json, plus the category-C cleaning pairs of
  TestCleanTextCategoryC with a vocabulary that separates joining, splitting
  and keeping.
* The vocab file rules of tokenizer.New (bufio line scanning: CRLF, a last
  line without newline, duplicates, empty lines) and its refusals.
* An independent check: HF `tokenizers`' BertWordPieceTokenizer — the
  implementation the reference's goldens were made with and its comments
  cite ("mirroring HF") — on the 135 input texts of the reference's golden
  files (tests/golden/tokenizer_texts.json) with a synthetic vocabulary, cased
  and uncased, must give the same ids; where HF and the reference disagree by
  design (documented in tokenizer.go) the reference's rule is asserted.
* encode_batch lays rows out for Model.embed; invalid UTF-8 is dropped.
"""
import json
import os
import unicodedata

import numpy as np
import pytest

from rembed_amd import _lib
from rembed_amd.tokenizer import WordPieceTokenizer

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = json.load(open(os.path.join(HERE, "golden", "wordpiece_cases.json"), encoding="utf-8"))
TEXTS = json.load(open(os.path.join(HERE, "golden", "tokenizer_texts.json"),
                       encoding="utf-8"))["texts"]


def vocab_file(tmp_path, lines, name="vocab.txt", sep="\n"):
    p = tmp_path / name
    p.write_bytes(sep.join(lines).encode("utf-8"))
    return str(p)


def tok_for(tmp_path, vocab, lower=True, specials=("", "", "")):
    return WordPieceTokenizer(vocab_file(tmp_path, vocab), lower, *specials)


@pytest.mark.parametrize("case", CASES["cases"], ids=lambda c: c["test"][:60])
def test_reference_cases(tmp_path, case):
    specials = tuple(case.get("specials", ("", "", "")))
    if "load_error" in case:
        with pytest.raises(_lib.RembedError) as e:
            tok_for(tmp_path, case["vocab"], case["lower"], specials)
        assert e.value.code == _lib.RH_ERR_MISSING
        return
    t = tok_for(tmp_path, case["vocab"], case["lower"], specials)
    text = case["text"] if "text" in case else case["text_repeat"][0] * case["text_repeat"][1]
    want = case["ids"] if "ids" in case else [i for v, n in case["ids_repeat"] for i in [v] * n]
    ids, mask = t.encode(text, case["max_len"])
    assert ids == want
    assert mask == [1] * len(ids)


def test_category_c_cleaning(tmp_path):
    cc = CASES["category_c"]
    t = tok_for(tmp_path, cc["vocab"])
    seen = set()
    for text, equiv in cc["pairs"]:
        got, want = t.encode(text)[0], t.encode(equiv)[0]
        assert got == want, (text, got, want)
        seen.add(tuple(want))
    # the equivalents themselves tokenize differently (the check is not vacuous)
    assert len(seen) >= 5


def test_vocab_file_rules(tmp_path):
    base = ["[PAD]", "[UNK]", "[CLS]", "[SEP]", "hello", "world"]
    # CRLF line ends, and a last line without a newline
    t = WordPieceTokenizer(vocab_file(tmp_path, base, "crlf.txt", "\r\n"))
    assert t.encode("hello world")[0] == [2, 4, 5, 3]
    assert t.vocab_size() == 6
    # a trailing newline adds no entry ("...world\n")
    t = WordPieceTokenizer(vocab_file(tmp_path, base + [""], "trail.txt"))
    assert t.vocab_size() == 6
    # an empty line inside the file takes an id (the empty token)
    t = WordPieceTokenizer(vocab_file(tmp_path, ["[PAD]", "", "[UNK]", "[CLS]", "[SEP]",
                                                  "hello"], "gap.txt"))
    assert t.encode("hello")[0] == [3, 5, 4]
    assert t.vocab_size() == 6
    # a later duplicate line wins; VocabSize counts distinct entries
    t = WordPieceTokenizer(vocab_file(tmp_path, base + ["hello"], "dup.txt"))
    assert t.encode("hello")[0] == [2, 6, 3]
    assert t.vocab_size() == 6
    with pytest.raises(_lib.RembedError) as e:
        WordPieceTokenizer(str(tmp_path / "absent.txt"))
    assert e.value.code == _lib.RH_ERR_INVALID
    with pytest.raises(_lib.RembedError) as e:
        WordPieceTokenizer(vocab_file(tmp_path, ["[PAD]", "[UNK]", "[CLS]"], "nosep.txt"))
    assert e.value.code == _lib.RH_ERR_MISSING


def test_invalid_utf8_is_dropped(tmp_path):
    t = tok_for(tmp_path, ["[PAD]", "[UNK]", "[CLS]", "[SEP]", "hello", "world"])
    for raw in (b"hel\xfflo world", b"hel\xc3lo world", b"hello\xed\xa0\x80 world",
                b"hel\xf8\x88\x80\x80\x80lo world", b"hello world\xe2\x82"):
        assert t.encode(raw)[0] == [2, 4, 5, 3], raw


def test_encode_batch_layout(tmp_path):
    t = tok_for(tmp_path, ["[PAD]", "[UNK]", "[CLS]", "[SEP]", "play", "##ing", "hello"])
    texts = ["playing hello", "", "hello " * 20, "zzz"]
    ids, lens = t.encode_batch(texts, max_len=8, pad_id=0)
    assert ids.shape == (4, 8) and ids.dtype == np.int64 and lens.dtype == np.int32
    for b, text in enumerate(texts):
        single = t.encode(text, 8)[0]
        assert lens[b] == len(single)
        assert ids[b, :lens[b]].tolist() == single
        assert np.all(ids[b, lens[b]:] == 0)
    assert lens.tolist() == [5, 2, 8, 3]


def _strip_lower(text):
    text = unicodedata.normalize("NFD", text.lower())
    return "".join(c for c in text if unicodedata.category(c) != "Mn")


def synthetic_vocab(texts, lower):
    """Specials, every character of the texts as a word and as a "##"
    continuation, and every whitespace-separated run of up to 6 characters
    (so whole words, pieces and [UNK] all occur)."""
    chars, words = set(), set()
    for t in texts:
        s = _strip_lower(t) if lower else t
        chars.update(c for c in s if not c.isspace())
        words.update(w for w in s.split() if len(w) <= 6)
    # characters that are not allowed in a vocab line (\n, \r) are dropped;
    # a few characters are left out on purpose so [UNK] also occurs
    chars = sorted(c for c in chars if c not in "\n\r" and ord(c) % 17 != 3)
    words = sorted(w for w in words if "\r" not in w)
    return ["[PAD]", "[UNK]", "[CLS]", "[SEP]"] + chars + ["##" + c for c in chars] + words


@pytest.mark.parametrize("lower", [True, False], ids=["uncased", "cased"])
def test_matches_hf_bert_wordpiece(tmp_path, lower):
    """HF tokenizers' BertWordPieceTokenizer (clean_text, CJK padding, accent
    stripping coupled to lowercasing, WordPiece with max 100 chars per word)
    against this tokenizer on the reference's golden texts."""
    tokenizers = pytest.importorskip("tokenizers")
    vocab = synthetic_vocab(TEXTS, lower)
    path = vocab_file(tmp_path, vocab)
    ours = WordPieceTokenizer(path, lower)
    hf = tokenizers.BertWordPieceTokenizer(path, clean_text=True, handle_chinese_chars=True,
                                           strip_accents=lower, lowercase=lower)
    hf.no_truncation()
    mismatched, compared = [], 0
    for text in TEXTS:
        got = ours.encode(text, 100000)[0]
        if any(sp in text for sp in ("[CLS]", "[SEP]", "[UNK]", "[PAD]", "[MASK]")):
            # HF matches registered special tokens inside the text; the
            # reference's basicTokens has no such step (tokenizer.go:110-162),
            # so "[CLS]" in a text is the three words "[", "cls", "]"
            words = (_strip_lower(text) if lower else text).replace("[", " [ ").replace(
                "]", " ] ").split()
            assert got[1:-1] == [i for w in words for i in ours.encode(w, 100000)[0][1:-1]]
            continue
        compared += 1
        want = hf.encode(text).ids
        if got != want:
            mismatched.append((text, got, want))
    assert compared >= 130
    assert not mismatched, mismatched[:3]
