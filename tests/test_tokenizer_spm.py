"""The SentencePiece Unigram (XLM-R family) and Gemma byte-fallback BPE
tokenizers behind rh_tokenizer_sentencepiece_load / rh_tokenizer_gemma_load
(host code, no GPU), after tokenizer/sentencepiece and tokenizer/gemma.

* SentencePiece: a unigram model trained with the `sentencepiece` package
  (the C++ reference implementation the Go port follows) on the reference's
  golden texts with the NMT-NFKC rule. Its normalizer must reproduce the
  "normalized" strings of the reference's own fixtures
  (tokenizer/sentencepiece/testdata/fixture.json, fixture-nfd.json: the
  charsmap of a real XLM-R model; the NMT-NFKC map is the same table), and
  the ids must equal sentencepiece's own encoding mapped into HF's fairseq
  id space the way sentencepiece.go:110-121 maps them.
* Gemma: a tokenizer.json built with HF `tokenizers` in Gemma's form
  (space -> U+2581 normalizer, whole-string BPE with byte fallback, <bos> /
  <eos> framing) from a BPE trained on the same texts with a limited
  alphabet, so byte fallback occurs; ids must equal HF's.
"""
import io
import json
import os

import pytest

from rembed_amd import _lib
from rembed_amd.tokenizer import GemmaTokenizer, SentencePieceTokenizer

HERE = os.path.dirname(os.path.abspath(__file__))
TEXTS = json.load(open(os.path.join(HERE, "golden", "tokenizer_texts.json"),
                       encoding="utf-8"))["texts"]
NORMALIZED = json.load(open(os.path.join(HERE, "golden", "spm_normalized.json"),
                            encoding="utf-8"))["cases"]
EXTRA = ["  leading and   inner   spaces  ", "", " ", "tab\tand\nnewline", "ｆｕｌｌｗｉｄｔｈ",
         "ﬁ ligature", "①②③", "x" * 600, "日本語 テキスト", "emoji 🚀", "a b c"]


@pytest.fixture(scope="module")
def spm_model(tmp_path_factory):
    spm = pytest.importorskip("sentencepiece")
    d = tmp_path_factory.mktemp("spm")
    buf = io.BytesIO()
    spm.SentencePieceTrainer.train(
        sentence_iterator=iter(TEXTS * 3), model_writer=buf, vocab_size=600,
        model_type="unigram", normalization_rule_name="nmt_nfkc", hard_vocab_limit=False,
        character_coverage=0.98, minloglevel=2)
    path = d / "sentencepiece.bpe.model"
    path.write_bytes(buf.getvalue())
    return str(path)


def fairseq(sp_ids):
    """sentencepiece.go:110-121: <unk> 0 -> 3, <s> 1 -> 0, </s> 2 -> 2, else +1."""
    return [{0: 3, 1: 0, 2: 2}.get(i, i + 1) for i in sp_ids]


def test_spm_normalizer_matches_reference_fixtures(spm_model):
    """The reference's fixtures hold the normalized text of each case, made
    with a real XLM-R model's NMT-NFKC charsmap (the table the trained model
    carries too): this normalizer must reproduce every one, including the
    decomposed-Hangul / kana cases of fixture-nfd.json."""
    ours = SentencePieceTokenizer(spm_model)
    bad = [(c["text"], ours.normalize(c["text"]), c["normalized"]) for c in NORMALIZED
           if ours.normalize(c["text"]) != c["normalized"]]
    assert not bad, bad[:3]
    assert len(NORMALIZED) >= 30


def test_spm_matches_sentencepiece(spm_model):
    spm = pytest.importorskip("sentencepiece")
    sp = spm.SentencePieceProcessor(model_file=spm_model)
    ours = SentencePieceTokenizer(spm_model)
    assert ours.vocab_size() == sp.get_piece_size() + 2
    texts = TEXTS + EXTRA + [c["text"] for c in NORMALIZED]
    bad = []
    for text in texts:
        got = ours.encode(text, 100000)[0]
        want = [0] + fairseq(sp.encode(text)) + [2]
        if got != want:
            bad.append((text, got, want))
    assert not bad, bad[:2]


def test_spm_truncation(spm_model):
    ours = SentencePieceTokenizer(spm_model)
    for max_len in (0, 1, 2):
        assert ours.encode("hello world", max_len)[0] == [0, 2]
    ids = ours.encode("the quick brown fox " * 100, 16)[0]
    assert len(ids) == 16 and ids[0] == 0 and ids[-1] == 2


def test_spm_refusals(tmp_path):
    junk = tmp_path / "junk.model"
    junk.write_bytes(b"\xff\xff\xff")
    with pytest.raises(_lib.RembedError):
        SentencePieceTokenizer(str(junk))
    with pytest.raises(_lib.RembedError):
        SentencePieceTokenizer(str(tmp_path / "absent.model"))


@pytest.fixture(scope="module")
def gemma_json(tmp_path_factory):
    tokenizers = pytest.importorskip("tokenizers")
    from tokenizers import AddedToken, Tokenizer, models, normalizers, trainers
    d = tmp_path_factory.mktemp("gemma")
    base = Tokenizer(models.BPE())
    base.normalizer = normalizers.Replace(" ", "▁")
    trainer = trainers.BpeTrainer(vocab_size=900, min_frequency=1, limit_alphabet=120,
                                  show_progress=False)
    base.train_from_iterator(TEXTS, trainer)
    trained = json.loads(base.to_str())["model"]
    vocab = {"<pad>": 0, "<eos>": 1, "<bos>": 2, "<unk>": 3}
    for b in range(256):
        vocab[f"<0x{b:02X}>"] = len(vocab)
    for tok, _ in sorted(trained["vocab"].items(), key=lambda kv: kv[1]):
        vocab.setdefault(tok, len(vocab))
    merges = [tuple(m.split(" ")) if isinstance(m, str) else tuple(m) for m in trained["merges"]]
    tok = Tokenizer(models.BPE(vocab, merges, unk_token="<unk>", byte_fallback=True))
    tok.normalizer = normalizers.Replace(" ", "▁")
    tok.add_special_tokens([AddedToken(t, special=True) for t in ("<pad>", "<eos>", "<bos>",
                                                                   "<unk>")])
    path = d / "tokenizer.json"
    tok.save(str(path))
    return str(path), tok


def test_gemma_matches_hf(gemma_json):
    path, hf = gemma_json
    ours = GemmaTokenizer(path)
    fallback = 0
    bad = []
    for text in TEXTS + EXTRA:
        got = ours.encode(text, 100000)[0]
        inner = hf.encode(text, add_special_tokens=False).ids
        fallback += sum(4 <= i < 260 for i in inner)
        want = [2] + inner + [1]
        if got != want:
            bad.append((text, got, want))
    assert not bad, bad[:2]
    assert fallback > 0  # byte fallback was exercised
    for max_len in (0, 1, 2):
        assert ours.encode("hello world", max_len)[0] == [2, 1]


def test_gemma_refusals(tmp_path, gemma_json):
    path, _ = gemma_json
    j = json.load(open(path, encoding="utf-8"))
    j["model"]["byte_fallback"] = False
    nofb = tmp_path / "nofb.json"
    nofb.write_text(json.dumps(j))
    with pytest.raises(_lib.RembedError):
        GemmaTokenizer(str(nofb))
    j = json.load(open(path, encoding="utf-8"))
    del j["model"]["vocab"]["<0x41>"]
    nobyte = tmp_path / "nobyte.json"
    nobyte.write_text(json.dumps(j))
    with pytest.raises(_lib.RembedError):
        GemmaTokenizer(str(nobyte))
