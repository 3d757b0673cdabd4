"""Python mirror of rembed's tokenizers over the C ABI.

WordPieceTokenizer follows tokenizer.New / Encode / VocabSize
(tokenizer/tokenizer.go:39-216); BpeTokenizer follows bpe.New,
NewFromTokenizerJSON and NewQwenFromTokenizerJSON
(tokenizer/bpe/bpe.go:104-324); SentencePieceTokenizer follows
sentencepiece.New (tokenizer/sentencepiece/sentencepiece.go:47-241);
GemmaTokenizer follows gemma.New (tokenizer/gemma/gemma.go:58-254). The tokenization itself runs in the library
(rh_tokenizer_*); these classes only marshal text and ids.
"""
import ctypes

import numpy as np

from ._lib import check, lib

MAX_SEQ_LEN = 512  # tokenizer.MaxSeqLen (tokenizer/tokenizer.go:19)


def _utf8(text):
    return text.encode("utf-8", "surrogatepass") if isinstance(text, str) else bytes(text)


class _Tokenizer:
    def __init__(self, h):
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib.rh_tokenizer_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def vocab_size(self):
        return int(lib.rh_tokenizer_vocab_size(self.h))

    def encode(self, text, max_len=MAX_SEQ_LEN):
        """(ids, mask) of one text as int64 lists, framed, at most max_len ids
        (the framing survives any max_len); the mask is all ones."""
        raw = _utf8(text)
        cap = max(int(max_len), 2)
        ids = np.empty(cap, np.int64)
        n = ctypes.c_int()
        check(lib.rh_tokenizer_encode(self.h, raw, len(raw), int(max_len), ids.ctypes.data, cap,
                                      ctypes.byref(n)))
        out = ids[:n.value].tolist()
        return out, [1] * len(out)

    def encode_batch(self, texts, max_len=MAX_SEQ_LEN, pad_id=0):
        """Padded int64 ids [batch][max(max_len, 2)] and int32 lengths: the
        inputs of Model.embed."""
        raws = [_utf8(t) for t in texts]
        stride = max(int(max_len), 2)
        ids = np.empty((len(raws), stride), np.int64)
        lens = np.empty(len(raws), np.int32)
        bufs = (ctypes.c_char_p * max(1, len(raws)))(*raws)
        sizes = (ctypes.c_size_t * max(1, len(raws)))(*[len(r) for r in raws])
        check(lib.rh_tokenizer_encode_batch(self.h, ctypes.cast(bufs, ctypes.c_void_p),
                                            ctypes.cast(sizes, ctypes.c_void_p), len(raws),
                                            int(max_len), int(pad_id), ids.ctypes.data,
                                            lens.ctypes.data))
        return ids, lens


class WordPieceTokenizer(_Tokenizer):
    """A BERT WordPiece vocab (one token per line, id = line number)."""

    def __init__(self, vocab_path, lower_case=True, cls_tok="", sep_tok="", unk_tok=""):
        h = ctypes.c_void_p()
        check(lib.rh_tokenizer_wordpiece_load(str(vocab_path).encode(), int(bool(lower_case)),
                                              cls_tok.encode(), sep_tok.encode(),
                                              unk_tok.encode(), ctypes.byref(h)))
        super().__init__(h)


class BpeTokenizer(_Tokenizer):
    """A byte-level BPE tokenizer (RoBERTa / GPT-2, ModernBERT, Qwen3)."""

    @classmethod
    def from_files(cls, vocab_json, merges_txt, cls_tok="<s>", sep_tok="</s>", unk_tok="<unk>"):
        """RoBERTa's vocab.json + merges.txt (bpe.New)."""
        h = ctypes.c_void_p()
        check(lib.rh_tokenizer_bpe_load(str(vocab_json).encode(), str(merges_txt).encode(),
                                        cls_tok.encode(), sep_tok.encode(), unk_tok.encode(),
                                        ctypes.byref(h)))
        return cls(h)

    @classmethod
    def from_tokenizer_json(cls, path, cls_tok="[CLS]", sep_tok="[SEP]", unk_tok="[UNK]"):
        """ModernBERT's tokenizer.json (bpe.NewFromTokenizerJSON)."""
        h = ctypes.c_void_p()
        check(lib.rh_tokenizer_bpe_load_json(str(path).encode(), 0, cls_tok.encode(),
                                             sep_tok.encode(), unk_tok.encode(),
                                             ctypes.byref(h)))
        return cls(h)

    @classmethod
    def qwen(cls, path, eos_tok="<|endoftext|>"):
        """Qwen3's tokenizer.json (bpe.NewQwenFromTokenizerJSON): the Qwen
        pre-tokenizer and a trailing eos alone."""
        h = ctypes.c_void_p()
        check(lib.rh_tokenizer_bpe_load_json(str(path).encode(), 1, None, eos_tok.encode(),
                                             None, ctypes.byref(h)))
        return cls(h)


class SentencePieceTokenizer(_Tokenizer):
    """An XLM-R-family SentencePiece Unigram model (sentencepiece.bpe.model),
    ids in HF's fairseq space."""

    def __init__(self, model_path):
        h = ctypes.c_void_p()
        check(lib.rh_tokenizer_sentencepiece_load(str(model_path).encode(), ctypes.byref(h)))
        super().__init__(h)

    def normalize(self, text):
        """The model's normalized text (Normalize, sentencepiece.go:244)."""
        raw = _utf8(text)
        cap = 4 * len(raw) + 64
        buf = ctypes.create_string_buffer(cap)
        n = ctypes.c_size_t()
        check(lib.rh_tokenizer_sentencepiece_normalize(self.h, raw, len(raw), buf, cap,
                                                       ctypes.byref(n)))
        return buf.raw[:n.value].decode("utf-8")


class GemmaTokenizer(_Tokenizer):
    """Gemma's byte-fallback BPE from its tokenizer.json."""

    def __init__(self, tokenizer_json):
        h = ctypes.c_void_p()
        check(lib.rh_tokenizer_gemma_load(str(tokenizer_json).encode(), ctypes.byref(h)))
        super().__init__(h)
