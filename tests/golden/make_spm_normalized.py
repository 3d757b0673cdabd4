"""Collects the (text, normalized) pairs of the reference's SentencePiece
fixtures (tokenizer/sentencepiece/testdata/fixture.json and fixture-nfd.json
under the reference tree) into spm_normalized.json: the NMT-NFKC
normalizer's expected output for each text, as the reference's tests hold
it. Only those two fields are kept.

Usage: python tests/golden/make_spm_normalized.py [/root/reference]
"""
import json
import os
import sys

ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
cases = []
for name in ("fixture.json", "fixture-nfd.json"):
    f = os.path.join(ref, "tokenizer", "sentencepiece", "testdata", name)
    for c in json.load(open(f, encoding="utf-8"))["cases"]:
        if "normalized" in c:
            cases.append({"text": c["text"], "normalized": c["normalized"], "fixture": name})
out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "spm_normalized.json")
json.dump({"source": "tokenizer/sentencepiece/testdata/{fixture,fixture-nfd}.json",
           "cases": cases}, open(out, "w"), ensure_ascii=True, indent=0)
print(f"{len(cases)} cases -> {out}")
