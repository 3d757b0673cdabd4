"""Collects the input texts of the reference's tokenizer and embedding
goldens (testdata/*.json, tokenizer/*/testdata/*.json under the reference
tree) into tokenizer_texts.json: a battery of multilingual, whitespace,
control-character and symbol cases for the tokenizer tests. Only the texts
are kept (the ids there belong to vocabularies this tree does not have).

Usage: python tests/golden/make_tokenizer_texts.py [/root/reference]
"""
import glob
import json
import os
import sys

ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
texts = set()
for f in sorted(glob.glob(os.path.join(ref, "testdata", "*.json")) +
                glob.glob(os.path.join(ref, "tokenizer", "*", "testdata", "*.json"))):
    for case in json.load(open(f, encoding="utf-8")).get("cases", []):
        if isinstance(case.get("text"), str):
            texts.add(case["text"])
out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tokenizer_texts.json")
json.dump({"source": "input texts of testdata/*.json and tokenizer/*/testdata/*.json",
           "texts": sorted(texts)}, open(out, "w"), ensure_ascii=True, indent=0)
print(f"{len(texts)} texts -> {out}")
