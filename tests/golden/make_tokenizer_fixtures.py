"""Writes tests/golden/tokenizer/metaspace.json and metaspace_cases.jsonl:
fixtures for the tokenizer's Metaspace pipeline (Gemma 3 as bekko ships
it: Metaspace(U+2581, prepend always, split), template <bos> A <eos> /
<bos> A <eos> B <eos>), which the reference's own fixtures cannot pin here
(their tokenizer.json files are not in the repository).

The reference's contract is exact parity with Hugging Face `tokenizers`
(tokenizer/tokenizer.go:4-6; its fixtures come from that library,
tools/oracle/tokenizer_fixtures.py), so the expected ids and offsets are
that library's, on the siglip2-tiny vocabulary and merges with the
pre-tokenizer, normalizer and template switched to the Metaspace form.
Texts: those of tokenizer_cases.jsonl, plus pairs for EncodePair.
Run once, here (tokenizers 0.22.2); the GPU boxes only read the output.
"""
import json
import os

from tokenizers import Tokenizer

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tokenizer")


def main():
    cfg = json.load(open(os.path.join(HERE, "tokenizer.json"), encoding="utf-8"))
    cfg["normalizer"] = None
    cfg["pre_tokenizer"] = {"type": "Metaspace", "replacement": "▁", "prepend_scheme": "always", "split": True}
    cfg["post_processor"] = {
        "type": "TemplateProcessing",
        "single": [{"SpecialToken": {"id": "<bos>", "type_id": 0}}, {"Sequence": {"id": "A", "type_id": 0}},
                   {"SpecialToken": {"id": "<eos>", "type_id": 0}}],
        "pair": [{"SpecialToken": {"id": "<bos>", "type_id": 0}}, {"Sequence": {"id": "A", "type_id": 0}},
                 {"SpecialToken": {"id": "<eos>", "type_id": 0}}, {"Sequence": {"id": "B", "type_id": 1}},
                 {"SpecialToken": {"id": "<eos>", "type_id": 1}}],
        "special_tokens": {"<bos>": {"id": "<bos>", "ids": [2], "tokens": ["<bos>"]},
                           "<eos>": {"id": "<eos>", "ids": [1], "tokens": ["<eos>"]}}}
    # one added token with lstrip: the spaces before it are absorbed into
    # its span (tokenizer.go:632-641). Not rstrip: there the reference
    # consumes the trailing spaces (tokenizer.go:642-656) while tokenizers
    # 0.22.2 also tokenizes them, so the library is no oracle for it.
    for a in cfg["added_tokens"]:
        if a["content"] == "<mask>":
            a["lstrip"] = True
    path = os.path.join(HERE, "metaspace.json")
    with open(path, "w", encoding="utf-8") as f:
        json.dump(cfg, f, ensure_ascii=False)
    tok = Tokenizer.from_file(path)
    texts = []
    for line in open(os.path.join(HERE, "tokenizer_cases.jsonl"), encoding="utf-8"):
        fx = json.loads(line)
        if not fx.get("pair"):
            texts.append(fx["text"])
    texts += ["a <mask> b", "a<mask>b", "<mask>", "  <mask>  x", "x \u00a0\u2003<mask>\u3000 y", "<mask><mask> <eos>",
              "\t<mask>\n", "caf\u00e9 <mask>", "<mask> \u00e9t\u00e9"]
    with open(os.path.join(HERE, "metaspace_cases.jsonl"), "w", encoding="utf-8") as f:
        for t in texts:
            e = tok.encode(t)
            b = t.encode("utf-8")
            # character offsets -> byte offsets (the reference's Offset)
            cb = [0]
            for ch in t:
                cb.append(cb[-1] + len(ch.encode("utf-8")))
            offs = [[cb[s], cb[e2]] for s, e2 in e.offsets]
            f.write(json.dumps({"text": t, "ids": e.ids, "offsets": offs}, ensure_ascii=False) + "\n")
            assert len(b) == cb[-1]
        for i in range(0, min(len(texts), 400) - 1, 2):
            c, t = texts[i], texts[i + 1]
            e = tok.encode(c, t)
            f.write(json.dumps({"context": c, "text": t, "pair": True, "ids": e.ids}, ensure_ascii=False) + "\n")


if __name__ == "__main__":
    main()
