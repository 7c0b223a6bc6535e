"""Writes gemma4_tokenizer_vectors.json: the Gemma 4 tokenizer's ids for a
fixed set of texts, as Hugging Face `tokenizers` (an independent
implementation of the same tokenizer.json semantics) computes them from the
reference's tokenizer/gemma4/tokenizer.json.

Each vector holds the text, its ids, and the decoding of those ids with and
without special tokens. Run from the repository root:

    python3 tests/golden/make_tokenizer_vectors.py [/root/reference/tokenizer/gemma4]
"""
import json
import os
import sys

from tokenizers import Tokenizer
import tokenizers

HERE = os.path.dirname(os.path.abspath(__file__))

TEXTS = [
    "",
    "Hello world!",
    "The quick brown fox jumps over the lazy dog.",
    " leading space",
    "trailing space ",
    "  two   three    four     spaces",
    "line one\nline two\r\nline three\n\n\n\nfour newlines",
    "\ttab\t\ttabs\t\t\t",
    " " * 40 + "forty spaces, then " + "\n" * 33 + "33 newlines",
    "def f(x):\n    return x ** 2  # square\n",
    '{"key": [1, 2.5, -3e10], "nested": {"a": null, "b": true}}',
    "3.14159 1,000,000 2024-12-01 0x1F 1e-7 99.9% $12.50",
    "https://example.com/path?query=1&other=two#frag",
    "Привет, мир! Ελληνικά. עברית. العربية. हिन्दी. ไทย. 한국어.",
    "日本語のテキストと中文文本，还有標點符號。",
    "emoji 🤖👍🏽 family 👨‍👩‍👧‍👦 flag 🇯🇵 keycap 1️⃣",
    "combining é vs é, Å vs Å, zero​width‍joiner",
    "rare 𝔘𝔫𝔦𝔠𝔬𝔡𝔢 𠀀𠀁 \U0001f9ff  private",
    "<|turn>user\nHi<turn|>\n<|turn>model\n",
    "<bos><|turn>system\n<|think|>\n<turn|>\n<|turn>user\nWhy?<turn|>\n<|turn>model\n",
    "<|turn><turn|><|turn>adjacent specials<eos><pad><unk><mask>",
    "partial specials <|tur <turn| |turn> <|think <channel",
    "<|channel>thought\nreasoning here<channel|>the answer",
    "<|image|><|audio|><|video|><|image><image|><|audio><audio|>",
    "<|tool_call>call<tool_call|><|tool_response>resp<tool_response|><|\"|>",
    "mixed<|turn>inside words<turn|>again",
    "UPPER lower MiXeD CamelCaseIdentifier snake_case_identifier kebab-case",
    "a" * 100,
    "ab" * 60,
    " non-breaking space　ideographic space",
    "control \x01\x02\x1f chars and DEL \x7f",
]


def main():
    src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tokenizer/gemma4"
    tok = Tokenizer.from_file(os.path.join(src, "tokenizer.json"))
    vectors = []
    for t in TEXTS:
        ids = tok.encode(t).ids
        vectors.append(dict(text=t, ids=ids, decoded=tok.decode(ids, skip_special_tokens=True),
                            decoded_raw=tok.decode(ids, skip_special_tokens=False)))
    out = dict(source="tokenizer/gemma4/tokenizer.json", generator="tokenizers %s" % tokenizers.__version__,
               vectors=vectors)
    with open(os.path.join(HERE, "gemma4_tokenizer_vectors.json"), "w", encoding="utf-8") as f:
        json.dump(out, f, ensure_ascii=False, indent=1)
    print("wrote %d vectors" % len(vectors))


if __name__ == "__main__":
    main()
