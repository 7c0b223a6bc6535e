"""The Node tokenizer and generation loop (gemma4-js_amd/node/tokenizer.js,
generate.js), the counterparts of custom-webgpu/standalone-tokenizer.js and
the generate handler of custom-webgpu/main.js:342-556.

The tokenizer is checked against Hugging Face `tokenizers`, an independent
implementation of the tokenizer.json semantics the reference restates:
- on seeded toy tokenizers in the Gemma 4 layout (always run);
- on the reference's Gemma 4 tokenizer.json, through the committed golden
  vectors and a seeded random corpus (run where that file is present).
Where the reference and `tokenizers` differ - invalid UTF-8 in byte-fallback
tokens, which the reference's TextDecoder replaces per maximal subpart and
`tokenizers` per byte - the reference's behaviour is pinned with Python's
UTF-8 decoder, which follows the same maximal-subpart rule.
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import toy_tokenizer as tt

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which("node")
GEMMA_DIR = "/root/reference/tokenizer/gemma4"
GOLDEN = os.path.join(ROOT, "tests", "golden", "gemma4_tokenizer_vectors.json")

pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")
tokenizers = pytest.importorskip("tokenizers")
needs_gemma = pytest.mark.skipif(not os.path.exists(os.path.join(GEMMA_DIR, "tokenizer.json")),
                                 reason="the Gemma 4 tokenizer.json is not present")


def run_tok(tok_dir, req, tmp_path, timeout=180):
    rp = tmp_path / "req.json"
    rp.write_text(json.dumps(req, ensure_ascii=False), encoding="utf-8")
    p = subprocess.run([NODE, os.path.join(ROOT, "tests", "js", "tokenizer_driver.js"), str(tok_dir), str(rp)],
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, timeout=timeout)
    assert p.returncode == 0, p.stderr.decode("utf-8", "replace")[-4000:]
    return json.loads(p.stdout.decode("utf-8").strip().splitlines()[-1])


@pytest.mark.parametrize("vocab,seed", [(512, 0), (4096, 3), (20000, 7)])
def test_toy_bpe_matches_hf_tokenizers(tmp_path, vocab, seed):
    """Encode and decode of random texts built from vocabulary pieces, with
    characters outside the vocabulary (byte fallback) and special tokens."""
    d = tmp_path / "tok"
    tj = tt.write_toy_dir(str(d), vocab, seed)
    hf = tokenizers.Tokenizer.from_str(json.dumps(tj))
    texts = tt.random_texts(seed + 100, 300, tj)
    want = [hf.encode(t).ids for t in texts]
    res = run_tok(d, dict(encode=texts, decode=want, decodeRaw=want), tmp_path)
    for t, w, g in zip(texts, want, res["encode"]):
        assert g == w, (t, w, g)
    assert res["decode"] == [hf.decode(w, skip_special_tokens=True) for w in want]
    assert res["decodeRaw"] == [hf.decode(w, skip_special_tokens=False) for w in want]
    assert res["decodeRaw"] == texts  # byte fallback makes every valid text round-trip


def test_merge_order_lowest_rank_then_leftmost(tmp_path):
    """Hand-made merges where the order decides the result: on "aaa" the
    leftmost of two equal-rank pairs merges first (aa|a, not a|aa), and a
    lower rank beats a pair further left ("xbc" -> x|bc before xb|c)."""
    d = tmp_path / "tok"
    tj = tt.write_toy_dir(str(d), 300, 1)
    v = tj["model"]["vocab"]
    mine = ["a", "b", "c", "x", "aa", "bc", "xb", "abc", "xbc"]
    for t in mine:
        v.setdefault(t, len(v))
    # only these merges apply to strings of a, b, c and x
    m = [["b", "c"], ["a", "a"], ["x", "b"], ["a", "bc"]]
    m += [p for p in tj["model"]["merges"] if p[0] not in mine and p[1] not in mine]
    tj["model"]["merges"] = m
    (d / "tokenizer.json").write_text(json.dumps(tj, ensure_ascii=False), encoding="utf-8")
    hf = tokenizers.Tokenizer.from_str(json.dumps(tj))
    texts = ["aaa", "aaaa", "xbc", "abc", "aabc", "xbcaaa"]
    res = run_tok(d, dict(encode=texts), tmp_path)
    assert res["encode"] == [hf.encode(t).ids for t in texts]
    assert res["encode"][0] == [v["aa"], v["a"]]
    assert res["encode"][2] == [v["x"], v["bc"]]


def test_byte_fallback_decode_follows_textdecoder(tmp_path):
    """Runs of <0xHH> tokens decode as UTF-8 with U+FFFD for each maximal
    invalid subpart (the reference's TextDecoder), as Python decodes them."""
    d = tmp_path / "tok"
    tj = tt.write_toy_dir(str(d), 512, 0)
    v = tj["model"]["vocab"]
    seqs = [[0xE4, 0xBD], [0xFF, 0xE4, 0xBD, 0xA0], [0xF0, 0x9F, 0xA4], [0xC3, 0xA9, 0xC3],
            [0xED, 0xA0, 0x80], [0x80, 0x80], [0xE4, 0xBD, 0xA0, 0xE5, 0xA5, 0xBD]]
    ids = [[v["<0x%02X>" % b] for b in s] + [v["a"]] for s in seqs]
    res = run_tok(d, dict(decode=ids), tmp_path)
    assert res["decode"] == [bytes(s).decode("utf-8", "replace") + "a" for s in seqs]


def test_chat_template_stop_ids_and_errors(tmp_path):
    """renderChat/encodeChat (standalone-tokenizer.js:736-780), stopTokenIds
    (782-814) and the reasoning split of main.js:127-161, by their closed
    forms."""
    d = tmp_path / "tok"
    tj = tt.write_toy_dir(str(d), 512, 0, eos_ids=(1, 7))
    hf = tokenizers.Tokenizer.from_str(json.dumps(tj))
    msgs = [{"role": "user", "content": "hi there"}, {"role": "assistant", "content": "yo"},
            {"role": "user", "content": 42}]
    split_cases = [
        ["plain answer", "plain answer"],
        ["<|channel>thought\nstep one", "x"],
        ["<|channel>thought\nwhy<channel|><|channel>final\n  the answer<channel|>", "plain"],
        ["<|channel>thought\nwhy<channel|>   ", "fallback"],
    ]
    res = run_tok(d, dict(
        chat=[dict(messages=msgs, opts={}), dict(messages=msgs[:1], opts=dict(enableThinking=True)),
              dict(messages=msgs[:1], opts=dict(addGenerationPrompt=False))],
        badChat=[[{"role": "system", "content": "s"}]], stop=True, split=split_cases), tmp_path)
    r0 = "<bos><|turn>user\nhi there<turn|>\n<|turn>assistant\nyo<turn|>\n<|turn>user\n42<turn|>\n<|turn>model\n"
    r1 = "<bos><|turn>system\n<|think|>\n<turn|>\n<|turn>user\nhi there<turn|>\n<|turn>model\n"
    r2 = "<bos><|turn>user\nhi there<turn|>\n"
    assert [c["rendered"] for c in res["chat"]] == [r0, r1, r2]
    assert [c["ids"] for c in res["chat"]] == [hf.encode(r).ids for r in (r0, r1, r2)]
    assert res["badChat"] == ["Standalone Gemma 4 text template currently supports user/assistant messages, got system."]
    assert res["stop"] == sorted({1, 7, tj["model"]["vocab"]["<turn|>"]})
    assert res["split"] == [
        {"reasoning": "", "answer": "plain answer"},
        {"reasoning": "step one", "answer": ""},
        {"reasoning": "why", "answer": "the answer"},
        {"reasoning": "why", "answer": "fallback"},
    ]


@needs_gemma
def test_gemma4_golden_vectors(tmp_path):
    """The committed vectors (ids by `tokenizers` on the reference's
    tokenizer.json): encode, both decodes, and the text round trip."""
    g = json.load(open(GOLDEN, encoding="utf-8"))
    vecs = g["vectors"]
    res = run_tok(GEMMA_DIR, dict(encode=[v["text"] for v in vecs], decode=[v["ids"] for v in vecs],
                                  decodeRaw=[v["ids"] for v in vecs], describe=True, stop=True), tmp_path)
    for v, ids in zip(vecs, res["encode"]):
        assert ids == v["ids"], v["text"]
    assert res["decode"] == [v["decoded"] for v in vecs]
    assert res["decodeRaw"] == [v["decoded_raw"] for v in vecs]
    assert res["decodeRaw"] == [v["text"] for v in vecs]
    assert res["describe"] == {"modelType": "BPE", "vocabSize": 262144, "merges": 514906, "byteFallback": True,
                               "pretokenizers": ["Split"], "decoders": ["Replace", "ByteFallback", "Fuse"],
                               "specialTokens": 24}
    # generation_config eos [1, 106, 50] with <eos> = 1 and <turn|> = 106
    assert res["stop"] == [1, 50, 106]


def random_unicode(rng, n):
    ranges = [(0x20, 0x7E), (0x0A, 0x0A), (0xA0, 0x24F), (0x370, 0x3FF), (0x400, 0x4FF), (0x590, 0x6FF),
              (0x900, 0x97F), (0xE00, 0xE7F), (0x3040, 0x30FF), (0x4E00, 0x9FFF), (0xAC00, 0xD7A3),
              (0x1F300, 0x1FAFF), (0x20000, 0x2A6DF), (0xE000, 0xF8FF)]
    out = []
    for _ in range(n):
        k = int(rng.integers(0, 60))
        s = []
        for _ in range(k):
            lo, hi = ranges[int(rng.integers(len(ranges)))] if rng.random() < 0.4 else ranges[0]
            s.append(chr(int(rng.integers(lo, hi + 1))))
        out.append("".join(s))
    return out


@needs_gemma
def test_gemma4_random_corpus_matches_hf_tokenizers(tmp_path):
    """400 seeded strings over ASCII, Latin, Greek, Cyrillic, Hebrew/Arabic,
    Devanagari, Thai, kana, CJK (BMP and plane 2), Hangul, emoji and private
    use, plus whole chat renderings."""
    hf = tokenizers.Tokenizer.from_file(os.path.join(GEMMA_DIR, "tokenizer.json"))
    rng = np.random.default_rng(2024)
    texts = random_unicode(rng, 400)
    texts += ["<bos><|turn>user\n%s<turn|>\n<|turn>model\n" % t for t in texts[:20]]
    want = [hf.encode(t).ids for t in texts]
    res = run_tok(GEMMA_DIR, dict(encode=texts, decodeRaw=want), tmp_path)
    for t, w, g in zip(texts, want, res["encode"]):
        assert g == w, t
    assert res["decodeRaw"] == texts


GEN_MOCK = r"""
'use strict';
// A scripted model: greedy() returns the next token of a fixed sequence and
// records (ids, position); decode(k) returns the next k.
const { generate } = require(process.argv[2]);
const cases = JSON.parse(process.argv[3]);
const tokenizer = {
  encodeChat: (m) => ({ rendered: 'R', ids: cases.prompt }),
  stopTokenIds: () => new Set(cases.stop),
  decode: (ids, o) => ids.map((i) => (o.skipSpecialTokens && cases.stop.includes(i) ? '' : String.fromCharCode(97 + (i % 26)))).join(''),
};
function model(seq) {
  let i = 0;
  const calls = [];
  return {
    calls,
    resetCache() { calls.push(['reset']); i = 0; },
    async greedy(ids, pos) { calls.push(['greedy', ids.length, pos]); return { nextTokenId: seq[i++] }; },
    decode(k) { calls.push(['decode', k]); const r = seq.slice(i, i + k); i += k; return Int32Array.from(r); },
  };
}
(async () => {
  const out = [];
  for (const c of cases.runs) {
    const m = model(cases.seq);
    const r = await generate(m, tokenizer, 'p', c);
    out.push({ generated: r.generated, stopReason: r.stopReason, text: r.text, calls: m.calls });
  }
  console.log(JSON.stringify(out));
})().catch((e) => { console.error(e.stack); process.exit(1); });
"""


def test_generate_loop_semantics(tmp_path):
    """main.js:342-556 with a scripted model: the stop token ends the loop
    before it is appended; maxNewTokens and the KV capacity end it; token g
    is fed at position prompt + g - 1; the chunked device decode returns the
    same tokens and never asks past either limit."""
    script = tmp_path / "gen_mock.js"
    script.write_text(GEN_MOCK)
    prompt = [2, 10, 11, 12]
    seq = [20, 21, 22, 23, 1, 24, 25, 26, 27, 28, 29, 30]
    runs = [dict(maxNewTokens=10, maxSeq=64), dict(maxNewTokens=10, maxSeq=64, chunk=3),
            dict(maxNewTokens=3, maxSeq=64), dict(maxNewTokens=3, maxSeq=64, chunk=8),
            dict(maxNewTokens=10, maxSeq=6), dict(maxNewTokens=10, maxSeq=6, chunk=8)]
    cases = dict(prompt=prompt, seq=seq, stop=[1], runs=runs)
    p = subprocess.run([NODE, str(script), os.path.join(ROOT, "gemma4-js_amd", "node", "generate.js"),
                        json.dumps(cases)], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=60)
    assert p.returncode == 0, p.stderr
    r = json.loads(p.stdout.strip().splitlines()[-1])
    # stop token 1 is the 5th token: 4 generated
    assert r[0]["generated"] == [20, 21, 22, 23] and r[0]["stopReason"] == "stop_token"
    assert r[0]["calls"] == [["reset"], ["greedy", 4, 0], ["greedy", 1, 4], ["greedy", 1, 5],
                             ["greedy", 1, 6], ["greedy", 1, 7]]
    assert r[0]["text"] == "uvwx"
    assert r[1]["generated"] == r[0]["generated"] and r[1]["stopReason"] == "stop_token"
    assert r[1]["calls"] == [["reset"], ["greedy", 4, 0], ["decode", 3], ["decode", 3]]
    # maxNewTokens 3: no model call after the third token
    assert r[2]["generated"] == [20, 21, 22] and r[2]["stopReason"] == "max_new_tokens"
    assert r[2]["calls"][-1] == ["greedy", 1, 5]
    assert r[3]["generated"] == [20, 21, 22] and r[3]["calls"] == [["reset"], ["greedy", 4, 0], ["decode", 2]]
    # capacity 6 with a 4-token prompt: positions 4 and 5 are fed, then the loop ends
    assert r[4]["generated"] == [20, 21, 22] and r[4]["stopReason"] == "kv_capacity"
    assert r[4]["calls"][-1] == ["greedy", 1, 5]
    assert r[5]["generated"] == [20, 21, 22] and r[5]["calls"] == [["reset"], ["greedy", 4, 0], ["decode", 2]]
