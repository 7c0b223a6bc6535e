"""Seeded toy tokenizer.json files in the Gemma 4 layout, for the tokenizer
and generation tests.

The layout is that of the Gemma 4 file: normalizer Replace(" " -> "▁"),
pre-tokenizer Split(" ", MergedWithPrevious), a BPE model with byte_fallback
and the 256 <0xHH> tokens, and decoder Replace("▁" -> " "), ByteFallback,
Fuse.  The merges are drawn at random over the growing vocabulary, so they
include chains, pairs of byte tokens, and several pairs that make the same
string; every merge result is in the vocabulary, as Hugging Face
`tokenizers` requires.
"""
import json
import os

import numpy as np

SPECIALS = ["<pad>", "<eos>", "<bos>", "<unk>", "<|turn>", "<turn|>", "<|think|>", "<|channel>",
            "<channel|>"]
ALPHABET = list("▁\nabcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789.,!?'-:;()")


def toy_tokenizer(vocab_size=512, seed=0, alphabet=ALPHABET):
    """Returns the tokenizer.json dict: specials first, then the byte tokens,
    the alphabet and merge results up to vocab_size tokens."""
    rng = np.random.default_rng(seed)
    vocab = {}
    for t in SPECIALS:
        vocab[t] = len(vocab)
    byte_tokens = ["<0x%02X>" % b for b in range(256)]
    for t in byte_tokens + list(alphabet):
        vocab.setdefault(t, len(vocab))
    # draws: mostly the alphabet and earlier merge results (so merges chain),
    # now and then a byte token
    merges, seen = [], set()
    tokens = list(alphabet)

    def pick():
        u = rng.random()
        if u < 0.05:
            return byte_tokens[int(rng.integers(256))]
        if u < 0.5:
            return alphabet[int(rng.integers(len(alphabet)))]
        return tokens[int(rng.integers(len(tokens)))]

    while len(vocab) < vocab_size and len(merges) < 4 * vocab_size:
        a, b = pick(), pick()
        if (a, b) in seen or len(a) + len(b) > 12:
            continue
        seen.add((a, b))
        merges.append([a, b])
        if a + b not in vocab:
            vocab[a + b] = len(vocab)
            tokens.append(a + b)
    return {
        "version": "1.0",
        "truncation": None,
        "padding": None,
        "added_tokens": [dict(id=vocab[t], content=t, single_word=False, lstrip=False, rstrip=False,
                              normalized=False, special=True) for t in SPECIALS],
        "normalizer": {"type": "Replace", "pattern": {"String": " "}, "content": "▁"},
        "pre_tokenizer": {"type": "Split", "pattern": {"String": " "}, "behavior": "MergedWithPrevious",
                          "invert": False},
        "post_processor": None,
        "decoder": {"type": "Sequence", "decoders": [
            {"type": "Replace", "pattern": {"String": "▁"}, "content": " "},
            {"type": "ByteFallback"}, {"type": "Fuse"}]},
        "model": {"type": "BPE", "dropout": None, "unk_token": "<unk>", "continuing_subword_prefix": None,
                  "end_of_word_suffix": None, "fuse_unk": True, "byte_fallback": True,
                  "ignore_merges": False, "vocab": vocab, "merges": merges},
    }


def write_toy_dir(path, vocab_size=512, seed=0, eos_ids=(1, 5)):
    """Writes tokenizer.json, tokenizer_config.json and generation_config.json
    of a toy tokenizer into path; returns the tokenizer.json dict."""
    os.makedirs(path, exist_ok=True)
    tj = toy_tokenizer(vocab_size, seed)
    with open(os.path.join(path, "tokenizer.json"), "w", encoding="utf-8") as f:
        json.dump(tj, f, ensure_ascii=False)
    cfg = dict(bos_token="<bos>", eos_token="<eos>", unk_token="<unk>", pad_token="<pad>",
               sot_token="<|turn>", eot_token="<turn|>", think_token="<|think|>")
    with open(os.path.join(path, "tokenizer_config.json"), "w") as f:
        json.dump(cfg, f)
    with open(os.path.join(path, "generation_config.json"), "w") as f:
        json.dump({"bos_token_id": 2, "eos_token_id": list(eos_ids), "pad_token_id": 0}, f)
    return tj


def random_texts(seed, n, tokenizer_json, extra=("é", "中", "🤖", "ß", "\t", "  ", "<|turn>", "<turn|>")):
    """n strings made of vocabulary token texts (so that merges apply and
    chain), with "▁" written as a space, plus characters outside the
    vocabulary and special-token texts.  Pieces that spell a byte token's
    name are left out: such text could merge into the byte token itself and
    not round-trip."""
    rng = np.random.default_rng(seed)
    words = [t.replace("▁", " ") for t in tokenizer_json["model"]["vocab"]
             if t not in SPECIALS and "<0x" not in t] + list(extra)
    out = []
    for _ in range(n):
        length = int(rng.integers(0, 24))
        out.append("".join(words[int(rng.integers(len(words)))] for _ in range(length)))
    return out
