"""The Node side of the bridge: the N-API addon and the JS runtime.

CPU: the addon loads in Node and the runtime's host logic (topK, bf16 decode,
safetensors reader, PLE manifest checks) behaves like the reference.
GPU: the reference-shaped JS surface (SafeFileReader -> GPUW4Linear.load ->
GPUOps.w4, W4PleShardBundle.rowsToGpu, GPUOps.headChunk) runs on the HIP
path and its outputs match the oracle.
"""
import json
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

import synthetic as syn

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "gemma4-js_amd", "node", "g4hip.node")
NODE = shutil.which("node")

pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


def run_node(script, *args, timeout=120):
    if not os.path.exists(ADDON):
        pytest.fail("the Node addon is not built (python3 gemma4-js_amd/build.py)")
    p = subprocess.run([NODE, os.path.join(ROOT, "tests", "js", script)] + list(args),
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=timeout)
    assert p.returncode == 0, p.stderr[-4000:]
    return json.loads(p.stdout.strip().splitlines()[-1])


def test_js_runtime_host_logic(tmp_path):
    res = run_node("cpu_checks.js", str(tmp_path), os.path.join(ROOT, "tests", "golden", "ple_w4_layout.json"))
    assert res["ok"] and len(res["checks"]) == 7


def write_safetensors(path, tensors):
    """tensors: name -> (dtype string, shape, raw bytes)"""
    header, off, blobs = {}, 0, []
    for name, (dt, shape, raw) in tensors.items():
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        off += len(raw)
        blobs.append(raw)
    hj = json.dumps(header).encode()
    hj += b" " * ((8 - len(hj) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for b in blobs:
            f.write(b)


@pytest.mark.gpu
def test_js_device_side_loaders_match_host_loaders():
    """W4Weight built from DeviceBuffers and PleTable shards uploaded from a
    DeviceBuffer (both filled by fillRandom) give bit-identical linear
    outputs and gathered rows to the same bytes loaded from the host."""
    res = run_node("device_loaders.js")
    assert res == {"w4": True, "scalesNonzero": True, "ple": True, "pleNonzero": True}


@pytest.mark.gpu
def test_js_surface_on_gpu_matches_oracle(tmp_path, oracle):
    d = tmp_path
    rows, n, k = 3, 2048, 1536
    packed, scales, q = syn.w4_weights(31, n, k)
    _, x = syn.activations(31, rows, k)
    vocab_head, chunk_rows = 9000, 4096
    rng = np.random.default_rng(31)
    E = syn.bf16_rne(rng.standard_normal((vocab_head, k)).astype(np.float32) * np.float32(0.05))
    h = rng.standard_normal(k).astype(np.float32)
    write_safetensors(str(d / "model.safetensors"), {
        "model.layers.0.mlp.gate_proj.weight_packed": ("I32", packed.shape, packed.tobytes()),
        "model.layers.0.mlp.gate_proj.weight_scale": ("BF16", scales.shape, scales.tobytes()),
        "model.embed_tokens.weight": ("BF16", E.shape, E.tobytes()),
    })
    x.astype(np.float32).tofile(str(d / "x.f32"))
    h.tofile(str(d / "h.f32"))
    # a 3-shard PLE distribution in the builder's layout, last shard short
    vocab, width, rps = 9000, 8960, 4096
    shards = syn.ple_table(31, vocab, width, rps, threads=4)
    (d / "ple").mkdir()
    entries = []
    for i, s in enumerate(shards):
        r0, r1 = i * rps, min(vocab, (i + 1) * rps)
        name = "ple-%05d-of-%05d.bin" % (i, len(shards))
        s.tofile(str(d / "ple" / name))
        pb = (r1 - r0) * width // 2
        entries.append({"index": i, "file": name, "row_start": r0, "row_end": r1, "rows": r1 - r0,
                        "packed_offset": 0, "packed_bytes": pb, "scales_offset": pb,
                        "scales_bytes": (r1 - r0) * (width // 32) * 2, "bytes": int(s.nbytes)})
    manifest = {"format": "gemma4-ple-w4-sharded-v1", "version": 1, "complete": True,
                "width": width, "vocab_size": vocab,
                "quantization": {"bits": 4, "group_size": 32},
                "layout": {"kind": "row_sharded_packed_then_scales", "rows_per_shard": rps,
                           "packed_row_bytes": width // 2, "scale_row_bytes": (width // 32) * 2},
                "shards": entries}
    (d / "ple" / "manifest.json").write_text(json.dumps(manifest))
    ple_ids = [0, 4095, 4096, 8999, 17, 17, 8192]
    (d / "meta.json").write_text(json.dumps({"rows": rows, "ple_ids": ple_ids, "vocab": vocab,
                                             "chunk_rows": chunk_rows}))

    res = run_node("gpu_parity.js", str(d), timeout=300)
    assert res["ok"]
    assert res["linear"] == {"inDim": k, "outDim": n, "groupSize": 32, "groups": 48}

    y = np.fromfile(str(d / "y.f32"), dtype=np.float32).reshape(rows, n)
    ref = oracle.w4_linear(x, packed, scales).astype(np.float64)
    rel = np.linalg.norm(y - ref, axis=1) / np.linalg.norm(ref, axis=1)
    assert rel.max() <= 1e-3
    y_one = np.fromfile(str(d / "y_one.f32"), dtype=np.float32)
    y_replay = np.fromfile(str(d / "y_replay.f32"), dtype=np.float32)
    assert np.array_equal(y_replay, y_one)  # same kernel, deterministic
    assert np.linalg.norm(y_one - ref[0]) / np.linalg.norm(ref[0]) <= 1e-3

    ple = np.fromfile(str(d / "ple.f32"), dtype=np.float32).reshape(len(ple_ids), width)
    want = oracle.ple_gather(np.concatenate(shards), vocab, width, rps, np.array(ple_ids, np.int32))
    assert np.array_equal(ple.view(np.uint32), want.view(np.uint32))
    assert res["ple_range_error"] == "PLE token id out of range: %d" % vocab

    logits = np.fromfile(str(d / "logits.f32"), dtype=np.float32)
    want_l = oracle.bf16_head(h, E, 1.0, 30.0)
    assert np.allclose(logits, want_l, rtol=1e-4, atol=1e-4)
    assert res["top10"][0] == int(oracle.topk(want_l, 10)[0][0])


def _bf16_bytes(a):
    return syn.bf16_rne(np.asarray(a, np.float32)).astype(np.uint16).tobytes()


def small_checkpoint(tmp_path, max_seq=32):
    """A 5-layer model in the reference's tensor layout - W4 projections, BF16
    norms and layer scalars, tied BF16 embedding, dense BF16 per-layer
    embeddings - written to tmp_path/core.safetensors, with the driver config
    in tmp_path/cfg.json.  Returns (cfg, oracle Model)."""
    import layer_oracle as lo
    H, heads, P, V, window = 128, 2, 32, 512, 8
    specs = [  # sliding/global, own or shared KV, as spec(i) describes E2B layers
        dict(full=False, headDim=64, intermediate=256, shared=False, storeShared=True,
             attentionType="sliding", ropeBase=10000, ropeProp=1.0),
        dict(full=True, headDim=128, intermediate=256, shared=False, storeShared=True,
             attentionType="full", ropeBase=1000000, ropeProp=0.25),
        dict(full=False, headDim=64, intermediate=512, shared=True, storeShared=False,
             attentionType="sliding", ropeBase=10000, ropeProp=1.0),
        dict(full=True, headDim=128, intermediate=512, shared=True, storeShared=False,
             attentionType="full", ropeBase=1000000, ropeProp=0.25),
        dict(full=False, headDim=64, intermediate=512, shared=True, storeShared=False,
             attentionType="sliding", ropeBase=10000, ropeProp=1.0),
    ]
    NL = len(specs)
    rng = np.random.default_rng(77)
    T = {}
    E = syn.bf16_rne(rng.standard_normal((V, H)).astype(np.float32) * np.float32(0.05))
    T["model.language_model.embed_tokens.weight"] = ("BF16", (V, H), E.tobytes())
    ple_dense = syn.bf16_rne(rng.standard_normal((V, NL * P)).astype(np.float32) * np.float32(0.05))
    T["model.language_model.embed_tokens_per_layer.weight"] = ("BF16", (V, NL * P), ple_dense.tobytes())
    seed = [100]

    def lin(name, n, k):
        seed[0] += 1
        packed, scales, _ = syn.w4_weights(seed[0], n, k)
        T[name + ".weight_packed"] = ("I32", (n, k // 8), packed.astype(np.uint32).tobytes())
        T[name + ".weight_scale"] = ("BF16", (n, k // 32), scales.astype(np.uint16).tobytes())
        return packed, scales

    def norm(name, n):
        bits = syn.bf16_rne(rng.uniform(0.8, 1.2, n).astype(np.float32))
        T[name] = ("BF16", (n,), bits.tobytes())
        return syn.bf16_to_f32(bits).astype(np.float32)

    top = lin("model.language_model.per_layer_model_projection", NL * P, H)
    ple_norm = norm("model.language_model.per_layer_projection_norm.weight", P)
    final_norm = norm("model.language_model.norm.weight", H)
    layers = []
    for i, s in enumerate(specs):
        root = "model.language_model.layers.%d" % i
        hd, inter = s["headDim"], s["intermediate"]
        L = dict(head_dim=hd, intermediate=inter, full=s["full"],
                 kv_source=-1 if not s["shared"] else (1 if s["full"] else 0),
                 rope_base=float(s["ropeBase"]), rope_prop=s["ropeProp"], linear={}, norm={})
        shapes = [("q", "self_attn.q_proj", heads * hd, H), ("o", "self_attn.o_proj", H, heads * hd),
                  ("gate", "mlp.gate_proj", inter, H), ("up", "mlp.up_proj", inter, H),
                  ("down", "mlp.down_proj", H, inter), ("ple_gate", "per_layer_input_gate", P, H),
                  ("ple_proj", "per_layer_projection", H, P)]
        if not s["shared"]:
            shapes += [("k", "self_attn.k_proj", hd, H), ("v", "self_attn.v_proj", hd, H)]
        for key, name, n, k in shapes:
            L["linear"][key] = lin(root + "." + name, n, k)
        for key, name, n in [("input", "input_layernorm", H), ("post_attn", "post_attention_layernorm", H),
                             ("pre_ffw", "pre_feedforward_layernorm", H),
                             ("post_ffw", "post_feedforward_layernorm", H),
                             ("post_ple", "post_per_layer_input_norm", H), ("q", "self_attn.q_norm", hd)]:
            L["norm"][key] = norm(root + "." + name + ".weight", n)
        if not s["shared"]:
            L["norm"]["k"] = norm(root + ".self_attn.k_norm.weight", hd)
        sk = syn.bf16_rne(np.array([rng.uniform(0.9, 1.1)], np.float32))
        T[root + ".layer_scalar"] = ("BF16", (1,), sk.tobytes())
        L["skip"] = float(syn.bf16_to_f32(sk)[0])
        layers.append(L)
    ckpt = tmp_path / "core.safetensors"
    write_safetensors(str(ckpt), T)
    prompt = [int(t) for t in syn.token_ids(21, 11, V)]
    steps = 4
    cfg = dict(hidden=H, heads=heads, pleDim=P, window=window, maxSeq=max_seq, lmChunkRows=200,
               specs=specs, prompt=prompt, steps=steps)
    (tmp_path / "cfg.json").write_text(json.dumps(cfg))
    ple_f32 = syn.bf16_to_f32(ple_dense).reshape(V, NL * P)
    ref = lo.Model(H, heads, P, V, layers, E, lambda ids: ple_f32[np.asarray(ids)], top, ple_norm,
                   final_norm, window=window)
    return cfg, ref


def near_tie(lg, tok):
    return float(np.max(lg) - lg[tok]) <= 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("driver", ["ops", "engine"])
def test_js_model_driver_matches_oracle(tmp_path, oracle, driver):
    """Gemma4WebGPU's load/forward/logits/greedy from Node on the small
    checkpoint against the oracle model.  Two drivers: Gemma4Hip (one GPUOps
    call per op, as gemma4-webgpu.js) and Gemma4HipEngine (the native
    engine).  Logits of the prompt within relative L2 1e-3; greedy tokens
    equal unless the oracle's top two are within 1e-3.  The engine's recorded
    decode step must choose exactly the tokens of its one-token greedy calls."""
    cfg, ref = small_checkpoint(tmp_path)
    prompt = cfg["prompt"]
    res = run_node("model_parity.js", str(tmp_path / "core.safetensors"), str(tmp_path / "cfg.json"),
                   driver, timeout=300)
    want_tok, want_lg = ref.greedy(prompt, 0)
    got_lg = np.asarray(res["logits0"], np.float64)
    assert np.linalg.norm(got_lg - want_lg) / np.linalg.norm(want_lg) < 1e-3
    toks = res["tokens"]
    assert toks[0] == want_tok or near_tie(want_lg, toks[0])
    pos = len(prompt)
    for t_prev, t in zip(toks[:-1], toks[1:]):
        w, lg = ref.greedy([t_prev], pos)
        assert t == w or near_tie(lg, t), (pos, t, w)
        pos += 1
    assert res["cache"]["caches"] == 2 and res["cache"]["bytes"] == pos * (64 + 128) * 4 * 2
    assert res["appendError"] == "KV append position %d != cache length %d" % (pos + 5, pos)
    if driver == "engine":
        assert res["decoded"] == toks[1:]


def _stats_of(line):
    """The numbers of one formatStats line (gemma4-webgpu.js:59-63)."""
    import re
    m = re.search(r"finite=(\d+)/(\d+) nan=(\d+) inf=(\d+) min=(\S+) max=(\S+) mean=(\S+) "
                  r"std=(\S+)$", line)
    assert m, line
    f, c, nan, inf = (int(m.group(i)) for i in range(1, 5))
    return dict(finite=f, count=c, nan=nan, inf=inf, min=float(m.group(5)),
                max=float(m.group(6)), mean=float(m.group(7)), std=float(m.group(8)))


def _assert_stats(line, values, what):
    got = _stats_of(line)
    a = np.asarray(values, np.float64).ravel()
    assert got["count"] == a.size and got["finite"] == a.size, (what, line)
    assert got["nan"] == 0 and got["inf"] == 0, (what, line)
    want = dict(min=a.min(), max=a.max(), mean=a.mean(), std=a.std())
    for k, v in want.items():
        # 4 significant digits printed; FP32 against binary64 underneath
        tol = 2e-3 * max(abs(v), want["std"], 1e-30)
        assert abs(got[k] - v) <= tol, (what, k, got[k], v)


@pytest.mark.gpu
@pytest.mark.parametrize("driver", ["ops", "engine"])
def test_js_diagnostic_lines_match_oracle(tmp_path, oracle, driver):
    """forward(prompt, 0, {diagnostic: true}) and logits(h, {diagnostic: true})
    (gemma4-webgpu.js:311-440) log the reference's lines in its order: top
    hidden, top PLE, then per layer its hidden state, with layer 1's 23
    encodeLayer stages before it, then the logits and their first 16 values.
    Every statistic is checked against the same read-out of the oracle model.
    A NaN planted in layer 1's post-attention norm weight must stop the
    forward at that stage, with the reference's message."""
    cfg, ref = small_checkpoint(tmp_path)
    ckpt, cfgp = str(tmp_path / "core.safetensors"), str(tmp_path / "cfg.json")
    res = run_node("diag_parity.js", ckpt, cfgp, driver, timeout=300)
    assert res["error"] is None, res["error"]
    probes = {}
    last = ref.forward(cfg["prompt"], 0, probes=probes)
    lines = res["lines"]
    NL = len(cfg["specs"])
    assert lines[0].startswith("[diag top hidden] ")
    _assert_stats(lines[0], probes["top hidden"], "top hidden")
    assert lines[1].startswith("[diag top PLE]    ")
    _assert_stats(lines[1], probes["top PLE"], "top PLE")
    i = 2
    for layer in range(NL):
        if layer == 1:
            assert lines[i] == "[diag layer 01 stages]"
            i += 1
            names = list(probes["stages"])
            assert len(names) == 23
            for name in names:
                assert lines[i].startswith("  " + name.ljust(20) + " "), (lines[i], name)
                _assert_stats(lines[i], probes["stages"][name], name)
                i += 1
        assert lines[i].startswith("[diag layer %02d] " % layer)
        _assert_stats(lines[i], probes["layer %d" % layer], "layer %d" % layer)
        i += 1
    lg = ref.logits(last)
    assert lines[i].startswith("[diag logits] ")
    _assert_stats(lines[i], lg, "logits")
    first = [float(v) for v in lines[i + 1][len("[diag logits first 16] "):].split()]
    assert len(first) == 16 and np.allclose(first, lg[:16], rtol=1e-3, atol=1e-4 * np.abs(lg).max())
    assert len(lines) == i + 2
    bad = run_node("diag_parity.js", ckpt, cfgp, driver,
                   "model.language_model.layers.1.post_attention_layernorm.weight", timeout=300)
    assert bad["error"] == "First non-finite Layer 1 stage: postAttentionNorm."
    assert bad["lines"][-1].startswith("  postAttentionNorm    ") and "nan=0 " not in bad["lines"][-1]


def reference_decode(tj, ids, skip_special):
    """standalone-tokenizer.js decode on a Gemma-layout tokenizer.json: ids to
    token texts (special added tokens dropped when skip_special), "▁" to
    space, runs of <0xHH> tokens as UTF-8 with U+FFFD per maximal invalid
    subpart, joined."""
    import re
    inv = {v: k for k, v in tj["model"]["vocab"].items()}
    special = {a["id"] for a in tj["added_tokens"] if a["special"]}
    out, buf = [], bytearray()
    for i in ids:
        if skip_special and i in special:
            continue
        t = inv[i].replace("▁", " ")
        m = re.fullmatch(r"<0x([0-9A-Fa-f]{2})>", t)
        if m:
            buf.append(int(m.group(1), 16))
            continue
        if buf:
            out.append(bytes(buf).decode("utf-8", "replace"))
            buf = bytearray()
        out.append(t)
    if buf:
        out.append(bytes(buf).decode("utf-8", "replace"))
    return "".join(out)


@pytest.mark.gpu
@pytest.mark.parametrize("driver", ["ops", "engine"])
def test_js_generate_matches_oracle(tmp_path, oracle, driver):
    """The generation loop of main.js:342-556 (gemma4-js_amd/node/generate.js)
    on the small checkpoint with a 512-token toy tokenizer: the chat prompt
    encodes as Hugging Face `tokenizers` encodes it; every generated token is
    the oracle model's greedy choice (or within 1e-3 of its top logit), fed
    back at position prompt + g - 1; the text is the reference's decoding; a
    stop token ends the loop before it is appended, and the KV capacity ends
    it after prompt + 4 positions.  The engine's chunked device decode gives
    the same tokens."""
    import toy_tokenizer as tt
    tokenizers = pytest.importorskip("tokenizers")
    cfg, ref = small_checkpoint(tmp_path, max_seq=64)
    cfg.update(genPrompt="hi there", genMax=12)
    (tmp_path / "cfg.json").write_text(json.dumps(cfg))
    tj = tt.write_toy_dir(str(tmp_path / "tok"), 512, 5)
    hf = tokenizers.Tokenizer.from_str(json.dumps(tj))
    res = run_node("generate_parity.js", str(tmp_path / "core.safetensors"), str(tmp_path / "cfg.json"),
                   str(tmp_path / "tok"), driver, timeout=300)
    runs = res["runs"]
    step = runs["step"]
    rendered = "<bos><|turn>user\nhi there<turn|>\n<|turn>model\n"
    assert step["rendered"] == rendered and step["inputIds"] == hf.encode(rendered).ids
    stops = {1, 5, tj["model"]["vocab"]["<turn|>"]}
    gen = step["generated"]
    assert not stops & set(gen)
    assert step["stopReason"] in ("max_new_tokens", "stop_token")
    seq = gen + ([step["stopTokenId"]] if step["stopReason"] == "stop_token" else [])
    if step["stopReason"] == "max_new_tokens":
        assert len(gen) == cfg["genMax"]
    ids = step["inputIds"]
    w, lg = ref.greedy(ids, 0)
    for g, t in enumerate(seq):
        assert t == w or near_tie(lg, t), (g, t, w)
        if g + 1 < len(seq):
            w, lg = ref.greedy([t], len(ids) + g)
    assert step["text"] == reference_decode(tj, gen, True)
    assert step["rawText"] == reference_decode(tj, gen, False)
    if driver == "engine":
        assert runs["chunk"]["generated"] == gen and runs["chunk"]["stopReason"] == step["stopReason"]
    k = res["k"]
    if k >= 0:
        for name in ["stop"] + (["stopChunk"] if driver == "engine" else []):
            assert runs[name]["generated"] == gen[:k], name
            assert runs[name]["stopReason"] == "stop_token" and runs[name]["stopTokenId"] == gen[k], name
    cap = runs["cap"]
    if len(gen) >= 5:
        assert cap["generated"] == gen[:5] and cap["stopReason"] == "kv_capacity"
    else:
        assert cap["generated"] == gen and cap["stopReason"] == step["stopReason"]
