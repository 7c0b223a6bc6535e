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
    assert res["ok"] and len(res["checks"]) == 6


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
