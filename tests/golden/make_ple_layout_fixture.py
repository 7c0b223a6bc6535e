"""Writes tests/golden/ple_w4_layout.json from the reference distribution manifest.

The fixture is data only: the PLE W4 table geometry and its shard table
(row ranges, packed/scales offsets and byte counts) exactly as the reference's
webgpu-distribution/ple-w4/manifest.json records them.  The sha256 digests are
dropped: the shard files themselves are not part of the reference checkout.

    python3 tests/golden/make_ple_layout_fixture.py [/path/to/gemma4-js]
"""
import json
import os
import sys

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
SRC = os.path.join(REF, "webgpu-distribution", "ple-w4", "manifest.json")
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ple_w4_layout.json")

KEYS = ["format", "version", "complete", "shape", "width", "vocab_size", "quantization",
        "layout", "source_bytes", "packed_bytes", "scale_bytes", "total_bytes", "ratio",
        "verification_rows"]
SHARD_KEYS = ["index", "file", "row_start", "row_end", "rows", "packed_offset", "packed_bytes",
              "scales_offset", "scales_bytes", "bytes"]

m = json.load(open(SRC))
fixture = {k: m[k] for k in KEYS}
fixture["shards"] = [{k: s[k] for k in SHARD_KEYS} for s in m["shards"]]
fixture["source"] = "webgpu-distribution/ple-w4/manifest.json (sha256 fields dropped)"
with open(OUT, "w") as f:
    json.dump(fixture, f, indent=1)
    f.write("\n")
print("wrote", OUT)
