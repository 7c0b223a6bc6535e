"""Build recipe for libg4hip (gfx950 HIP kernels + C ABI) and its Node addon.

    python3 gemma4-js_amd/build.py            # library + Node addon
    python3 gemma4-js_amd/build.py --lib      # library only

Outputs stay in the source tree (git-ignored):
    gemma4-js_amd/lib/libg4hip.so
    gemma4-js_amd/node/g4hip.node   (links libg4hip.so through $ORIGIN/../lib)
"""
import concurrent.futures
import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
OBJDIR = os.path.join(PKG, "_build")
LIB = os.path.join(LIBDIR, "libg4hip.so")
NODE_DIR = os.path.join(PKG, "node")
ADDON = os.path.join(NODE_DIR, "g4hip.node")
NODE_INCLUDE = "/usr/include/node"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed-FP32 VALU forms are kept out of every kernel: the compiler may not
# emit them for ordinary float code.
HIP_FLAGS = [
    "--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-Wall", "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE, "-I", CSRC,
]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so;
    # that line is noise, everything else is shown.
    out = "\n".join(l for l in p.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if p.returncode != 0:
        raise RuntimeError("command failed (%d): %s\n%s" % (p.returncode, " ".join(cmd), out))
    return out


def build_lib(verbose=False):
    os.makedirs(LIBDIR, exist_ok=True)
    os.makedirs(OBJDIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError("no HIP sources under " + CSRC)
    objs = []

    def compile_one(src):
        obj = os.path.join(OBJDIR, os.path.basename(src)[:-4] + ".o")
        out = _run([HIPCC] + HIP_FLAGS + ["-c", src, "-o", obj])
        return obj, out

    workers = min(len(sources), max(1, (os.cpu_count() or 2) // 2), 8)
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        for obj, out in ex.map(compile_one, sources):
            objs.append(obj)
            if verbose and out.strip():
                print(out)
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + objs)
    os.replace(tmp, LIB)
    return LIB


def build_node_addon():
    """The N-API addon; skipped (returns None) when Node headers are absent."""
    src = os.path.join(NODE_DIR, "g4_napi.cc")
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")) or not os.path.exists(src):
        return None
    tmp = ADDON + ".tmp"
    _run(["g++", "-O2", "-std=c++14", "-fPIC", "-shared", "-Wall",
          "-DNAPI_VERSION=8", "-DNODE_GYP_MODULE_NAME=g4hip", "-I", NODE_INCLUDE, "-I", INCLUDE, src,
          "-o", tmp, "-L", LIBDIR, "-lg4hip", "-Wl,-rpath,$ORIGIN/../lib"])
    os.replace(tmp, ADDON)
    return ADDON


def build_all(verbose=False):
    lib = build_lib(verbose)
    addon = build_node_addon()
    return lib, addon


if __name__ == "__main__":
    if "--lib" in sys.argv:
        print(build_lib(verbose=True))
    else:
        print(build_all(verbose=True))
