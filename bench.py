#!/usr/bin/env python3
"""Benchmark of the W4A16 / PLE hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]

Headline (`value`): decode W4A16 GEMV, M=1, K=1536, N=6144 (the E2B
gate/up shape; BF16 activations, BF16 group-32 scales, FP32 accumulate,
FP32 output).  The GEMV rotates over 120 distinct device copies of the
weights (640 MB, well beyond the 256 MB Infinity Cache and the 8 x 4 MB L2),
so every launch streams its 5.3 MB from HBM.  One step = one replay of the
whole rotation (120 GEMV launches recorded once as a command buffer, i.e. a
HIP graph), so the host launch path is not what is timed and the timed region
holds steps x 120 launches whatever the step count.  value = algorithmic
bytes of all timed launches / time; ms_per_step is per rotation and
roofline.avg_launch_us per GEMV.

Algorithmic bytes per GEMV = N*K/2 packed + N*(K/32)*2 scales + K*2 x (BF16)
+ N*4 y (FP32) = 5,336,064 B.

Extras (same JSON line, "extra"): one E2B sliding decoder layer of 7 GEMVs
(aggregate GB/s), PLE gather of 1 and 2048 ids over the full [262144, 8960]
table, the tied BF16 LM head over 262144 rows, the prefill GEMM (M=2048) at
both shapes in TFLOP/s, and the full random-init Gemma-4-E2B decode (prompt
of 512 random ids, then 256 greedy steps, max_seq 1024): decode tokens/s,
also reported as "decode_tok_s" on the line, and prefill tokens/s.

cpu_baseline: the oracle's TF.js-semantics FP32 dequant + matMul
restatement of the headline GEMV timed on the host, about 5 s per leg:
single-threaded JavaScript under Node (the reference's tfjs-backend-cpu is
single-threaded JS), C on one core and C on every core this process may use
(`value`, `cores` = those threads; `nproc` is the host's count).
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gemma4-js_amd"))

import numpy as np  # noqa: E402

import g4hip  # noqa: E402
import synthetic as syn  # noqa: E402

METRIC = "W4A16 GEMV GB/s (% of 8 TB/s HBM) + decode tok/s, E2B-shaped, 1 MI355X"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
COLD_BYTES = 640e6  # rotation footprint: > 2x the 256 MB Infinity Cache


def w4_bytes(n, k, m=1, x_bytes=2, y_bytes=4):
    return n * k // 2 + n * (k // 32) * 2 + m * k * x_bytes + m * n * y_bytes


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_cmdbufs(cbs, reps):
    """Submit each command buffer in `cbs` `reps` times; return elapsed ms."""
    e0, e1 = g4hip.Event(), g4hip.Event()
    e0.record()
    for _ in range(reps):
        for cb in cbs:
            cb.submit()
    e1.record()
    return e0.elapsed_ms(e1)


def record(fn):
    with g4hip.Encoder() as enc:
        fn()
    return enc.cmdbuf


def bench_gemv(n, k, steps, warmup, seed=0, copies=None):
    """One step = one replay of the full cold rotation: `copies` GEMV launches,
    each on its own device copy of the weights (>= 640 MB in all), recorded
    once as a command buffer.  The timed region is `steps` replays, so it never
    shrinks to one short graph, whatever `steps` is.  A given `copies` sets the
    rotation instead (a few copies stay in the memory-side cache: warm)."""
    packed, scales, _ = syn.w4_weights(seed, n, k)
    per = w4_bytes(n, k)
    if copies is None:
        copies = max(2, int(math.ceil(COLD_BYTES / per)))
        copies = min(copies, 128) if per > 4e6 else copies
    lins = [g4hip.W4Linear(packed, scales, gemm_tiles=False) for _ in range(copies)]
    # at least 120 launches per recorded step, cycling through the copies
    order = [lins[i % copies] for i in range(max(copies, 120))]
    x_bits, _ = syn.activations(seed, 1, k)
    x = g4hip.Buffer.from_array(x_bits)
    y = g4hip.Buffer(n * 4)

    def rotation():
        for lin in order:
            lin.linear(x.ptr, g4hip.BF16, 1, y.ptr, g4hip.F32)

    full = record(rotation)
    time_cmdbufs([full], max(1, warmup))
    g4hip.sync()
    ms = time_cmdbufs([full], steps)
    launches = steps * len(order)
    for lin in lins:
        lin.free()
    return {"bytes_per_launch": per, "copies": copies, "ms": ms, "steps": steps,
            "launches": launches, "us_per_launch": ms * 1e3 / launches,
            "gbs": per * launches / (ms * 1e-3) / 1e9}


def bench_gemv_stamps(n=6144, k=1536, seed=0, replays=3):
    """Where the time of one headline GEMV goes, from inside the launch: the
    same cold rotation as bench_gemv, recorded with g4_w4_gemv_stamps (the
    row-split kernel writing 5 real-time clock stamps per wave: start, x
    staged, staging barrier passed, weights landed, store issued; the stamp
    after the weights waits for all of them).  Medians over the launches of
    the last replay, in us; times of one launch are taken from the launch's
    first wave start (t0 min over waves), the gap from the previous launch's
    last store issue."""
    packed, scales, _ = syn.w4_weights(seed, n, k)
    per = w4_bytes(n, k)
    copies = min(128, max(2, int(math.ceil(COLD_BYTES / per))))
    lins = [g4hip.W4Linear(packed, scales, gemm_tiles=False) for _ in range(copies)]
    order = [lins[i % copies] for i in range(max(copies, 120))]
    x_bits, _ = syn.activations(seed, 1, k)
    x = g4hip.Buffer.from_array(x_bits)
    y = g4hip.Buffer(n * 4)
    waves = lins[0].stamp_waves()
    st = g4hip.Buffer(len(order) * waves * 5 * 8)

    def rotation():
        for i, lin in enumerate(order):
            lin.gemv_stamps(x.ptr, g4hip.BF16, y.ptr, st.ptr + i * waves * 5 * 8)

    cb = record(rotation)
    time_cmdbufs([cb], max(1, replays - 1))
    g4hip.sync()
    ms = time_cmdbufs([cb], 1)
    s = st.download(np.uint64).reshape(len(order), waves, 5).astype(np.int64)
    for lin in lins:
        lin.free()
    tick_us = 0.01  # 100 MHz
    base = s[:, :, 0].min(axis=1)  # first wave start per launch
    rel = (s - base[:, None, None]) * tick_us
    gaps = (s[1:, :, 0].min(axis=1) - s[:-1, :, 4].max(axis=1)) * tick_us

    def med(a):
        return round(float(np.median(a)), 3)

    return {
        "launches": len(order), "waves_per_launch": waves,
        "us_per_launch_events": round(ms * 1e3 / len(order), 3),
        "span_first_start_to_last_store": med(rel[:, :, 4].max(axis=1)),
        "last_wave_start": med(rel[:, :, 0].max(axis=1)),
        "x_staged_after_wave_start": med(np.median(s[:, :, 1] - s[:, :, 0], axis=1) * tick_us),
        "barrier_passed_after_wave_start": med(np.median(s[:, :, 2] - s[:, :, 0], axis=1) * tick_us),
        "weights_landed_after_wave_start": med(np.median(s[:, :, 3] - s[:, :, 0], axis=1) * tick_us),
        "weights_landed_last": med(rel[:, :, 3].max(axis=1)),
        "store_after_weights_landed": med(np.median(s[:, :, 4] - s[:, :, 3], axis=1) * tick_us),
        "gap_to_next_launch": med(gaps),
    }


E2B_SLIDING_LAYER = [("q", 2048, 1536), ("k", 256, 1536), ("v", 256, 1536), ("o", 1536, 2048),
                     ("gate", 6144, 1536), ("up", 6144, 1536), ("down", 1536, 6144)]


# The layer's GEMVs by shared input: q/k/v and gate/up each run as one launch.
E2B_SLIDING_LAUNCHES = [("q", "k", "v"), ("o",), ("gate", "up"), ("down",)]


def bench_layer(reps=50, seed=1):
    """One E2B sliding decoder layer: its 7 GEMVs at M=1, chained through
    their real input sizes, the ones that share an input in one launch
    (g4_w4_linear_multi: 4 launches per layer); rotated over enough layer
    copies to stay cold."""
    mats = {name: (syn.w4_weights(seed + i, n, k)[:2], n, k)
            for i, (name, n, k) in enumerate(E2B_SLIDING_LAYER)}
    layer_bytes = sum(w4_bytes(n, k) for _, n, k in mats.values())
    copies = int(math.ceil(COLD_BYTES / layer_bytes))
    layers = [{name: g4hip.W4Linear(*ps, gemm_tiles=False) for name, (ps, _, _) in mats.items()}
              for _ in range(copies)]
    xs = {k: g4hip.Buffer.from_array(syn.activations(seed, 1, k)[0]) for k in (1536, 2048, 6144)}
    ys = {name: g4hip.Buffer(n * 4) for name, (_, n, _) in mats.items()}

    def f():
        for layer in layers:
            for names in E2B_SLIDING_LAUNCHES:
                k = mats[names[0]][2]
                g4hip.W4Linear.linear_multi([layer[nm] for nm in names], xs[k].ptr, g4hip.BF16,
                                            1, [ys[nm].ptr for nm in names], g4hip.F32)

    cb = record(f)
    time_cmdbufs([cb], 2)
    ms = time_cmdbufs([cb], reps)
    n_layers = reps * copies
    return {"gemvs_per_layer": 7, "launches_per_layer": len(E2B_SLIDING_LAUNCHES),
            "bytes_per_layer": layer_bytes, "copies": copies,
            "us_per_layer": ms * 1e3 / n_layers,
            "gbs": layer_bytes * n_layers / (ms * 1e-3) / 1e9}


def bench_ple(reps=200, seed=2024):
    vocab, width, rps = 262144, 8960, 4096
    t0 = time.time()
    shards = syn.ple_table(seed, vocab, width, rps, threads=16)
    t = g4hip.PleTable(vocab, width, 32, rps)
    for i, s in enumerate(shards):
        t.upload_shard(i, s)
    del shards
    log("  PLE table generated+uploaded in %.1fs" % (time.time() - t0))
    res = {}
    for n in (1, 2048):
        # distinct id sets per replay so rows are not re-served from cache
        sets = [syn.token_ids(seed + r, n, vocab) for r in range(16)]
        idb = [g4hip.Buffer.from_array(s) for s in sets]
        for dtype, name in ((g4hip.F32, "f32"), (g4hip.BF16, "bf16")):
            ob = g4hip.Buffer(n * width * (4 if dtype == g4hip.F32 else 2))

            def f():
                for b in idb:
                    t.gather_dev(b.ptr, n, ob.ptr, dtype)

            cb = record(f)
            time_cmdbufs([cb], 2)
            ms = time_cmdbufs([cb], reps // 16 if n > 1 else reps)
            calls = len(idb) * (reps // 16 if n > 1 else reps)
            per = n * (width // 2 + (width // 32) * 2 + 4) + n * width * (4 if dtype == g4hip.F32 else 2)
            res["ids%d_%s" % (n, name)] = {"us_per_call": ms * 1e3 / calls, "bytes_per_call": per,
                                          "gbs": per * calls / (ms * 1e-3) / 1e9}
    t.free()
    return res


def bench_head(reps=20, seed=12):
    vocab, k = 262144, 1536
    rng = np.random.default_rng(seed)
    E = g4hip.Buffer(vocab * k * 2)
    step = 16384
    for r0 in range(0, vocab, step):
        E.upload(syn.bf16_rne(rng.standard_normal((step, k), dtype=np.float32) * np.float32(0.03)),
                 r0 * k * 2)
    h = g4hip.Buffer.from_array(rng.standard_normal(k).astype(np.float32))
    out = g4hip.Buffer(vocab * 4)
    cb = record(lambda: g4hip.bf16_head(h.ptr, E.ptr, vocab, k, out.ptr, 1.0, 30.0))
    time_cmdbufs([cb], 2)
    ms = time_cmdbufs([cb], reps)
    per = vocab * k * 2 + k * 4 + vocab * 4
    return {"us_per_call": ms * 1e3 / reps, "bytes_per_call": per,
            "gbs": per * reps / (ms * 1e-3) / 1e9}


def bench_gemm(reps=20, seed=3, calls=8):
    """Prefill GEMMs, M=2048, BF16 x, FP32 y, x pre-pass (and K-slice sum)
    included.  As for the GEMV, one step is one replay of a recorded sequence:
    `calls` GEMMs back to back, each on its own device copy of the weights,
    so the command buffer's own launch is paid once per `calls` GEMMs (one
    call per replay measured 52.6 / 69.6 us against 49.5 / 65.6 us per call
    with 8).  `ms` is per GEMM call."""
    res = {}
    for n, k in ((6144, 1536), (1536, 6144)):
        packed, scales, _ = syn.w4_weights(seed, n, k)
        lins = [g4hip.W4Linear(packed, scales) for _ in range(calls)]
        x = g4hip.Buffer.from_array(syn.activations(seed, 2048, k)[0])
        y = g4hip.Buffer(2048 * n * 4)
        lins[0].linear(x.ptr, g4hip.BF16, 2048, y.ptr, g4hip.F32)  # sizes the workspace

        def f():
            for lin in lins:
                lin.linear(x.ptr, g4hip.BF16, 2048, y.ptr, g4hip.F32)

        cb = record(f)
        time_cmdbufs([cb], 1)
        ms = time_cmdbufs([cb], reps) / calls
        flops = 2.0 * 2048 * n * k
        tf = flops * reps / (ms * 1e-3) / 1e12
        res["M2048_N%d_K%d" % (n, k)] = {"ms": ms / reps, "tflops": tf,
                                         "frac_of_bf16_peak": tf / BF16_PEAK_TFLOPS,
                                         "calls_per_replay": calls}
        del lins
    return res


def bench_decode(prompt=512, steps=256, max_seq=1024, seed=4):
    """E2B decode: random-init Gemma-4-E2B (35 layers, vocab 262144, W4 projections,
    W4 PLE table, BF16 tied head) - a prompt of random ids, then greedy decode
    steps, each a replay of the recorded one-token step.  The prefill figure
    is the median of three prefills of the prompt; the decode runs after the
    last one."""
    import e2b
    cfg = g4hip.e2b_config(max_seq)
    m = e2b.build(cfg, seed)
    ids = syn.token_ids(seed, prompt, cfg.vocab)
    m.reset()
    m.greedy(ids, 0)
    m.decode(4, want_tokens=False)  # records the decode step
    g4hip.sync()
    a, b, c = g4hip.Event(), g4hip.Event(), g4hip.Event()
    pre = []
    for _ in range(3):  # prefill: forward + head + argmax (synchronises); the median of 3
        m.reset()
        a.record()
        first = m.greedy(ids, 0)
        b.record()
        g4hip.sync()
        pre.append(a.elapsed_ms(b))
    d = g4hip.Event()
    d.record()
    m.decode(steps, want_tokens=False)
    c.record()
    g4hip.sync()
    pre_ms, dec_ms = sorted(pre)[1], d.elapsed_ms(c)
    w4 = e2b.w4_bytes(cfg)
    head = cfg.vocab * cfg.hidden * 2
    per_token = w4 + head
    m.free()
    return {"prompt": prompt, "steps": steps, "max_seq": max_seq,
            "prefill_ms": pre_ms, "prefill_tok_s": prompt / (pre_ms * 1e-3),
            "decode_ms": dec_ms, "ms_per_token": dec_ms / steps,
            "decode_tok_s": steps / (dec_ms * 1e-3),
            "weight_bytes_per_token": per_token,
            "weight_gbs": per_token * steps / (dec_ms * 1e-3) / 1e9,
            "first_token": int(first)}


def bench_decode_node(prompt=512, steps=256, max_seq=1024, seed=4, timeout=240):
    """The same E2B decode driven from Node through the N-API bridge
    (gemma4-js_amd/node/e2b-bench.js); None when node is not installed."""
    import shutil
    import subprocess
    node = shutil.which("node")
    if node is None:
        return None
    script = os.path.join(ROOT, "gemma4-js_amd", "node", "e2b-bench.js")
    p = subprocess.run([node, script, str(prompt), str(steps), str(max_seq), str(seed)],
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=timeout)
    if p.returncode != 0:
        raise RuntimeError("node decode bench failed: " + p.stderr[-2000:])
    return json.loads(p.stdout.strip().splitlines()[-1])


def bench_decode_eager(steps, prompt=512, max_seq=1024, seed=4):
    """The E2B prompt, then `steps` one-token greedy calls launched one by one
    (each a host round trip): the decode step's kernels without graph replay."""
    import e2b
    cfg = g4hip.e2b_config(max_seq)
    m = e2b.build(cfg, seed)
    ids = syn.token_ids(seed, prompt, cfg.vocab)
    m.reset()
    tok = m.greedy(ids, 0)
    t0 = time.perf_counter()
    for s in range(steps):
        tok = m.greedy([tok], prompt + s)
    el = time.perf_counter() - t0
    m.free()
    return {"steps": steps, "host_ms_per_token": el * 1e3 / steps, "last_token": int(tok)}


def _cpu_share():
    """Host threads this process may run on (the box's CPU share), and nproc."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = min(avail, int(omp)) if omp and omp.isdigit() and int(omp) > 0 else avail
    return threads, os.cpu_count() or 1


def _time_leg(fn, budget_s):
    fn()  # warm
    calls, t0 = 0, time.perf_counter()
    while True:
        fn()
        calls += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            return calls, el


def cpu_baseline(n, k, budget_s=5.0, seed=0):
    """The reference's CPU path for the headline GEMV, restated three ways and
    timed on this host: single-threaded JavaScript under Node (the reference's
    tfjs-backend-cpu is single-threaded JS), the C oracle on one core, and the
    C oracle's chunks over every core this process may use (`value`).  Each
    leg's output is checked against the single-core C oracle."""
    import shutil
    import subprocess
    import tempfile
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import g4oracle
    packed, scales, _ = syn.w4_weights(seed, n, k)
    _, x = syn.activations(seed, 1, k)
    per = w4_bytes(n, k)
    threads, nproc = _cpu_share()
    ref = g4oracle.w4_linear(x, packed, scales)
    legs = {}

    calls, el = _time_leg(lambda: g4oracle.w4_linear(x, packed, scales), budget_s)
    legs["c_1core"] = {"threads": 1, "calls": calls, "seconds": el, "ms_per_gemv": el / calls * 1e3,
                       "gbs": per * calls / el / 1e9}
    y_mt = [None]

    def mt():
        y_mt[0] = g4oracle.w4_linear_mt(x, packed, scales, threads)

    calls, el = _time_leg(mt, budget_s)
    assert np.array_equal(y_mt[0].view(np.uint32), ref.view(np.uint32)), "all-core leg differs"
    legs["c_allcores"] = {"threads": g4oracle.omp_threads(threads), "calls": calls, "seconds": el,
                          "ms_per_gemv": el / calls * 1e3, "gbs": per * calls / el / 1e9}
    node = shutil.which("node")
    if node is not None:
        with tempfile.TemporaryDirectory() as td:
            paths = [os.path.join(td, f) for f in ("p.bin", "s.bin", "x.bin", "y.bin")]
            np.ascontiguousarray(packed).view(np.int32).tofile(paths[0])
            np.ascontiguousarray(scales).view(np.uint16).tofile(paths[1])
            np.ascontiguousarray(x, dtype=np.float32).tofile(paths[2])
            p = subprocess.run([node, os.path.join(ROOT, "oracle", "w4_linear_cpu.js"), "1",
                                str(k), str(n)] + paths + [str(budget_s)],
                               stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                               timeout=budget_s * 10 + 60)
            if p.returncode != 0:
                raise RuntimeError("JS CPU leg failed: " + p.stderr[-2000:])
            r = json.loads(p.stdout.strip().splitlines()[-1])
            y_js = np.fromfile(paths[3], dtype=np.float32).reshape(ref.shape)
        assert np.array_equal(y_js.view(np.uint32), ref.view(np.uint32)), "JS leg differs"
        legs["js_1core"] = {"threads": 1, "calls": r["calls"], "seconds": r["seconds"],
                            "ms_per_gemv": r["ms_per_call"],
                            "gbs": per * r["calls"] / r["seconds"] / 1e9,
                            "node": subprocess.run([node, "--version"], stdout=subprocess.PIPE,
                                                   text=True).stdout.strip()}
    best = legs["c_allcores"]
    return {"value": best["gbs"], "unit": "GB/s", "cores": best["threads"], "kind": "port",
            "nproc": nproc,
            "sample": "M1 K%d N%d GEMVs through the oracle's TF.js-semantics restatement of "
                      "official-quantized-linear.js:82-128 (FP32 dequant per 256-row chunk, then "
                      "48-blocked FP32 matMul), about %.0f s per leg; value = C oracle over %d "
                      "threads (%.2f ms/GEMV); legs: single-threaded JS under Node, C on one "
                      "core, C on all cores; every leg's output bit-equal to the C oracle"
                      % (k, n, budget_s, best["threads"], best["ms_per_gemv"]),
            "legs": legs}


def _node_leg(script, args, budget_s):
    """One single-threaded JS restatement under Node: (parsed result, node version)."""
    import shutil
    import subprocess
    node = shutil.which("node")
    if node is None:
        return None, None
    p = subprocess.run([node, os.path.join(ROOT, "oracle", script)] + [str(a) for a in args]
                       + [str(budget_s)], stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                       text=True, timeout=budget_s * 10 + 60)
    if p.returncode != 0:
        raise RuntimeError("JS CPU leg %s failed: %s" % (script, p.stderr[-2000:]))
    ver = subprocess.run([node, "--version"], stdout=subprocess.PIPE, text=True).stdout.strip()
    return json.loads(p.stdout.strip().splitlines()[-1]), ver


def cpu_configs(budget_s=2.0, seed=0):
    """The reference's CPU path beside the PLE gather (1 and 2048 ids), the E2B
    sliding layer's 7 GEMVs and the two M2048 prefill GEMMs, each restated
    three ways and timed on this host: single-threaded JS under Node, the C
    oracle on one core, the C oracle over every core this process may use.
    Every leg's output is checked bit-equal to the single-core C oracle.  The
    GEMMs are timed on a bounded sample of their 2048 rows (the CPU's time
    is linear in the rows); the rate is per FLOP of the rows computed."""
    import tempfile
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import g4oracle
    threads, nproc = _cpu_share()
    nthr = g4oracle.omp_threads(threads)
    out = {"threads_all": nthr, "nproc": nproc, "seconds_per_leg": budget_s}

    # config 1: PLE readRows over the whole [262144, 8960] table
    vocab, width, rps = 262144, 8960, 4096
    table = np.concatenate(syn.ple_table(2024, vocab, width, rps, threads=threads))
    ple = {}
    for n in (1, 2048):
        ids = syn.token_ids(seed + n, n, vocab)
        ref = g4oracle.ple_gather(table, vocab, width, rps, ids)
        per = n * (width // 2 + (width // 32) * 2 + 4) + n * width * 4
        legs = {}
        calls, el = _time_leg(lambda: g4oracle.ple_gather(table, vocab, width, rps, ids), budget_s)
        legs["c_1core"] = {"threads": 1, "us_per_call": el / calls * 1e6,
                           "gbs": per * calls / el / 1e9}
        got = [None]

        def mt():
            got[0] = g4oracle.ple_gather_mt(table, vocab, width, rps, ids, threads)

        calls, el = _time_leg(mt, budget_s)
        assert np.array_equal(got[0].view(np.uint32), ref.view(np.uint32)), "PLE all-core leg"
        legs["c_allcores"] = {"threads": nthr, "us_per_call": el / calls * 1e6,
                              "gbs": per * calls / el / 1e9}
        # the JS leg gets each id's packed row and scale row, already read;
        # at 2048 ids it runs the first 128 (its time is linear in the ids)
        js_ids = ids[:128]
        recs = []
        for tid in js_ids:
            po, so = g4oracle.ple_row_offsets(vocab, width, rps, int(tid) // rps, int(tid) % rps)
            recs.append(table[po:po + width // 2])
            recs.append(table[so:so + width // 16])
        with tempfile.TemporaryDirectory() as td:
            rp, op = os.path.join(td, "rows.bin"), os.path.join(td, "out.bin")
            np.concatenate(recs).tofile(rp)
            r, ver = _node_leg("ple_rows_cpu.js", [js_ids.size, width, rp, op], budget_s)
            if r is not None:
                y = np.fromfile(op, dtype=np.float32).reshape(js_ids.size, width)
                assert np.array_equal(y.view(np.uint32), ref[:js_ids.size].view(np.uint32)), \
                    "PLE JS leg"
                scale = n / js_ids.size
                legs["js_1core"] = {"threads": 1, "ids_timed": int(js_ids.size),
                                    "us_per_call": r["ms_per_call"] * 1e3 * scale,
                                    "gbs": per * r["calls"] / (r["seconds"] * scale) / 1e9,
                                    "node": ver,
                                    "note": "the reader's per-row dequant loop on rows already "
                                            "read (no File.slice)"}
        ple["ids%d_f32" % n] = legs
    del table
    out["ple_gather"] = ple

    def linear_legs(shapes, m, with_js=True):
        """C 1-core, C all-core and JS 1-core time of the GEMVs/GEMMs `shapes`
        [(n, k)] at m rows, as one sequence per call."""
        mats = [(syn.w4_weights(seed + i, n, k)[:2], n, k) for i, (n, k) in enumerate(shapes)]
        xs = {k: np.random.default_rng([seed, k]).standard_normal((m, k)).astype(np.float32)
              for _, k in shapes}
        refs = [g4oracle.w4_linear(xs[k], pk, sc) for (pk, sc), n, k in mats]
        legs = {}
        calls, el = _time_leg(lambda: [g4oracle.w4_linear(xs[k], pk, sc)
                                       for (pk, sc), n, k in mats], budget_s)
        legs["c_1core"] = {"threads": 1, "ms_per_call": el / calls * 1e3}
        got = [None]

        def mt():
            got[0] = [g4oracle.w4_linear_mt(xs[k], pk, sc, threads) for (pk, sc), n, k in mats]

        calls, el = _time_leg(mt, budget_s)
        for a, b in zip(got[0], refs):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "all-core leg"
        legs["c_allcores"] = {"threads": nthr, "ms_per_call": el / calls * 1e3}
        if with_js:
            total_ms, ver = 0.0, None
            with tempfile.TemporaryDirectory() as td:
                for i, ((pk, sc), n, k) in enumerate(mats):
                    paths = [os.path.join(td, "%s%d.bin" % (f, i)) for f in "psxy"]
                    np.ascontiguousarray(pk).view(np.int32).tofile(paths[0])
                    np.ascontiguousarray(sc).view(np.uint16).tofile(paths[1])
                    xs[k].tofile(paths[2])
                    r, ver = _node_leg("w4_linear_cpu.js", [m, k, n] + paths,
                                       budget_s / len(mats))
                    if r is None:
                        break
                    y = np.fromfile(paths[3], dtype=np.float32).reshape(m, n)
                    assert np.array_equal(y.view(np.uint32), refs[i].view(np.uint32)), "JS leg"
                    total_ms += r["ms_per_call"]
                else:
                    legs["js_1core"] = {"threads": 1, "ms_per_call": total_ms, "node": ver}
        return legs

    # config 2: one E2B sliding layer's 7 GEMVs at one row
    lb = sum(w4_bytes(n, k) for _, n, k in E2B_SLIDING_LAYER)
    legs = linear_legs([(n, k) for _, n, k in E2B_SLIDING_LAYER], 1)
    for v in legs.values():
        v["gbs"] = lb / (v["ms_per_call"] * 1e-3) / 1e9
    out["layer_e2b_sliding_7gemv"] = legs

    # config 3: the M2048 GEMMs on a sample of rows
    gemm = {}
    for n, k in ((6144, 1536), (1536, 6144)):
        rows = 16
        legs = linear_legs([(n, k)], rows)
        for v in legs.values():
            v["gflops"] = 2.0 * rows * n * k / (v["ms_per_call"] * 1e-3) / 1e9
            v["ms_per_2048_rows"] = v["ms_per_call"] * 2048 / rows
        gemm["M2048_N%d_K%d" % (n, k)] = {"rows_timed": rows, "legs": legs}
    out["gemm_prefill"] = gemm
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20,
                    help="replays of the full cold rotation of headline GEMVs")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=5.0, help="seconds per CPU leg")
    ap.add_argument("--cpu-config-seconds", type=float, default=2.0,
                    help="seconds per CPU leg beside the PLE, layer and GEMM configurations")
    ap.add_argument("--skip-decode", action="store_true",
                    help="leave out the E2B decode extra")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the E2B decode leg and print its figures")
    ap.add_argument("--decode-eager", type=int, default=0, metavar="STEPS",
                    help="only run the E2B prompt and STEPS one-token greedy calls without "
                         "graph replay (for kernel profiles), then exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py runs on one GPU: --gpus %d is not supported (the path is measured on a "
              "single MI355X; multi-GPU sharding is design-only)" % args.gpus, file=sys.stderr)
        sys.exit(2)

    g4hip.init(0)
    info = g4hip.device_info()
    log("device:", info)
    if args.decode_only:
        print(json.dumps({"decode_e2b": bench_decode(), "decode_e2b_node": bench_decode_node()}),
              flush=True)
        return
    if args.decode_eager:
        print(json.dumps({"decode_eager": bench_decode_eager(args.decode_eager)}), flush=True)
        return
    # One 64 MiB device-to-device copy of known size before anything else:
    # the reference point that scales the FETCH_SIZE / WRITE_SIZE counters
    # when this command runs under `rocprofv3 --pmc`.
    cal_a, cal_b = g4hip.Buffer(64 << 20), g4hip.Buffer(64 << 20)
    g4hip.check(g4hip.lib().g4_copy(cal_b.ptr, 0, cal_a.ptr, 0, 64 << 20))
    g4hip.sync()
    cal_a.free()
    cal_b.free()
    n, k = 6144, 1536
    log("GEMV M1 K%d N%d: %d steps (+%d warmup)" % (k, n, args.steps, args.warmup))
    g = bench_gemv(n, k, args.steps, args.warmup)
    avg_us = g["us_per_launch"]
    achieved = g["bytes_per_launch"] / (avg_us * 1e-6) / 1e9
    log("  %d launches (%d steps x %d weight copies): %.3f us/GEMV, %.1f GB/s"
        % (g["launches"], g["steps"], g["copies"], avg_us, g["gbs"]))

    extra = {}
    if not args.no_extra:
        # the same GEMV with its weights resident in the 256 MB memory-side
        # cache: 4 copies (21 MB) rotate; labelled, never the headline value
        w = bench_gemv(n, k, args.steps, args.warmup, copies=4)
        extra["gemv_m1_k1536_n6144_mall_warm"] = {
            "label": "MALL-warm: 4 weight copies (21 MB) in rotation, not cold",
            "us_per_launch": w["us_per_launch"], "gbs": w["gbs"], "launches": w["launches"]}
        log("GEMV, MALL-warm (4 copies):", extra["gemv_m1_k1536_n6144_mall_warm"])
        extra["gemv_stamps_us"] = bench_gemv_stamps(n, k)
        log("GEMV clock stamps (us):", extra["gemv_stamps_us"])
        log("E2B sliding layer, 7 GEMVs at M=1 ...")
        extra["layer_e2b_sliding_7gemv"] = bench_layer()
        log("  ", extra["layer_e2b_sliding_7gemv"])
        log("PLE gather-dequant, 1 and 2048 ids ...")
        extra["ple_gather"] = bench_ple()
        log("  ", extra["ple_gather"])
        log("BF16 LM head ...")
        extra["lm_head_262144x1536"] = bench_head()
        log("  ", extra["lm_head_262144x1536"])
        log("prefill GEMM, M2048 ...")
        extra["gemm_prefill"] = bench_gemm()
        log("  ", extra["gemm_prefill"])
        if not args.skip_decode:
            log("E2B decode: prompt 512, 256 greedy steps ...")
            extra["decode_e2b"] = bench_decode()
            log("  ", extra["decode_e2b"])
            log("E2B decode from Node (N-API bridge) ...")
            extra["decode_e2b_node"] = bench_decode_node()
            log("  ", extra["decode_e2b_node"])

    cpu = None
    if not args.no_cpu:
        log("CPU baseline (JS 1 core, C 1 core, C all cores) ...")
        cpu = cpu_baseline(n, k, args.cpu_seconds)
        log("  ", cpu)
        log("CPU legs beside the PLE gather, the E2B layer and the M2048 GEMMs ...")
        cpu["configs"] = cpu_configs(args.cpu_config_seconds)
        log("  ", cpu["configs"])

    traffic, traffic_src, kname = None, None, "w4_gemv_r16_kernel"
    tpath = os.path.join(ROOT, "profiles", "w4_gemv_m1_k1536_n6144_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            t = json.load(f)
        traffic = t["hbm_bytes_per_launch"]
        kname = t.get("kernel", kname)
        traffic_src = "profiles/w4_gemv_m1_k1536_n6144_traffic.json (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE)"
    line = {
        "metric": METRIC, "value": round(g["gbs"], 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": g["ms"] / args.steps,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (seeded int4 weights in [-7,7], bf16 scales |N|*0.02, bf16 N(0,1) x)",
        "config": {"workload": "W4A16 decode GEMV M=1 K=1536 N=6144, cold (rotating weight "
                               "copies, >= 640 MB), BF16 x, FP32 y", "M": 1, "K": k, "N": n,
                   "group": 32, "weight_copies": g["copies"],
                   "step": "one replay of the rotation: %d GEMV launches" % g["copies"],
                   "launches_timed": g["launches"], "device": info["name"],
                   "cu_count": info["cu_count"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src, "kernel": kname, "avg_launch_us": round(avg_us, 4),
                     "bytes_per_launch": g["bytes_per_launch"],
                     "timing": "HIP events on the library stream around %d launches"
                               % g["launches"]},
        "cpu_baseline": cpu,
        "decode_tok_s": round(extra["decode_e2b"]["decode_tok_s"], 1) if "decode_e2b" in extra else None,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
