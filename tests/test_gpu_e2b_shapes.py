"""The decode kernels that the Gemma-4-E2B shapes select, against the oracle.

A 4-layer model at the E2B widths: hidden 1536, 8 query heads, PLE 256, a
sliding layer (head dim 256, MLP 6144), a global layer (head dim 512, MLP
6144, RoPE 1e6 / 0.25) and two later layers with MLP 12288 that reuse those
layers' KV caches, as layers 15-34 of E2B do (gemma4-webgpu.js:65-77).  The
vocabulary is 8192 rows.  At these widths the one-token step runs the fused
GEMVs of the 1536-wide input (48 groups per row), the split down projection
over 4 and 8 input slices, and the one-launch decode attention at head dims
256 and 512, whose key splits per head are 16 (sliding, 512-key window) and
24 (global, max_seq 576) or 32 (global, max_seq 1024).

A 520-token prompt (past the 512-key window; max_seq 576) or a 1000-token
prompt (max_seq 1024, the global layers' longest key range) is prefilled,
then 24 tokens are decoded by replaying the recorded step (and, separately,
by one-token calls).  At the prompt and after every step the final-norm hidden state and
the logits must be within relative L2 1e-3 of the float64 oracle model fed
the same tokens (layer_oracle.DequantModel, gemma4-webgpu.js:215-481), and
each chosen token must be the oracle's top-1 unless its top two logits are
within 1e-3."""
import copy

import numpy as np
import pytest

import layer_oracle as lo
import synthetic as syn

pytestmark = pytest.mark.gpu

H, HEADS, P, V, WINDOW = 1536, 8, 256, 8192, 512
LAYERS = [
    dict(head_dim=256, full=0, kv_source=-1, intermediate=6144, rope_base=1e4, rope_prop=1.0),
    dict(head_dim=512, full=1, kv_source=-1, intermediate=6144, rope_base=1e6, rope_prop=0.25),
    dict(head_dim=256, full=0, kv_source=0, intermediate=12288, rope_base=1e4, rope_prop=1.0),
    dict(head_dim=512, full=1, kv_source=1, intermediate=12288, rope_base=1e6, rope_prop=0.25),
]
# A second sliding layer with its own cache after the global one: in the
# prefill it takes its q/k/v input as the previous layer's prepared x', so q,
# k and v run as one GEMM launch split over K (3 slices at head dim 256; the
# global layer above splits in 2), whose slices the q/k/v norms add.
LAYERS_OWN3 = LAYERS[:2] + [
    dict(head_dim=256, full=0, kv_source=-1, intermediate=6144, rope_base=1e4, rope_prop=1.0)
] + LAYERS[2:]
STEPS, RPS = 24, 4096
CASES = [(520, 576), (1000, 1024)]  # (prompt, max_seq)


def rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return np.linalg.norm(a - b) / np.linalg.norm(b)


def near_tie(logits, tok, tol=1e-3):
    return float(np.max(logits) - logits[tok]) <= tol


def config(g4, max_seq, specs=LAYERS):
    c = g4.GemmaConfig()
    c.hidden, c.heads, c.ple_dim, c.vocab = H, HEADS, P, V
    c.layers, c.max_seq, c.window, c.eps, c.softcap = len(specs), max_seq, WINDOW, 1e-6, 30.0
    for i, L in enumerate(specs):
        c.head_dim[i], c.intermediate[i], c.full[i] = L["head_dim"], L["intermediate"], L["full"]
        c.kv_source[i], c.rope_base[i], c.rope_prop[i] = L["kv_source"], L["rope_base"], L["rope_prop"]
    return c


def spread_gate(packed, scales, q):
    """The same weight with its group scales multiplied by 2^(-24 r / (N - 1))
    on output row r, so that the rows' largest scales spread far beyond 2^12
    and the prefill GEMM shifts each output row on its own."""
    n = scales.shape[0]
    f = np.exp2(-24.0 * np.arange(n) / (n - 1)).astype(np.float32)[:, None]
    return packed, syn.bf16_rne(syn.bf16_to_f32(scales).reshape(scales.shape) * f)


def build_model(g4, full_range=False, specs=LAYERS):
    """A model of the layers `specs` at the E2B widths and its float64 oracle.  With
    full_range every W4 weight and the PLE table draw q over all of [-8, 7]
    (W4 nibble 0 and PLE nibble 8 in every group), and each gate weight has
    row-spread scales (spread_gate), so the prefill's gate/up GEMM (one
    launch, gelu(gate) * up in its epilogue) runs with per-row shifts."""
    NL = len(specs)
    rng = np.random.default_rng(1536)
    E = syn.bf16_rne(rng.standard_normal((V, H), dtype=np.float32) * np.float32(0.03))
    shards = [syn.ple_shard(17, s, RPS, NL * P, full_range=full_range) for s in range(V // RPS)]
    table = np.concatenate(shards)
    seed = [100]

    def w(n, k, gate=False):
        seed[0] += 1
        pw = syn.w4_weights(seed[0], n, k, full_range=full_range)
        return spread_gate(*pw) if gate and full_range else pw[:2]

    top = w(NL * P, H)
    layers = []
    for L in specs:
        hd, inter, shared = L["head_dim"], L["intermediate"], L["kv_source"] >= 0
        shapes = dict(q=(HEADS * hd, H), o=(H, HEADS * hd), gate=(inter, H), up=(inter, H),
                      down=(H, inter), ple_gate=(P, H), ple_proj=(H, P))
        if not shared:
            shapes.update(k=(hd, H), v=(hd, H))
        lin = {name: w(n, k, name == "gate") for name, (n, k) in shapes.items()}
        norm = {n: rng.uniform(0.9, 1.1, H).astype(np.float32)
                for n in ("input", "post_attn", "pre_ffw", "post_ffw", "post_ple")}
        norm["q"] = rng.uniform(0.9, 1.1, hd).astype(np.float32)
        if not shared:
            norm["k"] = rng.uniform(0.9, 1.1, hd).astype(np.float32)
        layers.append(dict(L, linear=lin, norm=norm, skip=float(rng.uniform(0.9, 1.1))))
    ple_norm = rng.uniform(0.9, 1.1, P).astype(np.float32)
    final_norm = rng.uniform(0.9, 1.1, H).astype(np.float32)

    def ple_rows(ids):
        import g4oracle
        return g4oracle.ple_gather(table, V, NL * P, RPS, ids)

    ref = lo.DequantModel(H, HEADS, P, V, layers, E, ple_rows, top, ple_norm, final_norm,
                          window=WINDOW)
    prefills = {}

    def prefill(prompt):
        """The oracle after the prompt (computed once per prompt length): the
        ids, the final-norm hidden state, and a function restoring the state."""
        if prompt not in prefills:
            ref.reset()
            ids = syn.token_ids(21, prompt, V)
            h0 = ref.forward(ids, 0)
            prefills[prompt] = (ids, h0, copy.deepcopy((ref.k, ref.v, ref.length)))
        ids, h0, snap = prefills[prompt]

        def restore():
            ref.k, ref.v, ref.length = copy.deepcopy(snap)

        return ids, h0, restore

    # device copies of every weight, shared by the engines of both tests
    E_dev = g4.Buffer.from_array(E)
    t = g4.PleTable(V, NL * P, 32, RPS)
    for s, data in enumerate(shards):
        t.upload_shard(s, data)
    w_top = g4.W4Linear(*top)
    w_layers = [{name: g4.W4Linear(*pw) for name, pw in L["linear"].items()} for L in layers]

    def make_engine(max_seq):
        m = g4.Gemma(config(g4, max_seq, specs))
        m.set_embedding(E_dev)
        m.set_ple(t)
        m.set_linear(-1, "top", w_top)
        m.set_norm(-1, "ple_projection", ple_norm)
        m.set_norm(-1, "final", final_norm)
        for i, L in enumerate(layers):
            for name, lin in w_layers[i].items():
                m.set_linear(i, name, lin)
            for name, v in L["norm"].items():
                m.set_norm(i, name, v)
            m.set_layer_scalar(i, L["skip"])
        return m

    return dict(ref=ref, prefill=prefill, make=make_engine)


@pytest.fixture(scope="module")
def mid(g4):
    return build_model(g4)


@pytest.fixture(scope="module")
def mid_full(g4):
    return build_model(g4, full_range=True)


@pytest.fixture(scope="module")
def mid_own3(g4):
    return build_model(g4, specs=LAYERS_OWN3)


@pytest.mark.parametrize("mode", ["graph", "eager"])
@pytest.mark.parametrize("prompt,max_seq", CASES)
def test_e2b_widths_prefill_past_window_then_decode_match_oracle(g4, mid, prompt, max_seq, mode):
    run_against_oracle(g4, mid, prompt, max_seq, mode)


def test_e2b_widths_split_qkv_prefill_then_decode_match_oracle(g4, mid_own3):
    # two layers with their own cache after the first: the prefill's one
    # K-split q/k/v launch per layer (2 and 3 slices), then recorded steps
    run_against_oracle(g4, mid_own3, 520, 576, "graph")


def test_e2b_widths_full_nibble_range_match_oracle(g4, mid_full):
    # every weight and the PLE table over the formats' whole q range, gate
    # weights with row-spread scales: prefill (the packed-weight gate/up GEMM
    # with per-row shifts) and recorded decode steps against the oracle
    run_against_oracle(g4, mid_full, 520, 576, "graph")


def run_against_oracle(g4, mid, prompt, max_seq, mode):
    ref = mid["ref"]
    ids, h0, restore = mid["prefill"](prompt)
    m = mid["make"](max_seq)
    lg = g4.Buffer(V * 4)
    hb = g4.Buffer(H * 4)
    tok = m.greedy(ids, 0, lg)
    m.last_hidden(hb)
    want_lg = ref.logits(h0)
    assert rel(hb.download(np.float32), h0) < 1e-3
    assert rel(lg.download(np.float32), want_lg) < 1e-3
    assert tok == int(np.argmax(want_lg)) or near_tie(want_lg, tok)
    restore()
    prev, pos = tok, prompt
    worst = 0.0
    for s in range(STEPS):
        if mode == "graph":
            t = int(m.decode(1)[0])  # replays the step recorded for max_seq keys
            m.last_hidden(hb)
            m.logits(hb, lg)
        else:
            t = m.greedy([prev], pos, lg)
            m.last_hidden(hb)
        got_h, got_lg = hb.download(np.float32), lg.download(np.float32)
        want_h = ref.forward([prev], pos)
        want_lg = ref.logits(want_h)
        eh, el = rel(got_h, want_h), rel(got_lg, want_lg)
        worst = max(worst, eh, el)
        assert eh < 1e-3 and el < 1e-3, (mode, s, pos, eh, el)
        assert t == int(np.argmax(got_lg)), (mode, s, t)  # the step's own argmax
        assert t == int(np.argmax(want_lg)) or near_tie(want_lg, t), (mode, s, t)
        prev, pos = t, pos + 1
    assert m.cache_length() == prompt + STEPS
    print("%s, prompt %d: worst relative L2 over %d steps %.2e" % (mode, prompt, STEPS, worst))


def test_e2b_widths_diagnostic_read_outs_match_oracle(g4, mid):
    # g4_gemma_forward_diag on 6 prompt rows: the top-level hidden and PLE
    # rows, every layer's output and all 23 encodeLayer stages of layer 1
    # (gemma4-webgpu.js:224-309, 311-397) against the oracle's read-outs,
    # each within relative L2 1e-3; the final-norm row equals the plain
    # forward's to 1e-5
    ref = mid["ref"]
    n, NL = 6, len(LAYERS)
    ids = syn.token_ids(33, n, V)
    ref.reset()
    probes = {}
    want_last = ref.forward(ids, 0, probes=probes)
    m = mid["make"](576)
    off = m.diag_stages(1, n)
    assert len(off) == g4.STAGES + 1
    top, tple = g4.Buffer(n * H * 4), g4.Buffer(n * NL * P * 4)
    lay, st, last = g4.Buffer(NL * n * H * 4), g4.Buffer(off[-1] * 4), g4.Buffer(H * 4)
    m.forward_diag(ids, 0, last, top, tple, lay, 1, st)
    assert m.cache_length() == n
    assert rel(top.download(np.float32), probes["top hidden"]) < 1e-5
    assert rel(tple.download(np.float32), probes["top PLE"]) < 1e-3
    layers = lay.download(np.float32).reshape(NL, n, H)
    for i in range(NL):
        assert rel(layers[i], probes["layer %d" % i]) < 1e-3, i
    stages = st.download(np.float32)
    for k, name in enumerate(g4.STAGE_NAMES):
        assert off[k + 1] - off[k] == np.asarray(probes["stages"][name]).size, name
        got = stages[off[k]:off[k + 1]]
        assert rel(got, probes["stages"][name]) < 1e-3, name
    assert rel(last.download(np.float32), want_last) < 1e-3
    m2 = mid["make"](576)
    last2 = g4.Buffer(H * 4)
    m2.forward(ids, 0, last2)
    assert rel(last.download(np.float32), last2.download(np.float32)) < 1e-5
    # a layer without its own KV has empty k/v stages
    off3 = m.diag_stages(2, n)
    for k in range(3, 7):
        assert off3[k + 1] == off3[k]
    with pytest.raises(g4.G4Error):
        m.forward_diag(ids, n, None, None, None, None, NL, st)  # stage layer out of range
    m.free()
    m2.free()
