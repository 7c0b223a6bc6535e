"""Random-init models of the Gemma-4-E2B shapes on the device engine.

The weights follow the synthetic distributions of the benchmark
configurations: W4 q uniform in [-7, 7] with bf16 scales |N(0,1)| * 0.02, the
PLE table's W4 rows with scales |N(0,1)| * 0.05, a BF16 N(0,1) * 0.03 tied
embedding, norm weights uniform in [0.9, 1.1] and layer scalars 1.  Every
large tensor is generated on the device (g4_fill_random), so a full model
(~2.2 GB: 1.0 GB of W4 projections, 0.8 GB embedding, 1.3 GB PLE table) is
ready in seconds.
"""
import numpy as np

import g4hip


def build(cfg, seed=0, ple_rows_per_shard=4096):
    """Gemma model + the handles it borrows, for a g4hip.GemmaConfig."""
    m = g4hip.Gemma(cfg)
    rng = np.random.default_rng([seed, 0xE2B])
    H, P, NL, V = cfg.hidden, cfg.ple_dim, cfg.layers, cfg.vocab
    s = [seed * 1000]

    def nxt():
        s[0] += 1
        return s[0]

    def lin(n, k):
        return g4hip.w4_random(n, k, nxt(), 0.02)

    def norm(n):
        return rng.uniform(0.9, 1.1, n).astype(np.float32)

    E = g4hip.Buffer(V * H * 2)
    g4hip.fill_random(E, V * H, g4hip.RAND_BF16_NORMAL, nxt(), 0.03)
    m.set_embedding(E)
    ple = g4hip.PleTable(V, NL * P, 32, ple_rows_per_shard)
    width = NL * P
    packed_row, scale_row = width // 2, (width // 32) * 2
    stage = None
    for shard in range(ple.num_shards):
        nbytes = ple.shard_bytes(shard)
        rows = nbytes // (packed_row + scale_row)
        if stage is None or stage.nbytes < nbytes:
            stage = g4hip.Buffer(nbytes)
        g4hip.fill_random(stage, rows * packed_row, g4hip.RAND_PLE_PACKED, nxt())
        g4hip.fill_random(stage.at(rows * packed_row), rows * (width // 32),
                          g4hip.RAND_BF16_ABS_NORMAL, nxt(), 0.05)
        g4hip.check(g4hip.lib().g4_ple_upload_shard_dev(ple.h, shard, stage.ptr, nbytes))
    g4hip.sync()
    stage.free()
    m.set_ple(ple)
    m.set_linear(-1, "top", lin(NL * P, H))
    m.set_norm(-1, "ple_projection", norm(P))
    m.set_norm(-1, "final", norm(H))
    for i in range(NL):
        hd, inter, shared = cfg.head_dim[i], cfg.intermediate[i], cfg.kv_source[i] >= 0
        m.set_linear(i, "q", lin(cfg.heads * hd, H))
        if not shared:
            m.set_linear(i, "k", lin(hd, H))
            m.set_linear(i, "v", lin(hd, H))
        m.set_linear(i, "o", lin(H, cfg.heads * hd))
        m.set_linear(i, "gate", lin(inter, H))
        m.set_linear(i, "up", lin(inter, H))
        m.set_linear(i, "down", lin(H, inter))
        m.set_linear(i, "ple_gate", lin(P, H))
        m.set_linear(i, "ple_proj", lin(H, P))
        for name in ("input", "post_attn", "pre_ffw", "post_ffw", "post_ple"):
            m.set_norm(i, name, norm(H))
        m.set_norm(i, "q", norm(hd))
        if not shared:
            m.set_norm(i, "k", norm(hd))
        m.set_layer_scalar(i, 1.0)
    return m


def w4_bytes(cfg):
    """Device bytes of the W4 projections (packed + scales) read per token."""
    H, P, NL = cfg.hidden, cfg.ple_dim, cfg.layers

    def b(n, k):
        return n * k // 2 + n * (k // 32) * 2

    total = b(NL * P, H)
    for i in range(NL):
        hd, inter = cfg.head_dim[i], cfg.intermediate[i]
        qd = cfg.heads * hd
        total += b(qd, H) + b(H, qd) + 2 * b(inter, H) + b(H, inter) + b(P, H) + b(H, P)
        if cfg.kv_source[i] < 0:
            total += 2 * b(hd, H)
    return total
