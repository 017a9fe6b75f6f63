"""The replayed decode graph (q38_decode_graph_*) on the GPU.

A graph replays the same kernels with the same arguments as the plain calls
(q38_attn_decode / q38_full_core, full_core ops.rs:813-940), so its outputs
must equal theirs bit for bit; the plain calls are held against the oracle
by tests/test_gpu_attn.py, and one graph output here is checked against the
oracle directly.  Positions move between replays across split-count changes
(the split kernel's grid is rewritten), one split, and a page boundary.
"""
import numpy as np
import pytest

from parity import check_attn

pytestmark = pytest.mark.gpu

LAYERS = (3, 7, 11)
POSITIONS = (4000, 4001, 300, 15, 8992)


def _cache(pkg, ctx, n_seq, n_tokens, seed):
    """A cache with n_seq sequences of n_tokens cached tokens in LAYERS."""
    kv = pkg.KVCache(ctx, n_slots=3, max_pages=n_seq * (n_tokens // 16 + 8), max_seqs=n_seq,
                     max_tokens_per_seq=n_tokens + 64)
    seqs = [kv.seq_create() for _ in range(n_seq)]
    d_k, d_v = ctx.empty((n_tokens, 1024)), ctx.empty((n_tokens, 1024))
    rows = {}
    for li, layer in enumerate(LAYERS):
        for b, s in enumerate(seqs):
            ctx.fill_normal(d_k, n_tokens * 1024, seed + 16 * li + 2 * b)
            ctx.fill_normal(d_v, n_tokens * 1024, seed + 16 * li + 2 * b + 1)
            kv.write(layer, s, 0, n_tokens, d_k, d_v)
            rows[(layer, b)] = (d_k.download(), d_v.download())
    return kv, seqs, rows


def test_graph_attn_decode_matches_plain_calls(pkg, ctx, ref, synth, margin):
    """Batch 1, three layers per replay, the attn_decode form with appends and
    gates.  Positions 4000 -> 4001 (same splits) -> 300 (fewer, shorter
    splits) -> 15 (one split: no merge work) -> 8992 (the first row of a
    page not yet reserved), each replay against the plain calls at the same
    positions."""
    n_tok = 8992
    kv, seqs, rows = _cache(pkg, ctx, 1, n_tok, 0x7100)
    try:
        q = {L: ctx.array(synth.normal(0x7200 + L, 6144)) for L in LAYERS}
        g = {L: ctx.array(synth.normal(0x7300 + L, 6144)) for L in LAYERS}
        kn = {L: ctx.array(synth.normal(0x7400 + L, 1024)) for L in LAYERS}
        vn = {L: ctx.array(synth.normal(0x7500 + L, 1024)) for L in LAYERS}
        out_g = {L: ctx.empty((24, 256)) for L in LAYERS}
        out_p = {L: ctx.empty((24, 256)) for L in LAYERS}
        calls = [{"layer": L, "q": q[L], "k_new": kn[L], "v_new": vn[L], "gate": g[L], "out": out_g[L]}
                 for L in LAYERS]
        with kv.decode_graph(seqs, [4000], calls) as graph:
            for pos in POSITIONS:
                graph.set_positions([pos])
                graph.launch()
                for L in LAYERS:
                    kv.attn_decode(L, seqs, [pos], q[L], out_p[L], k_new=kn[L], v_new=vn[L], gate=g[L])
                for L in LAYERS:
                    got, want = out_g[L].download(), out_p[L].download()
                    assert np.array_equal(got, want), (pos, L, float(np.max(np.abs(got - want))))
            # the last replay against the oracle: the cached rows with every
            # appended position holding the appended row
            L = LAYERS[1]
            K, V = rows[(L, 0)]
            K, V = np.concatenate([K, K[:1]]), np.concatenate([V, V[:1]])
            for p in POSITIONS:
                K[p], V[p] = kn[L].download(), vn[L].download()
            want = ref.attn_heads(q[L].download(), K, V, gate=g[L].download(), threads=16)
            check_attn(margin, out_g[L].download(), want)
    finally:
        kv.close()


def test_graph_full_core_batched_tokens(pkg, ctx, synth):
    """Two sequences of different lengths (the split kernel that reads page
    ids from the table), the full_core form (q|gate rows, raw key and value,
    norm weights), three consecutive tokens replayed with positions advanced
    each time, against plain q38_full_core calls."""
    n_tok = 5000
    kv, seqs, _ = _cache(pkg, ctx, 2, n_tok, 0x7600)
    try:
        qn = ctx.array(synth.normal(0x7700, 256, sigma=0.1, mean=1.0))
        kn_w = ctx.array(synth.normal(0x7701, 256, sigma=0.1, mean=1.0))
        qg = {L: ctx.array(synth.normal(0x7710 + L, 2 * 12288)) for L in LAYERS}
        key = {L: ctx.array(synth.normal(0x7720 + L, 2 * 1024)) for L in LAYERS}
        val = {L: ctx.array(synth.normal(0x7730 + L, 2 * 1024)) for L in LAYERS}
        out_g = {L: ctx.empty((2, 24, 256)) for L in LAYERS}
        out_p = {L: ctx.empty((2, 24, 256)) for L in LAYERS}
        calls = [{"layer": L, "q": qg[L], "k_new": key[L], "v_new": val[L], "q_norm": qn, "k_norm": kn_w,
                  "out": out_g[L]} for L in LAYERS]
        pos = [4990, 1200]
        with kv.decode_graph(seqs, pos, calls) as graph:
            for t in range(3):
                p = [pos[0] + t, pos[1] + t]
                graph.set_positions(p)
                graph.launch()
                for L in LAYERS:
                    kv.full_core(L, seqs, p, qn, kn_w, qg[L], key[L], val[L], out_p[L])
                for L in LAYERS:
                    assert np.array_equal(out_g[L].download(), out_p[L].download()), (t, L)
    finally:
        kv.close()


def test_graph_rejects_bad_positions_and_keeps_working(pkg, ctx, synth):
    """A position past the context limit fails in set_positions with nothing
    changed; the graph then replays at valid positions as before.  Calls on
    a DeltaNet layer or with a half-given append are refused at creation."""
    from q38amd import Q38Error
    n_tok = 2000
    kv, seqs, _ = _cache(pkg, ctx, 1, n_tok, 0x7800)
    try:
        L = LAYERS[0]
        q = ctx.array(synth.normal(0x7900, 6144))
        out_g, out_p = ctx.empty((24, 256)), ctx.empty((24, 256))
        with pytest.raises(Q38Error):
            kv.decode_graph(seqs, [100], [{"layer": 4, "q": q, "out": out_g}])
        with pytest.raises(Q38Error):
            kv.decode_graph(seqs, [100], [{"layer": L, "q": q, "k_new": q, "out": out_g}])
        free_before = kv.free_pages()
        with kv.decode_graph(seqs, [1500], [{"layer": L, "q": q, "out": out_g}]) as graph:
            with pytest.raises(Q38Error):
                graph.set_positions([n_tok + 64])
            with pytest.raises(Q38Error):
                graph.set_positions([-1])
            assert kv.free_pages() == free_before
            graph.set_positions([1999])
            graph.launch()
            kv.attn_decode(L, seqs, [1999], q, out_p)
            assert np.array_equal(out_g.download(), out_p.download())
    finally:
        kv.close()
