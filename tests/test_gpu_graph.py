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


def _linear_inputs(ctx, synth, seed):
    return [ctx.array(synth.normal(seed + i, m)) for i, m in enumerate((10240, 6144, 48, 48))]


def test_token_graph_interleaves_linear_core(pkg, ctx, synth):
    """A token graph in the model's layer order -- three one-token
    linear_core steps, then a full_core decode call, twice (DeltaNet layers
    0-2 and 4-6, attention layers 3 and 7) -- replayed for three tokens with
    positions advanced and new inputs written into the fixed buffers before
    each replay, against the plain calls in the same order on a twin cache
    and twin states: every output and the final states bit for bit."""
    n_tok = 3000
    kvs = [_cache(pkg, ctx, 1, n_tok, 0x7A00) for _ in range(2)]
    try:
        conv_w = ctx.array(synth.normal(0x7A10, 10240 * 4, sigma=0.5))
        dt = ctx.array(synth.normal(0x7A11, 48))
        a = ctx.array(-np.abs(synth.normal(0x7A12, 48)))
        norm = ctx.array(synth.normal(0x7A13, 128, sigma=0.1, mean=1.0))
        qn = ctx.array(synth.normal(0x7A14, 256, sigma=0.1, mean=1.0))
        kn = ctx.array(synth.normal(0x7A15, 256, sigma=0.1, mean=1.0))
        conv0 = synth.normal(0x7A16, 6 * 30720)
        delta0 = synth.normal(0x7A17, 6 * 48 * 128 * 128, sigma=0.02)
        conv = [ctx.array(conv0) for _ in range(2)]
        delta = [ctx.array(delta0) for _ in range(2)]
        lin_in = [_linear_inputs(ctx, synth, 0x7A20 + 8 * i) for i in range(6)]
        att_in = {L: [ctx.array(synth.normal(0x7A60 + L, 12288)), ctx.array(synth.normal(0x7A70 + L, 1024)),
                      ctx.array(synth.normal(0x7A80 + L, 1024))] for L in (3, 7)}
        outs = [{k: ctx.empty((6144,)) for k in range(8)} for _ in range(2)]

        kv_g, seqs_g, _ = kvs[0]
        pos0 = 2990
        graph = kv_g.decode_graph(seqs_g, [pos0])
        for layer in range(8):
            if layer in (3, 7):
                q, key, val = att_in[layer]
                graph.add_decode({"layer": layer, "q": q, "k_new": key, "v_new": val, "q_norm": qn, "k_norm": kn,
                                  "out": outs[0][layer]})
            else:
                r = layer if layer < 3 else layer - 1
                graph.add_linear_core(1, conv_w, dt, a, norm, conv[0].offset(r * 30720),
                                      delta[0].offset(r * 48 * 128 * 128), *lin_in[r], outs[0][layer])
        graph.end()
        kv_p, seqs_p, _ = kvs[1]
        with graph:
            for t in range(3):
                pos = pos0 + t
                # this token's inputs, written into the buffers both paths read
                for r in range(6):
                    for i, buf in enumerate(lin_in[r]):
                        buf.upload(synth.normal(0x7B00 + 100 * t + 8 * r + i, buf.shape[0]))
                for L in (3, 7):
                    for i, buf in enumerate(att_in[L]):
                        buf.upload(synth.normal(0x7C00 + 100 * t + 4 * L + i, buf.shape[0]))
                graph.set_positions([pos])
                graph.launch()
                for layer in range(8):
                    if layer in (3, 7):
                        q, key, val = att_in[layer]
                        kv_p.full_core(layer, seqs_p, [pos], qn, kn, q, key, val, outs[1][layer])
                    else:
                        r = layer if layer < 3 else layer - 1
                        ctx.linear_core(1, 1, conv_w, dt, a, norm, conv[1].offset(r * 30720),
                                        delta[1].offset(r * 48 * 128 * 128), *lin_in[r], outs[1][layer])
                for layer in range(8):
                    got, want = outs[0][layer].download(), outs[1][layer].download()
                    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (t, layer)
        assert np.array_equal(conv[0].download(), conv[1].download())
        assert np.array_equal(delta[0].download().view(np.uint32), delta[1].download().view(np.uint32))
    finally:
        for kv, _, _ in kvs:
            kv.close()


def test_token_graph_with_a_captured_child_graph(pkg, ctx, synth):
    """The caller's own work as a child step: a graph captured from the
    context's stream (a device copy of layer 3's output into layer 7's query
    buffer, a data dependency) sits between two decode calls; the replay
    equals the plain sequence decode, copy, decode bit for bit."""
    import ctypes
    import os
    hip = ctypes.CDLL(os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib", "libamdhip64.so"))
    hip.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    hip.hipGraphDestroy.argtypes = [ctypes.c_void_p]
    n_tok = 2000
    kv, seqs, _ = _cache(pkg, ctx, 1, n_tok, 0x7D00)
    try:
        q3 = ctx.array(synth.normal(0x7D10, 6144))
        q7 = ctx.empty((24, 256))
        o3, o7 = ctx.empty((24, 256)), ctx.empty((24, 256))
        stream = ctx.stream()
        ctx.sync()
        child = ctypes.c_void_p()
        assert hip.hipStreamBeginCapture(stream, 2) == 0  # relaxed capture mode
        ctx.copy(q7, o3, 6144 * 4)
        assert hip.hipStreamEndCapture(stream, ctypes.byref(child)) == 0
        graph = kv.decode_graph(seqs, [1500])
        graph.add_decode({"layer": 3, "q": q3, "out": o3})
        graph.add_graph(child.value)
        graph.add_decode({"layer": 7, "q": q7, "out": o7})
        graph.end()
        hip.hipGraphDestroy(child)
        with graph:
            graph.set_positions([1999])
            graph.launch()
            got3, got7 = o3.download(), o7.download()
        ctx.sync()
        o3.zero()
        q7.zero()
        kv.attn_decode(3, seqs, [1999], q3, o3)
        ctx.copy(q7, o3, 6144 * 4)
        kv.attn_decode(7, seqs, [1999], q7, o7)
        assert np.array_equal(got3, o3.download())
        assert np.array_equal(got7, o7.download())
        assert np.abs(got7).max() > 0
    finally:
        kv.close()
