"""Prefill's block images kept between q38_attn_prefill calls (the cache of
q38_kv_set_prefill_cache) on the GPU: a call sequence that prefills in
pieces, appends decode tokens into a partly converted block, truncates and
rewrites, run on two caches with the same contents -- images kept, and
images converted whole every call -- gives the same outputs bit for bit;
one output is also held against the oracle (ops.rs:1153-1172 token by
token through attention, ops.rs:868-938)."""
import numpy as np
import pytest

from parity import abs_rel

pytestmark = pytest.mark.gpu


def _kv(pkg, ctx, n):
    kv = pkg.KVCache(ctx, n_slots=2, max_pages=n // 16 + 8, max_seqs=2, max_tokens_per_seq=n)
    return kv, kv.seq_create()


def test_prefill_image_cache_equals_whole_conversion(pkg, ctx, ref, synth, margin):
    n = 2400
    layer = 3
    K = synth.normal(0x7E00, n * 1024)
    V = synth.normal(0x7E01, n * 1024)
    K2 = synth.normal(0x7E02, n * 1024)  # rewritten keys after the truncate
    V2 = synth.normal(0x7E03, n * 1024)
    Q = synth.normal(0x7E04, n * 6144)
    G = synth.normal(0x7E05, n * 6144)
    d = {name: ctx.array(x) for name, x in (("K", K), ("V", V), ("K2", K2), ("V2", V2), ("Q", Q), ("G", G))}
    steps = [("prefill", 0, 700, "K"), ("prefill", 700, 513, "K"), ("decode", 1213, 4, "K"),
             ("prefill", 1217, 300, "K"), ("truncate", 1000, 0, None), ("prefill", 1000, 400, "K2"),
             ("prefill", 1400, 1, "K2"), ("prefill", 1401, 999, "K2")]
    outs = {}
    for cached in (True, False):
        kv, seq = _kv(pkg, ctx, n)
        try:
            kv.set_prefill_cache(cached)
            got = []
            for kind, base, T, src in steps:
                if kind == "truncate":
                    kv.seq_truncate(seq, base)
                    continue
                kd, vd = (d["K"], d["V"]) if src == "K" else (d["K2"], d["V2"])
                if kind == "prefill":
                    o = ctx.empty((T, 24, 256))
                    kv.attn_prefill(layer, seq, base, T, d["Q"].offset(base * 6144), kd.offset(base * 1024),
                                    vd.offset(base * 1024), o, gate=d["G"].offset(base * 6144))
                    got.append(o.download())
                else:
                    for t in range(T):
                        p = base + t
                        o = ctx.empty((24, 256))
                        kv.attn_decode(layer, [seq], [p], d["Q"].offset(p * 6144), o, k_new=kd.offset(p * 1024),
                                       v_new=vd.offset(p * 1024), gate=d["G"].offset(p * 6144))
                        got.append(o.download())
            outs[cached] = got
        finally:
            kv.close()
    assert len(outs[True]) == len(outs[False])
    for i, (a, b) in enumerate(zip(outs[True], outs[False])):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), i
    # the last prefill (999 tokens after 1401) against the oracle: keys
    # 0..999 from K, 1000..2399 from K2
    Kr = np.concatenate([K[:1000 * 1024], K2[1000 * 1024:]]).reshape(n, 1024)
    Vr = np.concatenate([V[:1000 * 1024], V2[1000 * 1024:]]).reshape(n, 1024)
    last = outs[True][-1]
    worst = (0.0, 0.0)
    for t in (0, 1, 500, 998):
        pos = 1401 + t
        want = ref.attn_heads(Q[pos * 6144:(pos + 1) * 6144], Kr[:pos + 1], Vr[:pos + 1],
                              gate=G[pos * 6144:(pos + 1) * 6144], threads=16)
        worst = tuple(max(x, y) for x, y in zip(worst, abs_rel(last[t], want)))
    margin("out max-abs (rows of the last piece)", worst[0], 1e-3)
    margin("out rel (rows of the last piece)", worst[1], 1e-3)
