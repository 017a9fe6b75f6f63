"""q38_full_core_noalloc -- full_core with its split-K partials in the fixed
per-device scratch array instead of the context's growable workspace --
against q38_full_core on the same inputs, through the C ABI:

  - two calls in a row, the second with a smaller input (three sequences of
    9000-31000 cached tokens on 128-token splits, 471 splits; then one
    sequence of 9001 tokens on the automatic split): outputs bit-identical
    to q38_full_core's, the second also against the restatement;
  - a call whose partials exceed the scratch (939 splits) fails with -1 and
    leaves the pool and every sequence as they were.
"""
import numpy as np
import pytest
from parity import check_attn, decode_split

pytestmark = pytest.mark.gpu

SPLIT_PARTIAL_BYTES = 24 * (256 + 2) * 4


def _inputs(synth, seed, n):
    return (synth.normal(seed, n * 12288), synth.normal(seed + 1, n * 1024), synth.normal(seed + 2, n * 1024))


def test_noalloc_matches_full_core_two_calls(pkg, ctx, ref, margin, synth):
    layer = 7  # slot 1
    lengths = [20000, 9000, 31000]
    ctx_len = 32768
    pool = sum(p // 16 + 2 for p in lengths) + 16
    kv = pkg.KVCache(ctx, n_slots=2, max_pages=pool, max_seqs=3, max_tokens_per_seq=ctx_len)
    try:
        seqs = [kv.seq_create() for _ in lengths]
        rows_k, rows_v = ctx.empty((max(lengths), 1024)), ctx.empty((max(lengths), 1024))
        host_b = None
        for i, (s, P) in enumerate(zip(seqs, lengths)):
            ctx.fill_normal(rows_k, P * 1024, 0xD000 + 2 * i)
            ctx.fill_normal(rows_v, P * 1024, 0xD001 + 2 * i)
            kv.write(layer, s, 0, P, rows_k, rows_v)
            if i == 1:
                host_b = (rows_k.download(P), rows_v.download(P))
        rows_k.free()
        rows_v.free()
        qn = synth.normal(0xD100, 256, sigma=0.2, mean=1.0)
        kn = synth.normal(0xD101, 256, sigma=0.2, mean=1.0)
        d_qn, d_kn = ctx.array(qn), ctx.array(kn)

        # call 1: three sequences, 128-token splits (471 splits, 11.7 MB of partials)
        positions = list(lengths)
        assert sum((p + 128) // 128 for p in positions) * SPLIT_PARTIAL_BYTES <= pkg.NOALLOC_SCRATCH_BYTES
        qg, key, val = (ctx.array(x) for x in _inputs(synth, 0xD200, 3))
        out_a, out_b = ctx.empty((3, 24, 256)), ctx.empty((3, 24, 256))
        with decode_split(ctx, 128):
            kv.full_core(layer, seqs, positions, d_qn, d_kn, qg, key, val, out_a)
            kv.full_core_noalloc(layer, seqs, positions, d_qn, d_kn, qg, key, val, out_b)
        assert np.array_equal(out_a.download(), out_b.download())

        # call 2: one sequence, automatic split (a smaller input)
        b = seqs[1]
        qg2, key2, val2 = _inputs(synth, 0xD300, 1)
        d_qg2, d_key2, d_val2 = ctx.array(qg2), ctx.array(key2), ctx.array(val2)
        out_c, out_d = ctx.empty((24, 256)), ctx.empty((24, 256))
        out_d.upload(np.full((24, 256), np.nan, np.float32))
        kv.full_core(layer, [b], [9001], d_qn, d_kn, d_qg2, d_key2, d_val2, out_c)
        kv.full_core_noalloc(layer, [b], [9001], d_qn, d_kn, d_qg2, d_key2, d_val2, out_d)
        got = out_d.download()
        assert np.array_equal(out_c.download(), got)
        # and the restatement: b's cache as the device holds it (the row
        # appended at 9000 by call 1 included), then full_core at 9001
        r_k, r_v = ctx.empty((9001, 1024)), ctx.empty((9001, 1024))
        kv.read(layer, b, 0, 9001, r_k, r_v)
        kc = np.zeros(2 * ctx_len * 1024, np.float32)
        vc = np.zeros(2 * ctx_len * 1024, np.float32)
        kc[ctx_len * 1024: (ctx_len + 9001) * 1024] = r_k.download().reshape(-1)
        vc[ctx_len * 1024: (ctx_len + 9001) * 1024] = r_v.download().reshape(-1)
        assert np.array_equal(kc[ctx_len * 1024: (ctx_len + 9000) * 1024], host_b[0].reshape(-1))
        want, _ = ref.full_core(qn, kn, qg2, key2, val2, kc, vc, ctx_len, 9001, layer, threads=16)
        check_attn(margin, got, want)

        # partials past the scratch: 64-token splits, 939 splits
        before = (kv.free_pages(), [kv.seq_capacity(s) for s in seqs])
        positions = [20001, 9002, 31001]
        assert sum((p + 64) // 64 for p in positions) * SPLIT_PARTIAL_BYTES > pkg.NOALLOC_SCRATCH_BYTES
        with decode_split(ctx, 64):
            with pytest.raises(pkg.Q38Error, match="fixed scratch"):
                kv.full_core_noalloc(layer, seqs, positions, d_qn, d_kn, qg, key, val, out_b)
        assert (kv.free_pages(), [kv.seq_capacity(s) for s in seqs]) == before
    finally:
        kv.close()
