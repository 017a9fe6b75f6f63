"""Full-attention decode and prefill on the GPU against the CPU restatement
of full_core (src/model/ops.rs:813-940).  Tolerances (tests/parity.py):
max-abs <= 1e-3 and max-abs <= 1e-3 * max|want|."""
import numpy as np
import pytest
from parity import TOL_ABS, TOL_REL, abs_rel, check_attn, decode_split

pytestmark = pytest.mark.gpu


def _decode_one(pkg, ctx, P, seed, gate=True, layer=3, split=None):
    from q38amd import synth
    kv = pkg.KVCache(ctx, n_slots=17, max_pages=(P + 15) // 16 + 4, max_seqs=2, max_tokens_per_seq=P + 64)
    try:
        seq = kv.seq_create()
        K = synth.normal(seed + 1, P * 1024)
        V = synth.normal(seed + 2, P * 1024)
        Q = synth.normal(seed + 3, 6144)
        G = synth.normal(seed + 4, 6144) if gate else None
        d_k, d_v, d_q = ctx.array(K), ctx.array(V), ctx.array(Q)
        d_g = ctx.array(G) if gate else None
        d_o = ctx.empty((24, 256))
        if P > 1:
            kv.write(layer, seq, 0, P - 1, d_k, d_v)
        with decode_split(ctx, split):
            kv.attn_decode(layer, [seq], [P - 1], d_q, d_o, k_new=d_k.offset((P - 1) * 1024),
                           v_new=d_v.offset((P - 1) * 1024), gate=d_g)
        got = d_o.download()
        # the append must have landed in the cache
        d_kr, d_vr = ctx.empty((1, 1024)), ctx.empty((1, 1024))
        kv.read(layer, seq, P - 1, 1, d_kr, d_vr)
        assert np.array_equal(d_kr.download().reshape(-1), K[(P - 1) * 1024:])
        assert np.array_equal(d_vr.download().reshape(-1), V[(P - 1) * 1024:])
        for d in (d_k, d_v, d_q, d_o, d_kr, d_vr) + ((d_g,) if gate else ()):
            d.free()
        return got, Q, K.reshape(P, 1024), V.reshape(P, 1024), G
    finally:
        kv.close()


@pytest.mark.parametrize("gate", [False, True])
def test_decode_256_tokens(pkg, ctx, ref, margin, gate):
    """Config: 24 q / 4 kv heads, d 256, 256 cached tokens (position 255)."""
    got, Q, K, V, G = _decode_one(pkg, ctx, 256, 0x51333800, gate=gate)
    check_attn(margin, got, ref.attn_heads(Q, K, V, gate=G))


@pytest.mark.parametrize("P", [1, 2, 15, 16, 17, 63, 64, 65, 200, 1000])
def test_decode_ragged_lengths(pkg, ctx, ref, margin, P):
    """Edge lengths: one position (o = v exactly up to the gate), partial pages,
    partial half-pages, lengths around the split size."""
    got, Q, K, V, G = _decode_one(pkg, ctx, P, 7000 + P, gate=True)
    check_attn(margin, got, ref.attn_heads(Q, K, V, gate=G))


@pytest.mark.parametrize("split", [16, 32, 48, 64, 128, 512, 1024, 2048, 4096])
def test_decode_split_invariance(pkg, ctx, ref, margin, split):
    """Splits from one page per workgroup (two waves of four idle; 188 splits
    over 3000 tokens, the last one 8 tokens) to the whole context in one
    workgroup; 48-token splits (three pages) are no power of two."""
    got, Q, K, V, G = _decode_one(pkg, ctx, 3000, 9100, gate=True, split=split)
    check_attn(margin, got, ref.attn_heads(Q, K, V, gate=G))


def test_decode_merge_repeated(pkg, ctx, ref, margin):
    """The split-K partials and their merge over many launches in a row: 40
    decodes over 1 to 47 splits, sharing the partial workspace, the output
    poisoned with NaN before each launch and checked after it."""
    from q38amd import synth
    P = 3000
    kv = pkg.KVCache(ctx, n_slots=17, max_pages=(P + 15) // 16 + 4, max_seqs=1, max_tokens_per_seq=P + 64)
    try:
        seq = kv.seq_create()
        K = synth.normal(0x9200, P * 1024)
        V = synth.normal(0x9201, P * 1024)
        Q = synth.normal(0x9202, 6144)
        G = synth.normal(0x9203, 6144)
        d_k, d_v, d_q, d_g = ctx.array(K), ctx.array(V), ctx.array(Q), ctx.array(G)
        kv.write(3, seq, 0, P, d_k, d_v)
        want = ref.attn_heads(Q, K.reshape(P, 1024), V.reshape(P, 1024), gate=G)
        d_o = ctx.empty((24, 256))
        poison = np.full(6144, np.nan, np.float32)
        worst = np.zeros(6144)
        for i in range(40):
            split = [64, 128, 192, 384, 3008][i % 5]
            d_o.upload(poison)
            with decode_split(ctx, split):
                kv.attn_decode(3, [seq], [P - 1], d_q, d_o, gate=d_g)
            got = d_o.download().reshape(-1)
            assert np.all(np.isfinite(got)), (i, split)
            worst = np.maximum(worst, np.abs(got - want.reshape(-1)))
        check_attn(margin, want.reshape(-1) + worst, want.reshape(-1))
    finally:
        kv.close()


def test_decode_128k_context(pkg, ctx, ref, margin):
    """The full-stack context: 131072 cached tokens (2048-token splits)."""
    got, Q, K, V, G = _decode_one(pkg, ctx, 131072, 0x51333820, gate=True)
    check_attn(margin, got, ref.attn_heads(Q, K, V, gate=G, threads=16))


def test_decode_32k_metric_shape(pkg, ctx, ref, margin):
    """The benchmark shape: 32768 cached tokens."""
    got, Q, K, V, G = _decode_one(pkg, ctx, 32768, 0x51333810, gate=False)
    check_attn(margin, got, ref.attn_heads(Q, K, V, threads=16))


def test_decode_batched_paged_permuted(pkg, ctx, ref, margin):
    """Config: 32 sequences, context ~U[1K, 32K], 16-token pages, page table a
    random permutation of the pool, one decode token per sequence."""
    from q38amd import synth
    n = 32
    rng = np.random.default_rng(0x51333802)
    ctx_len = rng.integers(1024, 32768, size=n, endpoint=True)
    pages_needed = [(int(c) + 15) // 16 for c in ctx_len]
    pool = sum(pages_needed) + 8
    kv = pkg.KVCache(ctx, n_slots=1, max_pages=pool, max_seqs=n, max_tokens_per_seq=32768 + 16)
    perm = rng.permutation(pool)
    seqs, off = [], 0
    for i in range(n):
        s = kv.seq_create()
        kv.seq_set_pages(s, perm[off:off + pages_needed[i]].tolist())
        off += pages_needed[i]
        seqs.append(s)
    layer = 3
    Ks, Vs = [], []
    d_k, d_v = ctx.empty((32768, 1024)), ctx.empty((32768, 1024))
    for i in range(n):
        P = int(ctx_len[i])
        # seeded N(0,1) rows made on the device (same stream as synth.normal)
        ctx.fill_normal(d_k, P * 1024, 0x5000 + 2 * i)
        ctx.fill_normal(d_v, P * 1024, 0x5001 + 2 * i)
        kv.write(layer, seqs[i], 0, P, d_k, d_v)
        Ks.append(d_k.download(P))
        Vs.append(d_v.download(P))
    d_k.free()
    d_v.free()
    Q = synth.normal(0x6000, n * 6144)
    G = synth.normal(0x6001, n * 6144)
    d_q, d_g, d_o = ctx.array(Q), ctx.array(G), ctx.empty((n, 24, 256))
    kv.attn_decode(layer, seqs, [int(c) - 1 for c in ctx_len], d_q, d_o, gate=d_g)
    got = d_o.download()
    kv.close()
    wants = [ref.attn_heads(Q[i * 6144:(i + 1) * 6144], Ks[i], Vs[i], gate=G[i * 6144:(i + 1) * 6144], threads=16)
             for i in range(n)]
    # each sequence against its own scale (the relative bound per sequence)
    worst_rel = max(abs_rel(got[i], wants[i])[1] for i in range(n))
    worst_abs = max(abs_rel(got[i], wants[i])[0] for i in range(n))
    margin("out max-abs", worst_abs, TOL_ABS)
    margin("out rel (worst sequence)", worst_rel, TOL_REL)


@pytest.mark.parametrize("split", [None, 128, 64])
def test_decode_permuted_pages_both_launch_forms(pkg, ctx, ref, margin, split):
    """Five sequences (one page, two pages, and longer) on a permuted page
    table.  Launches of at most 256 splits carry each split's first two page
    ids in their arguments (default and 128-token splits: 135 splits at 128);
    64-token splits make 267 splits, which read every page id from the table."""
    from q38amd import synth
    lens = [5, 17, 3001, 7777, 6100]
    n = len(lens)
    rng = np.random.default_rng(0x51333803 + (split or 0))
    pages_needed = [(c + 15) // 16 for c in lens]
    pool = sum(pages_needed) + 8
    kv = pkg.KVCache(ctx, n_slots=1, max_pages=pool, max_seqs=n, max_tokens_per_seq=8192)
    perm = rng.permutation(pool)
    try:
        seqs, off = [], 0
        for i in range(n):
            s = kv.seq_create()
            kv.seq_set_pages(s, perm[off:off + pages_needed[i]].tolist())
            off += pages_needed[i]
            seqs.append(s)
        Ks, Vs = [], []
        for i, P in enumerate(lens):
            K = synth.normal(0x7100 + 2 * i, P * 1024)
            V = synth.normal(0x7101 + 2 * i, P * 1024)
            d_k, d_v = ctx.array(K), ctx.array(V)
            kv.write(3, seqs[i], 0, P, d_k, d_v)
            d_k.free()
            d_v.free()
            Ks.append(K.reshape(P, 1024))
            Vs.append(V.reshape(P, 1024))
        Q = synth.normal(0x7200, n * 6144)
        G = synth.normal(0x7201, n * 6144)
        d_q, d_g, d_o = ctx.array(Q), ctx.array(G), ctx.empty((n, 24, 256))
        with decode_split(ctx, split):
            kv.attn_decode(3, seqs, [P - 1 for P in lens], d_q, d_o, gate=d_g)
        got = d_o.download()
    finally:
        kv.close()
    for i in range(n):
        want = ref.attn_heads(Q[i * 6144:(i + 1) * 6144], Ks[i], Vs[i], gate=G[i * 6144:(i + 1) * 6144])
        check_attn(margin, got[i], want, f"seq {i} ({lens[i]} tokens)")


def test_decode_after_rollback_new_pages(pkg, ctx, ref, margin):
    """A rollback returns pages to the free stack, a second sequence takes some
    of them, and the first grows again into other physical pages, one row per
    decode call (64-token splits, so every split's first page ids come from
    the host copy of the page table, which must follow each change)."""
    from q38amd import synth
    P, keep, n_new = 900, 300, 40
    kv = pkg.KVCache(ctx, n_slots=1, max_pages=80, max_seqs=2, max_tokens_per_seq=1024)
    try:
        a = kv.seq_create()
        K = synth.normal(0x7300, P * 1024).reshape(P, 1024)
        V = synth.normal(0x7301, P * 1024).reshape(P, 1024)
        d_k, d_v = ctx.array(K), ctx.array(V)
        kv.write(3, a, 0, P, d_k, d_v)
        kv.seq_truncate(a, keep)
        b = kv.seq_create()
        kv.write(3, b, 0, 200, d_k, d_v)  # takes pages that a released
        Kn = synth.normal(0x7304, n_new * 1024).reshape(n_new, 1024)
        Vn = synth.normal(0x7305, n_new * 1024).reshape(n_new, 1024)
        Q = synth.normal(0x7306, 6144)
        G = synth.normal(0x7307, 6144)
        d_q, d_g, d_o = ctx.array(Q), ctx.array(G), ctx.empty((24, 256))
        with decode_split(ctx, 64):
            for i in range(n_new):
                d_kn, d_vn = ctx.array(Kn[i]), ctx.array(Vn[i])
                kv.attn_decode(3, [a], [keep + i], d_q, d_o, k_new=d_kn, v_new=d_vn, gate=d_g)
                if i % 13 == 0 or i == n_new - 1:
                    want = ref.attn_heads(Q, np.concatenate([K[:keep], Kn[:i + 1]]),
                                          np.concatenate([V[:keep], Vn[:i + 1]]), gate=G)
                    check_attn(margin, d_o.download(), want, f"token {i}")
                d_kn.free()
                d_vn.free()
    finally:
        kv.close()


def test_full_core_matches_reference(pkg, ctx, ref, margin):
    """full_core whole: q/gate split, q and k RMSNorm, RoPE, append, attention,
    gate, for consecutive tokens, including a position past 2^16 (RoPE angles
    of the iterative f32 recurrence at large arguments)."""
    from q38amd import synth
    ctx_len = 70000
    layer = 7
    qn = synth.normal(1, 256, sigma=0.2, mean=1.0)
    kn = synth.normal(2, 256, sigma=0.2, mean=1.0)
    # the reference caches: only slot 1 (layer 7) is used; keep [2][ctx][1024]
    kc = np.zeros(2 * ctx_len * 1024, np.float32)
    vc = np.zeros(2 * ctx_len * 1024, np.float32)
    kv = pkg.KVCache(ctx, n_slots=17, max_pages=ctx_len // 16 + 8, max_seqs=1, max_tokens_per_seq=ctx_len)
    seq = kv.seq_create()
    d_qn, d_kn = ctx.array(qn), ctx.array(kn)
    # fill positions 0..65599 directly (same rows in both caches), then run
    # full_core for positions 65600..65603
    base = 65600
    K0 = synth.normal(3, base * 1024)
    V0 = synth.normal(4, base * 1024)
    kc[ctx_len * 1024: ctx_len * 1024 + base * 1024] = K0
    vc[ctx_len * 1024: ctx_len * 1024 + base * 1024] = V0
    d_k0, d_v0 = ctx.array(K0), ctx.array(V0)
    kv.write(layer, seq, 0, base, d_k0, d_v0)
    d_k0.free()
    d_v0.free()
    for i in range(4):
        pos = base + i
        qg = synth.normal(100 + i, 12288)
        key = synth.normal(200 + i, 1024)
        val = synth.normal(300 + i, 1024)
        d_o = ctx.empty((24, 256))
        kv.full_core(layer, [seq], [pos], d_qn, d_kn, ctx.array(qg), ctx.array(key), ctx.array(val), d_o)
        want, _ = ref.full_core(qn, kn, qg, key, val, kc, vc, ctx_len, pos, layer, threads=16)
        check_attn(margin, d_o.download(), want, f"position {pos}")
    kv.close()


def test_full_core_batched_positions(pkg, ctx, ref, margin):
    """full_core for three sequences at different positions in one call (one
    pre launch with each sequence's own RoPE position, then the batched
    decode with appends), each against the reference on its own caches."""
    from q38amd import synth
    layer = 3
    ctx_len = 1024
    qn = synth.normal(11, 256, sigma=0.2, mean=1.0)
    kn = synth.normal(12, 256, sigma=0.2, mean=1.0)
    kv = pkg.KVCache(ctx, n_slots=17, max_pages=3 * ctx_len // 16, max_seqs=3, max_tokens_per_seq=ctx_len)
    positions = [100, 37, 500]
    seqs = [kv.seq_create() for _ in positions]
    caches = []
    for i, (sq, pos) in enumerate(zip(seqs, positions)):
        K0 = synth.normal(20 + i, pos * 1024)
        V0 = synth.normal(30 + i, pos * 1024)
        kc = np.zeros(ctx_len * 1024, np.float32)
        vc = np.zeros(ctx_len * 1024, np.float32)
        kc[:pos * 1024] = K0
        vc[:pos * 1024] = V0
        d_k0, d_v0 = ctx.array(K0), ctx.array(V0)
        kv.write(layer, sq, 0, pos, d_k0, d_v0)
        d_k0.free()
        d_v0.free()
        caches.append((kc, vc))
    qg = synth.normal(40, 3 * 12288)
    key = synth.normal(41, 3 * 1024)
    val = synth.normal(42, 3 * 1024)
    d_o = ctx.empty((3, 24, 256))
    kv.full_core(layer, seqs, positions, ctx.array(qn), ctx.array(kn), ctx.array(qg), ctx.array(key),
                 ctx.array(val), d_o)
    got = d_o.download().reshape(3, 6144)
    for b, pos in enumerate(positions):
        kc, vc = caches[b]
        want, _ = ref.full_core(qn, kn, qg[b * 12288:(b + 1) * 12288], key[b * 1024:(b + 1) * 1024],
                                val[b * 1024:(b + 1) * 1024], kc, vc, ctx_len, pos, layer, threads=8)
        check_attn(margin, got[b], np.asarray(want).reshape(-1), f"seq {b}")
    kv.close()


def test_full_core_many_splits(pkg, ctx, ref, margin):
    """full_core for five sequences with 64-token splits: 326 splits in one
    launch, more than the 256 whose first page ids ride in the launch
    arguments, so the fused-pre kernel form that reads every page id from the
    page table runs.  Permuted page table; each sequence against the
    restatement on its own caches; the appended key row (RMSNormed and
    rotated in the kernel) and value row read back."""
    from q38amd import synth
    layer = 11  # slot 2
    positions = [3001, 6100, 64, 4500, 7000]
    n, ctx_len = len(positions), 8192
    assert sum((p + 64) // 64 for p in positions) > 256
    qn = synth.normal(51, 256, sigma=0.2, mean=1.0)
    kn = synth.normal(52, 256, sigma=0.2, mean=1.0)
    pages_needed = [p // 16 + 1 for p in positions]
    pool = sum(pages_needed) + 16
    kv = pkg.KVCache(ctx, n_slots=17, max_pages=pool, max_seqs=n, max_tokens_per_seq=ctx_len)
    perm = np.random.default_rng(0x51333811).permutation(pool)
    try:
        seqs, off, caches = [], 0, []
        for i, P in enumerate(positions):
            s = kv.seq_create()
            kv.seq_set_pages(s, perm[off:off + pages_needed[i]].tolist())
            off += pages_needed[i]
            seqs.append(s)
            K0 = synth.normal(60 + 2 * i, P * 1024)
            V0 = synth.normal(61 + 2 * i, P * 1024)
            d_k0, d_v0 = ctx.array(K0), ctx.array(V0)
            kv.write(layer, s, 0, P, d_k0, d_v0)
            d_k0.free()
            d_v0.free()
            kc = np.zeros(3 * ctx_len * 1024, np.float32)
            vc = np.zeros(3 * ctx_len * 1024, np.float32)
            kc[2 * ctx_len * 1024: 2 * ctx_len * 1024 + P * 1024] = K0
            vc[2 * ctx_len * 1024: 2 * ctx_len * 1024 + P * 1024] = V0
            caches.append((kc, vc))
        qg = synth.normal(70, n * 12288)
        key = synth.normal(71, n * 1024)
        val = synth.normal(72, n * 1024)
        d_o = ctx.empty((n, 24, 256))
        with decode_split(ctx, 64):
            kv.full_core(layer, seqs, positions, ctx.array(qn), ctx.array(kn), ctx.array(qg), ctx.array(key),
                         ctx.array(val), d_o)
        got = d_o.download().reshape(n, 6144)
        r_k, r_v = ctx.empty((1, 1024)), ctx.empty((1, 1024))
        for b, P in enumerate(positions):
            kc, vc = caches[b]
            want, k_formed = ref.full_core(qn, kn, qg[b * 12288:(b + 1) * 12288], key[b * 1024:(b + 1) * 1024],
                                           val[b * 1024:(b + 1) * 1024], kc, vc, ctx_len, P, layer, threads=16)
            check_attn(margin, got[b], np.asarray(want).reshape(-1), f"seq {b}")
            kv.read(layer, seqs[b], P, 1, r_k, r_v)
            margin(f"seq {b} appended key max-abs", float(np.max(np.abs(r_k.download().reshape(-1) - k_formed))), 1e-5)
            assert np.array_equal(r_v.download().reshape(-1), val[b * 1024:(b + 1) * 1024])
    finally:
        kv.close()


def test_attn_pre_matches_reference(pkg, ctx, ref):
    """RMSNorm + RoPE prologue alone, bit for bit where the math is exact."""
    from q38amd import synth
    n = 8
    qn = synth.normal(11, 256, sigma=0.2, mean=1.0)
    kn = synth.normal(12, 256, sigma=0.2, mean=1.0)
    qg = synth.normal(13, n * 12288)
    key = synth.normal(14, n * 1024)
    pos0 = 123457
    d_q, d_g, d_k = ctx.empty((n, 6144)), ctx.empty((n, 6144)), ctx.empty((n, 1024))
    ctx.attn_pre(n, pos0, ctx.array(qn), ctx.array(kn), ctx.array(qg), ctx.array(key), d_q, d_g, d_k)
    gq, gg, gk = d_q.download(), d_g.download(), d_k.download()
    for t in range(n):
        src = qg[t * 12288:(t + 1) * 12288].reshape(24, 512)
        q = np.stack([ref.rmsnorm(src[h, :256], qn) for h in range(24)]).reshape(-1)
        q = ref.rope(q, 24, pos0 + t)
        k = np.stack([ref.rmsnorm(key[t * 1024 + h * 256: t * 1024 + (h + 1) * 256], kn) for h in range(4)])
        k = ref.rope(k.reshape(-1), 4, pos0 + t)
        assert np.array_equal(gg[t].reshape(24, 256), src[:, 256:])
        assert np.max(np.abs(gq[t] - q)) <= 1e-5
        assert np.max(np.abs(gk[t] - k)) <= 1e-5


def test_prefill_matches_reference_rows(pkg, ctx, ref, margin):
    """batch_full_attention (ops.rs:1153-1172) over a 1024-token prompt after
    a 300-token prefix; sampled rows against the restatement."""
    from q38amd import synth
    base, T = 300, 1024
    kv = pkg.KVCache(ctx, n_slots=17, max_pages=(base + T) // 16 + 8, max_seqs=1, max_tokens_per_seq=base + T)
    seq = kv.seq_create()
    layer = 11
    K = synth.normal(41, (base + T) * 1024)
    V = synth.normal(42, (base + T) * 1024)
    Q = synth.normal(43, T * 6144)
    G = synth.normal(44, T * 6144)
    d_k, d_v = ctx.array(K), ctx.array(V)
    kv.write(layer, seq, 0, base, d_k, d_v)
    d_o = ctx.empty((T, 24, 256))
    kv.attn_prefill(layer, seq, base, T, ctx.array(Q), d_k.offset(base * 1024), d_v.offset(base * 1024), d_o,
                    gate=ctx.array(G))
    got = d_o.download()
    Kr, Vr = K.reshape(-1, 1024), V.reshape(-1, 1024)
    rows = sorted(set([0, 1, 15, 16, 511, T - 1] + list(np.random.default_rng(5).integers(0, T, 10))))
    worst = (0.0, 0.0)
    for t in rows:
        n_pos = base + t + 1
        want = ref.attn_heads(Q[t * 6144:(t + 1) * 6144], Kr[:n_pos], Vr[:n_pos], gate=G[t * 6144:(t + 1) * 6144])
        worst = tuple(max(a, b) for a, b in zip(worst, abs_rel(got[t], want)))
    kv.close()
    _check_rows(margin, worst)


def _check_rows(margin, worst):
    margin("out max-abs (worst row)", worst[0], TOL_ABS)
    margin("out rel (worst row)", worst[1], TOL_REL)


def _prefill_case(pkg, ctx, ref, base, T, seed, gate=True, permute=False, rows=None):
    """Prefill of T tokens after a base-token prefix through q38_attn_prefill
    (bf16x3 MFMA kernel); rows (default: all) against the restatement.
    Returns the worst (max-abs, relative) error over the rows."""
    from q38amd import synth
    n_pages = (base + T + 15) // 16
    kv = pkg.KVCache(ctx, n_slots=17, max_pages=n_pages + 8, max_seqs=1, max_tokens_per_seq=base + T)
    try:
        seq = kv.seq_create()
        if permute:
            pages = np.random.default_rng(seed).permutation(n_pages + 8)[:n_pages]
            kv.seq_set_pages(seq, pages.tolist())
        layer = 7
        K = synth.normal(seed + 1, (base + T) * 1024)
        V = synth.normal(seed + 2, (base + T) * 1024)
        Q = synth.normal(seed + 3, T * 6144)
        G = synth.normal(seed + 4, T * 6144) if gate else None
        d_k, d_v = ctx.array(K), ctx.array(V)
        if base:
            kv.write(layer, seq, 0, base, d_k, d_v)
        d_o = ctx.empty((T, 24, 256))
        kv.attn_prefill(layer, seq, base, T, ctx.array(Q), d_k.offset(base * 1024), d_v.offset(base * 1024), d_o,
                        gate=ctx.array(G) if gate else None)
        got = d_o.download()
        Kr, Vr = K.reshape(-1, 1024), V.reshape(-1, 1024)
        worst = (0.0, 0.0)
        for t in (range(T) if rows is None else rows):
            n_pos = base + t + 1
            want = ref.attn_heads(Q[t * 6144:(t + 1) * 6144], Kr[:n_pos], Vr[:n_pos],
                                  gate=None if G is None else G[t * 6144:(t + 1) * 6144], threads=16)
            worst = tuple(max(a, b) for a, b in zip(worst, abs_rel(got[t], want)))
        return worst
    finally:
        kv.close()


@pytest.mark.parametrize("T", [1, 2, 15, 16, 17, 31, 33, 100])
def test_prefill_short_prompts_all_rows(pkg, ctx, ref, margin, T):
    """Ragged prompt lengths from position 0 (partial query and key blocks)."""
    _check_rows(margin, _prefill_case(pkg, ctx, ref, 0, T, 900 + T))


def test_prefill_permuted_pages_no_gate(pkg, ctx, ref, margin):
    """Randomly permuted page table, prefix of 37 tokens, no output gate."""
    _check_rows(margin, _prefill_case(pkg, ctx, ref, 37, 150, 960, gate=False, permute=True))


def test_prefill_4096_prompt(pkg, ctx, ref, margin):
    """The chunked-prefill workload: a 4096-token causal prompt; every one of
    the 4096 query rows, all 24 heads, against the restatement."""
    _check_rows(margin, _prefill_case(pkg, ctx, ref, 0, 4096, 980))


def test_prefill_past_64_query_blocks(pkg, ctx, ref, margin):
    """Prompts of more than 64 query blocks run one job per workgroup in the
    grid's own order (shorter ones on host-placed jobs): 4160 tokens after a
    100-token prefix (65 query blocks).  All 24 heads of one row in every
    64-query block (its row offset varies from block to block), plus the
    first, last and ragged rows and samples between."""
    T = 4160
    per_block = [qb * 64 + (qb * 37) % 64 for qb in range((T + 63) // 64)]
    rows = sorted(set([0, 1, 63, 64, 2047, 4095, 4096, 4127, 4128, T - 1] + [r for r in per_block if r < T] +
                      list(np.random.default_rng(11).integers(0, T, 12))))
    _check_rows(margin, _prefill_case(pkg, ctx, ref, 100, T, 990, rows=rows))


@pytest.mark.parametrize("base,T,step,gate,permute", [(0, 1024, 1, True, False), (3001, 700, 7, True, False),
                                                     (9000, 200, 1, True, False), (0, 512, 1, False, True)])
def test_prefill_split_jobs(pkg, ctx, ref, margin, base, T, step, gate, permute):
    """Prompts whose longest jobs pass 1.35 times a workgroup's share of key
    blocks (the last query blocks of a short prompt; every job after a long
    prefix): the host cuts jobs into pieces of key blocks that write partials,
    and q38_prefill_merge combines them.  1024 tokens from position 0 (36 of
    48 jobs cut), 700 after a 3001-token prefix (the prompt starts inside a
    key block), 200 after 9000 (every job in 16 pieces), 512 with permuted pages and
    no gate; every row, or every 7th and the last."""
    rows = sorted(set(range(0, T, step)) | {T - 1})
    _check_rows(margin, _prefill_case(pkg, ctx, ref, base, T, 1100 + T, gate=gate, permute=permute, rows=rows))


@pytest.mark.parametrize("base", [0, 2000])
def test_prefill_reference_restart(pkg, ctx, ref, margin, base):
    """Keys far above the first block's scores: the prefill kernel keeps one
    reference max per query taken from its first key block and restarts a
    workgroup's key loop when a later block passes it by more than 2^64.
    Heads 0-5 query one direction u; key base+70 of kv head 0 scores 60
    (natural units) and key base+150 scores 130, so queries 70.. restart and
    queries 150.. again.  After a 2000-token prefix every job is cut into
    pieces, so the restarts return to a piece's first block.  All rows
    against the restatement."""
    from q38amd import synth
    T = 200
    n = base + T
    kv = pkg.KVCache(ctx, n_slots=17, max_pages=n // 16 + 4, max_seqs=1, max_tokens_per_seq=n)
    try:
        seq = kv.seq_create()
        layer = 3
        K = synth.normal(1001, n * 1024).reshape(n, 4, 256)
        V = synth.normal(1002, n * 1024).reshape(n, 4, 256)
        Q = synth.normal(1003, T * 6144).reshape(T, 24, 256)
        u = synth.normal(1004, 256)
        Q[:, 0:6, :] = u
        un = u / np.linalg.norm(u)
        K[base + 70, 0] = (60.0 * 16.0 / np.linalg.norm(u)) * un
        K[base + 150, 0] = (130.0 * 16.0 / np.linalg.norm(u)) * un
        K, V, Q = K.astype(np.float32).reshape(-1), V.astype(np.float32).reshape(-1), Q.astype(np.float32).reshape(-1)
        d_k, d_v = ctx.array(K), ctx.array(V)
        if base:
            kv.write(layer, seq, 0, base, d_k, d_v)
        d_o = ctx.empty((T, 24, 256))
        kv.attn_prefill(layer, seq, base, T, ctx.array(Q), d_k.offset(base * 1024), d_v.offset(base * 1024), d_o)
        got = d_o.download()
        Kr, Vr = K.reshape(-1, 1024), V.reshape(-1, 1024)
        worst = (0.0, 0.0)
        for t in range(T):
            want = ref.attn_heads(Q[t * 6144:(t + 1) * 6144], Kr[:base + t + 1], Vr[:base + t + 1])
            worst = tuple(max(a, b) for a, b in zip(worst, abs_rel(got[t], want)))
        # the planted keys dominate: head 0 of query 120 returns v_70, of query 190 v_150
        assert np.max(np.abs(got[120, 0] - Vr[base + 70, :256])) <= 1e-3
        assert np.max(np.abs(got[190, 0] - Vr[base + 150, :256])) <= 1e-3
    finally:
        kv.close()
    _check_rows(margin, worst)


def test_kv_pages_roundtrip_and_rollback(pkg, ctx, synth):
    """Write/read through a permuted page table; truncate releases whole pages
    past the kept positions; reset releases all."""
    kv = pkg.KVCache(ctx, n_slots=2, max_pages=64, max_seqs=4, max_tokens_per_seq=512)
    a = kv.seq_create()
    kv.seq_set_pages(a, list(range(63, 43, -1)))  # 20 pages, reversed order
    K = synth.normal(51, 300 * 1024)
    V = synth.normal(52, 300 * 1024)
    d_k, d_v = ctx.array(K), ctx.array(V)
    kv.write(3, a, 0, 300, d_k, d_v)
    r_k, r_v = ctx.empty((300, 1024)), ctx.empty((300, 1024))
    kv.read(3, a, 0, 300, r_k, r_v)
    assert np.array_equal(r_k.download().reshape(-1), K)
    assert np.array_equal(r_v.download().reshape(-1), V)
    assert kv.seq_capacity(a) == 320 and kv.free_pages() == 44
    kv.seq_truncate(a, 100)  # keeps pages for positions < 100 (7 pages)
    assert kv.seq_capacity(a) == 112 and kv.free_pages() == 57
    kv.read(3, a, 0, 100, r_k, r_v)
    assert np.array_equal(r_k.download().reshape(-1)[:100 * 1024], K[:100 * 1024])
    kv.seq_reset(a)
    assert kv.seq_capacity(a) == 0 and kv.free_pages() == 64
    kv.close()


def test_device_generator_matches_host(pkg, ctx, synth):
    """The device fill reproduces the host generator (same SplitMix64 words,
    same Box-Muller), so device-made inputs are the documented inputs."""
    n = 100001
    d = ctx.empty((n,))
    ctx.fill_normal(d, n, 0x1234, sigma=0.5, mean=0.25)
    got = d.download()
    want = synth.normal(0x1234, n, sigma=0.5, mean=0.25)
    ulps = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert np.mean(ulps == 0) > 0.999 and int(ulps.max()) <= 1
