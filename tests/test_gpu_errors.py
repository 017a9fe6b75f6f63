"""The reference's one error contract on this path, Err(-1), through the C
ABI: the KV bounds check (src/model/ops.rs:860-864) and the context-full
check (ops.rs:1702), plus the checks of the paged cache that the dense
reference cache does not need (layer kind, pool exhaustion, page ownership,
repeated sequences).  Each failing call must return -1 with a message and
leave the cache as it was: free pages, every sequence's capacity and the
rows already cached.  The checks run on the host, so no kernel is launched
for a failing call."""
import numpy as np
import pytest
from parity import check_attn

pytestmark = pytest.mark.gpu


def _snapshot(kv, seqs):
    return kv.free_pages(), [kv.seq_capacity(s) for s in seqs]


def _fails(pkg, fn, match):
    with pytest.raises(pkg.Q38Error, match=match):
        fn()


@pytest.fixture
def small(pkg, ctx, synth):
    """A cache of 12 pages (192 tokens), context limit 128 tokens, two
    sequences: a holds positions 0..99 (7 pages), b is empty."""
    kv = pkg.KVCache(ctx, n_slots=17, max_pages=12, max_seqs=3, max_tokens_per_seq=128)
    a, b = kv.seq_create(), kv.seq_create()
    K = synth.normal(0xE1, 100 * 1024)
    V = synth.normal(0xE2, 100 * 1024)
    d_k, d_v = ctx.array(K), ctx.array(V)
    kv.write(3, a, 0, 100, d_k, d_v)
    bufs = {"q": ctx.array(synth.normal(0xE3, 2 * 6144)), "o": ctx.empty((2, 24, 256)),
            "kn": ctx.array(synth.normal(0xE4, 2 * 1024)), "vn": ctx.array(synth.normal(0xE5, 2 * 1024)),
            "qg": ctx.array(synth.normal(0xE6, 2 * 12288)), "w": ctx.array(np.ones(256, np.float32))}
    yield kv, a, b, K.reshape(100, 1024), V.reshape(100, 1024), bufs
    kv.close()


def _rows_intact(ctx, kv, a, K, V):
    r_k, r_v = ctx.empty((100, 1024)), ctx.empty((100, 1024))
    kv.read(3, a, 0, 100, r_k, r_v)
    assert np.array_equal(r_k.download(), K) and np.array_equal(r_v.download(), V)


def test_decode_past_context_limit(pkg, ctx, small):
    """ops.rs:860-864 / :1702: a position at or past the context limit."""
    kv, a, b, K, V, d = small
    before = _snapshot(kv, [a, b])
    _fails(pkg, lambda: kv.attn_decode(3, [a], [128], d["q"], d["o"], k_new=d["kn"], v_new=d["vn"]),
           "past the context limit")
    _fails(pkg, lambda: kv.full_core(3, [b], [200], d["w"], d["w"], d["qg"], d["kn"], d["vn"], d["o"]),
           "past the context limit")
    _fails(pkg, lambda: kv.attn_decode(3, [a], [-1], d["q"], d["o"]), "negative position")
    assert _snapshot(kv, [a, b]) == before
    _rows_intact(ctx, kv, a, K, V)


def test_prefill_and_write_past_context_limit(pkg, ctx, small):
    kv, a, b, K, V, d = small
    before = _snapshot(kv, [a, b])
    kn = ctx.empty((60, 1024))
    _fails(pkg, lambda: kv.attn_prefill(3, a, 100, 60, d["q"], kn, kn, ctx.empty((60, 24, 256))),
           "past the context limit")
    _fails(pkg, lambda: kv.write(3, b, 100, 60, kn, kn), "exceed the per-sequence limit")
    assert _snapshot(kv, [a, b]) == before
    _rows_intact(ctx, kv, a, K, V)


@pytest.mark.parametrize("layer", [0, 1, 2, 4, 62, 65, -1])
def test_not_a_full_attention_layer(pkg, ctx, small, layer):
    """Full attention is on layers 3, 7, ..., 63 and the MTP layer 64
    (ops.rs:38-41); every other layer is a DeltaNet layer."""
    kv, a, b, K, V, d = small
    before = _snapshot(kv, [a, b])
    _fails(pkg, lambda: kv.attn_decode(layer, [a], [100], d["q"], d["o"], k_new=d["kn"], v_new=d["vn"]),
           "not a full-attention layer")
    assert _snapshot(kv, [a, b]) == before


def test_layer_without_slot(pkg, ctx, synth):
    kv = pkg.KVCache(ctx, n_slots=16, max_pages=4, max_seqs=1, max_tokens_per_seq=64)
    try:
        s = kv.seq_create()
        q, o = ctx.empty((24, 256)), ctx.empty((24, 256))
        kn = ctx.empty((1024,))
        _fails(pkg, lambda: kv.attn_decode(64, [s], [0], q, o, k_new=kn, v_new=kn), "needs slot 16")
        assert kv.free_pages() == 4 and kv.seq_capacity(s) == 0
    finally:
        kv.close()


def test_pool_exhausted_batch_changes_nothing(pkg, ctx, small):
    """a (7 pages held) grows to position 120 (1 more page) and b needs 8
    pages for position 120: 9 pages against 5 free.  Neither reserves."""
    kv, a, b, K, V, d = small
    assert kv.free_pages() == 5
    before = _snapshot(kv, [a, b])
    _fails(pkg, lambda: kv.attn_decode(3, [a, b], [120, 120], d["q"], d["o"], k_new=d["kn"], v_new=d["vn"]),
           "KV pool exhausted")
    assert _snapshot(kv, [a, b]) == before
    _rows_intact(ctx, kv, a, K, V)
    _fails(pkg, lambda: kv.seq_reserve(b, 100), "KV pool exhausted")
    assert _snapshot(kv, [a, b]) == before


def test_repeated_sequence_in_appending_decode(pkg, ctx, small):
    kv, a, b, K, V, d = small
    before = _snapshot(kv, [a, b])
    _fails(pkg, lambda: kv.attn_decode(3, [a, a], [100, 101], d["q"], d["o"], k_new=d["kn"], v_new=d["vn"]),
           "appears twice")
    assert _snapshot(kv, [a, b]) == before


def test_unknown_or_unreserved_sequence(pkg, ctx, small):
    kv, a, b, K, V, d = small
    before = _snapshot(kv, [a, b])
    _fails(pkg, lambda: kv.attn_decode(3, [7], [0], d["q"], d["o"]), "does not exist")
    # without an append the positions must already be reserved
    _fails(pkg, lambda: kv.attn_decode(3, [a], [115], d["q"], d["o"]), "not reserved")
    assert _snapshot(kv, [a, b]) == before


def test_set_pages_rejects_held_duplicate_and_foreign_ids(pkg, ctx, small):
    """A rejected q38_seq_set_pages keeps the sequence's own mapping and the
    pool; the sequence's own pages may be reordered."""
    kv, a, b, K, V, d = small
    before = _snapshot(kv, [a, b])
    _fails(pkg, lambda: kv.seq_set_pages(b, [8, 8]), "not free")
    _fails(pkg, lambda: kv.seq_set_pages(b, [0]), "not free")            # held by a
    _fails(pkg, lambda: kv.seq_set_pages(b, [12]), "outside the pool")
    _fails(pkg, lambda: kv.seq_set_pages(a, [0, 1, 2, 3, 4, 5, 6, 99]), "outside the pool")
    assert _snapshot(kv, [a, b]) == before
    _rows_intact(ctx, kv, a, K, V)
    # a's own pages in another order: allowed, and the rows move with the ids
    kv.seq_set_pages(a, [6, 5, 4, 3, 2, 1, 0])
    assert _snapshot(kv, [a, b]) == before


def test_decode_works_after_failures(pkg, ctx, ref, margin, small):
    """After every rejected call above, the same cache decodes correctly."""
    kv, a, b, K, V, d = small
    _fails(pkg, lambda: kv.attn_decode(3, [a, b], [120, 120], d["q"], d["o"], k_new=d["kn"], v_new=d["vn"]),
           "KV pool exhausted")
    kv.attn_decode(3, [a], [100], d["q"], d["o"], k_new=d["kn"], v_new=d["vn"])
    got = d["o"].download()[0]
    kn = d["kn"].download()[:1024]
    vn = d["vn"].download()[:1024]
    want = ref.attn_heads(d["q"].download()[:6144], np.vstack([K, kn]), np.vstack([V, vn]))
    check_attn(margin, got, want)


def test_gdn_and_split_argument_checks(pkg, ctx):
    state = ctx.empty((2 * 48 * 128 * 128,))
    x = ctx.empty((2 * 6144,))
    _fails(pkg, lambda: ctx.gdn_step(2, state, x, x, x, x, x, x, state_stride=100), "overlaps states")
    for bad in (1, 8, 15, 63, 100, 8192, -64):
        _fails(pkg, lambda: ctx.set_decode_split(bad), "multiple of 16")
    ctx.set_decode_split(0)
    # linear_core over a prompt reads and writes 16-byte vectors: a buffer
    # one float off is refused before anything is launched
    T = 4
    w = [ctx.empty((n,)) for n in (40960, 48, 48, 128)]
    bufs = {"conv": ctx.empty((30720 + 4,)), "qkv": ctx.empty((T * 10240 + 4,)), "z": ctx.empty((T * 6144 + 4,)),
            "out": ctx.empty((T * 6144 + 4,))}
    delta, gates = ctx.empty((786432,)), ctx.empty((2 * T * 48,))
    for bad in bufs:
        p = {k: (v.offset(1) if k == bad else v.ptr) for k, v in bufs.items()}
        _fails(pkg, lambda: ctx.linear_core(1, T, *w, p["conv"], delta, p["qkv"], p["z"], gates, gates.offset(T * 48),
                                            p["out"]), "16-byte aligned")
    with pytest.raises(pkg.Q38Error, match="decode limit"):
        pkg.KVCache(ctx, n_slots=1, max_pages=1, max_seqs=1, max_tokens_per_seq=(1 << 24) + 16)
