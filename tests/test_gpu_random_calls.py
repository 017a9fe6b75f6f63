"""Seeded random calls through the projection and KV-cache entry points,
beside the fixed cases of test_gpu_proj.py, test_gpu_attn.py and
test_gpu_prefill_cache.py: shapes, token counts and call orders drawn from a
seed, so that the library's choice of kernel (GEMV, split-block on 16/8/4
waves, 128 x 64 tiles, shared multi-matrix launches, the f32 path's forms)
and the prefill block images' invalidation meet combinations no fixed case
names.  Each failure message names its seed and case.

- projections: q38_gemv_q8_k, q38_gemv_q8_k_multi (1-4 matrices, empty ones
  included, one past 5 split-block workgroups per CU), q38_quantize_project_q8_k
  and q38_gemv_f32, every Q8_K weight format and F32/F16/BF16/Q8_0, widths up
  to the 49152 maximum, 1-1500 tokens, against the oracle's restatement of
  tensor_gemv_q8_k / tensor_gemm_q8_k (src/kernel/tensor.rs:1131-1173,
  :1217-1270) bit for bit and of tensor_gemv_f32 (:1095-1129) within 1e-5 of
  the sum of |w x|;
- the KV cache: random sequences of prefill pieces, decode appends and
  truncates over two sequences and two full-attention layers, with the
  prefill images kept and converted whole every call (bit-identical outputs),
  rows held against the restatement of full_core's attention
  (src/model/ops.rs:868-938, :1153-1172) within 1e-3;
- linear_core: 1-3 sequences fed random pieces (one token, a few, 37-700)
  in consecutive calls, the conv and recurrent states carried between them,
  against the restatement run token by token (ops.rs:1088-1099, :744-804):
  outputs within 1e-3, the conv state bit-exact, the recurrent state within
  1e-4 relative;
- full_core (q38_full_core: the q/k norms, RoPE at each sequence's position,
  the append, attention and the gate; ops.rs:813-940): 1-4 sequences of
  random lengths advanced token by token, each step against the restatement
  on its own caches (appended rows included) within 1e-3;
- the replayed decode graph (q38_decode_graph_*): 1-3 sequences, positions
  drawn per replay anywhere in the cached range (split counts and page
  boundaries change between replays), every replay bit-identical to the
  plain q38_attn_decode calls at the same positions."""
import numpy as np
import pytest
from oracle_checks import _random_f32_path, _random_kquant
from parity import TOL_ABS, TOL_REL, abs_rel, state_rel

pytestmark = pytest.mark.gpu

Q8K_TYPES = [10, 11, 12, 13, 14, 20, 23, 16, 17, 22, 18, 21, 19, 29]
F32_TYPES = [0, 1, 30, 8]
TOKENS = list(range(1, 21)) + [24, 31, 32, 33, 40, 47, 48, 63, 64, 65, 96, 127, 128, 129, 200, 257, 300, 511,
                               777, 1024, 1500]


def _rows(rng):
    u = rng.random()
    if u < 0.3:
        return int(rng.integers(1, 64))
    if u < 0.8:
        return int(rng.integers(64, 3000))
    return int(rng.integers(3000, 9000))


def _f32_case(ctx, ref, rng, case):
    T = int(rng.choice(TOKENS))
    ty = int(rng.choice(F32_TYPES))
    mul = 64 if ty == 8 or rng.random() < 0.7 else 8  # Q8_0 rows are 64k wide
    W = int(mul * rng.integers(1, (6144 if T <= 64 else 2048) // mul + 1))
    rows = _rows(rng)
    while rows * W * T > 6e8:
        rows = max(1, rows // 2)
    x = rng.standard_normal((T, W)).astype(np.float32)
    wb, wv = _random_f32_path(ty, rows, W, int(rng.integers(1 << 30)))
    d_w, d_x, d_o = ctx.array(wb, np.uint8), ctx.array(x), ctx.empty((T, rows))
    try:
        ctx.gemv_f32(ty, rows, W, d_w, d_x, T, d_o)
        got = d_o.download().astype(np.float64)
    finally:
        for a_ in (d_w, d_x, d_o):
            a_.free()
    scale = np.abs(x.astype(np.float64)) @ np.abs(wv).T
    want = ref.gemv_f32(ty, wb, x, threads=16).astype(np.float64)
    err = float(np.max(np.abs(got - want) / (scale + 1e-30)))
    assert err <= 1e-5, (case, "f32", ty, rows, W, T, err)


def _q8k_case(ctx, ref, rng, case, kind, cus):
    T = int(rng.choice(TOKENS))
    ty = int(rng.choice(Q8K_TYPES))
    W = 256 * int(rng.integers(1, (68 if T <= 32 else 20) + 1))
    if rng.random() < 0.05:
        W, T = 49152, int(rng.integers(1, 4))  # the widest row: one token per pass
    n_m = 1 if kind == "single" else int(rng.integers(1, 5))
    rows = [_rows(rng) for _ in range(n_m)]
    if kind != "single" and rng.random() < 0.25:
        rows[int(rng.integers(n_m))] = 0
    if kind != "single" and T >= 8 and rng.random() < 0.2:
        rows[0] = 160 * cus + int(rng.integers(1, 300))  # past 5 split-block workgroups per CU
    while sum(rows) * W * T > 8e8:
        rows = [r // 2 for r in rows]
    x = (rng.standard_normal((T, W)) * rng.uniform(0.1, 4.0, (T, 1))).astype(np.float32)
    q8 = ref.quantize_q8_k(x)
    wbs = [_random_kquant(ty, max(r, 1), W, int(rng.integers(1 << 30)))[:r] for r in rows]
    d_ws = [ctx.array(wb, np.uint8) if r else None for wb, r in zip(wbs, rows)]
    d_os = [ctx.empty((T, max(r, 1))) for r in rows]
    d_x = ctx.array(x)
    d_q = ctx.empty((ctx.q8k_bytes(T, W),), np.uint8)
    try:
        if kind == "quantize_project":
            ctx.quantize_project_q8_k(ty, rows, W, d_ws, d_x, T, d_q, d_os)
        else:
            ctx.quantize_q8_k(T, W, d_x, d_q)
            if kind == "single":
                ctx.gemv_q8_k(ty, rows[0], W, d_ws[0], d_q, T, d_os[0])
            else:
                ctx.gemv_q8_k_multi(ty, rows, W, d_ws, d_q, T, d_os)
        what = (case, kind, ty, rows, W, T)
        assert np.array_equal(d_q.download(), q8), what
        for wb, r, d_o in zip(wbs, rows, d_os):
            if r:
                got = d_o.download()
                want = ref.gemv_q8_k(ty, wb, q8, T, W, threads=16)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (what, r)
    finally:
        for a_ in d_ws + d_os + [d_x, d_q]:
            if a_ is not None:
                a_.free()


@pytest.mark.parametrize("seed", [0x5133A000, 0x5133A001, 0x5133A002])
def test_random_projection_calls(ctx, ref, seed):
    rng = np.random.default_rng(seed)
    cus = ctx.info()["cu_count"]
    for case in range(120):
        kind = str(rng.choice(["single", "multi", "quantize_project", "f32"], p=[0.35, 0.25, 0.15, 0.25]))
        if kind == "f32":
            _f32_case(ctx, ref, rng, (seed, case))
        else:
            _q8k_case(ctx, ref, rng, (seed, case), kind, cus)


N_POS = 3000
LAYERS = (3, 7)


def _plan(rng):
    """(kind, sequence, layer, count or keep, bank, gate) steps of one run."""
    plan, length = [], [0, 0]
    for _ in range(int(rng.integers(6, 14))):
        s = int(rng.integers(2))
        layer = LAYERS[int(rng.integers(2))]
        u = rng.random()
        if u < 0.2 and length[s] > 0:
            keep = int(rng.integers(0, length[s] + 1))
            plan.append(("truncate", s, layer, keep, 0, False))
            length[s] = keep
        elif u < 0.45 and length[s] + 8 <= N_POS:
            T = int(rng.integers(1, 6))
            plan.append(("decode", s, layer, T, int(rng.integers(3)), bool(rng.random() < 0.8)))
            length[s] += T
        elif length[s] < N_POS:
            T = int(min(N_POS - length[s], rng.choice([1, 2, 31, 32, 33, 64, 100, 257, 513, 700, 1100])))
            plan.append(("prefill", s, layer, T, int(rng.integers(3)), bool(rng.random() < 0.8)))
            length[s] += T
    return plan


def _run_plan(pkg, ctx, ref, plan, banks, d_banks, Q, G, d_Q, d_G, cached, rng):
    """The plan's calls on a fresh cache; returns the outputs and the
    (max-abs, relative) errors of sampled rows against the restatement."""
    kv = pkg.KVCache(ctx, n_slots=17, max_pages=2 * (N_POS // 16) + 16, max_seqs=2, max_tokens_per_seq=N_POS)
    try:
        kv.set_prefill_cache(cached)
        seqs = [kv.seq_create(), kv.seq_create()]
        length = [0, 0]
        # what the cache holds per (sequence, layer), and how far each is written
        Kc = {(s, l): np.zeros((N_POS, 1024), np.float32) for s in range(2) for l in LAYERS}
        Vc = {(s, l): np.zeros((N_POS, 1024), np.float32) for s in range(2) for l in LAYERS}
        written = {(s, l): 0 for s in range(2) for l in LAYERS}
        got, errs = [], []
        for kind, s, layer, T, b, gate in plan:
            seq = seqs[s]
            if kind == "truncate":
                kv.seq_truncate(seq, T)
                length[s] = T
                for l in LAYERS:
                    written[(s, l)] = min(written[(s, l)], T)
                continue
            base = length[s]
            for l in LAYERS:  # every layer of the sequence holds positions < base
                w0 = written[(s, l)]
                if w0 < base:
                    kv.write(l, seq, w0, base - w0, d_banks[b][0].offset(w0 * 1024), d_banks[b][1].offset(w0 * 1024))
                    Kc[(s, l)][w0:base] = banks[b][0][w0:base]
                    Vc[(s, l)][w0:base] = banks[b][1][w0:base]
                    written[(s, l)] = base
            kd, vd = d_banks[b]
            if kind == "prefill":
                o = ctx.empty((T, 24, 256))
                kv.attn_prefill(layer, seq, base, T, d_Q.offset(base * 6144), kd.offset(base * 1024),
                                vd.offset(base * 1024), o, gate=d_G.offset(base * 6144) if gate else None)
                got.append(o.download())
                o.free()
                rows = sorted({0, T - 1} | set(int(r) for r in rng.integers(0, T, 3)))
            else:
                step = []
                for p in range(base, base + T):
                    o = ctx.empty((24, 256))
                    kv.attn_decode(layer, [seq], [p], d_Q.offset(p * 6144), o, k_new=kd.offset(p * 1024),
                                   v_new=vd.offset(p * 1024), gate=d_G.offset(p * 6144) if gate else None)
                    step.append(o.download())
                    o.free()
                got.append(np.stack(step))
                rows = list(range(T))
            Kc[(s, layer)][base:base + T] = banks[b][0][base:base + T]
            Vc[(s, layer)][base:base + T] = banks[b][1][base:base + T]
            written[(s, layer)] = length[s] = base + T
            for t in rows:
                pos = base + t
                want = ref.attn_heads(Q[pos * 6144:(pos + 1) * 6144], Kc[(s, layer)][:pos + 1],
                                      Vc[(s, layer)][:pos + 1],
                                      gate=G[pos * 6144:(pos + 1) * 6144] if gate else None, threads=16)
                errs.append(abs_rel(got[-1][t], want))
        return got, errs
    finally:
        kv.close()


@pytest.mark.parametrize("seed", [0x5133B000, 0x5133B001])
def test_random_kv_call_sequences(pkg, ctx, ref, synth, margin, seed):
    banks = [(synth.normal(seed + 3 * b + 1, N_POS * 1024).reshape(N_POS, 1024),
              synth.normal(seed + 3 * b + 2, N_POS * 1024).reshape(N_POS, 1024)) for b in range(3)]
    Q = synth.normal(seed + 10, N_POS * 6144)
    G = synth.normal(seed + 11, N_POS * 6144)
    d_banks = [(ctx.array(k), ctx.array(v)) for k, v in banks]
    d_Q, d_G = ctx.array(Q), ctx.array(G)
    worst = (0.0, 0.0)
    try:
        for run in range(16):
            plan = _plan(np.random.default_rng([seed, run]))
            kept, errs = _run_plan(pkg, ctx, ref, plan, banks, d_banks, Q, G, d_Q, d_G, True,
                                   np.random.default_rng([seed, run, 1]))
            whole, _ = _run_plan(pkg, ctx, ref, plan, banks, d_banks, Q, G, d_Q, d_G, False,
                                 np.random.default_rng([seed, run, 1]))
            assert len(kept) == len(whole)
            for i, (a_, b_) in enumerate(zip(kept, whole)):
                assert np.array_equal(a_.view(np.uint32), b_.view(np.uint32)), (seed, run, i, plan)
            for e in errs:
                assert e[0] <= 1e-3 and e[1] <= 1e-3, (seed, run, e, plan)
                worst = tuple(max(x, y) for x, y in zip(worst, e))
    finally:
        for d in [a_ for pair in d_banks for a_ in pair] + [d_Q, d_G]:
            d.free()
    margin("out max-abs (sampled rows, all runs)", worst[0], 1e-3)
    margin("out rel (sampled rows, all runs)", worst[1], 1e-3)


GDN_STATE = 48 * 128 * 128


@pytest.mark.parametrize("seed", [0x5133C000, 0x5133C001, 0x5133C002])
def test_random_linear_core_pieces(ctx, ref, margin, seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 4))
    f32 = lambda *shape, s=1.0: (rng.standard_normal(shape) * s).astype(np.float32)
    conv_w, dt = f32(10240 * 4, s=0.5), f32(48)
    a = -np.abs(f32(48))
    norm = (1.0 + f32(128, s=0.1)).astype(np.float32)
    conv = f32(n, 30720)
    delta = f32(n, GDN_STATE, s=0.02)
    d_w = [ctx.array(x) for x in (conv_w, dt, a, norm)]
    d_conv, d_delta = ctx.array(conv), ctx.array(delta)
    c_ref = [conv[s].copy() for s in range(n)]
    s_ref = [delta[s].copy() for s in range(n)]
    pieces = [int(rng.choice([1, 1, 1, 2, 3, 5, 8, 16, 37, 63, 64, 65, 129, 300, 700])) for _ in range(8)]
    worst = 0.0
    for call, T in enumerate(pieces):
        qkv, z = f32(n, T, 10240), f32(n, T, 6144)
        b, al = f32(n, T, 48), f32(n, T, 48)
        d_in = [ctx.array(x) for x in (qkv, z, b, al)]
        d_out = ctx.empty((n * T, 6144))
        ctx.linear_core(n, T, *d_w, d_conv, d_delta, *d_in, d_out)
        got = d_out.download().reshape(n, T, 6144)
        for d in d_in + [d_out]:
            d.free()
        for s in range(n):
            for t in range(T):
                o = ref.linear_core(conv_w, dt, a, norm, c_ref[s], s_ref[s], qkv[s, t], z[s, t], b[s, t], al[s, t],
                                    threads=16)
                e = float(np.max(np.abs(got[s, t] - o)))
                assert e <= TOL_ABS, (seed, n, pieces, call, s, t, e)
                worst = max(worst, e)
        got_conv = d_conv.download().reshape(n, 30720)
        got_delta = d_delta.download().reshape(n, GDN_STATE)
        for s in range(n):
            assert np.array_equal(got_conv[s], c_ref[s]), (seed, pieces, call, s)
            rel = state_rel(got_delta[s], s_ref[s])
            assert max(rel) <= 1e-4, (seed, n, pieces, call, s, rel)
    for d in d_w + [d_conv, d_delta]:
        d.free()
    margin("out max-abs (every row, every call)", worst, TOL_ABS)
    rel = max(max(state_rel(got_delta[s], s_ref[s])) for s in range(n))
    margin("final state rel (max and Frobenius)", rel, 1e-4)


@pytest.mark.parametrize("seed", [0x5133D000, 0x5133D001, 0x5133D002])
def test_random_graph_replays(pkg, ctx, seed):
    rng = np.random.default_rng(seed)
    n_seq, n_tok, layers = int(rng.integers(1, 4)), 6000, (3, 7)
    gate = bool(rng.random() < 0.7)
    kv = pkg.KVCache(ctx, n_slots=2, max_pages=n_seq * (n_tok // 16 + 8), max_seqs=n_seq,
                     max_tokens_per_seq=n_tok + 64)
    try:
        seqs = [kv.seq_create() for _ in range(n_seq)]
        d_k, d_v = ctx.empty((n_tok, 1024)), ctx.empty((n_tok, 1024))
        for li, layer in enumerate(layers):
            for b, sq in enumerate(seqs):
                ctx.fill_normal(d_k, n_tok * 1024, seed + 16 * li + 2 * b)
                ctx.fill_normal(d_v, n_tok * 1024, seed + 16 * li + 2 * b + 1)
                kv.write(layer, sq, 0, n_tok, d_k, d_v)
        f32 = lambda *shape: ctx.array(rng.standard_normal(shape).astype(np.float32))
        q = {L: f32(n_seq, 6144) for L in layers}
        g = {L: f32(n_seq, 6144) if gate else None for L in layers}
        kn = {L: f32(n_seq, 1024) for L in layers}
        vn = {L: f32(n_seq, 1024) for L in layers}
        out_g = {L: ctx.empty((n_seq, 24, 256)) for L in layers}
        out_p = {L: ctx.empty((n_seq, 24, 256)) for L in layers}
        calls = [{"layer": L, "q": q[L], "k_new": kn[L], "v_new": vn[L], "out": out_g[L],
                  **({"gate": g[L]} if gate else {})} for L in layers]
        draw = lambda: [int(rng.choice([rng.integers(0, 64), rng.integers(0, n_tok + 1)])) for _ in range(n_seq)]
        with kv.decode_graph(seqs, draw(), calls) as graph:
            for rep in range(8):
                pos = draw()
                graph.set_positions(pos)
                graph.launch()
                for L in layers:
                    kv.attn_decode(L, seqs, pos, q[L], out_p[L], k_new=kn[L], v_new=vn[L], gate=g[L])
                for L in layers:
                    got, want = out_g[L].download(), out_p[L].download()
                    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (seed, n_seq, rep, pos, L)
    finally:
        kv.close()


@pytest.mark.parametrize("seed", [0x5133E000, 0x5133E007, 0x5133E009, 0x5133E00E])  # 2-4 sequences, position 0 to 1949
def test_random_full_core_steps(pkg, ctx, ref, margin, seed):
    rng = np.random.default_rng(seed)
    n_seq, ctx_len, layer = int(rng.integers(1, 5)), 2048, 3  # the first full-attention layer: the
    # restatement indexes its caches by full-attention layer ([layer / 4][ctx_len][1024])
    f32 = lambda *shape, s=1.0, m=0.0: (m + rng.standard_normal(shape) * s).astype(np.float32)
    qn, kn = f32(256, s=0.2, m=1.0), f32(256, s=0.2, m=1.0)
    pos = [int(rng.choice([rng.integers(0, 40), rng.integers(0, ctx_len - 8)])) for _ in range(n_seq)]
    kv = pkg.KVCache(ctx, n_slots=17, max_pages=n_seq * ctx_len // 16 + 8, max_seqs=n_seq, max_tokens_per_seq=ctx_len)
    worst = (0.0, 0.0)
    try:
        seqs = [kv.seq_create() for _ in range(n_seq)]
        caches = []
        for sq, p in zip(seqs, pos):
            kc, vc = np.zeros((ctx_len, 1024), np.float32), np.zeros((ctx_len, 1024), np.float32)
            if p:
                kc[:p], vc[:p] = f32(p, 1024), f32(p, 1024)
                d_k0, d_v0 = ctx.array(kc[:p]), ctx.array(vc[:p])
                kv.write(layer, sq, 0, p, d_k0, d_v0)
                d_k0.free()
                d_v0.free()
            caches.append((kc, vc))
        d_qn, d_kn = ctx.array(qn), ctx.array(kn)
        for step in range(4):
            qg, key, val = f32(n_seq, 12288), f32(n_seq, 1024), f32(n_seq, 1024)
            d_in = [ctx.array(x) for x in (qg, key, val)]
            d_o = ctx.empty((n_seq, 24, 256))
            kv.full_core(layer, seqs, pos, d_qn, d_kn, *d_in, d_o)
            got = d_o.download().reshape(n_seq, 6144)
            for d in d_in + [d_o]:
                d.free()
            for b in range(n_seq):
                kc, vc = caches[b]
                want, _ = ref.full_core(qn, kn, qg[b], key[b], val[b], kc, vc, ctx_len, pos[b], layer, threads=16)
                e = abs_rel(got[b], np.asarray(want).reshape(-1))
                assert e[0] <= TOL_ABS and e[1] <= TOL_REL, (seed, n_seq, step, b, pos[b], e)
                worst = tuple(max(x, y) for x, y in zip(worst, e))
            pos = [p + 1 for p in pos]
        d_qn.free()
        d_kn.free()
    finally:
        kv.close()
    margin("out max-abs (every sequence and step)", worst[0], TOL_ABS)
    margin("out rel (every sequence and step)", worst[1], TOL_REL)
