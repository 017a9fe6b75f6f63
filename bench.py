"""Benchmark of the MI355X attention path.

Default workload (the headline metric): one full-attention GQA decode step at
32,768 cached tokens, batch 1, 24 query / 4 kv heads, head_dim 256, f32 KV
cache in 16-token pages, with the new token's K/V appended and the output
gate applied (full_core's attention part, src/model/ops.rs:858-938).  Steps
rotate over the 16 full-attention layers of the model, each with its own
268 MB of K/V, so every step streams its cache from HBM (4.3 GB total, far
above the 256 MB last-level cache).

Prints ONE JSON line.  `value` is decode steps per second over the timed
region (inputs resident in HBM): the timed steps recorded once as a HIP graph
(q38_decode_graph, the replay form of a token's decode calls) and replayed;
the same steps as plain q38_attn_decode calls are reported beside it
(extra.plain_step_us).  `roofline` is for the dominant kernel,
q38_attn_decode_split_one (a decode step is this launch plus the small
q38_attn_decode_merge that combines the split-K partials): algorithmic bytes
per launch (K + V each read once + q) over its mean duration, from start/stop
events stamped by each dispatch on the launch stream in the timed region.
`cpu_baseline` times the oracle's attention (a C restatement of the
reference's) on the same data.

Also measured under "extra" (all, or those --only names): prefill attention
and chunked DeltaNet prefill of a 4096-token prompt, linear_core over that
prompt (with its conv/L2/gates and gated-norm kernels), prefill attention at
512-8192-token prompts and after a prefix, the decode step at 1K to 128K
context, batched paged decode,
the launch floor, one-token linear_core over 48 layers, the 64-layer full
stack at 128K, the bare DeltaNet step for one and for 32 states per launch,
the Q4_K/Q6_K FFN projections for 1 and 8 tokens and for prompts, a decode
layer's projection chain (quantise then project per input, as two calls and
as one) for 1, 8 and 32 tokens, one token and a 4096-token prompt through
one matrix in every Q8_K weight format, the FFN projections' kernel and time
at 1-4096 tokens, the F32/F16/BF16/Q8_0 projection
path at 1, 16 and 4096 tokens, and the recurrent-state checkpoint, each
rotating over enough buffers to defeat the cache where the weights are
streamed.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
import __graft_entry__ as entry  # noqa: E402

HBM_PEAK_GBS = 8000.0
CTX = 32768
LAYERS = [3 + 4 * i for i in range(16)]
KV_BYTES = CTX * 1024 * 4 * 2                 # K + V of one layer: 268,435,456
SPLIT_BYTES = KV_BYTES + 24 * 256 * 4         # + q: bytes the split kernel must read
DECODE_KERNEL = "q38_attn_decode_split_one"   # the split kernel of a one-sequence decode
STEP_BYTES = KV_BYTES + 2 * 24 * 256 * 4      # + q + o: the decode step's unique bytes
COPY_BYTES = 512 << 20
GDN_STATE_BYTES = 48 * 128 * 128 * 4
GDN_STEP_BYTES = 2 * GDN_STATE_BYTES + 4 * (2 * 2048 + 6144 + 2 * 48 + 6144)  # state R+W + q,k,v,beta,g,o


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def attention_decode(pkg, ctx, steps: int, warmup: int):
    kv = pkg.KVCache(ctx, n_slots=16, max_pages=CTX // 16, max_seqs=1, max_tokens_per_seq=CTX)
    seq = kv.seq_create()
    rows_k = ctx.empty((CTX, 1024))
    rows_v = ctx.empty((CTX, 1024))
    for i, layer in enumerate(LAYERS):
        ctx.fill_normal(rows_k, CTX * 1024, 0x51333900 + 2 * i)
        ctx.fill_normal(rows_v, CTX * 1024, 0x51333901 + 2 * i)
        kv.write(layer, seq, 0, CTX, rows_k, rows_v)
    ctx.sync()
    d_q = ctx.empty((24, 256))
    d_g = ctx.empty((24, 256))
    d_o = ctx.empty((24, 256))
    ctx.fill_normal(d_q, 6144, 0x51333990)
    ctx.fill_normal(d_g, 6144, 0x51333991)
    # the new token of every step: row CTX-1 of the last layer's rows
    k_new = rows_k.offset((CTX - 1) * 1024)
    v_new = rows_v.offset((CTX - 1) * 1024)

    def step(i):
        kv.attn_decode(LAYERS[i % 16], [seq], [CTX - 1], d_q, d_o, k_new=k_new, v_new=v_new, gate=d_g)

    for i in range(warmup):
        step(i)
    ctx.sync()
    # plain launches: one q38_attn_decode call per step, bracketed by two
    # stream events (reported beside `value`)
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for i in range(steps):
        step(warmup + i)
    ctx.record(e1)
    ms_plain = ctx.elapsed_ms(e0, e1)
    ctx.sync()
    # the same steps recorded once as a HIP graph (q38_decode_graph: the
    # attention calls of a token, replayed per token) -- `value`.  The
    # per-token update of positions and page ids (q38_decode_graph_set_positions)
    # runs on the host before the timed replay, as a serving loop prepares
    # the next token while the GPU works.
    calls = [{"layer": LAYERS[(warmup + i) % 16], "q": d_q, "k_new": k_new, "v_new": v_new, "gate": d_g,
              "out": d_o} for i in range(steps)]
    graph = kv.decode_graph([seq], [CTX - 1], calls)
    graph.launch()  # untimed: the graph's first replay
    graph.set_positions([CTX - 1])
    ctx.sync()
    e2, e3 = ctx.event(), ctx.event()
    ctx.record(e2)
    graph.launch()
    ctx.record(e3)
    ms_total = ctx.elapsed_ms(e2, e3)
    ctx.sync()
    graph.close()
    # the split kernel's own duration, from the same steps again with each
    # split launch carrying start/stop events (not part of `value`: the
    # per-dispatch events are instrumentation)
    ctx.kernel_timer_start(DECODE_KERNEL, steps)
    for i in range(steps):
        step(warmup + i)
    k_ms, k_n = ctx.kernel_timer_stop()
    ctx.sync()
    # merge-kernel time, from a separate short loop (not part of `value`)
    ctx.kernel_timer_start("q38_attn_decode_merge", 64)
    for i in range(64):
        step(i)
    m_ms, m_n = ctx.kernel_timer_stop()
    # the same steps on one layer's cache only (268 MB against the 256 MB
    # last-level cache: the labelled same-buffer figure, not part of `value`)
    ctx.sync()
    e2, e3 = ctx.event(), ctx.event()
    ctx.record(e2)
    for i in range(100):
        kv.attn_decode(LAYERS[0], [seq], [CTX - 1], d_q, d_o, k_new=k_new, v_new=v_new, gate=d_g)
    ctx.record(e3)
    same_ms = ctx.elapsed_ms(e2, e3) / 100
    ctx.sync()
    last_layer = LAYERS[(warmup + steps - 1) % 16]
    # outputs of the last timed layer, for the parity line of the CPU leg
    step(warmup + steps - 1)
    out = d_o.download()
    res = {
        "ms_per_step": ms_total / steps,
        "plain_ms_per_step": ms_plain / steps,
        "kernel_ms": k_ms / max(k_n, 1),
        "kernel_launches": k_n,
        "merge_ms": m_ms / max(m_n, 1),
        "same_buffer_ms_per_step": same_ms,
        "out": out,
        "layer": last_layer,
        "kv": kv, "seq": seq, "rows": (rows_k, rows_v), "q": d_q, "g": d_g,
    }
    return res


def gdn_steps(pkg, ctx, n_seq: int, n_states: int, steps: int, warmup: int):
    """Gated-DeltaNet decode step over n_seq states per launch, rotating over
    n_states distinct state buffers (so the states stream from HBM)."""
    per = 48 * 128 * 128
    n_groups = n_states // n_seq
    states = ctx.empty((n_groups * n_seq * per,))
    ctx.fill_normal(states, n_groups * n_seq * per, 0x51334000, sigma=0.02)
    from q38amd import synth
    q, k, v, beta, g = synth.GdnStepInputs(0x51334001, n_seq=n_seq).step(0)
    dq, dk, dv, db, dg = (ctx.array(x) for x in (q, k, v, beta, g))
    d_o = ctx.empty((n_seq, 6144))

    def step(i):
        ctx.gdn_step(n_seq, states, dq, dk, dv, db, dg, d_o, state_offset=(i % n_groups) * n_seq * per)

    for i in range(warmup):
        step(i)
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for i in range(steps):
        step(warmup + i)
    ctx.record(e1)
    ms_total = ctx.elapsed_ms(e0, e1)
    ctx.sync()
    ctx.kernel_timer_start("q38_gdn_step_rows", steps)
    for i in range(steps):
        step(warmup + i)
    k_ms, k_n = ctx.kernel_timer_stop()
    states.free()
    kern = k_ms / max(k_n, 1)
    return {
        "n_seq": n_seq,
        "states_rotated": n_groups * n_seq,
        "ms_per_launch": ms_total / steps,
        "kernel_ms": kern,
        "kernel_gb_s": n_seq * GDN_STEP_BYTES / (kern * 1e-3) / 1e9,
        "kernel_frac_hbm": n_seq * GDN_STEP_BYTES / (kern * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "us_per_state_step": kern * 1e3 / n_seq,
    }


def launch_floor(ctx, n: int):
    """An empty kernel: n launches back to back (events around the loop) and
    the same launches with dispatch-stamped events (per-launch kernel time)."""
    for _ in range(16):
        ctx.noop()
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for _ in range(n):
        ctx.noop()
    ctx.record(e1)
    back_to_back = ctx.elapsed_ms(e0, e1) / n
    ctx.kernel_timer_start("q38_noop", n)
    for _ in range(n):
        ctx.noop()
    k_ms, k_n = ctx.kernel_timer_stop()
    return {"us_per_launch_back_to_back": back_to_back * 1e3, "us_event_stamped": k_ms * 1e3 / max(k_n, 1)}


# linear_core, one token: DeltaNet state read + written, conv state read +
# written, raw qkv, conv weights, z and out, gates and norm weight
LINEAR_CORE_BYTES = (2 * GDN_STATE_BYTES + 2 * 10240 * 3 * 4 + 10240 * 4 + 10240 * 4 * 4 + 2 * 6144 * 4
                     + 4 * 48 * 4 + 128 * 4)


def linear_core_decode(pkg, ctx, tokens: int, warmup: int):
    """linear_core for one decode token (conv, gates, recurrence, gated norm:
    one q38_gdn_decode launch) over the 48 DeltaNet layers' states in layer
    order, back to back: time per layer, and the kernel's own duration."""
    per = 48 * 128 * 128
    states = ctx.empty((48 * per,))
    ctx.fill_normal(states, 48 * per, 0x51334b00, sigma=0.02)
    conv = ctx.empty((48 * 30720,))
    ctx.fill_normal(conv, 48 * 30720, 0x51334b01)
    bufs = {}
    for name, m in (("conv_w", 40960), ("dt", 48), ("a", 48), ("norm", 128), ("qkv", 10240), ("z", 6144),
                    ("beta", 48), ("alpha", 48), ("out", 6144)):
        bufs[name] = ctx.empty((m,))
        ctx.fill_normal(bufs[name], m, 0x51334b10 + len(bufs))
    b = bufs

    def token():
        for li in range(48):
            ctx.linear_core(1, 1, b["conv_w"], b["dt"], b["a"], b["norm"], conv.offset(li * 30720),
                            states.offset(li * per), b["qkv"], b["z"], b["beta"], b["alpha"], b["out"])

    for _ in range(warmup):
        token()
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for _ in range(tokens):
        token()
    ctx.record(e1)
    us_layer = ctx.elapsed_ms(e0, e1) * 1e3 / (48 * tokens)
    ctx.kernel_timer_start("q38_gdn_decode", 48 * tokens)
    for _ in range(tokens):
        token()
    k_ms, k_n = ctx.kernel_timer_stop()
    states.free()
    conv.free()
    for v in bufs.values():
        v.free()
    kern_us = k_ms * 1e3 / max(k_n, 1)
    return {"layers": 48, "tokens": tokens, "us_per_layer_back_to_back": us_layer, "kernel_us": kern_us,
            "algorithmic_bytes_per_layer": LINEAR_CORE_BYTES,
            "gb_s_back_to_back": LINEAR_CORE_BYTES / (us_layer * 1e-6) / 1e9,
            "kernel_gb_s": LINEAR_CORE_BYTES / (kern_us * 1e-6) / 1e9,
            "note": "one q38_gdn_decode launch per layer (conv1d, SiLU, L2 norms, gates, recurrence, gated "
                    "RMSNorm); 48 layers' states (151 MB) rotated"}


PREFILL_T = 4096
# causal attention flops of a 4096-token prompt: per (query t, head) (t+1)
# keys x 256 dims x 2 (QK^T) + the same for PV
PREFILL_FLOPS = 24 * 4 * 256 * (PREFILL_T * (PREFILL_T + 1) // 2)
BF16_PEAK_TFLOPS = 2500.0


def prefill_attention(pkg, ctx, reps: int, T: int = PREFILL_T, base: int = 0):
    """Causal prefill attention of a T-token prompt after a base-token prefix
    (batch_full_attention, ops.rs:1153-1172) on the bf16x3 MFMA kernel: kernel
    time per prompt (the attention kernel, plus the merge of split jobs where
    the host cut any; the K/V split apart)."""
    n = base + T
    flops = 24 * 1024 * (T * base + T * (T + 1) // 2)
    kv = pkg.KVCache(ctx, n_slots=1, max_pages=(n + 15) // 16, max_seqs=1, max_tokens_per_seq=n)
    seq = kv.seq_create()
    k, v = ctx.empty((n, 1024)), ctx.empty((n, 1024))
    q, g, o = ctx.empty((T, 24, 256)), ctx.empty((T, 24, 256)), ctx.empty((T, 24, 256))
    for i, (buf, cnt) in enumerate(((k, n * 1024), (v, n * 1024), (q, T * 6144), (g, T * 6144))):
        ctx.fill_normal(buf, cnt, 0x51334200 + i)
    if base:
        kv.write(3, seq, 0, base, k, v)
    k_new, v_new = k.offset(base * 1024), v.offset(base * 1024)

    def run():
        kv.seq_truncate(seq, base)
        kv.attn_prefill(3, seq, base, T, q, k_new, v_new, o, gate=g)

    for _ in range(2):
        run()
    ctx.sync()
    timed = {}
    for name in ("q38_attn_prefill_mfma", "q38_prefill_merge", "q38_kv_split_mfma"):
        ctx.kernel_timer_start(name, reps)
        for _ in range(reps):
            run()
        k_ms, k_n = ctx.kernel_timer_stop()
        timed[name] = k_ms / k_n if k_n else 0.0
    kv.close()
    for b in (k, v, q, g, o):
        b.free()
    ms = timed["q38_attn_prefill_mfma"] + timed["q38_prefill_merge"]
    tflops = flops / (ms * 1e-3) / 1e12
    return {"tokens": T, "prefix": base, "kernel_ms": ms, "merge_ms": timed["q38_prefill_merge"],
            "kv_split_ms": timed["q38_kv_split_mfma"], "algorithmic_gflop": flops / 1e9, "tflop_s": tflops,
            "frac_bf16_peak": tflops / BF16_PEAK_TFLOPS,
            "mfma_tflop_s_executed": 3 * tflops,
            "note": "bf16x3 (hi*hi + hi*lo + lo*hi) MFMA products with f32 accumulation; "
                    "algorithmic flops count each product once"}


def prefill_attention_sweep(pkg, ctx, cases=((0, 512), (0, 1024), (0, 2048), (0, 8192), (8192, 512))):
    """Prefill attention at other (prefix, prompt) lengths (the 4096-token
    prompt is its own entry): kernel (+ merge) and K/V split times,
    algorithmic TFLOP/s."""
    res = {}
    for base, T in cases:
        r = prefill_attention(pkg, ctx, 4 if T > 4096 else 10, T, base)
        res[f"{base}+{T}"] = {k: r[k] for k in ("kernel_ms", "merge_ms", "kv_split_ms", "tflop_s", "frac_bf16_peak")}
    return res


def decode_context_sweep(pkg, ctx, contexts=(1024, 4096, 16384, 65536, 131072), steps: int = 48):
    """The headline's decode step (batch 1, append + gate) at other context
    lengths, rotating over the 16 full-attention layers as the headline does
    (16 x ctx x 8 KiB of K/V: 128 MB at 1K tokens sits in the 256 MB
    last-level cache, as a 16-layer model's whole cache would; from 4K tokens
    on every step streams from HBM).  Per context: step, split and merge
    times and the step's bandwidth."""
    res = {}
    for c in contexts:
        kv = pkg.KVCache(ctx, n_slots=16, max_pages=c // 16, max_seqs=1, max_tokens_per_seq=c)
        seq = kv.seq_create()
        rows_k, rows_v = ctx.empty((c, 1024)), ctx.empty((c, 1024))
        for i, layer in enumerate(LAYERS):
            ctx.fill_normal(rows_k, c * 1024, 0x51333a00 + 2 * i)
            ctx.fill_normal(rows_v, c * 1024, 0x51333a01 + 2 * i)
            kv.write(layer, seq, 0, c, rows_k, rows_v)
        d_q, d_g, d_o = ctx.empty((24, 256)), ctx.empty((24, 256)), ctx.empty((24, 256))
        ctx.fill_normal(d_q, 6144, 0x51333a90)
        ctx.fill_normal(d_g, 6144, 0x51333a91)
        k_new, v_new = rows_k.offset((c - 1) * 1024), rows_v.offset((c - 1) * 1024)

        def step(i):
            kv.attn_decode(LAYERS[i % 16], [seq], [c - 1], d_q, d_o, k_new=k_new, v_new=v_new, gate=d_g)

        for i in range(16):
            step(i)
        ctx.sync()
        e0, e1 = ctx.event(), ctx.event()
        ctx.record(e0)
        for i in range(steps):
            step(i)
        ctx.record(e1)
        step_us = ctx.elapsed_ms(e0, e1) * 1e3 / steps
        timed = {}
        for name in (DECODE_KERNEL, "q38_attn_decode_merge"):
            ctx.kernel_timer_start(name, steps)
            for i in range(steps):
                step(i)
            k_ms, k_n = ctx.kernel_timer_stop()
            timed[name] = k_ms * 1e3 / max(k_n, 1) if k_n else 0.0
        nbytes = c * 8192 + 2 * 24 * 256 * 4
        res[str(c)] = {"step_us": step_us, "split_us": timed[DECODE_KERNEL],
                       "merge_us": timed["q38_attn_decode_merge"], "step_gb_s": nbytes / (step_us * 1e-6) / 1e9,
                       "step_frac_hbm": nbytes / (step_us * 1e-6) / 1e9 / HBM_PEAK_GBS}
        for e in (e0, e1):
            ctx.destroy_event(e)
        for b in (rows_k, rows_v, d_q, d_g, d_o):
            b.free()
        kv.close()
    return res


def batched_decode(pkg, ctx, steps: int, warmup: int):
    """Batched paged decode: 32 sequences, context lengths ~U[1024, 32768]
    (seeded), 16-token pages placed by a random permutation of the pool, one
    decode token per sequence (append + attention + gate)."""
    rng = np.random.default_rng(0x51334300)
    n = 32
    ctxs = rng.integers(1024, 32769, n)
    pages = [(int(c) + 15) // 16 for c in ctxs]
    pool = sum(pages) + 64
    kv = pkg.KVCache(ctx, n_slots=1, max_pages=pool, max_seqs=n, max_tokens_per_seq=32768)
    perm = rng.permutation(pool)
    seqs, at = [], 0
    rows_k, rows_v = ctx.empty((32768, 1024)), ctx.empty((32768, 1024))
    for i in range(n):
        s = kv.seq_create()
        kv.seq_set_pages(s, perm[at:at + pages[i]].tolist())
        at += pages[i]
        c = int(ctxs[i])
        ctx.fill_normal(rows_k, c * 1024, 0x51334310 + 2 * i)
        ctx.fill_normal(rows_v, c * 1024, 0x51334311 + 2 * i)
        kv.write(3, s, 0, c, rows_k, rows_v)
        seqs.append(s)
    q, g, o = ctx.empty((n, 6144)), ctx.empty((n, 6144)), ctx.empty((n, 6144))
    kn, vn = ctx.empty((n, 1024)), ctx.empty((n, 1024))
    for i, (b, m) in enumerate(((q, n * 6144), (g, n * 6144), (kn, n * 1024), (vn, n * 1024))):
        ctx.fill_normal(b, m, 0x51334390 + i)
    positions = [int(c) - 1 for c in ctxs]

    def step():
        kv.attn_decode(3, seqs, positions, q, o, k_new=kn, v_new=vn, gate=g)

    for _ in range(warmup):
        step()
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for _ in range(steps):
        step()
    ctx.record(e1)
    ms = ctx.elapsed_ms(e0, e1) / steps
    ctx.sync()
    # more than 256 splits in the launch: the form that reads every page id
    # from the page table
    ctx.kernel_timer_start("q38_attn_decode_split_many", steps)
    for _ in range(steps):
        step()
    k_ms, k_n = ctx.kernel_timer_stop()
    kv.close()
    for b in (rows_k, rows_v, q, g, o, kn, vn):
        b.free()
    total = int(ctxs.sum())
    alg = total * 8192 + n * 2 * 6144 * 4
    kern = k_ms / max(k_n, 1)
    return {"sequences": n, "total_context_tokens": total, "algorithmic_bytes": alg,
            "step_ms": ms, "split_kernel_ms": kern,
            "step_gb_s": alg / (ms * 1e-3) / 1e9, "step_frac_hbm": alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "split_kernel_gb_s": alg / (kern * 1e-3) / 1e9,
            "split_kernel_frac_hbm": alg / (kern * 1e-3) / 1e9 / HBM_PEAK_GBS}


def full_stack(pkg, ctx, tokens: int, warmup: int):
    """One decode token through the attention path of all 64 layers of the
    hybrid (layer % 4 == 3 full attention, the other 48 Gated DeltaNet),
    batch 1, 131072 cached tokens: full_core (norms, RoPE, append, attention,
    gate) and linear_core (conv, gates, recurrence, gated norm) per layer, in
    layer order.  Projections are outside the path and not run."""
    CTXF = 131072
    pos = CTXF - 1
    kv = pkg.KVCache(ctx, n_slots=16, max_pages=CTXF // 16, max_seqs=1, max_tokens_per_seq=CTXF)
    seq = kv.seq_create()
    rows_k, rows_v = ctx.empty((CTXF, 1024)), ctx.empty((CTXF, 1024))
    full_layers = [l for l in range(64) if (l + 1) % 4 == 0]
    lin_layers = [l for l in range(64) if (l + 1) % 4 != 0]
    for i, layer in enumerate(full_layers):
        ctx.fill_normal(rows_k, CTXF * 1024, 0x51334400 + 2 * i)
        ctx.fill_normal(rows_v, CTXF * 1024, 0x51334401 + 2 * i)
        kv.write(layer, seq, 0, pos, rows_k, rows_v)
    rows_k.free()
    rows_v.free()
    per = 48 * 128 * 128
    states = ctx.empty((48 * per,))
    ctx.fill_normal(states, 48 * per, 0x51334480, sigma=0.02)
    conv = ctx.empty((48 * 30720,))
    ctx.fill_normal(conv, 48 * 30720, 0x51334481)
    bufs = {}
    for name, m in (("qn", 256), ("kn", 256), ("qg", 12288), ("key", 1024), ("val", 1024), ("conv_w", 40960),
                    ("dt", 48), ("a", 48), ("norm", 128), ("qkv", 10240), ("z", 6144), ("beta", 48),
                    ("alpha", 48), ("out_a", 6144), ("out_l", 6144)):
        bufs[name] = ctx.empty((m,))
        ctx.fill_normal(bufs[name], m, 0x51334490 + len(bufs))
    b = bufs

    def token():
        li = 0
        for layer in range(64):
            if (layer + 1) % 4 == 0:
                kv.full_core(layer, [seq], [pos], b["qn"], b["kn"], b["qg"], b["key"], b["val"], b["out_a"])
            else:
                ctx.linear_core(1, 1, b["conv_w"], b["dt"], b["a"], b["norm"], conv.offset(li * 30720),
                                states.offset(li * per), b["qkv"], b["z"], b["beta"], b["alpha"], b["out_l"])
                li += 1

    for _ in range(warmup):
        token()
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for _ in range(tokens):
        token()
    ctx.record(e1)
    ms_plain = ctx.elapsed_ms(e0, e1) / tokens
    ctx.sync()
    # the same token recorded once as a HIP graph (q38_decode_graph: 48
    # linear_core steps and 16 full_core calls in layer order) and replayed
    # per token, its positions set on the host before each replay
    graph = kv.decode_graph([seq], [pos])
    li = 0
    for layer in range(64):
        if (layer + 1) % 4 == 0:
            graph.add_decode({"layer": layer, "q": b["qg"], "k_new": b["key"], "v_new": b["val"], "q_norm": b["qn"],
                              "k_norm": b["kn"], "out": b["out_a"]})
        else:
            graph.add_linear_core(1, b["conv_w"], b["dt"], b["a"], b["norm"], conv.offset(li * 30720),
                                  states.offset(li * per), b["qkv"], b["z"], b["beta"], b["alpha"], b["out_l"])
            li += 1
    graph.end()
    graph.launch()  # untimed first replay
    g_ms = []
    for _ in range(tokens):
        graph.set_positions([pos])
        e2, e3 = ctx.event(), ctx.event()
        ctx.record(e2)
        graph.launch()
        ctx.record(e3)
        g_ms.append(ctx.elapsed_ms(e2, e3))
        for e in (e2, e3):
            ctx.destroy_event(e)
    graph.close()
    ms = sum(g_ms) / len(g_ms)
    kv.close()
    states.free()
    conv.free()
    for v in bufs.values():
        v.free()
    alg = 16 * CTXF * 8192 + 48 * 2 * per * 4
    return {"layers": 64, "full_attention_layers": len(full_layers), "deltanet_layers": len(lin_layers),
            "context": CTXF, "ms_per_token": ms, "tokens_per_s": 1e3 / ms, "algorithmic_bytes": alg,
            "gb_s": alg / (ms * 1e-3) / 1e9, "frac_hbm": alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "plain_ms_per_token": ms_plain, "plain_frac_hbm": alg / (ms_plain * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "note": "ms_per_token: the token replayed from one HIP graph (q38_decode_graph, 64 steps), "
                    "positions set before each replay; plain_ms_per_token: the same calls as plain launches"}


# chunked Gated-DeltaNet flops per (value head, 64-token chunk): KK^T, QK^T,
# W = T(bgK), U' = T(bV) (4 x 64*64*128*2), the triangular inverse (~64^3/3*2),
# and the state products W S^T, Q S^T, U^T K (3 x 64*128*128*2) and Bm U
GDN_CHUNK_FLOPS = 4 * 64 * 64 * 128 * 2 + (64 ** 3 // 3) * 2 + 3 * 64 * 128 * 128 * 2 + 64 * 64 * 128 * 2


def gdn_prefill(pkg, ctx, reps: int):
    """Chunked Gated-DeltaNet prefill of a 4096-token prompt (one layer, 48
    value heads, 64-token chunks on bf16x3 MFMA): prep + scan time per prompt."""
    from q38amd import synth
    T = PREFILL_T
    per = 48 * 128 * 128
    state = ctx.empty((per,))
    q, k, v, beta, g = synth.GdnStepInputs(0x51334a00).steps(0, T)
    dq, dk, dv, db, dg = (ctx.array(x) for x in (q, k, v, beta, g))
    out = ctx.empty((T, 6144))
    ctx.fill_normal(state, per, 0x51334a01, sigma=0.02)
    ctx.gdn_prefill(state, T, dq, dk, dv, db, dg, out)
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for _ in range(reps):
        ctx.gdn_prefill(state, T, dq, dk, dv, db, dg, out)
    ctx.record(e1)
    ms = ctx.elapsed_ms(e0, e1) / reps
    for b in (state, dq, dk, dv, db, dg, out):
        b.free()
    flops = GDN_CHUNK_FLOPS * 48 * (T // 64)
    tflops = flops / (ms * 1e-3) / 1e12
    return {"tokens": T, "ms": ms, "algorithmic_gflop": flops / 1e9, "tflop_s": tflops,
            "frac_bf16_peak": tflops / BF16_PEAK_TFLOPS,
            "note": "prep (KK^T, QK^T, triangular inverse, W, U') and scan (state products) kernels, "
                    "bf16x3 MFMA products"}


# linear_core over a prompt, per token: the conv/SiLU/L2/gates kernel reads
# the raw qkv row (40,960 B) and the two raw gates (384 B) and writes the
# same again; the gated RMSNorm reads o and z (2 x 24,576 B) and writes the
# output (24,576 B)
LC_PRE_BYTES_PER_TOKEN = 2 * (10240 * 4 + 2 * 48 * 4)
LC_POST_BYTES_PER_TOKEN = 3 * 6144 * 4


def linear_core_prefill(pkg, ctx, reps: int):
    """linear_core over a 4096-token prompt of one layer (conv, SiLU, L2
    norms and gates; the chunked recurrence; the gated RMSNorm): time per
    call, and the two elementwise kernels' durations and bandwidth."""
    T = PREFILL_T
    sizes = {"conv_w": 10240 * 4, "dt": 48, "a": 48, "norm": 128}
    w = {k: ctx.empty((n,)) for k, n in sizes.items()}
    for i, (k, buf) in enumerate(w.items()):
        ctx.fill_normal(buf, sizes[k], 0x51334c00 + i, sigma=0.1)
    conv, delta = ctx.empty((30720,)), ctx.empty((48 * 128 * 128,))
    ctx.fill_normal(conv, 30720, 0x51334c10)
    ctx.fill_normal(delta, 48 * 128 * 128, 0x51334c11, sigma=0.02)
    ins = [ctx.empty((T * n,)) for n in (10240, 6144, 48, 48)]
    for i, (buf, n) in enumerate(zip(ins, (10240, 6144, 48, 48))):
        ctx.fill_normal(buf, T * n, 0x51334c20 + i)
    out = ctx.empty((T * 6144,))

    def call():
        ctx.linear_core(1, T, w["conv_w"], w["dt"], w["a"], w["norm"], conv, delta, *ins, out)

    call()
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for _ in range(reps):
        call()
    ctx.record(e1)
    ms = ctx.elapsed_ms(e0, e1) / reps
    res = {"tokens": T, "ms": ms}
    for name, per_token in (("q38_gdn_pre", LC_PRE_BYTES_PER_TOKEN), ("q38_gdn_post", LC_POST_BYTES_PER_TOKEN)):
        ctx.kernel_timer_start(name, reps)
        for _ in range(reps):
            call()
        k_ms, k_n = ctx.kernel_timer_stop()
        us = k_ms * 1e3 / max(k_n, 1)
        res[name] = {"us": us, "algorithmic_bytes": per_token * T,
                     "gb_s": per_token * T / (us * 1e-6) / 1e9}
    for b in (conv, delta, out, *ins, *w.values()):
        b.free()
    return res


FFN_MATS = ((12, 17408, 5120, "gate"), (12, 17408, 5120, "up"), (14, 5120, 17408, "down"))
QUANT_BLOCK_BYTES = {12: 144, 13: 176, 14: 210, 10: 84, 11: 110, 20: 144, 23: 136, 16: 66, 17: 74, 22: 82, 18: 98,
                     21: 110, 19: 50, 29: 56}
GEMV_KERNELS = {12: "q38_gemv_q8k_q4k", 13: "q38_gemv_q8k_q5k", 14: "q38_gemv_q8k_q6k", 10: "q38_gemv_q8k_q2k",
                11: "q38_gemv_q8k_q3k", 20: "q38_gemv_q8k_iq4nl", 23: "q38_gemv_q8k_iq4xs",
                16: "q38_gemv_q8k_iq2xxs", 17: "q38_gemv_q8k_iq2xs", 22: "q38_gemv_q8k_iq2s",
                18: "q38_gemv_q8k_iq3xxs", 21: "q38_gemv_q8k_iq3s", 19: "q38_gemv_q8k_iq1s", 29: "q38_gemv_q8k_iq1m"}
FORMAT_NAMES = {12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 10: "Q2_K", 11: "Q3_K", 20: "IQ4_NL", 23: "IQ4_XS", 16: "IQ2_XXS",
                17: "IQ2_XS", 22: "IQ2_S", 18: "IQ3_XXS", 21: "IQ3_S", 19: "IQ1_S", 29: "IQ1_M"}


def gemv_bytes(ty: int, rows: int, width: int, n_tokens: int) -> int:
    """Algorithmic bytes of one projection launch: the weight rows once, the
    Q8_K activations (292 bytes per 256 values per token) and the f32 outputs."""
    return rows * (width // 256) * QUANT_BLOCK_BYTES[ty] + n_tokens * (width // 256) * 292 + n_tokens * rows * 4


def _graph_replay_us(ctx, work, reps: int):
    """Capture work() from the context's stream into a HIP graph, replay it
    reps times and return the microseconds per replay (None when the HIP
    runtime's graph calls are not available)."""
    import ctypes
    try:
        hip = ctypes.CDLL(os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib", "libamdhip64.so"))
    except OSError:
        return None
    hip.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_size_t]
    hip.hipGraphLaunch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipGraphExecDestroy.argtypes = [ctypes.c_void_p]
    hip.hipGraphDestroy.argtypes = [ctypes.c_void_p]
    stream = ctx.stream()
    ctx.sync()
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipStreamBeginCapture(stream, 2) != 0:  # relaxed capture mode
        return None
    work()
    if hip.hipStreamEndCapture(stream, ctypes.byref(graph)) != 0:
        return None
    try:
        if hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) != 0:
            return None
        hip.hipGraphLaunch(exe, stream)  # untimed first replay
        ctx.sync()
        e0, e1 = ctx.event(), ctx.event()
        ctx.record(e0)
        for _ in range(reps):
            hip.hipGraphLaunch(exe, stream)
        ctx.record(e1)
        us = ctx.elapsed_ms(e0, e1) * 1e3 / reps
        ctx.sync()
        for e in (e0, e1):
            ctx.destroy_event(e)
        return us
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)


def layer_projections(pkg, ctx, n_tokens: int, reps: int, layers: int = 4):
    """The projections of `layers` attention-layer decode steps in order, each
    input quantised then projected (ops.rs:617-639): x -> q|gate 12288, k
    1024, v 1024 rows; the attention output (6144) -> o 5120 rows; x -> gate
    and up 17408 rows; the FFN activation (17408) -> down 5120 rows (Q4_K,
    the down projection Q6_K; 232 MB a layer, 929 MB for 4).  Two forms of
    the same chain, bit-identical outputs: q38_quantize_q8_k then
    q38_gemv_q8_k_multi per input (8 launches a layer), and
    q38_quantize_project_q8_k (4 launches a layer); microseconds per layer,
    as plain launches and replayed from a captured HIP graph."""
    mats = []
    for li in range(layers):
        lm = []
        for ty, rows_list, width in ((12, [12288, 1024, 1024], 5120), (12, [5120], 6144), (12, [17408, 17408], 5120),
                                     (14, [5120], 17408)):
            ws = []
            for mi, rows in enumerate(rows_list):
                nbytes = rows * (width // 256) * QUANT_BLOCK_BYTES[ty]
                w = ctx.empty((nbytes,), np.uint8)
                ctx.fill_normal(w, nbytes // 4, 0x51335400 + 16 * li + 4 * mi + ty)
                ws.append(w)
            lm.append((ty, rows_list, width, ws))
        mats.append(lm)
    xs = {}
    for width in (5120, 6144, 17408):
        x = ctx.empty((n_tokens, width))
        ctx.fill_normal(x, n_tokens * width, 0x51335500 + width)
        xs[width] = (x, ctx.empty((ctx.q8k_bytes(n_tokens, width),), np.uint8))
    outs = [ctx.empty((n_tokens, 17408)) for _ in range(3)]

    def chain(fused):
        for lm in mats:
            for ty, rows_list, width, ws in lm:
                x, q = xs[width]
                o = outs[:len(rows_list)]
                if fused:
                    ctx.quantize_project_q8_k(ty, rows_list, width, ws, x, n_tokens, q, o)
                else:
                    ctx.quantize_q8_k(n_tokens, width, x, q)
                    ctx.gemv_q8_k_multi(ty, rows_list, width, ws, q, n_tokens, o)

    res = {"tokens": n_tokens, "layers": layers}
    e0, e1 = ctx.event(), ctx.event()
    for label, fused in (("separate", False), ("fused", True)):
        chain(fused)
        ctx.sync()
        ctx.record(e0)
        for _ in range(reps):
            chain(fused)
        ctx.record(e1)
        res[f"{label}_us_per_layer"] = ctx.elapsed_ms(e0, e1) * 1e3 / (reps * layers)
        g_us = _graph_replay_us(ctx, lambda: chain(fused), reps)
        if g_us is not None:
            res[f"{label}_graph_us_per_layer"] = g_us / layers
    for lm in mats:
        for _, _, _, ws in lm:
            for w in ws:
                w.free()
    for x, q in xs.values():
        x.free()
        q.free()
    for o in outs:
        o.free()
    return res


def ffn_projections(pkg, ctx, n_tokens: int, reps: int, layers: int = 4):
    """The FFN projections of `layers` layers (gate and up 17408x5120 Q4_K,
    down 5120x17408 Q6_K; 173 MB a layer, 693 MB for 4, beyond the 256 MB
    last-level cache) for n_tokens tokens, in layer order: per-kernel duration
    and bandwidth of q38_gemv_q8_k.  Weights are random bytes."""
    mats = []
    for li in range(layers):
        for ty, rows, width, name in FFN_MATS:
            nbytes = rows * (width // 256) * QUANT_BLOCK_BYTES[ty]
            w = ctx.empty((nbytes,), np.uint8)
            ctx.fill_normal(w, nbytes // 4, 0x51335000 + 8 * li + ty)
            mats.append((ty, rows, width, w))
    x5 = ctx.empty((n_tokens, 5120))
    ctx.fill_normal(x5, n_tokens * 5120, 0x51335100)
    x17 = ctx.empty((n_tokens, 17408))
    ctx.fill_normal(x17, n_tokens * 17408, 0x51335101)
    q5 = ctx.empty((ctx.q8k_bytes(n_tokens, 5120),), np.uint8)
    q17 = ctx.empty((ctx.q8k_bytes(n_tokens, 17408),), np.uint8)
    ctx.quantize_q8_k(n_tokens, 5120, x5, q5)
    ctx.quantize_q8_k(n_tokens, 17408, x17, q17)
    out = ctx.empty((n_tokens, 17408))

    def sweep():
        for ty, rows, width, w in mats:
            ctx.gemv_q8_k(ty, rows, width, w, q5 if width == 5120 else q17, n_tokens, out)

    sweep()
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for _ in range(reps):
        sweep()
    ctx.record(e1)
    sweep_us = ctx.elapsed_ms(e0, e1) * 1e3 / reps
    total_bytes = sum(gemv_bytes(ty, rows, width, n_tokens) for ty, rows, width, _ in mats)
    res = {"tokens": n_tokens, "layers": layers, "sweep_us": sweep_us,
           "sweep_gb_s": total_bytes / (sweep_us * 1e-6) / 1e9}
    # gate and up of a layer read the same input: one q38_gemv_q8_k_multi
    # launch for the pair, then down
    out2 = ctx.empty((n_tokens, 17408))

    def sweep_fused():
        for li in range(layers):
            g, u, d = mats[3 * li: 3 * li + 3]
            ctx.gemv_q8_k_multi(12, [17408, 17408], 5120, [g[3], u[3]], q5, n_tokens, [out, out2])
            ctx.gemv_q8_k(d[0], d[1], d[2], d[3], q17, n_tokens, out)

    sweep_fused()
    ctx.sync()
    ctx.record(e0)
    for _ in range(reps):
        sweep_fused()
    ctx.record(e1)
    fused_us = ctx.elapsed_ms(e0, e1) * 1e3 / reps
    res["fused_gate_up_sweep_us"] = fused_us
    res["fused_gate_up_sweep_gb_s"] = total_bytes / (fused_us * 1e-6) / 1e9
    # the same sweep captured from the context's stream into one HIP graph and
    # replayed, as a token graph replays a layer's projections
    g_us = _graph_replay_us(ctx, sweep_fused, reps)
    if g_us is not None:
        res["fused_gate_up_sweep_graph_us"] = g_us
        res["fused_gate_up_sweep_graph_gb_s"] = total_bytes / (g_us * 1e-6) / 1e9
    kern, k_ms, k_n = _timed_q8k_kernel(ctx, 12, sweep_fused, reps, reps * layers)
    us = k_ms * 1e3 / k_n
    b = 2 * gemv_bytes(12, 17408, 5120, n_tokens)
    res["q4k_gate_up_2x17408x5120"] = {"kernel": kern, "kernel_us": us, "launches": k_n, "algorithmic_bytes": b,
                                       "gb_s": b / (us * 1e-6) / 1e9,
                                       "frac_hbm": b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}
    out2.free()
    for ty, label in ((12, "q4k_17408x5120"), (14, "q6k_5120x17408")):
        kern, k_ms, k_n = _timed_q8k_kernel(ctx, ty, sweep, reps, reps * 3 * layers)
        us = k_ms * 1e3 / k_n
        rows, width = (17408, 5120) if ty == 12 else (5120, 17408)
        b = gemv_bytes(ty, rows, width, n_tokens)
        res[label] = {"kernel": kern, "kernel_us": us, "launches": k_n, "algorithmic_bytes": b,
                      "gb_s": b / (us * 1e-6) / 1e9, "frac_hbm": b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}
    for *_, w in mats:
        w.free()
    for a in (x5, x17, q5, q17, out):
        a.free()
    for e in (e0, e1):
        ctx.destroy_event(e)
    return res


def weight_formats(pkg, ctx, reps: int):
    """One token through a 17408 x 5120 matrix (the FFN gate's shape) in every
    Q8_K weight format: q38_gemv_q8_k's kernel duration and bandwidth, the
    weights rotated over copies totalling >= 512 MB (beyond the last-level
    cache).  Weights are random bytes (timing only)."""
    rows, width = 17408, 5120
    x = ctx.empty((1, width))
    ctx.fill_normal(x, width, 0x51335200)
    q = ctx.empty((ctx.q8k_bytes(1, width),), np.uint8)
    ctx.quantize_q8_k(1, width, x, q)
    out = ctx.empty((1, rows))
    res = {}
    for ty in (10, 11, 12, 13, 14, 20, 23, 16, 17, 22, 18, 21, 19, 29):
        nbytes = rows * (width // 256) * QUANT_BLOCK_BYTES[ty]
        copies = -(-512 * 2**20 // nbytes)
        ws = []
        for c in range(copies):
            w = ctx.empty((nbytes,), np.uint8)
            ctx.fill_normal(w, nbytes // 4, 0x51335210 + 64 * ty + c)
            ws.append(w)
        for w in ws:
            ctx.gemv_q8_k(ty, rows, width, w, q, 1, out)
        ctx.sync()
        ctx.kernel_timer_start(GEMV_KERNELS[ty], reps * copies)
        for _ in range(reps):
            for w in ws:
                ctx.gemv_q8_k(ty, rows, width, w, q, 1, out)
        k_ms, k_n = ctx.kernel_timer_stop()
        us = k_ms * 1e3 / max(k_n, 1)
        b = gemv_bytes(ty, rows, width, 1)
        res[FORMAT_NAMES[ty]] = {"kernel_us": round(us, 2), "weight_mb": round(nbytes / 1e6, 1),
                                 "gb_s": round(b / (us * 1e-6) / 1e9, 1),
                                 "frac_hbm": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 3)}
        for w in ws:
            w.free()
    for a in (x, q, out):
        a.free()
    return res


def weight_formats_prompt(pkg, ctx, n_tokens: int, reps: int):
    """A prompt of n_tokens tokens through a 17408 x 5120 matrix in every Q8_K
    weight format on the int8 matrix unit: kernel duration and useful int8
    operations per second.  Weights are random
    bytes (timing only)."""
    rows, width = 17408, 5120
    x = ctx.empty((n_tokens, width))
    ctx.fill_normal(x, n_tokens * width, 0x51335300)
    q = ctx.empty((ctx.q8k_bytes(n_tokens, width),), np.uint8)
    ctx.quantize_q8_k(n_tokens, width, x, q)
    out = ctx.empty((n_tokens, rows))
    res = {}
    for ty in (12, 13, 14, 10, 11, 23, 20, 16, 17, 22, 18, 21, 19, 29):
        nbytes = rows * (width // 256) * QUANT_BLOCK_BYTES[ty]
        w = ctx.empty((nbytes,), np.uint8)
        ctx.fill_normal(w, nbytes // 4, 0x51335310 + ty)
        ctx.gemv_q8_k(ty, rows, width, w, q, n_tokens, out)
        ctx.sync()
        kern, ms = _timed_projection(ctx, ty, rows, width, w, q, n_tokens, out, reps)
        tops = 2.0 * rows * width * n_tokens / (ms * 1e-3) / 1e12
        res[FORMAT_NAMES[ty]] = {"kernel": kern, "ms": round(ms, 3), "int8_tops": round(tops, 1),
                                 "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        w.free()
    for a in (x, q, out):
        a.free()
    return res


INT8_PEAK_TOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
F32_PATH_TYPES = {0: ("F32", 4.0), 1: ("F16", 2.0), 30: ("BF16", 2.0), 8: ("Q8_0", 34.0 / 32.0)}


def _f32_path_kernels(ty: int) -> list:
    """The kernels q38_gemv_f32 may launch for weight type ty."""
    sfx = F32_PATH_TYPES[ty][0].lower()
    kerns = ["q38_gemm_f32_" + sfx, "q38_gemm_f32s_" + sfx] + (["q38_gemm_f32w_" + sfx] if ty != 0 else [])
    if ty == 8:
        return kerns + ["q38_gemv_f32_q8_0s_r2_t1", "q38_gemv_f32_q8_0s_r2_t2", "q38_gemv_f32_q8_0s_r2_t4",
                        "q38_gemv_f32_q8_0s_r4_t8"]
    return kerns + ["q38_gemv_f32_" + sfx]


def f32_path(pkg, ctx, reps: int):
    """The projection path of weights project() does not quantise for
    (q38_gemv_f32: F32, F16, BF16, Q8_0) through 17408 x 5120 at 1, 16 and
    4096 tokens and the 48-row beta / alpha shape (48 x 5120) at 4096: kernel
    duration, the kernel the library chose (the GEMV for few tokens, the
    bf16 matrix unit's split-k or 128 x 64 form), weight bytes per second and useful f32
    operations per second (2 x rows x width x tokens; the matrix unit runs 3,
    5 or 6 bf16 products per multiply for BF16/Q8_0, F16, F32 weights).
    Weights are random bytes (timing only)."""
    res = {}
    for rows, width, n_tokens in ((17408, 5120, 1), (17408, 5120, 16), (17408, 5120, 4096), (48, 5120, 4096)):
        x = ctx.empty((n_tokens, width))
        ctx.fill_normal(x, n_tokens * width, 0x51335600 + n_tokens)
        out = ctx.empty((n_tokens, rows))
        for ty, (name, bpw) in F32_PATH_TYPES.items():
            nbytes = int(rows * width * bpw)
            w = ctx.empty((nbytes + 16,), np.uint8)
            ctx.fill_normal(w, (nbytes + 16) // 4, 0x51335610 + ty, sigma=0.05)
            ctx.gemv_f32(ty, rows, width, w, x, n_tokens, out)
            ctx.sync()
            for kern in _f32_path_kernels(ty):
                ctx.kernel_timer_start(kern, reps)
                for _ in range(reps):
                    ctx.gemv_f32(ty, rows, width, w, x, n_tokens, out)
                k_ms, k_n = ctx.kernel_timer_stop()
                if k_n > 0:
                    break
            ms = k_ms / reps
            res[f"{name}_{rows}x{width}_T{n_tokens}"] = {
                "kernel": kern, "ms": round(ms, 4), "weights_gb_s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                "tflop_s": round(2.0 * rows * width * n_tokens / (ms * 1e-3) / 1e12, 2)}
            w.free()
        x.free()
        out.free()
    return res


def _q8k_kernels(ty: int) -> tuple:
    """The kernels q38_gemv_q8_k may launch for weight type ty: the
    split-block matrix-unit forms (16, 8, 4 waves), the 128 x 64 one, the
    GEMV (IQ4_NL: the last two)."""
    gemv = GEMV_KERNELS[ty]
    kernels = (gemv.replace("q38_gemv_q8k_", "q38_gemm_ks16_q8k_"), gemv.replace("q38_gemv_q8k_", "q38_gemm_ks_q8k_"),
               gemv.replace("q38_gemv_q8k_", "q38_gemm_ks4_q8k_"), gemv.replace("gemv", "gemm"), gemv)
    return kernels if ty != 20 else kernels[3:]


def _timed_q8k_kernel(ctx, ty, work, reps, max_launches):
    """(kernel, total ms, launches) of the weight-type-ty projection kernel
    that reps calls of work() launch (the first of _q8k_kernels(ty) that
    runs)."""
    for kern in _q8k_kernels(ty):
        ctx.kernel_timer_start(kern, max_launches)
        for _ in range(reps):
            work()
        k_ms, k_n = ctx.kernel_timer_stop()
        if k_n > 0:
            return kern, k_ms, k_n
    raise RuntimeError(f"no projection kernel of type {ty} was launched")


def _timed_projection(ctx, ty, rows, width, w, q, n_tokens, out, reps):
    """Kernel time per call of one projection and the kernel that ran it:
    the split-block matrix-unit form (16, 8 or 4 waves), the 128 x 64 one or
    the GEMV, as the library chose for the shape."""
    kern, k_ms, _ = _timed_q8k_kernel(ctx, ty, lambda: ctx.gemv_q8_k(ty, rows, width, w, q, n_tokens, out), reps,
                                      reps * 64)
    return kern, k_ms / reps


def projection_sweep(pkg, ctx, reps: int):
    """The FFN gate (17408 x 5120 Q4_K) and down (5120 x 17408 Q6_K)
    projections at 1 to 4096 tokens: the kernel q38_gemv_q8_k chose (GEMV,
    split-block matrix-unit form of 16 / 8 / 4 waves, 128 x 64 tiles), its
    duration and its rate in weight bytes and int8 operations.  One matrix,
    reused (cache-resident below ~200 MB); random weights (timing only)."""
    res = {}
    for ty, rows, width, label in ((12, 17408, 5120, "q4k_17408x5120"), (14, 5120, 17408, "q6k_5120x17408")):
        nbytes = rows * (width // 256) * QUANT_BLOCK_BYTES[ty]
        w = ctx.empty((nbytes,), np.uint8)
        ctx.fill_normal(w, nbytes // 4, 0x51335700 + ty)
        per = {}
        for n_tokens in (1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 4096):
            x = ctx.empty((n_tokens, width))
            ctx.fill_normal(x, n_tokens * width, 0x51335710 + n_tokens)
            q = ctx.empty((ctx.q8k_bytes(n_tokens, width),), np.uint8)
            ctx.quantize_q8_k(n_tokens, width, x, q)
            out = ctx.empty((n_tokens, rows))
            ctx.gemv_q8_k(ty, rows, width, w, q, n_tokens, out)
            ctx.sync()
            kern, ms = _timed_projection(ctx, ty, rows, width, w, q, n_tokens, out, reps)
            per[n_tokens] = {"kernel": kern, "us": round(ms * 1e3, 2),
                             "weights_gb_s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                             "int8_tops": round(2.0 * rows * width * n_tokens / (ms * 1e-3) / 1e12, 1)}
            for a in (x, q, out):
                a.free()
        res[label] = per
        w.free()
    return res


def prompt_projections(pkg, ctx, n_tokens: int, reps: int):
    """The FFN projections of one layer for a prompt of n_tokens (gate
    17408 x 5120 Q4_K, down 5120 x 17408 Q6_K; the int8 matrix-unit form
    from 8 tokens on): kernel time and int8 operations per second
    (2 x rows x width x tokens; the K-quant expansion and the block terms
    are not counted)."""
    res = {"tokens": n_tokens}
    for ty, rows, width, label in ((12, 17408, 5120, "q4k_17408x5120"), (14, 5120, 17408, "q6k_5120x17408")):
        nbytes = rows * (width // 256) * QUANT_BLOCK_BYTES[ty]
        w = ctx.empty((nbytes,), np.uint8)
        ctx.fill_normal(w, nbytes // 4, 0x51335200 + ty)
        x = ctx.empty((n_tokens, width))
        ctx.fill_normal(x, n_tokens * width, 0x51335201)
        q = ctx.empty((ctx.q8k_bytes(n_tokens, width),), np.uint8)
        ctx.quantize_q8_k(n_tokens, width, x, q)
        out = ctx.empty((n_tokens, rows))
        ctx.gemv_q8_k(ty, rows, width, w, q, n_tokens, out)
        ctx.sync()
        kern, ms = _timed_projection(ctx, ty, rows, width, w, q, n_tokens, out, reps)
        ops = 2.0 * rows * width * n_tokens
        res[label] = {"kernel": kern, "ms": ms, "int8_tops": ops / (ms * 1e-3) / 1e12,
                      "frac_int8_peak": ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS}
        for arr in (w, x, q, out):
            arr.free()
    return res


def recurrent_checkpoint(pkg, ctx, reps: int):
    """checkpoint_state's device form: conv_state (5.9 MB) and delta_state
    (151 MB) of a sequence copied to the checkpoint; each copy reads and
    writes its bytes once."""
    n_conv, n_delta = 48 * 30720, 48 * 786432
    bufs = [ctx.empty((n,)) for n in (n_conv, n_delta, n_conv, n_delta)]
    pkg.recurrent_checkpoint(ctx, bufs[0], bufs[1], n_conv, n_delta, bufs[2], bufs[3])
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    for _ in range(reps):
        pkg.recurrent_checkpoint(ctx, bufs[0], bufs[1], n_conv, n_delta, bufs[2], bufs[3])
    ctx.record(e1)
    us = ctx.elapsed_ms(e0, e1) * 1e3 / reps
    for b in bufs:
        b.free()
    for e in (e0, e1):
        ctx.destroy_event(e)
    moved = 2 * 4 * (n_conv + n_delta)
    return {"us": us, "bytes_read_and_written": moved, "gb_s": moved / (us * 1e-6) / 1e9}


def cpu_baseline(ref, q, k_rows, v_rows, gate, budget_s: float, threads: int = 0):
    """The CPU restatement of the reference's attention (ops.rs:868-938) on the
    32K workload, all cores of this host (heads split across threads as the
    reference's rayon dispatch does), or `threads` of them: decode steps per
    second."""
    threads = threads or ref.cores()
    out = ref.attn_heads(q, k_rows, v_rows, gate=gate, threads=threads)  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        ref.attn_heads(q, k_rows, v_rows, gate=gate, threads=threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 200:
            break
    return {"value": n / el, "unit": "decode-steps/s", "cores": min(threads, 24), "kind": "port",
            "sample": f"{n} decode steps of the 32768-token workload (one layer's K/V, 24 heads), "
                      f"{el:.1f} s, {threads} threads available, heads split over min(threads, 24)"}, out


def copy_calibration(ctx, steps: int) -> None:
    """A plain copy of a known size: each launch reads and writes COPY_BYTES."""
    n = COPY_BYTES // 4
    src, dst = ctx.empty((n,)), ctx.empty((n,))
    ctx.fill_normal(src, n, 0x51334100)
    for _ in range(3):
        ctx.copy(dst, src, COPY_BYTES)
    ctx.sync()
    ctx.kernel_timer_start("q38_copy_f32", steps)
    for _ in range(steps):
        ctx.copy(dst, src, COPY_BYTES)
    k_ms, k_n = ctx.kernel_timer_stop()
    us = k_ms * 1e3 / max(k_n, 1)
    print(json.dumps({"mode": "copy-calibration", "kernel": "q38_copy_f32", "bytes_read": COPY_BYTES,
                      "bytes_written": COPY_BYTES, "launches": k_n, "kernel_us": us,
                      "gb_s": 2 * COPY_BYTES / (us * 1e-6) / 1e9}), flush=True)


EXTRAS = {
    "prefill_attention_4096": ("prefill attention, 4096-token causal prompt",
                               lambda pkg, ctx: prefill_attention(pkg, ctx, 5)),
    "gdn_prefill_4096": ("chunked Gated-DeltaNet prefill, 4096 tokens", lambda pkg, ctx: gdn_prefill(pkg, ctx, 5)),
    "linear_core_prefill_4096": ("linear_core over a 4096-token prompt (one layer)",
                                 lambda pkg, ctx: linear_core_prefill(pkg, ctx, 5)),
    "prefill_attention_sweep": ("prefill attention at 512-8192-token prompts and 512 after 8192",
                                lambda pkg, ctx: prefill_attention_sweep(pkg, ctx)),
    "decode_context_sweep": ("decode step at 1K-128K context (16 layers rotated)",
                             lambda pkg, ctx: decode_context_sweep(pkg, ctx)),
    "batched_decode_32": ("batched paged decode, 32 sequences, context ~U[1K, 32K]",
                          lambda pkg, ctx: batched_decode(pkg, ctx, 20, 3)),
    "launch_floor": ("empty kernel launches", lambda pkg, ctx: launch_floor(ctx, 500)),
    "linear_core_decode": ("linear_core decode over 48 DeltaNet layers", lambda pkg, ctx: linear_core_decode(
        pkg, ctx, 20, 3)),
    "full_stack_128k": ("64 layers (48 DeltaNet + 16 attention), 128K context, one token",
                        lambda pkg, ctx: full_stack(pkg, ctx, 10, 2)),
    "gdn_step_1": ("Gated-DeltaNet step, 1 state per launch over 192 states",
                   lambda pkg, ctx: gdn_steps(pkg, ctx, 1, 192, 384, 32)),
    "gdn_step_32": ("Gated-DeltaNet step, 32 states per launch over 192",
                    lambda pkg, ctx: gdn_steps(pkg, ctx, 32, 192, 60, 6)),
    "gdn_step_1_same_state": ("Gated-DeltaNet step, one state stepped in place (labelled same-buffer figure)",
                              lambda pkg, ctx: gdn_steps(pkg, ctx, 1, 1, 384, 32)),
    "recurrent_checkpoint": ("recurrent-state checkpoint of one sequence (157 MB)",
                             lambda pkg, ctx: recurrent_checkpoint(pkg, ctx, 20)),
    "projection_sweep": ("FFN gate and down projections at 1-4096 tokens: the kernel chosen and its time",
                         lambda pkg, ctx: projection_sweep(pkg, ctx, 3)),
    "prompt_projections_64": ("FFN projections of one layer for 64 prompt tokens",
                              lambda pkg, ctx: prompt_projections(pkg, ctx, 64, 5)),
    "prompt_projections_4096": ("FFN projections of one layer for a 4096-token prompt",
                                lambda pkg, ctx: prompt_projections(pkg, ctx, 4096, 3)),
    "layer_projections_1": ("the projections of 4 attention layers' decode steps, 1 token: quantise then project "
                            "per input, as two calls and as one",
                            lambda pkg, ctx: layer_projections(pkg, ctx, 1, 20)),
    "layer_projections_8": ("the same projections for a batch of 8 tokens",
                            lambda pkg, ctx: layer_projections(pkg, ctx, 8, 10)),
    "layer_projections_32": ("the same projections for a batch of 32 tokens",
                             lambda pkg, ctx: layer_projections(pkg, ctx, 32, 10)),
    "ffn_projections_1": ("FFN projections (Q4_K gate/up, Q6_K down) of 4 layers, 1 token",
                          lambda pkg, ctx: ffn_projections(pkg, ctx, 1, 20)),
    "ffn_projections_8": ("FFN projections (Q4_K gate/up, Q6_K down) of 4 layers, 8 tokens",
                          lambda pkg, ctx: ffn_projections(pkg, ctx, 8, 20)),
    "weight_formats_1": ("one token through a 17408x5120 matrix in each Q8_K weight format",
                         lambda pkg, ctx: weight_formats(pkg, ctx, 3)),
    "weight_formats_prompt_4096": ("a 4096-token prompt through a 17408x5120 matrix in each Q8_K weight format",
                                   lambda pkg, ctx: weight_formats_prompt(pkg, ctx, 4096, 2)),
    "f32_path_projections": ("F32/F16/BF16/Q8_0 weights (the f32-input path) at 1, 16 and 4096 tokens",
                             lambda pkg, ctx: f32_path(pkg, ctx, 3)),
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="skip every measurement besides the headline")
    ap.add_argument("--only", default=None,
                    help="comma-separated subset of the extra measurements (" + ",".join(EXTRAS) + ")")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="instead of the benchmark: time a plain 512 MiB device copy (q38_copy_f32), "
                    "the reference figure that scales the HBM byte counters")
    ap.add_argument("--module-dir", default=None, help="load the code objects from this directory "
                    "(default: next to the library), to compare builds")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: one GPU only; --gpus {args.gpus} is not supported "
              "(the path would shard over kv heads or context, with one split-K merge step)",
              file=sys.stderr)
        sys.exit(2)

    pkg = entry.load_package()
    ctx = pkg.Context(0, module_dir=args.module_dir)
    info = ctx.info()
    if args.copy_calibration:
        copy_calibration(ctx, args.steps)
        ctx.close()
        return
    log(f"device {info}")
    log(f"attention decode 32K: warmup {args.warmup}, steps {args.steps}")
    r = attention_decode(pkg, ctx, args.steps, args.warmup)
    k_ms = r["kernel_ms"]
    achieved = SPLIT_BYTES / (k_ms * 1e-3) / 1e9
    step_gbs = STEP_BYTES / (r["ms_per_step"] * 1e-3) / 1e9
    log(f"step {r['ms_per_step'] * 1e3:.2f} us (graph; plain launches {r['plain_ms_per_step'] * 1e3:.2f} us), "
        f"split kernel {k_ms * 1e3:.2f} us ({achieved:.0f} GB/s), "
        f"merge {r['merge_ms'] * 1e3:.2f} us")

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "attn_decode_split_32k_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            rec = json.load(f)
        # a record of another kernel says nothing about this one
        if rec.get("kernel") == DECODE_KERNEL:
            traffic = rec.get("hbm_bytes_per_launch")

    extra = {
        "split_kernel_us": k_ms * 1e3,
        "merge_kernel_us": r["merge_ms"] * 1e3,
        "step_us": r["ms_per_step"] * 1e3,
        "step_note": "value: the timed steps replayed from one HIP graph (q38_decode_graph); "
                     "plain_step_us: the same steps as plain q38_attn_decode calls",
        "plain_step_us": r["plain_ms_per_step"] * 1e3,
        "plain_step_frac_hbm": STEP_BYTES / (r["plain_ms_per_step"] * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "step_gb_s": step_gbs,
        "step_frac_hbm": step_gbs / HBM_PEAK_GBS,
        "same_buffer_step_us": r["same_buffer_ms_per_step"] * 1e3,
        "same_buffer_note": "100 steps on one layer's 268 MB cache (the timed steps rotate over 16 layers' caches)",
        "device": info["name"],
        "cu_count": info["cu_count"],
    }

    cpu = None
    if not args.no_cpu:
        ref = entry.load_oracle()
        kvc, seq = r["kv"], r["seq"]
        rows_k, rows_v = r["rows"]
        kvc.read(r["layer"], seq, 0, CTX, rows_k, rows_v)
        K = rows_k.download()
        V = rows_v.download()
        q = r["q"].download().reshape(-1)
        g = r["g"].download().reshape(-1)
        log(f"cpu baseline: restatement on {ref.cores()} host threads, ~{args.cpu_seconds:.0f} s")
        cpu, want = cpu_baseline(ref, q, K, V, g, args.cpu_seconds)
        extra["parity_max_abs_vs_cpu"] = float(np.max(np.abs(r["out"] - want)))
        one, _ = cpu_baseline(ref, q, K, V, g, min(args.cpu_seconds, 4.0), threads=1)
        extra["cpu_1_thread_steps_per_s"] = one["value"]
        log(f"cpu {cpu['value']:.2f} steps/s; GPU vs CPU max-abs {extra['parity_max_abs_vs_cpu']:.2e}")
    r["kv"].close()

    wanted = [] if args.no_extra else (args.only.split(",") if args.only else list(EXTRAS))
    unknown = [w for w in wanted if w not in EXTRAS]
    if unknown:
        print(f"bench.py: unknown measurement(s) {unknown}; choose from {list(EXTRAS)}", file=sys.stderr)
        sys.exit(2)
    for name in wanted:
        log(f"{name}: {EXTRAS[name][0]}")
        try:
            extra[name] = EXTRAS[name][1](pkg, ctx)
        except Exception as e:  # a failure in one extra is recorded; the headline line still prints
            extra[name] = {"error": f"{type(e).__name__}: {e}"}
        log(f"{name}: {json.dumps(extra[name])}")

    line = {
        "metric": "attn decode-steps/s & achieved HBM GB/s (% of 8 TB/s) at 32K ctx, 1 MI355X",
        "value": 1e3 / r["ms_per_step"],
        "unit": "decode-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded N(0,1) K/V/q/gate (SplitMix64 + Box-Muller), 16 layers' caches rotated",
        "config": {"workload": "full-attention GQA decode step, batch 1, 32768 cached tokens, 24 q / 4 kv "
                               "heads, head_dim 256, f32 paged KV (16-token pages), append + gate",
                   "context": CTX, "batch": 1, "q_heads": 24, "kv_heads": 4, "head_dim": 256,
                   "page_tokens": 16, "layers_rotated": 16},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "traffic_source": "profiled, not measured in this run: profiles/attn_decode_split_32k_traffic.json "
                                       "(rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of this kernel on this workload, "
                                       "scaled by the same counters on a plain copy)",
                     "kernel": DECODE_KERNEL, "algorithmic_bytes_per_launch": SPLIT_BYTES},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    ctx.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
