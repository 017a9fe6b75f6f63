"""Checks that pin the CPU restatement (oracle/) of the reference's attention
path.  Each check returns None when it holds and a message when it fails, so
the same list runs against the real restatement (tests/test_oracle.py) and
against builds with a planted mistake (tests/test_oracle_mutants.py), each of
which must be rejected by at least one check.

Three kinds of evidence, none of which retypes the restatement's formulas:
  - golden fixtures (tests/golden/attention_path.npz) written by an
    independent float64 numpy formulation (tests/golden/make_fixtures.py);
  - closed forms and invariants that the mathematics fixes (a single position
    returns v; identical keys average v; beta = 0 is pure decay; the delta
    rule stores v under k; RMSNorm/L2 norms; RoPE at position 0 is the
    identity and preserves pair norms);
  - the reference's own contract for its dispatch: serial and parallel runs
    agree bit for bit (the pattern of src/kernel/tensor.rs:791-926).
"""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "attention_path.npz")


def _fx():
    return np.load(FIXTURE, allow_pickle=False)


def _close(got, want, atol, rtol=0.0, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    if np.any(~np.isfinite(got)) or np.any(bad):
        return f"{what}: max err {np.nanmax(err):.3e} (atol {atol}, rtol {rtol})"
    return None


# ------------------------------------------------------------------ fixtures
def check_generator(ref, synth):
    f = _fx()
    seed = int(f["gen_seed"][0])
    if not np.array_equal(synth.splitmix64(seed, 0, 8), f["gen_words"]):
        return "SplitMix64 words differ from the fixture"
    return _close(synth.normal(seed, 8), f["gen_normals"], 0.0, 1e-7, "Box-Muller normals")


def check_attention_fixture(ref, synth):
    f = _fx()
    P = 256
    q = synth.normal(0x51333801, 6144)
    K = synth.normal(0x51333802, P * 1024).reshape(P, 1024)
    V = synth.normal(0x51333803, P * 1024).reshape(P, 1024)
    G = synth.normal(0x51333804, 6144)
    return (_close(ref.attn_heads(q, K, V), f["attn256_nogate"], 2e-6, 0, "attention 256, no gate")
            or _close(ref.attn_heads(q, K, V, gate=G), f["attn256_gate"], 2e-6, 0, "attention 256, gate"))


def check_full_core_fixture(ref, synth):
    f = _fx()
    pos, ctx_len, layer = 37, 40, 7
    qn = synth.normal(0x51333811, 256, sigma=0.2, mean=1.0)
    kn = synth.normal(0x51333812, 256, sigma=0.2, mean=1.0)
    qg = synth.normal(0x51333813, 12288)
    key = synth.normal(0x51333814, 1024)
    val = synth.normal(0x51333815, 1024)
    kc = np.zeros(2 * ctx_len * 1024, np.float32)
    vc = np.zeros(2 * ctx_len * 1024, np.float32)
    kc[ctx_len * 1024: ctx_len * 1024 + pos * 1024] = synth.normal(0x51333816, pos * 1024)
    vc[ctx_len * 1024: ctx_len * 1024 + pos * 1024] = synth.normal(0x51333817, pos * 1024)
    out, k = ref.full_core(qn, kn, qg, key, val, kc, vc, ctx_len, pos, layer)
    row = (ctx_len + pos) * 1024
    if not np.array_equal(kc[row:row + 1024], k) or not np.array_equal(vc[row:row + 1024], val):
        return "full_core did not append k/v at slot layer/4, row pos"
    return (_close(k, f["full_core37_k"], 1e-5, 0, "full_core k after norm+RoPE")
            or _close(out, f["full_core37"], 2e-6, 0, "full_core output"))


def check_full_core_bounds(ref, synth):
    """The cache-row bounds check of ops.rs:860-864 returns Err(-1)."""
    kc = np.zeros(4 * 1024, np.float32)
    try:
        ref.full_core(np.ones(256, np.float32), np.ones(256, np.float32), np.ones(12288, np.float32),
                      np.ones(1024, np.float32), np.ones(1024, np.float32), kc, kc.copy(), 4, 4, 3)
    except ValueError:
        return None
    return "position == context_length was accepted"


def check_rope_fixture(ref, synth):
    f = _fx()
    x = synth.normal(0x51333821, 512)
    for p in (0, 1, 1000, 131071):
        msg = _close(ref.rope(x, 2, p), f[f"rope_{p}"], 2e-6, 1e-6, f"rope at {p}")
        if msg:
            return msg
    return None


def check_softplus_fixture(ref, synth):
    f = _fx()
    got = [ref.scalar_fn("softplus", x) for x in f["softplus_in"]]
    return _close(got, f["softplus"], 1e-6, 1e-6, "softplus")


def check_rms_fixture(ref, synth):
    f = _fx()
    v = synth.normal(0x51333822, 256)
    return _close([ref.rms_scale(v)], f["rms_scale_256"], 0, 1e-6, "rms_scale")


def check_gdn_fixture(ref, synth):
    f = _fx()
    S = synth.normal(0x51333831, 48 * 128 * 128, sigma=0.02)
    gen = synth.GdnStepInputs(0x51333832)
    outs = []
    for t in range(64):
        outs.append(ref.gdn_heads(S, *gen.step(t), threads=4))
    idx = f["gdn64_sample_idx"]
    scale = np.max(np.abs(f["gdn64_state_sample"]))
    return (_close(S[idx], f["gdn64_state_sample"], 1e-5 * scale, 0, "gdn state after 64 steps")
            or _close((S.astype(np.float64).reshape(48, -1) ** 2).sum(1), f["gdn64_state_head_sumsq"], 0, 1e-4,
                      "gdn per-head state energy")
            or _close(outs[-1], f["gdn64_out_last"], 1e-5, 0, "gdn last output")
            or _close(np.stack([o[:128] for o in outs]), f["gdn64_out_head0"], 1e-5, 0, "gdn head 0 outputs")
            or _close(np.stack([o[17 * 128:18 * 128] for o in outs]), f["gdn64_out_head17"], 1e-5, 0,
                      "gdn head 17 outputs"))


def check_linear_core_fixture(ref, synth):
    f = _fx()
    conv_w = synth.normal(0x51333841, 10240 * 4, sigma=0.5)
    dt = synth.normal(0x51333842, 48)
    a = -np.abs(synth.normal(0x51333843, 48))
    norm = synth.normal(0x51333844, 128, sigma=0.1, mean=1.0)
    cs = synth.normal(0x51333845, 10240 * 3)
    S = synth.normal(0x51333846, 48 * 128 * 128, sigma=0.02)
    raw = []
    for t in range(4):
        qkv = synth.normal(0x51333850 + t, 10240)
        raw.append(qkv)
        o = ref.linear_core(conv_w, dt, a, norm, cs, S, qkv, synth.normal(0x51333860 + t, 6144),
                            synth.normal(0x51333870 + t, 48), synth.normal(0x51333880 + t, 48))
        msg = _close(o, f["linear4_out"][t], 2e-5, 1e-5, f"linear_core output, token {t}")
        if msg:
            return msg
    # the conv state holds the last three raw inputs, channel-major (closed form)
    want_cs = np.stack([raw[1], raw[2], raw[3]], axis=1).reshape(-1)
    if not np.array_equal(cs, want_cs):
        return "conv state is not the last three raw inputs"
    scale = np.max(np.abs(f["linear4_state_sample"]))
    return _close(S[f["gdn64_sample_idx"]], f["linear4_state_sample"], 1e-5 * scale, 0, "linear_core state")


# -------------------------------------------------------------- closed forms
def check_single_position(ref, synth):
    """One position: softmax weight 1, so o == v exactly (ops.rs:905-913)."""
    q = synth.normal(1, 6144)
    K = synth.normal(2, 1024).reshape(1, 1024)
    V = synth.normal(3, 1024).reshape(1, 1024)
    o = ref.attn_heads(q, K, V)
    want = np.repeat(V.reshape(4, 256), 6, axis=0)
    return None if np.array_equal(o, want) else "single position does not return v"


def check_identical_keys(ref, synth):
    """Identical keys: uniform weights, o = mean of the value rows."""
    P = 50
    q = synth.normal(4, 6144)
    K = np.tile(synth.normal(5, 1024), (P, 1))
    V = synth.normal(6, P * 1024).reshape(P, 1024)
    o = ref.attn_heads(q, K, V)
    want = np.repeat(V.astype(np.float64).mean(0).reshape(4, 256), 6, axis=0)
    return _close(o, want, 2e-6, 0, "identical keys")


def check_gqa_grouping(ref, synth):
    """Query heads 6j..6j+5 read kv head j: equal q rows give equal outputs,
    and permuting kv head j's rows changes exactly heads 6j..6j+5."""
    P = 40
    q1 = synth.normal(7, 256)
    q = np.tile(q1, 24)
    K = synth.normal(8, P * 1024).reshape(P, 1024)
    V = synth.normal(9, P * 1024).reshape(P, 1024)
    o = ref.attn_heads(q, K, V)
    for j in range(4):
        if not all(np.array_equal(o[6 * j], o[6 * j + i]) for i in range(6)):
            return f"heads of group {j} differ"
    K2 = K.copy()
    K2[:, 256:512] = K2[::-1, 256:512]  # change kv head 1 only
    o2 = ref.attn_heads(q, K2, V)
    changed = [h for h in range(24) if not np.array_equal(o[h], o2[h])]
    return None if changed == list(range(6, 12)) else f"changing kv head 1 changed heads {changed}"


def check_position_permutation(ref, synth):
    P = 64
    q = synth.normal(10, 6144)
    K = synth.normal(11, P * 1024).reshape(P, 1024)
    V = synth.normal(12, P * 1024).reshape(P, 1024)
    perm = np.random.default_rng(3).permutation(P)
    return _close(ref.attn_heads(q, K[perm], V[perm]), ref.attn_heads(q, K, V), 2e-6, 0, "position permutation")


def check_rope_identities(ref, synth):
    x = synth.normal(13, 24 * 256)
    if not np.array_equal(ref.rope(x, 24, 0)[:64], x[:64]):
        # theta_p = 0 for every pair at position 0: cos 1, sin 0
        return "RoPE at position 0 is not the identity"
    y = ref.rope(x, 24, 5000).reshape(24, 256)
    xr = x.reshape(24, 256)
    if not np.array_equal(y[:, 64:], xr[:, 64:]):
        return "RoPE touched lanes 64..255"
    n0 = np.hypot(xr[:, :32], xr[:, 32:64])
    n1 = np.hypot(y[:, :32], y[:, 32:64])
    return _close(n1, n0, 1e-5, 1e-6, "RoPE pair norms")


def check_norms(ref, synth):
    x = synth.normal(14, 256)
    w = synth.normal(15, 256)
    want = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    msg = _close(ref.rmsnorm(x, w), want, 1e-6, 1e-6, "rmsnorm closed form")
    if msg:
        return msg
    y = ref.l2norm(x)
    if abs(np.linalg.norm(y.astype(np.float64)) - 1.0) > 1e-6:
        return "l2norm result is not unit length"
    z = ref.l2norm(np.zeros(128, np.float32))
    return None if np.all(z == 0) else "l2norm of zero is not zero (floor 1e-6 missing)"


def check_gdn_beta_zero(ref, synth):
    """beta = 0: S_t = exp(g) S_{t-1}, o = S_t q / sqrt(128)."""
    S0 = synth.normal(16, 48 * 128 * 128, sigma=0.02)
    q, k, v, beta, g = synth.GdnStepInputs(17).step(0)
    S = S0.copy()
    o = ref.gdn_heads(S, q, k, v, np.zeros_like(beta), g)
    want_S = S0.reshape(48, 128, 128).astype(np.float64) * np.exp(g.astype(np.float64))[:, None, None]
    qh = q.reshape(16, 128)[np.arange(48) % 16].astype(np.float64)
    want_o = np.einsum("hcd,hd->hc", want_S, qh) / np.sqrt(128.0)
    return (_close(S.reshape(48, 128, 128), want_S, 1e-8, 1e-6, "beta=0 state")
            or _close(o.reshape(48, 128), want_o, 1e-6, 0, "beta=0 output"))


def check_gdn_write(ref, synth):
    """decay 1, beta 1, |k| = 1: after the step S k = v for every row."""
    S = synth.normal(18, 48 * 128 * 128, sigma=0.02)
    q, k, v, beta, g = synth.GdnStepInputs(19).step(0)
    ref.gdn_heads(S, q, k, v, np.ones_like(beta), np.zeros_like(g))
    kh = k.reshape(16, 128)[np.arange(48) % 16].astype(np.float64)
    Sk = np.einsum("hcd,hd->hc", S.reshape(48, 128, 128).astype(np.float64), kh)
    return _close(Sk, v.reshape(48, 128), 1e-5, 0, "delta-rule write S k = v")


def check_gdn_zero_state(ref, synth):
    """S_0 = 0: o = beta (k.q) v / sqrt(128)."""
    S = np.zeros(48 * 128 * 128, np.float32)
    q, k, v, beta, g = synth.GdnStepInputs(20).step(0)
    o = ref.gdn_heads(S, q, k, v, beta, g)
    kh = k.reshape(16, 128)[np.arange(48) % 16].astype(np.float64)
    qh = q.reshape(16, 128)[np.arange(48) % 16].astype(np.float64)
    want = beta.astype(np.float64)[:, None] * (kh * qh).sum(1)[:, None] * v.reshape(48, 128) / np.sqrt(128.0)
    return _close(o.reshape(48, 128), want, 1e-6, 0, "zero initial state")


def check_serial_equals_parallel(ref, synth):
    P = 300
    q = synth.normal(21, 6144)
    K = synth.normal(22, P * 1024).reshape(P, 1024)
    V = synth.normal(23, P * 1024).reshape(P, 1024)
    if not np.array_equal(ref.attn_heads(q, K, V, threads=1), ref.attn_heads(q, K, V, threads=7)):
        return "attention: serial and parallel differ"
    S1 = synth.normal(24, 48 * 128 * 128, sigma=0.02)
    S2 = S1.copy()
    ins = synth.GdnStepInputs(25).step(0)
    o1 = ref.gdn_heads(S1, *ins, threads=1)
    o2 = ref.gdn_heads(S2, *ins, threads=5)
    return None if np.array_equal(o1, o2) and np.array_equal(S1, S2) else "gdn: serial and parallel differ"


def check_layer_maps(ref, synth):
    full = [l for l in range(65) if ref.lib().q38r_is_full_attention(l)]
    if full != [3 + 4 * i for i in range(16)] + [64]:
        return f"full-attention layers {full}"
    rec = [ref.lib().q38r_recurrent_index(l) for l in range(64) if l not in full]
    return None if rec == list(range(48)) else "recurrent indices are not 0..47 in order"


# ------------------------------------------------------- weight projections
# Independent formulations of the projection path (src/kernel/quant.rs,
# src/kernel/tensor.rs): the Q8_K quantiser restated with numpy's float32
# arithmetic and round-half-to-even, and the K-quant weights DEQUANTISED the
# way the reference's decoded path reads them (dot_q4/q5/q6_k_scalar,
# tensor.rs:187-327) and multiplied out in float64 -- against the integer
# dots (tensor.rs:365-457) the oracle restates.

def _np_quantize_q8_k(x):
    """quantize_block (quant.rs:55-95) in numpy: first maximum of |x| sets the
    sign, float32 -127/max, round half to even, clamp at 127, 16-wide sums."""
    blocks = np.asarray(x, np.float32).reshape(-1, 256)
    q = np.zeros(blocks.shape, np.int8)
    sums = np.zeros((blocks.shape[0], 16), np.int16)
    scales = np.zeros(blocks.shape[0], np.float32)
    for b, blk in enumerate(blocks):
        k = int(np.argmax(np.abs(blk)))  # first occurrence
        if np.abs(blk[k]) == 0:
            continue
        inv = np.float32(-127.0) / np.float32(blk[k])
        v = np.rint((inv * blk).astype(np.float32))
        q[b] = np.minimum(v, 127).astype(np.int8)
        sums[b] = q[b].astype(np.int32).reshape(16, 16).sum(1).astype(np.int16)
        scales[b] = np.float32(1.0) / inv
    return q, sums, scales


def _q8k_dequant(planar, T, W, ref):
    q, _, sc = ref.q8k_split(planar, T, W)
    return q.reshape(T, W // 256, 256).astype(np.float64) * sc.astype(np.float64)[:, :, None]


def _f16(b0, b1):
    return np.frombuffer(np.array([b0, b1], np.uint8).tobytes(), np.float16)[0].astype(np.float64)


def _f16_bits(h):
    return np.array([h], np.uint16).view(np.float16)[0].astype(np.float64)


def _scale_min(s, j):
    if j < 4:
        return s[j] & 63, s[j + 4] & 63
    return (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4), (s[j + 4] >> 4) | ((s[j] >> 6) << 4)


# ggml's published IQ4_NL / IQ4_XS code book
_KVALUES_IQ4 = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.int64)


_GRIDS_H = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "qwen3.8_27b_in_rust_amd",
                        "csrc", "q38_iq_grids.h")
_GRID_BYTES = {"Q38_IQ2XXS_GRID": 8, "Q38_IQ2XS_GRID": 8, "Q38_IQ2S_GRID": 8, "Q38_IQ3XXS_GRID": 4,
               "Q38_IQ3S_GRID": 4, "Q38_IQ1S_GRID": 8}


def _iq_grids():
    """The IQ lattice grids of q38_iq_grids.h as byte arrays [entries][4 or 8]."""
    import re
    text = open(_GRIDS_H).read()
    out = {}
    for name, nb in _GRID_BYTES.items():
        body = re.search(r"#define %s \{(.*?)\}" % name, text, re.S).group(1)
        vals = np.array([int(v, 16) for v in re.findall(r"0x[0-9a-f]+", body)], np.uint64)
        out[name] = np.frombuffer(vals.astype("<u8").tobytes(), np.uint8).reshape(-1, 8)[:, :nb].astype(np.int64)
    return out


def _ksign_mask(i):
    """ggml's ksigns_iq2xs entry i as 8 signs: the 7 stored bits and an eighth
    that makes the number of minus signs even."""
    bits = [(i >> j) & 1 for j in range(7)]
    bits.append(sum(bits) & 1)
    return np.where(np.array(bits) == 1, -1, 1)


def _q3k_scales(sc12):
    """The 16 6-bit Q3_K scales as ggml's dequantize_row_q3_K unpacks them:
    four little-endian words, the high 2-bit pairs spread from the third."""
    aux = np.frombuffer(np.asarray(sc12, np.uint8).tobytes(), np.uint32).astype(np.uint64)
    k1, k2 = 0x03030303, 0x0F0F0F0F
    tmp = aux[2]
    words = [(aux[0] & k2) | (((tmp >> 0) & k1) << 4), (aux[1] & k2) | (((tmp >> 2) & k1) << 4),
             ((aux[0] >> 4) & k2) | (((tmp >> 4) & k1) << 4), ((aux[1] >> 4) & k2) | (((tmp >> 6) & k1) << 4)]
    return np.frombuffer(np.array(words, np.uint32).tobytes(), np.int8).astype(np.int64) - 32


_BLOCK_BYTES = {10: 84, 11: 110, 12: 144, 13: 176, 14: 210, 20: 144, 23: 136, 16: 66, 17: 74, 22: 82, 18: 98,
                21: 110, 19: 50, 29: 56}


def _dequant_iq(ty, blk, grids):
    """ggml's dequantize_row_iq2_xxs / _iq2_xs / _iq2_s / _iq3_xxs / _iq3_s /
    _iq1_s / _iq1_m for one 256-value block (float64)."""
    w = np.zeros(256)
    u16 = lambda o: int(blk[o]) | (int(blk[o + 1]) << 8)
    u32 = lambda o: u16(o) | (u16(o + 2) << 16)
    if ty == 29:  # IQ1_M: qs[32] | qh[16] | scales u16[4], d in their top nibbles
        sc = [u16(48 + 2 * k) for k in range(4)]
        d = _f16_bits((sc[0] >> 12) | ((sc[1] >> 8) & 0x00F0) | ((sc[2] >> 4) & 0x0F00) | (sc[3] & 0xF000))
    else:
        d = _f16(blk[0], blk[1])
    for ib in range(8):
        y = w[32 * ib:32 * ib + 32]
        if ty == 16:  # IQ2_XXS
            aux = u32(2 + 8 * ib + 4)
            db = d * (0.5 + (aux >> 28)) * 0.25
            for l in range(4):
                y[8 * l:8 * l + 8] = db * grids["Q38_IQ2XXS_GRID"][blk[2 + 8 * ib + l]] * _ksign_mask((aux >> (7 * l)) & 127)
        elif ty == 17:  # IQ2_XS
            sc = blk[66 + ib]
            for l in range(4):
                q = u16(2 + 8 * ib + 2 * l)
                db = d * (0.5 + ((sc >> (4 * (l // 2))) & 15)) * 0.25
                y[8 * l:8 * l + 8] = db * grids["Q38_IQ2XS_GRID"][q & 511] * _ksign_mask(q >> 9)
        elif ty == 22:  # IQ2_S: qs[32] | signs[32] | qh[8] | scales[8]
            sc, qh = blk[74 + ib], blk[66 + ib]
            for l in range(4):
                db = d * (0.5 + ((sc >> (4 * (l // 2))) & 15)) * 0.25
                idx = blk[2 + 4 * ib + l] | ((qh << (8 - 2 * l)) & 0x300)
                signs = np.where((blk[34 + 4 * ib + l] >> np.arange(8)) & 1, -1, 1)
                y[8 * l:8 * l + 8] = db * grids["Q38_IQ2S_GRID"][idx] * signs
        elif ty == 18:  # IQ3_XXS: qs[64] | scales-and-signs u32[8]
            aux = u32(66 + 4 * ib)
            db = d * (0.5 + (aux >> 28)) * 0.5
            for l in range(4):
                s8 = _ksign_mask((aux >> (7 * l)) & 127)
                y[8 * l:8 * l + 4] = db * grids["Q38_IQ3XXS_GRID"][blk[2 + 8 * ib + 2 * l]] * s8[:4]
                y[8 * l + 4:8 * l + 8] = db * grids["Q38_IQ3XXS_GRID"][blk[2 + 8 * ib + 2 * l + 1]] * s8[4:]
        elif ty == 21:  # IQ3_S: qs[64] | qh[8] | signs[32] | scales[4]
            db = d * (1 + 2 * ((blk[106 + ib // 2] >> (4 * (ib % 2))) & 15))
            qh = blk[66 + ib]
            for l in range(4):
                signs = np.where((blk[74 + 4 * ib + l] >> np.arange(8)) & 1, -1, 1)
                g1 = grids["Q38_IQ3S_GRID"][blk[2 + 8 * ib + 2 * l] | ((qh << (8 - 2 * l)) & 256)]
                g2 = grids["Q38_IQ3S_GRID"][blk[2 + 8 * ib + 2 * l + 1] | ((qh << (7 - 2 * l)) & 256)]
                y[8 * l:8 * l + 4] = db * g1 * signs[:4]
                y[8 * l + 4:8 * l + 8] = db * g2 * signs[4:]
        elif ty == 19:  # IQ1_S: qs[32] | qh u16[8]
            qh = u16(34 + 2 * ib)
            dl = d * (2 * ((qh >> 12) & 7) + 1)
            delta = -0.125 if qh & 0x8000 else 0.125
            for l in range(4):
                g = grids["Q38_IQ1S_GRID"][blk[2 + 4 * ib + l] | (((qh >> (3 * l)) & 7) << 8)]
                y[8 * l:8 * l + 8] = dl * (np.where(g > 127, g - 256, g) + delta)
        else:  # IQ1_M
            sc = u16(48 + 2 * (ib // 2))
            dl = [d * (2 * ((sc >> (6 * (ib % 2) + 3 * h)) & 7) + 1) for h in range(2)]
            qh = [blk[32 + 2 * ib], blk[32 + 2 * ib + 1]]
            for l in range(4):
                hb = qh[l // 2]
                idx = blk[4 * ib + l] | ((hb << (8 if l % 2 == 0 else 4)) & 0x700)
                delta = -0.125 if hb & (0x08 if l % 2 == 0 else 0x80) else 0.125
                g = grids["Q38_IQ1S_GRID"][idx]
                y[8 * l:8 * l + 8] = dl[l // 2] * (np.where(g > 127, g - 256, g) + delta)
    return w


def _dequant_row(ty, row):
    """A weight row's values the way the decoded path reads them."""
    out = []
    bb = _BLOCK_BYTES[ty]
    grids = _iq_grids() if ty in (16, 17, 18, 19, 21, 22, 29) else None
    for blk in np.asarray(row, np.uint8).reshape(-1, bb).astype(np.int64):
        w = np.zeros(256)
        if grids is not None:
            w = _dequant_iq(ty, blk, grids)
        elif ty == 10:
            # ggml's dequantize_row_q2_K: per 128 values, four 2-bit shifts,
            # each 32 values as two 16-value groups with scale d * (sc & 15)
            # and minimum dmin * (sc >> 4)
            sc, qs = blk[0:16], blk[16:80]
            d, dmin = _f16(blk[80], blk[81]), _f16(blk[82], blk[83])
            i = 0
            for n in range(2):
                for shift in range(0, 8, 2):
                    for part in range(2):
                        q = (qs[32 * n + 16 * part + np.arange(16)] >> shift) & 3
                        w[128 * n + 32 * (shift // 2) + 16 * part + np.arange(16)] = \
                            d * (sc[i] & 15) * q - dmin * (sc[i] >> 4)
                        i += 1
        elif ty == 20:
            for g in range(8):
                sub = blk[18 * g:18 * g + 18]
                d, q = _f16(sub[0], sub[1]), sub[2:18]
                w[32 * g:32 * g + 16] = d * _KVALUES_IQ4[q & 15]
                w[32 * g + 16:32 * g + 32] = d * _KVALUES_IQ4[q >> 4]
        elif ty == 11:
            hm, qs, d = blk[0:32], blk[32:96], _f16(blk[108], blk[109])
            sc = _q3k_scales(blk[96:108].astype(np.uint8))
            m, i = 0, 0
            for n in range(2):
                for shift in range(0, 8, 2):
                    for part in range(2):
                        lanes = np.arange(16 * part, 16 * part + 16)
                        qv = ((qs[32 * n + lanes] >> shift) & 3) - np.where(hm[lanes] & (1 << m), 0, 4)
                        w[128 * n + 32 * (shift // 2) + 16 * part + np.arange(16)] = d * sc[i] * qv
                        i += 1
                    m += 1
        elif ty == 23:
            d, sh, sl, qs = _f16(blk[0], blk[1]), int(blk[2]) | (int(blk[3]) << 8), blk[4:8], blk[8:136]
            for ib in range(8):
                ls = ((sl[ib // 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4)
                q = qs[16 * ib:16 * ib + 16]
                w[32 * ib:32 * ib + 16] = d * (ls - 32) * _KVALUES_IQ4[q & 15]
                w[32 * ib + 16:32 * ib + 32] = d * (ls - 32) * _KVALUES_IQ4[q >> 4]
        elif ty in (12, 13):
            d, dmin = _f16(blk[0], blk[1]), _f16(blk[2], blk[3])
            s = blk[4:16]
            qs = blk[16:144] if ty == 12 else blk[48:176]
            qh = blk[16:48] if ty == 13 else None
            for c in range(4):
                sc0, m0 = _scale_min(s, 2 * c)
                sc1, m1 = _scale_min(s, 2 * c + 1)
                lo = qs[32 * c:32 * c + 32] & 15
                hi = qs[32 * c:32 * c + 32] >> 4
                if qh is not None:
                    lo = lo + 16 * ((qh >> (2 * c)) & 1)
                    hi = hi + 16 * ((qh >> (2 * c + 1)) & 1)
                w[64 * c:64 * c + 32] = d * sc0 * lo - dmin * m0
                w[64 * c + 32:64 * c + 64] = d * sc1 * hi - dmin * m1
        else:
            ql, qh, sc = blk[0:128], blk[128:192], blk[192:208].astype(np.uint8).view(np.int8).astype(np.int64)
            d = _f16(blk[208], blk[209])
            for h in range(2):
                i = np.arange(32)
                a, b2, hh = ql[64 * h + i], ql[64 * h + 32 + i], qh[32 * h + i]
                parts = [(a & 15) | ((hh & 3) << 4), (b2 & 15) | (((hh >> 2) & 3) << 4),
                         (a >> 4) | (((hh >> 4) & 3) << 4), (b2 >> 4) | (((hh >> 6) & 3) << 4)]
                for k, qv in enumerate(parts):
                    w[128 * h + 32 * k + i] = d * sc[8 * h + i // 16 + 2 * k] * (qv - 32)
        out.append(w)
    return np.concatenate(out)


def _random_kquant(ty, rows, width, seed):
    """Weight rows of random bytes with finite, moderate f16 scales."""
    rng = np.random.default_rng(seed)
    bb = _BLOCK_BYTES[ty]
    w = rng.integers(0, 256, (rows, width // 256, bb), dtype=np.uint8)
    f16 = lambda lo, hi, n: np.frombuffer(rng.uniform(lo, hi, n).astype(np.float16).tobytes(), np.uint8).reshape(n, 2)
    n = rows * (width // 256)
    if ty in (12, 13):
        w.reshape(n, bb)[:, 0:2] = f16(1e-3, 4e-2, n)
        w.reshape(n, bb)[:, 2:4] = f16(1e-3, 4e-2, n)
    elif ty == 14:
        w.reshape(n, bb)[:, 208:210] = f16(1e-3, 4e-2, n)
    elif ty == 11:
        w.reshape(n, bb)[:, 108:110] = f16(1e-3, 4e-2, n)
    elif ty == 10:
        w.reshape(n, bb)[:, 80:82] = f16(1e-3, 4e-2, n)
        w.reshape(n, bb)[:, 82:84] = f16(1e-3, 4e-2, n)
    elif ty == 20:
        for g in range(8):
            w.reshape(n, bb)[:, 18 * g:18 * g + 2] = f16(1e-4, 4e-3, n)
    elif ty == 29:
        # IQ1_M: the f16 d is the top nibbles of the four scale halfwords
        h = np.frombuffer(f16(1e-3, 4e-2, n).tobytes(), np.uint16)
        blk = w.reshape(n, bb)
        for k in range(4):
            nib = ((h >> (4 * k)) & 15).astype(np.uint8)
            blk[:, 49 + 2 * k] = (blk[:, 49 + 2 * k] & 0x0F) | (nib << 4)
    else:
        w.reshape(n, bb)[:, 0:2] = f16(1e-4, 4e-3, n)
    return w.reshape(rows, -1)


def check_q8k_quantize(ref, synth):
    rng = np.random.default_rng(0x51333870)
    x = rng.standard_normal((3, 1024)).astype(np.float32) * np.float32(3.0)
    x[0, :256] = 0.0                                   # an all-zero block
    x[1, 256:512] = 0.25
    x[1, 256 + 2] = -3.0
    x[1, 256 + 5] = 3.0                                # |max| tie: the first (negative) sets the sign
    x[2, :256] = 0.0
    x[2, 0] = -127.0                                   # inverse scale 1: halves round to even
    x[2, 1:9] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, 126.5]
    # the reference's own activation pattern (tensor.rs:582-586)
    x[2, 256:512] = ((np.arange(256) * 7919) % 101) / np.float32(50.0) - np.float32(1.0)
    p = ref.quantize_q8_k(x)
    q, sums, scales = ref.q8k_split(p, 3, 1024)
    nq, nsums, nscales = _np_quantize_q8_k(x.reshape(-1))
    if not np.array_equal(q.reshape(-1, 256), nq):
        return "Q8_K quants differ from the numpy formulation"
    if not np.array_equal(sums.reshape(-1, 16), nsums):
        return "Q8_K group sums differ"
    if not np.array_equal(scales.reshape(-1).view(np.uint32), nscales.view(np.uint32)):
        return "Q8_K scales differ"
    if not (q[1, 256 + 2] == -127 and q[1, 256 + 5] == 127 and scales[1, 1] > 0):
        return "the first |maximum| does not set the sign"
    if list(q[2, 1:9]) != [2, 4, -2, -4, 0, 0, 2, 126]:
        return f"rounding is not half-to-even: {list(q[2, 1:9])}"
    return None


def check_kquant_dots_against_dequantised_rows(ref, synth):
    """Integer dots of every K-quant type equal the float64 dot of the
    dequantised weights with the dequantised activations."""
    W, T = 1024, 3
    rng = np.random.default_rng(0x51333871)
    x = rng.standard_normal((T, W)).astype(np.float32)
    x[1] = ((np.arange(W) * 7919) % 101) / np.float32(50.0) - np.float32(1.0)
    p = ref.quantize_q8_k(x)
    a = _q8k_dequant(p, T, W, ref).reshape(T, W)
    for ty in (ref.GGML_Q2_K, ref.GGML_Q3_K, ref.GGML_Q4_K, ref.GGML_Q5_K, ref.GGML_Q6_K, ref.GGML_IQ4_NL,
               ref.GGML_IQ4_XS, ref.GGML_IQ2_XXS, ref.GGML_IQ2_XS, ref.GGML_IQ2_S, ref.GGML_IQ3_XXS, ref.GGML_IQ3_S,
               ref.GGML_IQ1_S, ref.GGML_IQ1_M):
        wb = _random_kquant(ty, 7, W, 0x51333872 + ty)
        got = ref.gemv_q8_k(ty, wb, p, T, W)
        for r in range(7):
            w = _dequant_row(ty, wb[r])
            for t in range(T):
                want = float(np.dot(w, a[t]))
                scale = float(np.dot(np.abs(w), np.abs(a[t])))
                if abs(got[t, r] - want) > 2e-6 * scale:
                    return f"type {ty} row {r} token {t}: {got[t, r]} vs {want} (scale {scale:.3e})"
    return None


def check_gemv_serial_equals_threaded(ref, synth):
    W = 512
    x = np.random.default_rng(0x51333873).standard_normal((2, W)).astype(np.float32)
    p = ref.quantize_q8_k(x)
    for ty in (ref.GGML_Q2_K, ref.GGML_Q3_K, ref.GGML_Q4_K, ref.GGML_Q6_K, ref.GGML_IQ4_NL, ref.GGML_IQ4_XS):
        wb = _random_kquant(ty, 37, W, 0x51333874 + ty)
        if not np.array_equal(ref.gemv_q8_k(ty, wb, p, 2, W, threads=1), ref.gemv_q8_k(ty, wb, p, 2, W, threads=5)):
            return f"type {ty}: threaded GEMV differs from serial"
    return None


def _random_f32_path(ty, rows, width, seed):
    """Weight rows of an F32/F16/BF16/Q8_0 type: finite values of ~N(0, 0.05)
    (Q8_0: random quants, f16 scales 1e-4..1e-2), and their values decoded in
    numpy (float16 / the bf16 high half / d * q) as float64."""
    rng = np.random.default_rng(seed)
    if ty == 0:
        v = (rng.standard_normal((rows, width)) * 0.05).astype(np.float32)
        return v.view(np.uint8).reshape(rows, -1), v.astype(np.float64)
    if ty == 1:
        v = (rng.standard_normal((rows, width)) * 0.05).astype(np.float16)
        return v.view(np.uint8).reshape(rows, -1), v.astype(np.float64)
    if ty == 30:
        f = (rng.standard_normal((rows, width)) * 0.05).astype(np.float32)
        hi = (f.view(np.uint32) >> 16).astype(np.uint16)
        return hi.view(np.uint8).reshape(rows, -1), (hi.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    nb = width // 32
    q = rng.integers(-128, 128, (rows, nb, 32)).astype(np.int8)
    d = rng.uniform(1e-4, 1e-2, (rows, nb)).astype(np.float16)
    blk = np.zeros((rows, nb, 34), np.uint8)
    blk[:, :, 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:] = q.view(np.uint8)
    vals = (d.astype(np.float64)[:, :, None] * q.astype(np.float64)).reshape(rows, width)
    return blk.reshape(rows, -1), vals


def check_f32_path_dots(ref, synth):
    """tensor_gemv_f32's row dots (F32, F16, BF16, Q8_0) against the float64
    dot of the weights decoded independently in numpy: within 1e-5 of the
    sum of |w x| (a sequential f32 chain of ~1000 products), over random
    inputs and the reference's own activation pattern (tensor.rs:582-586);
    one row also against the closed form of a one-hot input (the weight
    itself, exactly)."""
    W, T, R = 1024, 3, 9
    rng = np.random.default_rng(0x51333875)
    x = rng.standard_normal((T, W)).astype(np.float32)
    x[1] = ((np.arange(W) * 7919) % 101) / np.float32(50.0) - np.float32(1.0)
    x[2] = 0.0
    x[2, 37] = 1.0
    for ty in (ref.GGML_F32, ref.GGML_F16, ref.GGML_BF16, ref.GGML_Q8_0):
        wb, wv = _random_f32_path(ty, R, W, 0x51333876 + ty)
        got = ref.gemv_f32(ty, wb, x)
        for r in range(R):
            for t in range(2):
                want = float(np.dot(wv[r], x[t].astype(np.float64)))
                scale = float(np.dot(np.abs(wv[r]), np.abs(x[t].astype(np.float64))))
                if abs(got[t, r] - want) > 1e-5 * scale:
                    return f"type {ty} row {r} token {t}: {got[t, r]} vs {want} (scale {scale:.3e})"
            if got[2, r] != np.float32(wv[r, 37]):
                return f"type {ty} row {r}: one-hot input gives {got[2, r]}, not the weight {wv[r, 37]}"
        if not np.array_equal(got, ref.gemv_f32(ty, wb, x, threads=4)):
            return f"type {ty}: threaded f32 GEMV differs from serial"
    return None


CHECKS = [v for k, v in sorted(globals().items()) if k.startswith("check_")]
