"""Writes tests/golden/*.npz: expected outputs of the attention path computed
by an independent float64 numpy formulation (vectorised softmax, einsum
recurrence) on seeded inputs from synth.py.

The reference (StepfenShawn/qwen3.8_27b_in_rust) ships no golden vectors or
fixtures for full_core / linear_core (its only tests need a 16 GB GGUF), so
these fixtures are built from the published algorithm, restated here in
float64 independently of the C restatement under oracle/.  Inputs are not
stored: they are regenerated from the seeds, and the first generator words
are stored to pin the generator itself.

Run:  python tests/golden/make_fixtures.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
import __graft_entry__ as entry  # noqa: E402

pkg = entry.load_package()
from q38amd import synth  # noqa: E402

F64 = np.float64


def rms_scale64(x):
    x = x.astype(F64)
    return 1.0 / np.sqrt(np.mean(x * x) + 1e-6)


def rope64(x, heads, position):
    """Rotation of lanes (p, p+32), p < 32, per 256-wide head.  The angle
    follows the reference's f32 recurrence theta_{p+1} = theta_p * s
    (ops.rs:599-607) exactly; cos/sin are taken in float64."""
    s = np.float32(np.float32(1e7) ** np.float32(-2.0 / 64.0))
    s64 = np.float32(F64(1e7) ** (-2.0 / 64.0))
    assert s == s64
    theta = np.empty(32, np.float32)
    t = np.float32(position)
    for p in range(32):
        theta[p] = t
        t = np.float32(t * s)
    c, si = np.cos(theta.astype(F64)), np.sin(theta.astype(F64))
    y = x.astype(F64).reshape(heads, 256).copy()
    x0, x1 = y[:, :32].copy(), y[:, 32:64].copy()
    y[:, :32] = x0 * c - x1 * si
    y[:, 32:64] = x0 * si + x1 * c
    return y.reshape(-1), theta


def attention64(q, K, V, gate=None):
    """q [24*256], K/V [P][1024] -> [24][256]; query head h reads kv head h//6."""
    q = q.astype(F64).reshape(24, 256)
    K = K.astype(F64).reshape(-1, 4, 256)
    V = V.astype(F64).reshape(-1, 4, 256)
    out = np.empty((24, 256))
    for h in range(24):
        j = h // 6
        s = K[:, j, :] @ q[h] / 16.0
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ V[:, j, :]
    if gate is not None:
        out *= 1.0 / (1.0 + np.exp(-gate.astype(F64).reshape(24, 256)))
    return out


def gdn_step64(S, q, k, v, beta, g):
    """S [48][128][128] (row c = value dim), q/k [16][128], v [48][128]."""
    qh = q.astype(F64).reshape(16, 128)[np.arange(48) % 16]
    kh = k.astype(F64).reshape(16, 128)[np.arange(48) % 16]
    S = S * np.exp(g.astype(F64))[:, None, None]
    pred = np.einsum("hcd,hd->hc", S, kh)
    delta = (v.astype(F64).reshape(48, 128) - pred) * beta.astype(F64)[:, None]
    S = S + delta[:, :, None] * kh[:, None, :]
    o = np.einsum("hcd,hd->hc", S, qh) / np.sqrt(128.0)
    return S, o


def linear_core64(conv_w, dt, a, norm, conv_state, S, qkv, z, beta, alpha):
    w = conv_w.astype(F64).reshape(10240, 4)
    cs = conv_state.astype(F64).reshape(10240, 3)
    x = qkv.astype(F64)
    y = cs[:, 0] * w[:, 0] + cs[:, 1] * w[:, 1] + cs[:, 2] * w[:, 2] + x * w[:, 3]
    new_cs = np.stack([cs[:, 1], cs[:, 2], x], axis=1)
    y = y / (1.0 + np.exp(-y))
    q = y[:2048].reshape(16, 128)
    k = y[2048:4096].reshape(16, 128)
    v = y[4096:].reshape(48, 128)
    q = q / np.maximum(np.linalg.norm(q, axis=1, keepdims=True), 1e-6)
    k = k / np.maximum(np.linalg.norm(k, axis=1, keepdims=True), 1e-6)
    b = 1.0 / (1.0 + np.exp(-beta.astype(F64)))
    xa = alpha.astype(F64) + dt.astype(F64)
    sp = np.where(xa > 20.0, xa, np.log1p(np.exp(np.minimum(xa, 20.0))))
    gg = a.astype(F64) * sp
    S, o = gdn_step64(S, q, k, v, b, gg)
    o = o / np.sqrt(np.mean(o * o, axis=1, keepdims=True) + 1e-6) * norm.astype(F64)[None, :]
    zz = z.astype(F64).reshape(48, 128)
    o = o * (zz / (1.0 + np.exp(-zz)))
    return o.reshape(-1), new_cs.reshape(-1), S


def main():
    out = {}
    # ---- generator pin
    out["gen_seed"] = np.array([0x51333800], np.uint64)
    out["gen_words"] = synth.splitmix64(0x51333800, 0, 8)
    out["gen_normals"] = synth.normal(0x51333800, 8).astype(F64)

    # ---- attention, 256 positions (24 q / 4 kv heads, head_dim 256), with and without gate
    P = 256
    q = synth.normal(0x51333801, 6144)
    K = synth.normal(0x51333802, P * 1024)
    V = synth.normal(0x51333803, P * 1024)
    G = synth.normal(0x51333804, 6144)
    out["attn256_nogate"] = attention64(q, K, V)
    out["attn256_gate"] = attention64(q, K, V, G)

    # ---- full_core at position 37 with 37 cached rows in slot 1 (layer 7)
    pos = 37
    qn = synth.normal(0x51333811, 256, sigma=0.2, mean=1.0)
    kn = synth.normal(0x51333812, 256, sigma=0.2, mean=1.0)
    qg = synth.normal(0x51333813, 12288)
    key = synth.normal(0x51333814, 1024)
    val = synth.normal(0x51333815, 1024)
    Kc = synth.normal(0x51333816, pos * 1024)
    Vc = synth.normal(0x51333817, pos * 1024)
    src = qg.astype(F64).reshape(24, 512)
    qq = np.concatenate([src[h, :256] * rms_scale64(src[h, :256]) * qn for h in range(24)])
    kk = np.concatenate([key[h * 256:(h + 1) * 256] * rms_scale64(key[h * 256:(h + 1) * 256]) * kn
                         for h in range(4)])
    qq, _ = rope64(qq, 24, pos)
    kk, _ = rope64(kk, 4, pos)
    Kall = np.concatenate([Kc.astype(F64), kk]).reshape(pos + 1, 1024)
    Vall = np.concatenate([Vc.astype(F64), val.astype(F64)]).reshape(pos + 1, 1024)
    out["full_core37"] = attention64(qq, Kall, Vall, src[:, 256:])
    out["full_core37_k"] = kk

    # ---- RoPE and primitive values
    x = synth.normal(0x51333821, 512)
    for p in (0, 1, 1000, 131071):
        out[f"rope_{p}"], theta = rope64(x, 2, p)
        out[f"rope_theta_{p}"] = theta.astype(F64)
    sp_in = np.array([-30, -1, 0, 1, 19.9, 20, 20.5, 50, 100], np.float32)
    out["softplus_in"] = sp_in.astype(F64)
    out["softplus"] = np.where(sp_in > 20, sp_in.astype(F64), np.log1p(np.exp(np.minimum(sp_in, 20).astype(F64))))
    v = synth.normal(0x51333822, 256)
    out["rms_scale_256"] = np.array([rms_scale64(v)])

    # ---- DeltaNet: 64 steps of the recurrence from S ~ N(0, 0.02^2)
    T = 64
    S = synth.normal(0x51333831, 48 * 128 * 128, sigma=0.02).astype(F64).reshape(48, 128, 128)
    gen = synth.GdnStepInputs(0x51333832)
    outs = []
    for t in range(T):
        S, o = gdn_step64(S, *gen.step(t))
        outs.append(o)
    rng = np.random.default_rng(7)
    idx = np.sort(rng.choice(S.size, 4096, replace=False))
    out["gdn64_sample_idx"] = idx.astype(np.int64)
    out["gdn64_state_sample"] = S.reshape(-1)[idx]
    out["gdn64_state_head_sumsq"] = (S * S).sum(axis=(1, 2))
    out["gdn64_out_last"] = outs[-1].reshape(-1)
    out["gdn64_out_head0"] = np.stack([o[0] for o in outs])
    out["gdn64_out_head17"] = np.stack([o[17] for o in outs])

    # ---- linear_core whole, 4 tokens
    conv_w = synth.normal(0x51333841, 10240 * 4, sigma=0.5)
    dt = synth.normal(0x51333842, 48)
    a = -np.abs(synth.normal(0x51333843, 48))
    norm = synth.normal(0x51333844, 128, sigma=0.1, mean=1.0)
    cs = synth.normal(0x51333845, 10240 * 3).astype(F64)
    S = synth.normal(0x51333846, 48 * 128 * 128, sigma=0.02).astype(F64).reshape(48, 128, 128)
    louts = []
    for t in range(4):
        qkv = synth.normal(0x51333850 + t, 10240)
        z = synth.normal(0x51333860 + t, 6144)
        b = synth.normal(0x51333870 + t, 48)
        al = synth.normal(0x51333880 + t, 48)
        o, cs, S = linear_core64(conv_w, dt, a, norm, cs, S, qkv, z, b, al)
        louts.append(o)
    out["linear4_out"] = np.stack(louts)
    out["linear4_state_sample"] = S.reshape(-1)[idx]

    # outputs are compared at tolerances >= 1e-5: float32 keeps them exactly
    # enough and halves the file
    for name in list(out):
        if out[name].dtype == F64 and not name.startswith(("gdn64_state", "linear4_state", "gen_")):
            out[name] = out[name].astype(np.float32)

    path = os.path.join(HERE, "attention_path.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {os.path.getsize(path)} bytes, {len(out)} arrays")


if __name__ == "__main__":
    main()
