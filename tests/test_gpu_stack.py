"""The 64-layer hybrid as a stack: one decode token through the attention
path of every layer, in forward_token's layer order (src/model/ops.rs:1701-1736
-> layer_forward :1555-1625), against the restatement.

Layers with (layer + 1) % 4 == 0 run full_core (ops.rs:813-940) on KV slot
layer/4; the other 48 run linear_core (ops.rs:648-742) on their own conv and
DeltaNet states (recurrent index layer - (layer + 1)/4, ops.rs:43-47).  The
projections between layers are outside the path, so every layer reads its
own seeded inputs; what the stack checks is that 16 slots, 48 state pairs
and two consecutive tokens keep to their own memory and come out as the
reference's layer loop leaves them."""
import numpy as np
import pytest
from parity import check_attn, check_state

pytestmark = pytest.mark.gpu

STATE = 48 * 128 * 128
CONV = 10240 * 3


def _fill(ctx, buf, n, seed, sigma=1.0, mean=0.0):
    ctx.fill_normal(buf, n, seed, sigma=sigma, mean=mean)
    return buf.download().reshape(-1)[:n].copy()


def test_stack_64_layers_two_tokens(pkg, ctx, ref, margin, synth):
    """8192-token context (16 slots of 8190 cached rows), two decode tokens at
    positions 8190 and 8191 through all 64 layers; every layer's output, the
    appended rows of every slot, and the final conv and DeltaNet states."""
    C = 8192
    base = C - 2
    full_layers = [layer for layer in range(64) if (layer + 1) % 4 == 0]
    lin_layers = [layer for layer in range(64) if (layer + 1) % 4 != 0]
    assert [ref.lib().q38r_recurrent_index(layer) for layer in lin_layers] == list(range(48))
    kv = pkg.KVCache(ctx, n_slots=16, max_pages=C // 16, max_seqs=1, max_tokens_per_seq=C)
    try:
        seq = kv.seq_create()
        kc = np.zeros(16 * C * 1024, np.float32)
        vc = np.zeros(16 * C * 1024, np.float32)
        rows_k, rows_v = ctx.empty((C, 1024)), ctx.empty((C, 1024))
        for i, layer in enumerate(full_layers):
            kc[i * C * 1024: i * C * 1024 + base * 1024] = _fill(ctx, rows_k, base * 1024, 0xA000 + 2 * i)
            vc[i * C * 1024: i * C * 1024 + base * 1024] = _fill(ctx, rows_v, base * 1024, 0xA001 + 2 * i)
            kv.write(layer, seq, 0, base, rows_k, rows_v)
        rows_k.free()
        rows_v.free()
        d_states, d_conv = ctx.empty((48 * STATE,)), ctx.empty((48 * CONV,))
        s_ref = _fill(ctx, d_states, 48 * STATE, 0xA100, sigma=0.02).reshape(48, STATE)
        c_ref = _fill(ctx, d_conv, 48 * CONV, 0xA101).reshape(48, CONV)
        # per-layer weights
        norms = {layer: (synth.normal(0xA200 + layer, 256, sigma=0.2, mean=1.0),
                         synth.normal(0xA300 + layer, 256, sigma=0.2, mean=1.0)) for layer in full_layers}
        lw = {layer: (synth.normal(0xA400 + layer, 40960, sigma=0.5), synth.normal(0xA500 + layer, 48),
                      -np.abs(synth.normal(0xA600 + layer, 48)), synth.normal(0xA700 + layer, 128, sigma=0.1,
                                                                            mean=1.0))
              for layer in lin_layers}
        d_norms = {layer: tuple(ctx.array(x) for x in w) for layer, w in norms.items()}
        d_lw = {layer: tuple(ctx.array(x) for x in w) for layer, w in lw.items()}
        d_out = ctx.empty((6144,))
        worst_full, worst_lin = (0.0, 0.0), (0.0, 0.0)
        from parity import abs_rel
        for tok in range(2):
            pos = base + tok
            for layer in range(64):
                sd = 0xB000 + 256 * tok + 4 * layer
                if (layer + 1) % 4 == 0:
                    qg = synth.normal(sd, 12288)
                    key = synth.normal(sd + 1, 1024)
                    val = synth.normal(sd + 2, 1024)
                    qn, kn = norms[layer]
                    kv.full_core(layer, [seq], [pos], *d_norms[layer], ctx.array(qg), ctx.array(key),
                                 ctx.array(val), d_out)
                    want, _ = ref.full_core(qn, kn, qg, key, val, kc, vc, C, pos, layer, threads=16)
                    worst_full = tuple(max(a, b) for a, b in zip(worst_full, abs_rel(d_out.download(), want)))
                else:
                    li = ref.lib().q38r_recurrent_index(layer)
                    qkv = synth.normal(sd, 10240)
                    z = synth.normal(sd + 1, 6144)
                    beta = synth.normal(sd + 2, 48)
                    alpha = synth.normal(sd + 3, 48)
                    ctx.linear_core(1, 1, *d_lw[layer], d_conv.offset(li * CONV), d_states.offset(li * STATE),
                                    ctx.array(qkv), ctx.array(z), ctx.array(beta), ctx.array(alpha), d_out)
                    want = ref.linear_core(*lw[layer], c_ref[li], s_ref[li], qkv, z, beta, alpha, threads=16)
                    worst_lin = tuple(max(a, b) for a, b in zip(worst_lin, abs_rel(d_out.download(), want)))
        margin("full-attention layers out max-abs", worst_full[0], 1e-3)
        margin("full-attention layers out rel", worst_full[1], 1e-3)
        margin("DeltaNet layers out max-abs", worst_lin[0], 1e-3)
        # the two appended rows of every slot, as the reference's cache holds them
        r_k, r_v = ctx.empty((2, 1024)), ctx.empty((2, 1024))
        worst_row = 0.0
        for i, layer in enumerate(full_layers):
            kv.read(layer, seq, base, 2, r_k, r_v)
            at = (i * C + base) * 1024
            worst_row = max(worst_row, float(np.max(np.abs(r_k.download().reshape(-1) - kc[at:at + 2048]))))
            assert np.array_equal(r_v.download().reshape(-1), vc[at:at + 2048]), layer
        margin("appended key rows max-abs", worst_row, 1e-5)
        # conv states bit-exact, DeltaNet states within the state tolerance
        assert np.array_equal(d_conv.download().reshape(48, CONV), c_ref)
        got_s = d_states.download().reshape(48, STATE)
        check_state(margin, got_s, s_ref, "48 DeltaNet states")
    finally:
        kv.close()


@pytest.mark.parametrize("layer", [63, 64])
def test_full_core_131072_last_slots(pkg, ctx, ref, margin, layer):
    """full_core at position 131071 (131071 cached tokens) on slot 15 (layer
    63) and slot 16 (the MTP layer 64) of a 17-slot cache sized for 128K
    tokens: the benchmark's fused launch at pool offsets past 4 GiB (slot 15
    starts 7.5 GiB into each pool).  The restatement runs the same layer core
    on a one-slot cache holding the same rows."""
    from q38amd import synth
    C = 131072
    pos = C - 1
    kv = pkg.KVCache(ctx, n_slots=17, max_pages=C // 16, max_seqs=1, max_tokens_per_seq=C)
    try:
        seq = kv.seq_create()
        rows_k, rows_v = ctx.empty((C, 1024)), ctx.empty((C, 1024))
        rows_k.zero()
        rows_v.zero()
        ctx.fill_normal(rows_k, pos * 1024, 0xC000 + layer)
        ctx.fill_normal(rows_v, pos * 1024, 0xC100 + layer)
        kv.write(layer, seq, 0, pos, rows_k, rows_v)
        kc = rows_k.download().reshape(-1)
        vc = rows_v.download().reshape(-1)
        rows_k.free()
        rows_v.free()
        qn = synth.normal(0xC200, 256, sigma=0.2, mean=1.0)
        kn = synth.normal(0xC201, 256, sigma=0.2, mean=1.0)
        qg = synth.normal(0xC202 + layer, 12288)
        key = synth.normal(0xC203 + layer, 1024)
        val = synth.normal(0xC204 + layer, 1024)
        d_o = ctx.empty((24, 256))
        kv.full_core(layer, [seq], [pos], ctx.array(qn), ctx.array(kn), ctx.array(qg), ctx.array(key),
                     ctx.array(val), d_o)
        want, k_formed = ref.full_core(qn, kn, qg, key, val, kc, vc, C, pos, 3, threads=16)
        check_attn(margin, d_o.download(), want)
        r_k, r_v = ctx.empty((1, 1024)), ctx.empty((1, 1024))
        kv.read(layer, seq, pos, 1, r_k, r_v)
        margin("appended key max-abs", float(np.max(np.abs(r_k.download().reshape(-1) - k_formed))), 1e-5)
        assert np.array_equal(r_v.download().reshape(-1), val)
    finally:
        kv.close()
