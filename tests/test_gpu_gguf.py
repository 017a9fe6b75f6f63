"""The model file on the device: q38_gguf_upload places every tensor's bytes
at base + offset (compared byte for byte with the file), the uploaded
matrices feed q38_gemv_q8_k and the uploaded norm weight feeds full_core
directly; and the recurrent-state checkpoint (src/model/ops.rs:1627-1647)
restores the states bit for bit after steps that changed them."""
import numpy as np
import pytest

import gguf_files as gf
from oracle_checks import _random_kquant
from parity import check_attn

pytestmark = pytest.mark.gpu


def test_upload_places_every_tensor(pkg, ctx, ref, tmp_path):
    rows, W = 96, 5120
    wq = _random_kquant(12, rows, W, 0x51334000)
    w6 = _random_kquant(14, 40, 1024, 0x51334001)
    norm = np.random.default_rng(0x51334002).standard_normal(256).astype(np.float32)
    tensors = [("blk.3.attn_q_norm.weight", 0, [256], norm.tobytes()),
               ("blk.3.attn_q.weight", 12, [W, rows], wq.tobytes()),
               ("blk.3.ffn_down.weight", 14, [1024, 40], w6.tobytes()),
               ("blk.3.odd.weight", 8, [32, 3], gf.tensor_bytes(8, [32, 3], 5))]
    blob, offsets, data_offset = gf.build(tensors, alignment=64)
    path = tmp_path / "m.gguf"
    path.write_bytes(blob)
    with pkg.Gguf(str(path)) as g:
        base, nbytes = g.upload(ctx)
        try:
            end = max(o + n for o, n in offsets.values())
            assert nbytes == end
            h = np.empty(nbytes, np.uint8)
            pkg.lib().q38_download(ctx.handle, h.ctypes.data, base, nbytes)
            assert h.tobytes() == blob[data_offset:data_offset + end]
            # the uploaded Q4_K matrix through the GEMV, in place
            t = g.tensor(g.find_tensor("blk.3.attn_q.weight"))
            assert t["shape"] == [W, rows] and (base + t["offset"]) % 16 == 0
            x = np.random.default_rng(0x51334003).standard_normal((2, W)).astype(np.float32)
            d_x = ctx.array(x)
            d_q = ctx.empty((ctx.q8k_bytes(2, W),), np.uint8)
            ctx.quantize_q8_k(2, W, d_x, d_q)
            d_o = ctx.empty((2, rows))
            ctx.gemv_q8_k(t["type"], rows, W, base + t["offset"], d_q, 2, d_o)
            want = ref.gemv_q8_k(12, wq, ref.quantize_q8_k(x), 2, W, threads=16)
            assert np.array_equal(d_o.download().view(np.uint32), want.view(np.uint32))
            t6 = g.tensor(g.find_tensor("blk.3.ffn_down.weight"))
            x6 = np.random.default_rng(0x51334004).standard_normal((1, 1024)).astype(np.float32)
            d_x6 = ctx.array(x6)
            d_q6 = ctx.empty((ctx.q8k_bytes(1, 1024),), np.uint8)
            ctx.quantize_q8_k(1, 1024, d_x6, d_q6)
            d_o6 = ctx.empty((1, 40))
            ctx.gemv_q8_k(14, 40, 1024, base + t6["offset"], d_q6, 1, d_o6)
            want6 = ref.gemv_q8_k(14, w6, ref.quantize_q8_k(x6), 1, 1024, threads=16)
            assert np.array_equal(d_o6.download().view(np.uint32), want6.view(np.uint32))
        finally:
            pkg.lib().q38_free(ctx.handle, base)


def test_uploaded_norm_feeds_full_core(pkg, ctx, ref, margin, synth, tmp_path):
    """q_norm and k_norm read as F32 tensors from the uploaded file
    (scalar()/f32_at(), ops.rs:456-473, read them from the mapping)."""
    qn = synth.normal(0x51334010, 256, sigma=0.2, mean=1.0)
    kn = synth.normal(0x51334011, 256, sigma=0.2, mean=1.0)
    blob, offsets, _ = gf.build([("blk.3.attn_q_norm.weight", 0, [256], qn.tobytes()),
                                 ("blk.3.attn_k_norm.weight", 0, [256], kn.tobytes())])
    path = tmp_path / "n.gguf"
    path.write_bytes(blob)
    layer, ctx_len, pos = 3, 256, 100
    K0 = synth.normal(0x51334012, pos * 1024)
    V0 = synth.normal(0x51334013, pos * 1024)
    qg = synth.normal(0x51334014, 12288)
    key = synth.normal(0x51334015, 1024)
    val = synth.normal(0x51334016, 1024)
    with pkg.Gguf(str(path)) as g:
        base, _ = g.upload(ctx)
        kv = pkg.KVCache(ctx, n_slots=1, max_pages=ctx_len // 16, max_seqs=1, max_tokens_per_seq=ctx_len)
        try:
            seq = kv.seq_create()
            kv.write(layer, seq, 0, pos, ctx.array(K0), ctx.array(V0))
            d_o = ctx.empty((24, 256))
            kv.full_core(layer, [seq], [pos], base + offsets["blk.3.attn_q_norm.weight"][0],
                         base + offsets["blk.3.attn_k_norm.weight"][0], ctx.array(qg), ctx.array(key),
                         ctx.array(val), d_o)
            kc = np.zeros(ctx_len * 1024, np.float32)
            vc = np.zeros(ctx_len * 1024, np.float32)
            kc[:pos * 1024] = K0
            vc[:pos * 1024] = V0
            want, _ = ref.full_core(qn, kn, qg, key, val, kc, vc, ctx_len, pos, layer, threads=16)
            check_attn(margin, d_o.download(), want)
        finally:
            kv.close()
            pkg.lib().q38_free(ctx.handle, base)


def test_recurrent_checkpoint_restore(pkg, ctx, synth):
    """checkpoint -> two linear_core tokens (the states change) -> restore:
    the states are the checkpointed ones bit for bit, and a repeated token
    from the restored state reproduces the first run's output."""
    n_conv, n_delta = 48 * 30720, 48 * 786432
    conv = ctx.empty((n_conv,))
    delta = ctx.empty((n_delta,))
    ctx.fill_normal(conv, n_conv, 0x51334020)
    ctx.fill_normal(delta, n_delta, 0x51334021, sigma=0.02)
    ck_conv, ck_delta = ctx.empty((n_conv,)), ctx.empty((n_delta,))
    conv0, delta0 = conv.download(), delta.download()
    pkg.recurrent_checkpoint(ctx, conv, delta, n_conv, n_delta, ck_conv, ck_delta)
    assert np.array_equal(ck_conv.download().view(np.uint32), conv0.view(np.uint32))
    assert np.array_equal(ck_delta.download().view(np.uint32), delta0.view(np.uint32))

    w = {k: ctx.array(synth.normal(0x51334030 + i, n)) for i, (k, n) in
         enumerate((("conv_w", 40960), ("dt", 48), ("a", 48), ("norm", 128)))}
    ins = [{k: synth.normal(0x51334040 + 8 * t + i, n) for i, (k, n) in
            enumerate((("qkv", 10240), ("z", 6144), ("beta", 48), ("alpha", 48)))} for t in range(2)]
    r = 5  # the recurrent index of the layer

    def token(inp):
        out = ctx.empty((6144,))
        ctx.linear_core(1, 1, w["conv_w"], w["dt"], w["a"], w["norm"], conv.offset(r * 30720),
                        delta.offset(r * 786432), ctx.array(inp["qkv"]), ctx.array(inp["z"]),
                        ctx.array(inp["beta"]), ctx.array(inp["alpha"]), out)
        return out.download()

    first = token(ins[0])
    token(ins[1])
    assert not np.array_equal(delta.download(), delta0)
    pkg.recurrent_restore(ctx, ck_conv, ck_delta, n_conv, n_delta, conv, delta)
    assert np.array_equal(conv.download().view(np.uint32), conv0.view(np.uint32))
    assert np.array_equal(delta.download().view(np.uint32), delta0.view(np.uint32))
    again = token(ins[0])
    assert np.array_equal(again.view(np.uint32), first.view(np.uint32))
    with pytest.raises(pkg.Q38Error, match="multiples of 4"):
        pkg.recurrent_checkpoint(ctx, conv, delta, 6, n_delta, ck_conv, ck_delta)
