"""The weight projections on the GPU (q38_quantize_q8_k, q38_gemv_q8_k,
q38_gemv_f32) against the oracle's restatement of quantize_q8_k
(src/kernel/quant.rs:55-128), of the scalar Q2_K..Q6_K x Q8_K row dots
(src/kernel/tensor.rs:301-457) and the IQ ones -- IQ4_NL, IQ4_XS, IQ3_S,
IQ3_XXS, IQ2_XXS, IQ2_XS, IQ2_S, IQ1_S, IQ1_M (src/kernel/iq.rs:355-667)
driven per row as tensor_gemv_q8_k / tensor_gemm_q8_k do
(tensor.rs:1131-1173, :1217-1270), and of the f32-input row dots of
tensor_gemv_f32 (tensor.rs:79-117, :1095-1129).  The integer parts and the
f32 block terms follow the reference's operation order, so the Q8_K path is
held bit-exact; the f32 path's sums are reassociated and held within 1e-5
of the sum of |w x|."""
import numpy as np
import pytest
from oracle_checks import _random_f32_path, _random_kquant
from parity import check_attn

pytestmark = pytest.mark.gpu

TYPES = {"Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ4_NL": 20, "IQ4_XS": 23,
         "IQ2_XXS": 16, "IQ2_XS": 17, "IQ2_S": 22, "IQ3_XXS": 18, "IQ3_S": 21, "IQ1_S": 19, "IQ1_M": 29}
F32_TYPES = {"F32": 0, "F16": 1, "BF16": 30, "Q8_0": 8}
HIDDEN = 5120


def _activations(T, W, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((T, W)) * rng.uniform(0.1, 4.0, (T, 1))).astype(np.float32)
    if T > 1:
        x[1] = ((np.arange(W) * 7919) % 101) / np.float32(50.0) - np.float32(1.0)  # tensor.rs:582-586
    if W >= 512:
        x[0, 256:512] = 0.0                      # an all-zero block
        x[0, 600] = -9.0
        x[0, 601] = 9.0                          # a |max| tie in block 2: the first sets the sign
    return x


def _quantize_on_device(ctx, x):
    T, W = x.shape
    d_x = ctx.array(x)
    d_q = ctx.empty((ctx.q8k_bytes(T, W),), np.uint8)
    ctx.quantize_q8_k(T, W, d_x, d_q)
    return d_q


@pytest.mark.parametrize("T,W", [(1, 256), (3, HIDDEN), (9, 17408)])
def test_quantize_q8_k_bit_exact(ctx, ref, T, W):
    x = _activations(T, W, 0x51333880 + W)
    got = _quantize_on_device(ctx, x).download()
    want = ref.quantize_q8_k(x)
    assert got.shape == want.shape
    assert np.array_equal(got, want)


@pytest.mark.parametrize("name", sorted(TYPES))
@pytest.mark.parametrize("rows,W,T", [(257, HIDDEN, 1), (61, 768, 3), (33, 1280, 9), (4, 256, 17),
                                      (1100, 17408, 4), (517, 17408, 8), (700, 2304, 1)])
def test_gemv_q8_k_bit_exact(ctx, ref, name, rows, W, T):
    """Row counts that leave a partial last workgroup, several token passes
    (9 and 17 tokens), a width whose token passes hold at most 3 tokens
    (17408: 8 tokens as passes of 3, 3 and 2, the passes of a row group
    numbered 8 workgroups apart over a row-group count that is not a
    multiple of 8), and matrices small enough to get one row per
    workgroup."""
    ty = TYPES[name]
    x = _activations(T, W, 0x51333890 + T)
    d_q = _quantize_on_device(ctx, x)
    wb = _random_kquant(ty, rows, W, 0x513338A0 + ty + rows)
    d_w = ctx.array(wb, np.uint8)
    d_o = ctx.empty((T, rows))
    ctx.gemv_q8_k(ty, rows, W, d_w, d_q, T, d_o)
    got = d_o.download()
    want = ref.gemv_q8_k(ty, wb, ref.quantize_q8_k(x), T, W, threads=16)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), float(np.max(np.abs(got - want)))


@pytest.mark.parametrize("name", sorted(TYPES))
def test_gemv_q8_k_subnormal_scales_and_widest_rows(ctx, ref, name):
    """f16 block scales that are subnormal (m * 2^-24) or zero, and the widest
    accepted row (49152 weights, 192 blocks: one token per pass)."""
    ty = TYPES[name]
    for rows, W, T in ((45, 1024, 2), (5, 49152, 2)):
        x = _activations(T, W, 0x513338A8 + W)
        d_q = _quantize_on_device(ctx, x)
        wb = _random_kquant(ty, rows, W, 0x513338A9 + ty)
        blocks = wb.reshape(rows * (W // 256), -1)
        off = {14: 208, 11: 108, 10: 80}.get(ty, 0)  # the block's (first) f16 scale
        sub = np.array([0x0001, 0x03ff, 0x8200, 0x0000, 0x8000], np.uint16)
        for i in range(0, blocks.shape[0], 3):
            if ty == 29:  # IQ1_M: the f16 is the top nibbles of the halfwords at 48, 50, 52, 54
                for k in range(4):
                    nib = (int(sub[i % 5]) >> (4 * k)) & 15
                    blocks[i, 49 + 2 * k] = (blocks[i, 49 + 2 * k] & 0x0F) | (nib << 4)
            else:
                blocks[i, off:off + 2] = np.frombuffer(sub[i % 5].tobytes(), np.uint8)
        if ty in (12, 13):  # dmin
            blocks[1::4, 2:4] = np.frombuffer(np.uint16(0x0155).tobytes(), np.uint8)
        d_w = ctx.array(wb, np.uint8)
        d_o = ctx.empty((T, rows))
        ctx.gemv_q8_k(ty, rows, W, d_w, d_q, T, d_o)
        want = ref.gemv_q8_k(ty, wb, ref.quantize_q8_k(x), T, W, threads=16)
        assert np.array_equal(d_o.download().view(np.uint32), want.view(np.uint32)), (rows, W, T)


@pytest.mark.parametrize("name", sorted(TYPES))
def test_gemv_q8_k_model_shapes(ctx, ref, name):
    """One token through an FFN-sized matrix (17408 rows of 5120)."""
    ty = TYPES[name]
    rows, W = 17408, HIDDEN
    x = _activations(1, W, 0x513338B0)
    d_q = _quantize_on_device(ctx, x)
    wb = _random_kquant(ty, rows, W, 0x513338B1 + ty)
    d_w = ctx.array(wb, np.uint8)
    d_o = ctx.empty((1, rows))
    ctx.gemv_q8_k(ty, rows, W, d_w, d_q, 1, d_o)
    want = ref.gemv_q8_k(ty, wb, ref.quantize_q8_k(x), 1, W, threads=16)
    assert np.array_equal(d_o.download().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name", sorted(TYPES))
@pytest.mark.parametrize("T", [1, 3, 9, 40])
def test_gemv_multi_equals_single(ctx, ref, name, T):
    """Several matrices on one input in one launch (q|gate, k, v of a layer
    are 12288, 1024, 1024 rows; here smaller, with an empty matrix and a
    one-row one): every output bit for bit as the single-matrix launch and
    the oracle.  At 40 tokens the three share one split-block launch."""
    ty = TYPES[name]
    W = 1280
    x = _activations(T, W, 0x513338E0 + T)
    d_q = _quantize_on_device(ctx, x)
    q8 = ref.quantize_q8_k(x)
    rows = [1500, 0, 96, 1]
    wbs = [_random_kquant(ty, max(r, 1), W, 0x513338E1 + ty + i)[:r] for i, r in enumerate(rows)]
    d_ws = [ctx.array(wb, np.uint8) if r else None for wb, r in zip(wbs, rows)]
    d_os = [ctx.empty((T, max(r, 1))) for r in rows]
    ctx.gemv_q8_k_multi(ty, rows, W, d_ws, d_q, T, d_os)
    for wb, r, d_w, d_o in zip(wbs, rows, d_ws, d_os):
        if r == 0:
            continue
        got = d_o.download()
        single = ctx.empty((T, r))
        ctx.gemv_q8_k(ty, r, W, d_w, d_q, T, single)
        assert np.array_equal(got.view(np.uint32), single.download().view(np.uint32))
        want = ref.gemv_q8_k(ty, wb, q8, T, W, threads=16)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name", sorted(TYPES))
@pytest.mark.parametrize("rows,W,T", [([1500, 0, 96, 1], 1280, 1), ([257, 64], HIDDEN, 3),
                                      ([300, 40], 17408, 9), ([1500, 96], 1280, 40)])
def test_quantize_project_equals_separate_calls(ctx, ref, name, rows, W, T):
    """quantize_input then project in one call (q38_quantize_project_q8_k):
    every output and every byte of the quantised input as
    q38_quantize_q8_k + q38_gemv_q8_k_multi, and the oracle.  For one token
    the GEMV quantises the input itself (the first row group storing it);
    from two tokens (3 and 9 here, the latter 17408 wide) and where a matrix
    takes the matrix unit (the 1500-row one at 40 tokens) the input is
    quantised by its own launch first."""
    ty = TYPES[name]
    x = _activations(T, W, 0x51333900 + T + W)
    d_x = ctx.array(x)
    q8 = ref.quantize_q8_k(x)
    wbs = [_random_kquant(ty, max(r, 1), W, 0x51333901 + ty + i)[:r] for i, r in enumerate(rows)]
    d_ws = [ctx.array(wb, np.uint8) if r else None for wb, r in zip(wbs, rows)]
    nq = ctx.q8k_bytes(T, W)
    d_q_sep = ctx.empty((nq,), np.uint8)
    d_q_fused = ctx.empty((nq,), np.uint8)
    ctx.fill_normal(d_q_fused, nq // 4, 0x5133390F)  # stale bytes that the call must overwrite
    outs_sep = [ctx.empty((T, max(r, 1))) for r in rows]
    outs_fused = [ctx.empty((T, max(r, 1))) for r in rows]
    ctx.quantize_q8_k(T, W, d_x, d_q_sep)
    ctx.gemv_q8_k_multi(ty, rows, W, d_ws, d_q_sep, T, outs_sep)
    ctx.quantize_project_q8_k(ty, rows, W, d_ws, d_x, T, d_q_fused, outs_fused)
    assert np.array_equal(d_q_fused.download(), d_q_sep.download())
    assert np.array_equal(d_q_fused.download(), q8)
    for wb, r, a_, b_ in zip(wbs, rows, outs_sep, outs_fused):
        if r == 0:
            continue
        got = b_.download()
        assert np.array_equal(got.view(np.uint32), a_.download().view(np.uint32))
        want = ref.gemv_q8_k(ty, wb, q8, T, W, threads=16)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name", sorted(TYPES))
@pytest.mark.parametrize("rows,W,T", [(130, 1280, 32), (2050, 256, 33), (1100, 1280, 65), (700, HIDDEN, 130),
                                      (2100, 2304, 64), (8200, 256, 16), (4200, 2304, 40), (4100, 768, 1000)])
def test_gemm_many_tokens_bit_exact(ctx, ref, name, rows, W, T):
    """The matrix-unit forms from 8 tokens on, bit for bit against the
    oracle, with partial row and token tiles.  The split-block form (32 rows
    x 32 tokens per workgroup, a row's blocks split over the waves) where
    its grid has 64 to 1280 workgroups: on 16 waves up to 256 workgroups
    (1, 5, 9 and 20 blocks, so the last round is partial), on 8 beyond
    (8200 x 16 with 1 block, 4200 x 40 with 9); 4100 x 1000 (4128 such
    workgroups) takes the 128-row x 64-token tiles, as IQ4_NL does from 32
    tokens (16 for 8192+ rows); 130 x 1280 (5 workgroups) stays on the
    GEMV."""
    ty = TYPES[name]
    x = _activations(T, W, 0x513338F0 + T + W)
    d_q = _quantize_on_device(ctx, x)
    wb = _random_kquant(ty, rows, W, 0x513338F1 + ty + rows)
    d_w = ctx.array(wb, np.uint8)
    d_o = ctx.empty((T, rows))
    ctx.gemv_q8_k(ty, rows, W, d_w, d_q, T, d_o)
    got = d_o.download()
    want = ref.gemv_q8_k(ty, wb, ref.quantize_q8_k(x), T, W, threads=16)
    bad = np.flatnonzero(got.view(np.uint32).reshape(-1) != want.view(np.uint32).reshape(-1))
    assert bad.size == 0, (bad.size, bad[:5], got.reshape(-1)[bad[:5]], want.reshape(-1)[bad[:5]])


def _ran(ctx, kernel, call):
    """Whether call() launched kernel (the library's per-dispatch timer)."""
    ctx.kernel_timer_start(kernel, 8)
    call()
    _, n = ctx.kernel_timer_stop()
    return n > 0


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K", "IQ2_S", "IQ4_NL"])
def test_projection_path_boundaries(ctx, ref, name):
    """The library's choice between the GEMV and the matrix-unit forms at
    each of its boundaries (8 tokens; 64 split-block workgroups of 32 rows
    x 32 tokens; one workgroup per CU for the 16-wave form, 1.5 for the
    8-wave one, 5 for the 4-wave one, past which the 128 x 64 tiles run):
    the expected kernel runs on each side, and
    every output is the oracle's bit for bit.  IQ4_NL has no split-block
    form and takes the 128 x 64 tiles from 32 tokens (16 for 8192+ rows)."""
    ty = TYPES[name]
    sfx = {"Q4_K": "q4k", "Q6_K": "q6k", "IQ2_S": "iq2s", "IQ4_NL": "iq4nl"}[name]
    cus = ctx.info()["cu_count"]
    W = 256
    cases = [  # rows, tokens, kernel expected
        (2048, 7, "q38_gemv_q8k_"), (2048, 8, "q38_gemm_ks16_q8k_"), (2016, 8, "q38_gemv_q8k_"),
        (32 * cus, 8, "q38_gemm_ks16_q8k_"), (32 * cus + 1, 8, "q38_gemm_ks_q8k_"),
        (48 * cus, 8, "q38_gemm_ks_q8k_"), (48 * cus + 1, 8, "q38_gemm_ks4_q8k_"),
        (32 * 5 * cus, 8, "q38_gemm_ks4_q8k_"), (32 * 5 * cus + 1, 8, "q38_gemm_q8k_"),
    ]
    if name == "IQ4_NL":
        cases = [(2048, 31, "q38_gemv_q8k_"), (2048, 32, "q38_gemm_q8k_"), (8191, 16, "q38_gemv_q8k_"),
                 (8192, 16, "q38_gemm_q8k_")]
    for rows, T, kern in cases:
        x = _activations(T, W, 0x51333A00 + T + rows)
        d_q = _quantize_on_device(ctx, x)
        wb = _random_kquant(ty, rows, W, 0x51333A01 + ty + rows)
        d_w = ctx.array(wb, np.uint8)
        d_o = ctx.empty((T, rows))
        assert _ran(ctx, kern + sfx, lambda: ctx.gemv_q8_k(ty, rows, W, d_w, d_q, T, d_o)), (rows, T, kern)
        want = ref.gemv_q8_k(ty, wb, ref.quantize_q8_k(x), T, W, threads=16)
        assert np.array_equal(d_o.download().view(np.uint32), want.view(np.uint32)), (rows, T)
        for arr in (d_q, d_w, d_o):
            arr.free()


@pytest.mark.parametrize("name", ["Q4_K", "Q5_K", "IQ3_S"])
def test_multi_matrices_share_the_split_block_launch(ctx, ref, name):
    """The path of a multi-matrix call at 8 tokens: a matrix past 5
    split-block workgroups per CU takes the 128 x 64 tiles on its own, and
    the others share one split-block launch when their grids add up to 64
    workgroups, though neither would take it alone (63 and 2); every output
    is the single-matrix call's and the oracle's bit for bit."""
    ty = TYPES[name]
    sfx = {"Q4_K": "q4k", "Q5_K": "q5k", "IQ3_S": "iq3s"}[name]
    cus = ctx.info()["cu_count"]
    W, T = 256, 8
    x = _activations(T, W, 0x51333B00)
    d_q = _quantize_on_device(ctx, x)
    q8 = ref.quantize_q8_k(x)
    rows = [2016, 160 * cus + 1, 0, 33]
    wbs = [_random_kquant(ty, max(r, 1), W, 0x51333B01 + ty + i)[:r] for i, r in enumerate(rows)]
    d_ws = [ctx.array(wb, np.uint8) if r else None for wb, r in zip(wbs, rows)]
    d_os = [ctx.empty((T, max(r, 1))) for r in rows]
    call = lambda: ctx.gemv_q8_k_multi(ty, rows, W, d_ws, d_q, T, d_os)
    assert _ran(ctx, "q38_gemm_q8k_" + sfx, call)
    assert _ran(ctx, "q38_gemm_ks16_q8k_" + sfx, call)
    assert not _ran(ctx, "q38_gemv_q8k_" + sfx, call)
    for i, (wb, r, d_w, d_o) in enumerate(zip(wbs, rows, d_ws, d_os)):
        if r == 0:
            continue
        got = d_o.download()
        want = ref.gemv_q8_k(ty, wb, q8, T, W, threads=16)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), r
        if i != 1:  # alone, the small matrices take the GEMV: the same bits
            single = ctx.empty((T, r))
            assert _ran(ctx, "q38_gemv_q8k_" + sfx, lambda: ctx.gemv_q8_k(ty, r, W, d_w, d_q, T, single))
            assert np.array_equal(got.view(np.uint32), single.download().view(np.uint32)), r


F32_PATH_SHAPES = [(48, HIDDEN, 1), (48, HIDDEN, 3), (257, 1024, 9), (5, 6144, 17), (1031, 2048, 1),
                   (48, HIDDEN, 64), (300, 1024, 100), (129, 768, 33), (64, 320, 16), (40, 1032, 20), (37, 64, 5),
                   (19, 17408, 2), (70, 14528, 3), (33, 6144, 15), (2048, 256, 512), (100, 1024, 9),
                   (70, 17408, 12), (4100, 128, 4096)]


@pytest.mark.parametrize("name,rows,W,T", [(n, r, w, t) for n in sorted(F32_TYPES) for r, w, t in F32_PATH_SHAPES
                                           if not (n == "Q8_0" and w % 64)])  # Q8_0 rows are 64k wide
def test_gemv_f32_path(ctx, ref, margin, name, rows, W, T):
    """tensor_gemv_f32 / tensor_gemm_f32 for the weight types project()
    does not quantise for (the 48-row beta / alpha projections of a DeltaNet
    layer and other shapes; several token passes; from 4 tokens on the
    matrix-unit forms, with partial row and token tiles and k ranges that
    leave a wave empty, and the GEMV where the width is not a multiple of
    64): every element within 1e-5 of the
    sum of |w x| of the oracle's sequential chain, and of the float64 dot of
    the weights decoded in numpy; a one-hot input row gives each weight
    exactly."""
    ty = F32_TYPES[name]
    sfx = {0: "f32", 1: "f16", 30: "bf16", 8: "q8_0"}[ty]
    if W % 64 or T < (9 if ty == 8 else 4):  # the GEMV; Q8_0: activations staged in LDS
        tp = min(t for t in (1, 2, 4, 8) if t >= min(T, 8))
        kern = "q38_gemv_f32_" + sfx + ("s_r%d_t%d" % (4 if tp == 8 else 2, tp) if ty == 8 else "")
    else:  # the matrix unit: k split over the waves up to 32 tokens or on small grids
        cus = ctx.info()["cu_count"]
        big_wgs = -(-rows // 128) * -(-T // 64)
        skinny = T <= 32 or 2 * big_wgs < cus
        wide = ty != 0 and -(-rows // 128) * -(-T // 128) >= 4 * cus  # 128-token tiles (not F32)
        kern = ("q38_gemm_f32s_" if skinny else "q38_gemm_f32w_" if wide else "q38_gemm_f32_") + sfx
    rng = np.random.default_rng(0x51333940 + ty + rows)
    x = rng.standard_normal((T, W)).astype(np.float32)
    if T > 1:
        x[1] = ((np.arange(W) * 7919) % 101) / np.float32(50.0) - np.float32(1.0)  # tensor.rs:582-586
        x[T - 1] = 0.0
        x[T - 1, W - 3] = 1.0
    wb, wv = _random_f32_path(ty, rows, W, 0x51333941 + ty + W)
    d_o = ctx.empty((T, rows))
    d_w, d_x = ctx.array(wb, np.uint8), ctx.array(x)
    assert _ran(ctx, kern, lambda: ctx.gemv_f32(ty, rows, W, d_w, d_x, T, d_o))
    got = d_o.download().astype(np.float64)
    want = ref.gemv_f32(ty, wb, x, threads=16).astype(np.float64)
    exact = x.astype(np.float64) @ wv.T
    scale = np.abs(x.astype(np.float64)) @ np.abs(wv).T
    margin("error vs oracle / sum of abs(w x)", np.max(np.abs(got - want) / (scale + 1e-30)), 1e-5)
    margin("error vs float64 dot / sum of abs(w x)", np.max(np.abs(got - exact) / (scale + 1e-30)), 1e-5)
    if T > 1:
        assert np.array_equal(got[T - 1], wv[:, W - 3].astype(np.float32).astype(np.float64))


def test_gemv_f32_argument_checks(pkg, ctx):
    w = ctx.empty((4096,), np.uint8)
    x = ctx.empty((1024,))
    o = ctx.empty((16,))
    with pytest.raises(pkg.Q38Error, match="unsupported weight type"):
        ctx.gemv_f32(12, 4, 256, w, x, 1, o)
    with pytest.raises(pkg.Q38Error, match="multiple of 8"):
        ctx.gemv_f32(0, 4, 100, w, x, 1, o)
    with pytest.raises(pkg.Q38Error, match="multiple of 64"):
        ctx.gemv_f32(8, 4, 96, w, x, 1, o)
    with pytest.raises(pkg.Q38Error, match="aligned"):
        ctx.gemv_f32(1, 4, 256, w.ptr + 2, x, 1, o)


def test_projection_argument_checks(pkg, ctx):
    x = ctx.empty((300,))
    q = ctx.empty((4096,), np.uint8)
    o = ctx.empty((16,))
    with pytest.raises(pkg.Q38Error, match="multiple of 256"):
        ctx.quantize_q8_k(1, 300, x, q)
    with pytest.raises(pkg.Q38Error, match="unsupported quant type"):
        ctx.gemv_q8_k(8, 4, 256, q, q, 1, o)
    with pytest.raises(pkg.Q38Error, match="multiple of 256"):
        ctx.gemv_q8_k(12, 4, 300, q, q, 1, o)
    with pytest.raises(pkg.Q38Error, match="above 49152"):
        ctx.gemv_q8_k(12, 4, 49408, q, q, 1, o)
    with pytest.raises(pkg.Q38Error, match="n_mats 5 outside"):
        ctx.gemv_q8_k_multi(12, [4] * 5, 256, [q] * 5, q, 1, [o] * 5)
    with pytest.raises(pkg.Q38Error, match="NULL weights or output"):
        ctx.gemv_q8_k_multi(12, [4, 4], 256, [q, None], q, 1, [o, o])
    with pytest.raises(pkg.Q38Error, match="multiple of 256"):
        pkg.Context.q8k_bytes(1, 100)
    with pytest.raises(pkg.Q38Error, match="d_x is NULL"):
        ctx.quantize_project_q8_k(12, [4], 256, [q], None, 1, q, [o])
    with pytest.raises(pkg.Q38Error, match="d_x must be 16-byte aligned"):
        ctx.quantize_project_q8_k(12, [4], 256, [q], x.offset(1), 1, q, [o])
    with pytest.raises(pkg.Q38Error, match="unsupported quant type"):
        ctx.quantize_project_q8_k(8, [4], 256, [q], x, 1, q, [o])
    # every matrix empty: only the quantisation runs
    xs = ctx.array(np.linspace(-2.0, 2.0, 256, dtype=np.float32))
    q2 = ctx.empty((ctx.q8k_bytes(1, 256),), np.uint8)
    ctx.quantize_project_q8_k(12, [0], 256, [None], xs, 1, q2, [None])
    q3 = ctx.empty((ctx.q8k_bytes(1, 256),), np.uint8)
    ctx.quantize_q8_k(1, 256, xs, q3)
    assert np.array_equal(q2.download(), q3.download())


def test_projections_feed_full_core(pkg, ctx, ref, margin, synth):
    """The reference's full_attention (ops.rs:942-982) around full_core: the
    layer input quantised once (quantize_input), q|gate (12288 rows, Q4_K),
    k and v (1024 rows each, Q6_K) projected on the device and handed to
    q38_full_core as device pointers, against the oracle running the same
    chain."""
    layer, ctx_len, pos = 3, 2048, 1500
    x = _activations(1, HIDDEN, 0x513338C0)
    wq = _random_kquant(12, 12288, HIDDEN, 0x513338C1)
    wk = _random_kquant(14, 1024, HIDDEN, 0x513338C2)
    wv = _random_kquant(14, 1024, HIDDEN, 0x513338C3)
    qn = synth.normal(0x513338C4, 256, sigma=0.2, mean=1.0)
    kn = synth.normal(0x513338C5, 256, sigma=0.2, mean=1.0)
    K0 = synth.normal(0x513338C6, pos * 1024)
    V0 = synth.normal(0x513338C7, pos * 1024)
    kv = pkg.KVCache(ctx, n_slots=1, max_pages=ctx_len // 16, max_seqs=1, max_tokens_per_seq=ctx_len)
    try:
        seq = kv.seq_create()
        d_k0, d_v0 = ctx.array(K0), ctx.array(V0)
        kv.write(layer, seq, 0, pos, d_k0, d_v0)
        d_q8 = _quantize_on_device(ctx, x)
        d_qg, d_key, d_val = ctx.empty((1, 12288)), ctx.empty((1, 1024)), ctx.empty((1, 1024))
        ctx.gemv_q8_k(12, 12288, HIDDEN, ctx.array(wq, np.uint8), d_q8, 1, d_qg)
        ctx.gemv_q8_k(14, 1024, HIDDEN, ctx.array(wk, np.uint8), d_q8, 1, d_key)
        ctx.gemv_q8_k(14, 1024, HIDDEN, ctx.array(wv, np.uint8), d_q8, 1, d_val)
        d_o = ctx.empty((24, 256))
        kv.full_core(layer, [seq], [pos], ctx.array(qn), ctx.array(kn), d_qg, d_key, d_val, d_o)
        got = d_o.download()
        # the oracle's chain
        q8 = ref.quantize_q8_k(x)
        qg = ref.gemv_q8_k(12, wq, q8, 1, HIDDEN, threads=16)[0]
        key = ref.gemv_q8_k(14, wk, q8, 1, HIDDEN, threads=16)[0]
        val = ref.gemv_q8_k(14, wv, q8, 1, HIDDEN, threads=16)[0]
        assert np.array_equal(d_qg.download()[0], qg)
        kc = np.zeros(ctx_len * 1024, np.float32)
        vc = np.zeros(ctx_len * 1024, np.float32)
        kc[:pos * 1024] = K0
        vc[:pos * 1024] = V0
        want, _ = ref.full_core(qn, kn, qg, key, val, kc, vc, ctx_len, pos, layer, threads=16)
        check_attn(margin, got, want)
    finally:
        kv.close()


def test_linear_attention_chain(pkg, ctx, ref, margin, synth):
    """The reference's linear_attention (ops.rs:744-804) on the device: the
    layer input quantised once (quantize_input), the qkv (10240 rows, Q4_K)
    and z (6144 rows, Q5_K) projections on the Q8_K path, beta and alpha
    (48 rows each, BF16 and Q8_0) on the f32 path, linear_core, the
    attention output quantised again and the ssm_out projection (5120 rows
    of 6144, Q6_K).  Each stage against the oracle on the device's input to
    that stage: the quantisations and Q8_K projections bit for bit, the f32
    projections within 1e-5 of the sum of |w x|, linear_core's output within
    1e-3 with its conv state bit-exact and its state within 1e-4 relative.
    The whole chain against the oracle's own chain is recorded too: there
    the ssm_out input is quantised from two linear_core outputs that differ
    by up to ~1e-4, so a few of its int8 quants may differ by one step."""
    H, V = HIDDEN, 6144
    rng = np.random.default_rng(0x51333950)
    x = (rng.standard_normal((1, H)) * 0.002).astype(np.float32)
    w_qkv = _random_kquant(12, 10240, H, 0x51333951)
    w_z = _random_kquant(13, V, H, 0x51333952)
    w_b, _ = _random_f32_path(30, 48, H, 0x51333953)
    w_a, _ = _random_f32_path(8, 48, H, 0x51333954)
    w_out = _random_kquant(14, H, V, 0x51333955)
    conv_w = synth.normal(0x51333956, 10240 * 4, sigma=0.5)
    dt = synth.normal(0x51333957, 48)
    a = -np.abs(synth.normal(0x51333958, 48))
    norm = synth.normal(0x51333959, 128, sigma=0.1, mean=1.0)
    conv0 = synth.normal(0x5133395A, 10240 * 3)
    delta0 = synth.normal(0x5133395B, 48 * 128 * 128, sigma=0.02)

    # the device chain
    d_q8 = _quantize_on_device(ctx, x)
    d_qkv, d_z = ctx.empty((1, 10240)), ctx.empty((1, V))
    d_beta, d_alpha = ctx.empty((1, 48)), ctx.empty((1, 48))
    ctx.gemv_q8_k(12, 10240, H, ctx.array(w_qkv, np.uint8), d_q8, 1, d_qkv)
    ctx.gemv_q8_k(13, V, H, ctx.array(w_z, np.uint8), d_q8, 1, d_z)
    d_x = ctx.array(x)
    ctx.gemv_f32(30, 48, H, ctx.array(w_b, np.uint8), d_x, 1, d_beta)
    ctx.gemv_f32(8, 48, H, ctx.array(w_a, np.uint8), d_x, 1, d_alpha)
    got_proj = [d.download()[0] for d in (d_qkv, d_z, d_beta, d_alpha)]
    d_conv, d_delta = ctx.array(conv0), ctx.array(delta0)
    d_attn = ctx.empty((1, V))
    ctx.linear_core(1, 1, *[ctx.array(v) for v in (conv_w, dt, a, norm)], d_conv, d_delta, d_qkv, d_z, d_beta,
                    d_alpha, d_attn)
    attn = d_attn.download()
    d_q8o = ctx.empty((ctx.q8k_bytes(1, V),), np.uint8)
    ctx.quantize_q8_k(1, V, d_attn, d_q8o)
    d_out = ctx.empty((1, H))
    ctx.gemv_q8_k(14, H, V, ctx.array(w_out, np.uint8), d_q8o, 1, d_out)
    out = d_out.download()[0]

    # stage by stage against the oracle
    q8 = ref.quantize_q8_k(x)
    assert np.array_equal(d_q8.download(), q8)
    assert np.array_equal(got_proj[0], ref.gemv_q8_k(12, w_qkv, q8, 1, H)[0])
    assert np.array_equal(got_proj[1], ref.gemv_q8_k(13, w_z, q8, 1, H)[0])
    for got, ty, w in ((got_proj[2], 30, w_b), (got_proj[3], 8, w_a)):
        _, wv = _random_f32_path(ty, 48, H, 0x51333953 if ty == 30 else 0x51333954)
        want = ref.gemv_f32(ty, w, x)[0]
        scale = np.abs(wv) @ np.abs(x[0].astype(np.float64))
        assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-5 * scale), ty
    c_ref, s_ref = conv0.copy(), delta0.copy()
    attn_ref = ref.linear_core(conv_w, dt, a, norm, c_ref, s_ref, *got_proj, threads=16)
    margin("linear_core out max-abs (device projections)", float(np.max(np.abs(attn[0] - attn_ref))), 1e-3)
    assert np.array_equal(d_conv.download(), c_ref)
    from parity import check_state
    check_state(margin, d_delta.download(), s_ref)
    q8o = ref.quantize_q8_k(attn)
    assert np.array_equal(d_q8o.download(), q8o)
    assert np.array_equal(out, ref.gemv_q8_k(14, w_out, q8o, 1, V)[0])

    # the oracle's chain on its own, end to end (recorded)
    proj = [ref.gemv_q8_k(12, w_qkv, q8, 1, H)[0], ref.gemv_q8_k(13, w_z, q8, 1, H)[0],
            ref.gemv_f32(30, w_b, x)[0], ref.gemv_f32(8, w_a, x)[0]]
    c2, s2 = conv0.copy(), delta0.copy()
    attn2 = ref.linear_core(conv_w, dt, a, norm, c2, s2, *proj, threads=16)
    out2 = ref.gemv_q8_k(14, w_out, ref.quantize_q8_k(attn2.reshape(1, -1)), 1, V)[0]
    rel = float(np.max(np.abs(out - out2)) / np.max(np.abs(out2)))
    margin("chain end to end, ssm_out rel to max|out|", rel, 1e-2)
