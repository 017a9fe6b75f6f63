"""ctypes binding of the CPU restatement (oracle/_build/libq38ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the oracle its GPU run is compared against, and by bench.py's cpu_baseline leg.  The product never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_float, c_int, c_size_t, c_uint32

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ORACLE_DIR, "_build", "libq38ref.so")

_F = POINTER(c_float)
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = open_library(LIB_PATH)
    return _lib


def use_library(path: str | None):
    """Point the module at another build of q38_ref.c (None: the default).
    Returns the previous binding so a caller can restore it."""
    global _lib
    prev = _lib
    _lib = None if path is None else open_library(path)
    return prev


def restore_library(prev) -> None:
    global _lib
    _lib = prev


def open_library(path: str):
    h = ctypes.CDLL(path)
    sig = {
        "q38r_rms_scale": (c_float, [_F, c_int]),
        "q38r_rmsnorm_inplace": (None, [_F, _F, c_int]),
        "q38r_sigmoid": (c_float, [c_float]),
        "q38r_silu": (c_float, [c_float]),
        "q38r_softplus": (c_float, [c_float]),
        "q38r_l2norm": (None, [_F, c_int]),
        "q38r_dot_128": (c_float, [_F, _F]),
        "q38r_mad_dot_128": (c_float, [_F, _F, c_float, _F]),
        "q38r_rope_theta_scale": (c_float, []),
        "q38r_rope": (None, [_F, c_int, c_uint32]),
        "q38r_attn_heads": (None, [_F, _F, _F, _F, c_size_t, c_int, _F, _F, c_int]),
        "q38r_full_core": (c_int, [_F, _F, _F, _F, _F, _F, _F, _F, _F, _F, _F, c_size_t, c_size_t,
                                   c_uint32, c_int, c_int]),
        "q38r_gdn_heads": (None, [_F, _F, _F, _F, _F, _F, _F, c_int]),
        "q38r_linear_core": (None, [_F, _F, _F, _F, _F, _F, _F, _F, _F, _F, _F, c_int]),
        "q38r_f16_to_f32": (c_float, [ctypes.c_uint16]),
        "q38r_quantize_q8_k": (c_int, [_F, c_int, c_int, ctypes.c_void_p]),
        "q38r_quant_block_bytes": (c_int, [c_int]),
        "q38r_gemv_q8_k": (c_int, [c_int, c_int, c_int, ctypes.c_void_p, ctypes.c_void_p, c_int, _F, c_int]),
        "q38r_f32_block": (c_int, [c_int, ctypes.POINTER(c_int)]),
        "q38r_gemv_f32": (c_int, [c_int, c_int, c_int, ctypes.c_void_p, _F, c_int, _F, c_int]),
        "q38r_is_full_attention": (c_int, [c_int]),
        "q38r_recurrent_index": (c_int, [c_int]),
        "q38r_available_cores": (c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(h, name)
        fn.restype = res
        fn.argtypes = args
    return h


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def _opt(a):
    return None if a is None else _f(a)


def cores() -> int:
    return lib().q38r_available_cores()


# ------------------------------------------------------------------ primitives
def rms_scale(x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, np.float32)
    return lib().q38r_rms_scale(_f(x), x.size)


def rmsnorm(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    y = np.array(x, np.float32, copy=True)
    lib().q38r_rmsnorm_inplace(_f(y), _f(np.ascontiguousarray(w, np.float32)), y.size)
    return y


def l2norm(x: np.ndarray) -> np.ndarray:
    y = np.array(x, np.float32, copy=True)
    lib().q38r_l2norm(_f(y), y.size)
    return y


def rope(x: np.ndarray, heads: int, position: int) -> np.ndarray:
    y = np.array(x, np.float32, copy=True)
    lib().q38r_rope(_f(y), heads, position)
    return y


def scalar_fn(name: str, x: float) -> float:
    return getattr(lib(), "q38r_" + name)(float(x))


# ---------------------------------------------------------------- attention
def attn_heads(q: np.ndarray, k_rows: np.ndarray, v_rows: np.ndarray, gate: np.ndarray | None = None,
               threads: int = 1) -> np.ndarray:
    """run_head for 24 heads over rows [positions][1024] (ops.rs:868-938)."""
    q = np.ascontiguousarray(q, np.float32).reshape(-1)
    k_rows = np.ascontiguousarray(k_rows, np.float32)
    v_rows = np.ascontiguousarray(v_rows, np.float32)
    positions = k_rows.shape[0]
    assert k_rows.shape == (positions, 1024) and v_rows.shape == (positions, 1024)
    scores = np.empty(24 * positions, np.float32)
    out = np.empty(24 * 256, np.float32)
    g = None if gate is None else np.ascontiguousarray(gate, np.float32).reshape(-1)
    lib().q38r_attn_heads(_f(q), _opt(g), _f(k_rows), _f(v_rows), 1024, positions, _f(scores), _f(out),
                          threads)
    return out.reshape(24, 256)


def full_core(q_norm, k_norm, q_and_gate, key, value, key_cache, value_cache, context_length, position,
              layer, threads=1):
    """full_core whole (ops.rs:813-940); caches are updated in place."""
    qg = np.ascontiguousarray(q_and_gate, np.float32).reshape(-1)
    k = np.array(key, np.float32, copy=True).reshape(-1)
    v = np.ascontiguousarray(value, np.float32).reshape(-1)
    q = np.empty(6144, np.float32)
    gate = np.empty(6144, np.float32)
    scores = np.empty(24 * context_length, np.float32)
    out = np.empty(6144, np.float32)
    assert key_cache.dtype == np.float32 and key_cache.flags.c_contiguous
    rc = lib().q38r_full_core(_f(np.ascontiguousarray(q_norm, np.float32)),
                              _f(np.ascontiguousarray(k_norm, np.float32)), _f(qg), _f(k), _f(v), _f(q),
                              _f(gate), _f(scores), _f(out), _f(key_cache), _f(value_cache),
                              key_cache.size, context_length, position, layer, threads)
    if rc != 0:
        raise ValueError("full_core: cache row out of bounds")
    return out.reshape(24, 256), k


# ------------------------------------------------------------------ DeltaNet
def gdn_heads(state: np.ndarray, q, k, v, beta, g, threads: int = 1) -> np.ndarray:
    """One recurrence step on `state` [48*128*128] in place (ops.rs:689-733)."""
    assert state.dtype == np.float32 and state.flags.c_contiguous and state.size == 48 * 128 * 128
    out = np.empty(6144, np.float32)
    args = [np.ascontiguousarray(a, np.float32).reshape(-1) for a in (q, k, v, beta, g)]
    lib().q38r_gdn_heads(_f(state), *[_f(a) for a in args], _f(out), threads)
    return out


def linear_core(conv_w, dt, a, norm_w, conv_state, delta_state, qkv, z, beta, alpha, threads=1):
    """linear_core whole (ops.rs:648-742); states are updated in place."""
    qkv = np.array(qkv, np.float32, copy=True).reshape(-1)
    beta = np.array(beta, np.float32, copy=True).reshape(-1)
    alpha = np.array(alpha, np.float32, copy=True).reshape(-1)
    out = np.empty(6144, np.float32)
    for s in (conv_state, delta_state):
        assert s.dtype == np.float32 and s.flags.c_contiguous
    lib().q38r_linear_core(*[_f(np.ascontiguousarray(x, np.float32).reshape(-1)) for x in (conv_w, dt, a, norm_w)],
                           _f(conv_state), _f(delta_state), _f(qkv),
                           _f(np.ascontiguousarray(z, np.float32).reshape(-1)), _f(beta), _f(alpha), _f(out),
                           threads)
    return out


# ------------------------------------------------------- weight projections
GGML_Q2_K, GGML_Q3_K, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K = 10, 11, 12, 13, 14
GGML_IQ4_NL, GGML_IQ4_XS = 20, 23
GGML_IQ2_XXS, GGML_IQ2_XS, GGML_IQ3_XXS, GGML_IQ1_S, GGML_IQ3_S, GGML_IQ2_S, GGML_IQ1_M = 16, 17, 18, 19, 21, 22, 29
QUANT_BLOCK_BYTES = {GGML_Q2_K: 84, GGML_Q3_K: 110, GGML_Q4_K: 144, GGML_Q5_K: 176, GGML_Q6_K: 210,
                     GGML_IQ4_NL: 144, GGML_IQ4_XS: 136, GGML_IQ2_XXS: 66, GGML_IQ2_XS: 74, GGML_IQ2_S: 82,
                     GGML_IQ3_XXS: 98, GGML_IQ3_S: 110, GGML_IQ1_S: 50, GGML_IQ1_M: 56}
# the f32-input path's weight types: (weights per block, bytes per block)
GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30
F32_PATH_BLOCKS = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_BF16: (1, 2), GGML_Q8_0: (32, 34)}


def q8k_bytes(n_tokens: int, width: int) -> int:
    """Bytes of a planar Q8_K buffer: int8 quants, int16 group sums, f32 scales."""
    blocks = width // 256
    return n_tokens * blocks * (256 + 32 + 4)


def q8k_split(planar: np.ndarray, n_tokens: int, width: int):
    """(quants int8 [T][W], sums int16 [T][B][16], scales f32 [T][B]) views."""
    blocks = width // 256
    buf = np.asarray(planar, np.uint8).reshape(-1)
    q = buf[:n_tokens * width].view(np.int8).reshape(n_tokens, width)
    off = n_tokens * width
    sums = buf[off:off + n_tokens * blocks * 32].view(np.int16).reshape(n_tokens, blocks, 16)
    off += n_tokens * blocks * 32
    scales = buf[off:off + n_tokens * blocks * 4].view(np.float32).reshape(n_tokens, blocks)
    return q, sums, scales


def quantize_q8_k(x: np.ndarray) -> np.ndarray:
    """quantize_q8_k (quant.rs:97-128) of x [T][W] into a planar uint8 buffer."""
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    T, W = x.shape
    out = np.zeros(q8k_bytes(T, W), np.uint8)
    if lib().q38r_quantize_q8_k(_f(x), T, W, out.ctypes.data) != 0:
        raise ValueError("width is not a multiple of 256")
    return out


def gemv_q8_k(ggml_type: int, weights: np.ndarray, planar: np.ndarray, n_tokens: int, width: int,
              threads: int = 1) -> np.ndarray:
    """tensor_gemv_q8_k / tensor_gemm_q8_k: out [T][rows] for weights [rows][row_bytes]."""
    w = np.ascontiguousarray(weights, np.uint8)
    rows = w.shape[0]
    out = np.empty((n_tokens, rows), np.float32)
    p = np.ascontiguousarray(planar, np.uint8)
    if lib().q38r_gemv_q8_k(ggml_type, rows, width, w.ctypes.data, p.ctypes.data, n_tokens, _f(out), threads) != 0:
        raise ValueError("unsupported type or width")
    return out


def gemv_f32(ggml_type: int, weights: np.ndarray, x: np.ndarray, threads: int = 1) -> np.ndarray:
    """tensor_gemv_f32 / tensor_gemm_f32 (tensor.rs:1095-1129, :1175-1215):
    out [T][rows] for weights [rows][row_bytes] of an F32/F16/BF16/Q8_0 type
    and f32 input x [T][width]."""
    w = np.ascontiguousarray(weights, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    T, W = x.shape
    rows = w.shape[0]
    out = np.empty((T, rows), np.float32)
    if lib().q38r_gemv_f32(ggml_type, rows, W, w.ctypes.data, _f(x), T, _f(out), threads) != 0:
        raise ValueError("unsupported type or width")
    return out
