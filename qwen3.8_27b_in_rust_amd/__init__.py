"""ctypes binding of libq38attn.so, the MI355X attention path (include/q38_attn.h).

The library is the product: hand-written gfx950 kernels behind a C ABI.  This
module only marshals numpy arrays and device pointers across that ABI for the
tests and the bench.  There is no CPU fallback: if the library or its code
objects are missing, or no MI355X is present, every call raises Q38Error.

The directory name is not a Python identifier; load it with
`importlib.util.spec_from_file_location` (see `load_package` in
__graft_entry__.py), or call the library through any FFI directly.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_uint32, c_void_p

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libq38attn.so")
INCLUDE_DIR = os.path.join(os.path.dirname(PKG_DIR), "include")
HEADER_PATH = os.path.join(INCLUDE_DIR, "q38_attn.h")

# shapes: reference src/model/mod.rs:13-24
ATTN_HEADS, ATTN_KV_HEADS, ATTN_HEAD_DIM = 24, 4, 256
ATTN_Q_DIM, ATTN_QG_DIM, ATTN_KV_DIM = 6144, 12288, 1024
LIN_QK_HEADS, LIN_V_HEADS, LIN_HEAD_DIM = 16, 48, 128
LIN_QK_DIM, LIN_V_DIM, LIN_QKV_DIM = 2048, 6144, 10240
LIN_STATE_FLOATS = LIN_V_HEADS * LIN_HEAD_DIM * LIN_HEAD_DIM
PAGE_TOKENS = 16
NOALLOC_SCRATCH_BYTES = 16 << 20  # Q38_NOALLOC_SCRATCH_BYTES of include/q38_attn.h


class Q38Error(RuntimeError):
    pass


class _LinearWeights(ctypes.Structure):
    _fields_ = [("d_conv_w", c_void_p), ("d_dt", c_void_p), ("d_a", c_void_p), ("d_norm", c_void_p)]


class _DecodeCall(ctypes.Structure):
    _fields_ = [("layer", c_int32), ("pad_", c_int32), ("d_q", c_void_p), ("d_k_new", c_void_p),
                ("d_v_new", c_void_p), ("d_gate", c_void_p), ("d_q_norm", c_void_p), ("d_k_norm", c_void_p),
                ("d_out", c_void_p)]


_P = c_void_p
_I32P = POINTER(c_int32)
_SIGNATURES = {
    "q38_last_error": (c_char_p, []),
    "q38_device_count": (c_int, [POINTER(c_int)]),
    "q38_ctx_create": (c_int, [POINTER(c_void_p), c_int, c_char_p]),
    "q38_ctx_destroy": (c_int, [_P]),
    "q38_ctx_stream": (c_void_p, [_P]),
    "q38_sync": (c_int, [_P]),
    "q38_device_info": (c_int, [_P, POINTER(c_int), POINTER(c_int), POINTER(c_int), c_char_p, c_size_t]),
    "q38_set_decode_split": (c_int, [_P, c_int]),
    "q38_alloc": (c_int, [_P, c_size_t, POINTER(c_void_p)]),
    "q38_free": (c_int, [_P, _P]),
    "q38_upload": (c_int, [_P, _P, _P, c_size_t]),
    "q38_download": (c_int, [_P, _P, _P, c_size_t]),
    "q38_zero": (c_int, [_P, _P, c_size_t]),
    "q38_event_create": (c_int, [_P, POINTER(c_void_p)]),
    "q38_event_record": (c_int, [_P, _P]),
    "q38_event_elapsed_ms": (c_int, [_P, _P, POINTER(c_float)]),
    "q38_event_destroy": (c_int, [_P]),
    "q38_kernel_timer_start": (c_int, [_P, c_char_p, c_int]),
    "q38_kernel_timer_stop": (c_int, [_P, POINTER(c_float), POINTER(c_int)]),
    "q38_fill_normal": (c_int, [_P, _P, c_size_t, ctypes.c_uint64, c_float, c_float]),
    "q38_device_copy": (c_int, [_P, _P, _P, c_size_t]),
    "q38_device_noop": (c_int, [_P]),
    "q38_kv_create": (c_int, [_P, c_int, c_int, c_int, c_int, POINTER(c_void_p)]),
    "q38_kv_destroy": (c_int, [_P]),
    "q38_kv_free_pages": (c_int, [_P, POINTER(c_int)]),
    "q38_kv_set_prefill_cache": (c_int, [_P, c_int]),
    "q38_seq_create": (c_int, [_P, POINTER(c_int)]),
    "q38_seq_free": (c_int, [_P, c_int]),
    "q38_seq_reset": (c_int, [_P, c_int]),
    "q38_seq_truncate": (c_int, [_P, c_int, c_int]),
    "q38_seq_reserve": (c_int, [_P, c_int, c_int]),
    "q38_seq_set_pages": (c_int, [_P, c_int, c_int, _I32P]),
    "q38_seq_capacity": (c_int, [_P, c_int, POINTER(c_int)]),
    "q38_kv_write": (c_int, [_P, c_int, c_int, c_int, c_int, _P, _P]),
    "q38_kv_read": (c_int, [_P, c_int, c_int, c_int, c_int, _P, _P]),
    "q38_attn_decode": (c_int, [_P, c_int, c_int, _I32P, _I32P, _P, _P, _P, _P, _P]),
    "q38_full_core": (c_int, [_P, c_int, c_int, _I32P, _I32P, _P, _P, _P, _P, _P, _P]),
    "q38_full_core_noalloc": (c_int, [_P, c_int, c_int, _I32P, _I32P, _P, _P, _P, _P, _P, _P]),
    "q38_attn_pre": (c_int, [_P, c_int, c_int, _P, _P, _P, _P, _P, _P, _P]),
    "q38_decode_graph_create": (c_int, [_P, c_int, _I32P, _I32P, c_int, POINTER(_DecodeCall), POINTER(c_void_p)]),
    "q38_decode_graph_begin": (c_int, [_P, c_int, _I32P, _I32P, POINTER(c_void_p)]),
    "q38_decode_graph_add_decode": (c_int, [_P, POINTER(_DecodeCall)]),
    "q38_decode_graph_add_linear_core": (c_int, [_P, c_int, POINTER(_LinearWeights), _P, _P, _P, _P, _P, _P, _P]),
    "q38_decode_graph_add_graph": (c_int, [_P, _P]),
    "q38_decode_graph_end": (c_int, [_P]),
    "q38_decode_graph_set_positions": (c_int, [_P, _I32P]),
    "q38_decode_graph_launch": (c_int, [_P]),
    "q38_decode_graph_destroy": (c_int, [_P]),
    "q38_q8k_bytes": (c_int, [c_int, c_int, POINTER(c_size_t)]),
    "q38_quantize_q8_k": (c_int, [_P, c_int, c_int, _P, _P]),
    "q38_gemv_q8_k": (c_int, [_P, c_int, c_int, c_int, _P, _P, c_int, _P]),
    "q38_gemv_f32": (c_int, [_P, c_int, c_int, c_int, _P, _P, c_int, _P]),
    "q38_gemv_q8_k_multi": (c_int, [_P, c_int, c_int, _I32P, c_int, POINTER(c_void_p), _P, c_int,
                                    POINTER(c_void_p)]),
    "q38_quantize_project_q8_k": (c_int, [_P, c_int, c_int, _I32P, c_int, POINTER(c_void_p), _P, c_int, _P,
                                          POINTER(c_void_p)]),
    "q38_attn_prefill": (c_int, [_P, c_int, c_int, c_int, c_int, _P, _P, _P, _P, _P]),
    "q38_gdn_step": (c_int, [_P, c_int, _P, c_int64, _P, _P, _P, _P, _P, _P]),
    "q38_gdn_prefill": (c_int, [_P, _P, c_int, _P, _P, _P, _P, _P, _P]),
    "q38_linear_core": (c_int, [_P, c_int, c_int, POINTER(_LinearWeights), _P, _P, _P, _P, _P, _P, _P]),
    "q38_gguf_open": (c_int, [c_char_p, POINTER(c_void_p)]),
    "q38_gguf_close": (c_int, [_P]),
    "q38_gguf_info": (c_int, [_P, POINTER(c_uint32), POINTER(c_uint32), POINTER(ctypes.c_uint64), POINTER(c_int),
                              POINTER(c_int)]),
    "q38_gguf_find_tensor": (c_int, [_P, c_char_p, POINTER(c_int)]),
    "q38_gguf_tensor": (c_int, [_P, c_int, POINTER(c_char_p), POINTER(c_int), POINTER(c_int),
                                POINTER(ctypes.c_uint64), POINTER(ctypes.c_uint64), POINTER(ctypes.c_uint64)]),
    "q38_gguf_meta_u32": (c_int, [_P, c_char_p, POINTER(c_uint32)]),
    "q38_gguf_upload": (c_int, [_P, _P, POINTER(c_void_p), POINTER(c_size_t)]),
    "q38_recurrent_checkpoint": (c_int, [_P, _P, _P, c_size_t, c_size_t, _P, _P]),
    "q38_recurrent_restore": (c_int, [_P, _P, _P, c_size_t, c_size_t, _P, _P]),
}

_lib = None


def library_built() -> bool:
    return os.path.exists(LIB_PATH)


def lib():
    """The loaded libq38attn.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not library_built():
            raise Q38Error(f"{LIB_PATH} is missing: build it first (__graft_entry__.build())")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().q38_last_error().decode(errors="replace")
        raise Q38Error(f"{what}: {msg}")


def device_count() -> int:
    n = c_int(0)
    _check(lib().q38_device_count(ctypes.byref(n)), "q38_device_count")
    return n.value


def _i32(seq) -> ctypes.Array:
    a = (c_int32 * len(seq))()
    for i, v in enumerate(seq):
        a[i] = int(v)
    return a


class DeviceArray:
    """A device buffer with a numpy shape and dtype, owned by a Context."""

    def __init__(self, ctx: "Context", shape, dtype=np.float32):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = c_void_p()
        _check(lib().q38_alloc(ctx.handle, self.nbytes, ctypes.byref(p)), "q38_alloc")
        self.ptr = p.value

    def offset(self, elements: int) -> int:
        return self.ptr + int(elements) * self.dtype.itemsize

    def upload(self, host: np.ndarray) -> "DeviceArray":
        h = np.ascontiguousarray(host, dtype=self.dtype)
        if h.nbytes != self.nbytes:
            raise Q38Error(f"upload of {h.nbytes} bytes into a {self.nbytes}-byte buffer")
        _check(lib().q38_upload(self.ctx.handle, self.ptr, h.ctypes.data, h.nbytes), "q38_upload")
        return self

    def download(self, rows: int | None = None) -> np.ndarray:
        """The whole buffer, or its first `rows` rows along the leading axis."""
        shape = self.shape if rows is None else (int(rows),) + tuple(self.shape[1:])
        h = np.empty(shape, dtype=self.dtype)
        if h.nbytes > self.nbytes:
            raise Q38Error("download larger than the buffer")
        _check(lib().q38_download(self.ctx.handle, h.ctypes.data, self.ptr, h.nbytes), "q38_download")
        return h

    def zero(self) -> "DeviceArray":
        _check(lib().q38_zero(self.ctx.handle, self.ptr, self.nbytes), "q38_zero")
        return self

    def free(self) -> None:
        if self.ptr:
            _check(lib().q38_free(self.ctx.handle, self.ptr), "q38_free")
            self.ptr = None


class Context:
    """One device, one stream, the loaded code objects."""

    def __init__(self, device: int = 0, module_dir: str | None = None):
        """module_dir: where the code objects are (default: $Q38_MODULE_DIR,
        else next to the library)."""
        module_dir = module_dir or os.environ.get("Q38_MODULE_DIR") or None
        h = c_void_p()
        md = module_dir.encode() if module_dir else None
        _check(lib().q38_ctx_create(ctypes.byref(h), device, md), "q38_ctx_create")
        self.handle = h.value

    def close(self) -> None:
        if self.handle:
            lib().q38_ctx_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self) -> dict:
        cu, clk, lds = c_int(), c_int(), c_int()
        name = ctypes.create_string_buffer(256)
        _check(lib().q38_device_info(self.handle, ctypes.byref(cu), ctypes.byref(clk),
                                     ctypes.byref(lds), name, 256), "q38_device_info")
        return {"cu_count": cu.value, "clock_khz": clk.value, "lds_bytes": lds.value,
                "name": name.value.decode()}

    def set_decode_split(self, tokens: int) -> None:
        """Context tokens per decode workgroup (multiple of 16), 0 = automatic."""
        _check(lib().q38_set_decode_split(self.handle, int(tokens)), "q38_set_decode_split")

    def stream(self) -> int:
        return lib().q38_ctx_stream(self.handle)

    def sync(self) -> None:
        _check(lib().q38_sync(self.handle), "q38_sync")

    def empty(self, shape, dtype=np.float32) -> DeviceArray:
        return DeviceArray(self, shape, dtype)

    def array(self, host: np.ndarray, dtype=np.float32) -> DeviceArray:
        h = np.ascontiguousarray(host, dtype=dtype)
        return DeviceArray(self, h.shape, dtype).upload(h)

    # -- events on the context's stream
    def event(self) -> int:
        e = c_void_p()
        _check(lib().q38_event_create(self.handle, ctypes.byref(e)), "q38_event_create")
        return e.value

    def record(self, event: int) -> None:
        _check(lib().q38_event_record(self.handle, event), "q38_event_record")

    @staticmethod
    def elapsed_ms(start: int, stop: int) -> float:
        ms = c_float()
        _check(lib().q38_event_elapsed_ms(start, stop, ctypes.byref(ms)), "q38_event_elapsed_ms")
        return ms.value

    @staticmethod
    def destroy_event(event: int) -> None:
        lib().q38_event_destroy(event)

    def kernel_timer_start(self, kernel: str, max_launches: int) -> None:
        _check(lib().q38_kernel_timer_start(self.handle, kernel.encode(), max_launches),
               "q38_kernel_timer_start")

    def kernel_timer_stop(self):
        """(summed kernel milliseconds, number of timed launches)"""
        ms, n = c_float(), c_int()
        _check(lib().q38_kernel_timer_stop(self.handle, ctypes.byref(ms), ctypes.byref(n)),
               "q38_kernel_timer_stop")
        return ms.value, n.value

    def fill_normal(self, dst, n: int, seed: int, sigma: float = 1.0, mean: float = 0.0) -> None:
        _check(lib().q38_fill_normal(self.handle, _ptr(dst), n, seed & 0xFFFFFFFFFFFFFFFF, sigma, mean),
               "q38_fill_normal")

    def noop(self) -> None:
        """Launch an empty kernel (the launch floor)."""
        _check(lib().q38_device_noop(self.handle), "q38_device_noop")

    def copy(self, dst, src, nbytes: int) -> None:
        _check(lib().q38_device_copy(self.handle, _ptr(dst), _ptr(src), nbytes), "q38_device_copy")

    # -- DeltaNet
    def gdn_step(self, n_seq, state: DeviceArray, q, k, v, beta, g, out, state_stride=LIN_STATE_FLOATS,
                 state_offset=0):
        _check(lib().q38_gdn_step(self.handle, n_seq, state.offset(state_offset), state_stride,
                                  _ptr(q), _ptr(k), _ptr(v), _ptr(beta), _ptr(g), _ptr(out)),
               "q38_gdn_step")

    def gdn_prefill(self, state: DeviceArray, n_tokens, q, k, v, beta, g, out, state_offset=0):
        _check(lib().q38_gdn_prefill(self.handle, state.offset(state_offset), n_tokens, _ptr(q), _ptr(k),
                                     _ptr(v), _ptr(beta), _ptr(g), _ptr(out)), "q38_gdn_prefill")

    def linear_core(self, n_seq, n_tokens, conv_w, dt, a, norm, conv_state, delta_state, qkv, z, beta,
                    alpha, out):
        w = _LinearWeights(_ptr(conv_w), _ptr(dt), _ptr(a), _ptr(norm))
        _check(lib().q38_linear_core(self.handle, n_seq, n_tokens, ctypes.byref(w), _ptr(conv_state),
                                     _ptr(delta_state), _ptr(qkv), _ptr(z), _ptr(beta), _ptr(alpha),
                                     _ptr(out)), "q38_linear_core")

    # -- weight projections
    @staticmethod
    def q8k_bytes(n_tokens: int, width: int) -> int:
        n = c_size_t()
        _check(lib().q38_q8k_bytes(n_tokens, width, ctypes.byref(n)), "q38_q8k_bytes")
        return n.value

    def quantize_q8_k(self, n_tokens, width, x, q8k):
        _check(lib().q38_quantize_q8_k(self.handle, n_tokens, width, _ptr(x), _ptr(q8k)), "q38_quantize_q8_k")

    def gemv_f32(self, ggml_type, rows, width, weights, x, n_tokens, out):
        _check(lib().q38_gemv_f32(self.handle, ggml_type, rows, width, _ptr(weights), _ptr(x), n_tokens, _ptr(out)),
               "q38_gemv_f32")

    def gemv_q8_k(self, ggml_type, rows, width, weights, q8k, n_tokens, out):
        _check(lib().q38_gemv_q8_k(self.handle, ggml_type, rows, width, _ptr(weights), _ptr(q8k), n_tokens,
                                   _ptr(out)), "q38_gemv_q8_k")

    def gemv_q8_k_multi(self, ggml_type, rows, width, weights, q8k, n_tokens, outs):
        n = len(rows)
        w = (c_void_p * n)(*[_ptr(x) for x in weights])
        o = (c_void_p * n)(*[_ptr(x) for x in outs])
        _check(lib().q38_gemv_q8_k_multi(self.handle, ggml_type, n, _i32(rows), width, w, _ptr(q8k), n_tokens, o),
               "q38_gemv_q8_k_multi")

    def quantize_project_q8_k(self, ggml_type, rows, width, weights, x, n_tokens, q8k, outs):
        n = len(rows)
        w = (c_void_p * n)(*[_ptr(v) for v in weights])
        o = (c_void_p * n)(*[_ptr(v) for v in outs])
        _check(lib().q38_quantize_project_q8_k(self.handle, ggml_type, n, _i32(rows), width, w, _ptr(x), n_tokens,
                                               _ptr(q8k), o), "q38_quantize_project_q8_k")

    def attn_pre(self, n_tokens, pos0, q_norm, k_norm, q_and_gate, key, q_out, gate_out, k_out):
        _check(lib().q38_attn_pre(self.handle, n_tokens, pos0, _ptr(q_norm), _ptr(k_norm), _ptr(q_and_gate),
                                  _ptr(key), _ptr(q_out), _ptr(gate_out), _ptr(k_out)), "q38_attn_pre")


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, DeviceArray):
        return x.ptr
    return int(x)


class KVCache:
    """Paged device KV cache (q38_kv_*)."""

    def __init__(self, ctx: Context, n_slots: int, max_pages: int, max_seqs: int, max_tokens_per_seq: int):
        self.ctx = ctx
        h = c_void_p()
        _check(lib().q38_kv_create(ctx.handle, n_slots, max_pages, max_seqs, max_tokens_per_seq,
                                   ctypes.byref(h)), "q38_kv_create")
        self.handle = h.value

    def close(self) -> None:
        if self.handle:
            lib().q38_kv_destroy(self.handle)
            self.handle = None

    def set_prefill_cache(self, enable: bool) -> None:
        _check(lib().q38_kv_set_prefill_cache(self.handle, int(bool(enable))), "q38_kv_set_prefill_cache")

    def free_pages(self) -> int:
        n = c_int()
        _check(lib().q38_kv_free_pages(self.handle, ctypes.byref(n)), "q38_kv_free_pages")
        return n.value

    def seq_create(self) -> int:
        s = c_int()
        _check(lib().q38_seq_create(self.handle, ctypes.byref(s)), "q38_seq_create")
        return s.value

    def seq_free(self, seq):
        _check(lib().q38_seq_free(self.handle, seq), "q38_seq_free")

    def seq_reset(self, seq):
        _check(lib().q38_seq_reset(self.handle, seq), "q38_seq_reset")

    def seq_truncate(self, seq, n_tokens):
        _check(lib().q38_seq_truncate(self.handle, seq, n_tokens), "q38_seq_truncate")

    def seq_reserve(self, seq, n_tokens):
        _check(lib().q38_seq_reserve(self.handle, seq, n_tokens), "q38_seq_reserve")

    def seq_set_pages(self, seq, page_ids):
        _check(lib().q38_seq_set_pages(self.handle, seq, len(page_ids), _i32(page_ids)), "q38_seq_set_pages")

    def seq_capacity(self, seq) -> int:
        n = c_int()
        _check(lib().q38_seq_capacity(self.handle, seq, ctypes.byref(n)), "q38_seq_capacity")
        return n.value

    def write(self, layer, seq, pos0, n_tokens, d_k, d_v):
        _check(lib().q38_kv_write(self.handle, layer, seq, pos0, n_tokens, _ptr(d_k), _ptr(d_v)),
               "q38_kv_write")

    def read(self, layer, seq, pos0, n_tokens, d_k, d_v):
        _check(lib().q38_kv_read(self.handle, layer, seq, pos0, n_tokens, _ptr(d_k), _ptr(d_v)),
               "q38_kv_read")

    def attn_decode(self, layer, seq_ids, positions, q, out, k_new=None, v_new=None, gate=None):
        n = len(seq_ids)
        _check(lib().q38_attn_decode(self.handle, layer, n, _i32(seq_ids), _i32(positions), _ptr(q),
                                     _ptr(k_new), _ptr(v_new), _ptr(gate), _ptr(out)), "q38_attn_decode")

    def full_core(self, layer, seq_ids, positions, q_norm, k_norm, q_and_gate, key, value, out):
        n = len(seq_ids)
        _check(lib().q38_full_core(self.handle, layer, n, _i32(seq_ids), _i32(positions), _ptr(q_norm),
                                   _ptr(k_norm), _ptr(q_and_gate), _ptr(key), _ptr(value), _ptr(out)),
               "q38_full_core")

    def full_core_noalloc(self, layer, seq_ids, positions, q_norm, k_norm, q_and_gate, key, value, out):
        n = len(seq_ids)
        _check(lib().q38_full_core_noalloc(self.handle, layer, n, _i32(seq_ids), _i32(positions), _ptr(q_norm),
                                           _ptr(k_norm), _ptr(q_and_gate), _ptr(key), _ptr(value), _ptr(out)),
               "q38_full_core_noalloc")

    def decode_graph(self, seq_ids, positions, calls=None):
        """A DecodeGraph: `calls` are dicts with layer, q, out and optionally
        k_new, v_new, gate (the attn_decode form) or q_norm, k_norm with
        q = q|gate rows and k_new/v_new the raw key/value (full_core); with
        no calls, an open graph to fill with add_* and end()."""
        return DecodeGraph(self, seq_ids, positions, calls)

    def attn_prefill(self, layer, seq, base_pos, n_tokens, q, k, v, out, gate=None):
        _check(lib().q38_attn_prefill(self.handle, layer, seq, base_pos, n_tokens, _ptr(q), _ptr(k), _ptr(v),
                                      _ptr(gate), _ptr(out)), "q38_attn_prefill")


def _decode_call(c: dict) -> _DecodeCall:
    d = _DecodeCall()
    d.layer = c["layer"]
    d.d_q = _ptr(c["q"])
    d.d_k_new = _ptr(c.get("k_new"))
    d.d_v_new = _ptr(c.get("v_new"))
    d.d_gate = _ptr(c.get("gate"))
    d.d_q_norm = _ptr(c.get("q_norm"))
    d.d_k_norm = _ptr(c.get("k_norm"))
    d.d_out = _ptr(c["out"])
    return d


class DecodeGraph:
    """q38_decode_graph_*: a token's work recorded once as a HIP graph.  With
    `calls`, the graph of those decode calls (q38_decode_graph_create);
    without, an open graph to fill with add_* and close with end()."""

    def __init__(self, kv, seq_ids, positions, calls=None):
        self.kv = kv
        self.n_seq = len(seq_ids)
        h = c_void_p()
        if calls is not None:
            arr = (_DecodeCall * len(calls))(*[_decode_call(c) for c in calls])
            _check(lib().q38_decode_graph_create(kv.handle, self.n_seq, _i32(seq_ids), _i32(positions), len(calls),
                                                 arr, ctypes.byref(h)), "q38_decode_graph_create")
        else:
            _check(lib().q38_decode_graph_begin(kv.handle, self.n_seq, _i32(seq_ids), _i32(positions),
                                                ctypes.byref(h)), "q38_decode_graph_begin")
        self.handle = h.value

    def add_decode(self, call: dict) -> None:
        c = _decode_call(call)
        _check(lib().q38_decode_graph_add_decode(self.handle, ctypes.byref(c)), "q38_decode_graph_add_decode")

    def add_linear_core(self, n_seq, conv_w, dt, a, norm, conv_state, delta_state, qkv, z, beta, alpha, out):
        w = _LinearWeights(_ptr(conv_w), _ptr(dt), _ptr(a), _ptr(norm))
        _check(lib().q38_decode_graph_add_linear_core(self.handle, n_seq, ctypes.byref(w), _ptr(conv_state),
                                                      _ptr(delta_state), _ptr(qkv), _ptr(z), _ptr(beta),
                                                      _ptr(alpha), _ptr(out)), "q38_decode_graph_add_linear_core")

    def add_graph(self, hip_graph: int) -> None:
        _check(lib().q38_decode_graph_add_graph(self.handle, hip_graph), "q38_decode_graph_add_graph")

    def end(self) -> None:
        _check(lib().q38_decode_graph_end(self.handle), "q38_decode_graph_end")

    def set_positions(self, positions) -> None:
        _check(lib().q38_decode_graph_set_positions(self.handle, _i32(positions)), "q38_decode_graph_set_positions")

    def launch(self) -> None:
        _check(lib().q38_decode_graph_launch(self.handle), "q38_decode_graph_launch")

    def close(self) -> None:
        if self.handle:
            _check(lib().q38_decode_graph_destroy(self.handle), "q38_decode_graph_destroy")
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Gguf:
    """A parsed GGUF file (q38_gguf_open); host-only until upload()."""

    MAX_DIMS = 8

    def __init__(self, path: str):
        h = c_void_p()
        _check(lib().q38_gguf_open(os.fsencode(path), ctypes.byref(h)), "q38_gguf_open")
        self.handle = h.value

    def close(self) -> None:
        if self.handle:
            lib().q38_gguf_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self) -> dict:
        v, al, off = c_uint32(), c_uint32(), ctypes.c_uint64()
        nt, nm = c_int(), c_int()
        _check(lib().q38_gguf_info(self.handle, ctypes.byref(v), ctypes.byref(al), ctypes.byref(off),
                                   ctypes.byref(nt), ctypes.byref(nm)), "q38_gguf_info")
        return {"version": v.value, "alignment": al.value, "data_offset": off.value, "n_tensors": nt.value,
                "n_metadata": nm.value}

    def find_tensor(self, name: str) -> int:
        i = c_int()
        _check(lib().q38_gguf_find_tensor(self.handle, name.encode("utf-8", "surrogateescape"), ctypes.byref(i)),
               "q38_gguf_find_tensor")
        return i.value

    def tensor(self, index: int) -> dict:
        name = c_char_p()
        ty, nd = c_int(), c_int()
        shape = (ctypes.c_uint64 * self.MAX_DIMS)()
        off, nb = ctypes.c_uint64(), ctypes.c_uint64()
        _check(lib().q38_gguf_tensor(self.handle, index, ctypes.byref(name), ctypes.byref(ty), ctypes.byref(nd),
                                     shape, ctypes.byref(off), ctypes.byref(nb)), "q38_gguf_tensor")
        # names are bytes in the file (not necessarily UTF-8); surrogateescape
        # round-trips them through find_tensor
        return {"name": name.value.decode("utf-8", "surrogateescape"), "type": ty.value,
                "shape": list(shape[:nd.value]),
                "offset": off.value, "nbytes": nb.value}

    def meta_u32(self, key: str) -> int:
        v = c_uint32()
        _check(lib().q38_gguf_meta_u32(self.handle, key.encode("utf-8", "surrogateescape"), ctypes.byref(v)),
               "q38_gguf_meta_u32")
        return v.value

    def upload(self, ctx: "Context") -> tuple[int, int]:
        """(device base pointer, bytes); free with ctx's q38_free."""
        p, n = c_void_p(), c_size_t()
        _check(lib().q38_gguf_upload(ctx.handle, self.handle, ctypes.byref(p), ctypes.byref(n)),
               "q38_gguf_upload")
        return p.value, n.value


def recurrent_checkpoint(ctx: "Context", conv_state, delta_state, n_conv, n_delta, conv_ckpt, delta_ckpt):
    _check(lib().q38_recurrent_checkpoint(ctx.handle, _ptr(conv_state), _ptr(delta_state), n_conv, n_delta,
                                          _ptr(conv_ckpt), _ptr(delta_ckpt)), "q38_recurrent_checkpoint")


def recurrent_restore(ctx: "Context", conv_ckpt, delta_ckpt, n_conv, n_delta, conv_state, delta_state):
    _check(lib().q38_recurrent_restore(ctx.handle, _ptr(conv_ckpt), _ptr(delta_ckpt), n_conv, n_delta,
                                       _ptr(conv_state), _ptr(delta_state)), "q38_recurrent_restore")


def header_functions(paths=None) -> list[str]:
    """Names of the functions the headers under include/ declare."""
    import glob
    import re
    names = set()
    for path in paths or sorted(glob.glob(os.path.join(INCLUDE_DIR, "*.h"))):
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(q38_[a-z0-9_]+)\s*\(", text))
    return sorted(names)
