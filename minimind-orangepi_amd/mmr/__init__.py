"""ctypes binding of libmmr.so, the MiniMind gfx950 decode runtime.

Everything here is a thin wrapper over the C ABI declared in include/mmr.h.
Device memory is plain HIP memory owned by DeviceArray objects (no torch):
numpy arrays go in and out through explicit copies.

The library must have been built (python minimind-orangepi_amd/build.py);
importing this module without it raises ImportError instead of falling back to
any CPU implementation.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent.parent
LIB_PATH = PKG / "lib" / "libmmr.so"

if not LIB_PATH.exists():
    raise ImportError(f"libmmr.so not built: run python {PKG / 'build.py'} (expected {LIB_PATH})")

_lib = C.CDLL(str(LIB_PATH))

OK, ERR_INVALID_ARGUMENT, ERR_OUT_OF_RANGE, ERR_RUNTIME, ERR_LENGTH = 0, 1, 2, 3, 4
KV_F16, KV_F32 = 0, 1
PRO_PLAIN, PRO_RMSNORM, PRO_RMSNORM_FINAL = 0, 1, 2
EPI_STORE, EPI_RESIDUAL, EPI_SWIGLU = 0, 1, 2
KERNEL_QKV, KERNEL_ATTENTION, KERNEL_O, KERNEL_GATE_UP, KERNEL_DOWN, KERNEL_LM_HEAD, KERNEL_FINALIZE = range(7)


class MmrError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"mmr error {code}: {message}")
        self.code = code


class InvalidArgument(MmrError, ValueError):
    pass


class OutOfRange(MmrError, IndexError):
    pass


class LengthError(MmrError):
    pass


_ERRORS = {ERR_INVALID_ARGUMENT: InvalidArgument, ERR_OUT_OF_RANGE: OutOfRange, ERR_LENGTH: LengthError}


class Config(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_int64),
        ("num_hidden_layers", C.c_int64),
        ("vocab_size", C.c_int64),
        ("num_attention_heads", C.c_int64),
        ("num_key_value_heads", C.c_int64),
        ("head_dim", C.c_int64),
        ("intermediate_size", C.c_int64),
        ("max_position_embeddings", C.c_int64),
        ("bos_token_id", C.c_int32),
        ("eos_token_id", C.c_int32),
        ("use_moe", C.c_int32),
        ("tie_word_embeddings", C.c_int32),
        ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_float),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


VP, I64, I32, U64, F32, SZ = C.c_void_p, C.c_int64, C.c_int32, C.c_uint64, C.c_float, C.c_size_t
P_I32 = C.POINTER(C.c_int32)
P_F32 = C.POINTER(C.c_float)

_SIGS = {
    "mmr_last_error": ([], C.c_char_p),
    "mmr_version": ([], C.c_int),
    "mmr_device_count": ([C.POINTER(C.c_int)], C.c_int),
    "mmr_launch_floor_us": ([C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_float)], C.c_int),
    "mmr_graph_capture_begin": ([VP], C.c_int),
    "mmr_graph_capture_end": ([VP, C.POINTER(VP)], C.c_int),
    "mmr_graph_launch": ([VP, VP], C.c_int),
    "mmr_graph_destroy": ([VP], C.c_int),
    "mmr_malloc": ([C.POINTER(VP), SZ], C.c_int),
    "mmr_free": ([VP], C.c_int),
    "mmr_memcpy_h2d": ([VP, VP, SZ], C.c_int),
    "mmr_memcpy_d2h": ([VP, VP, SZ], C.c_int),
    "mmr_memset": ([VP, C.c_int, SZ], C.c_int),
    "mmr_memcpy_d2d_async": ([VP, VP, SZ, VP], C.c_int),
    "mmr_stream_create": ([C.POINTER(VP)], C.c_int),
    "mmr_stream_destroy": ([VP], C.c_int),
    "mmr_stream_synchronize": ([VP], C.c_int),
    "mmr_device_synchronize": ([], C.c_int),
    "mmr_event_create": ([C.POINTER(VP)], C.c_int),
    "mmr_event_destroy": ([VP], C.c_int),
    "mmr_event_record": ([VP, VP], C.c_int),
    "mmr_event_elapsed_ms": ([VP, VP, P_F32], C.c_int),
    "mmr_gemm_k_splits": ([I64, I64, I64, C.POINTER(C.c_int)], C.c_int),
    "mmr_prefill_partial_floats": ([C.POINTER(Config), I64, C.POINTER(I64)], C.c_int),
    "mmr_splitk_block_tile": ([C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)], C.c_int),
    "mmr_decode_attention_splits": ([I64, I64, C.POINTER(C.c_int)], C.c_int),
    "mmr_f32_to_f16": ([VP, VP, SZ], C.c_int),
    "mmr_f16_to_f32": ([VP, VP, SZ], C.c_int),
    "mmr_matvec_f16": ([VP, I64, I64, VP, VP, VP, VP], C.c_int),
    "mmr_matvec_f16_ex": ([VP, I64, I64, VP, VP, F32, C.c_int, C.c_int, VP, VP, C.c_int, C.c_int, VP], C.c_int),
    "mmr_matvec_f16x": ([VP, I64, I64, VP, VP, VP, VP], C.c_int),
    "mmr_matvec_argmax_f16x": ([VP, I64, I64, VP, VP, VP, VP, SZ, VP], C.c_int),
    "mmr_matvec_argmax_workspace_size": ([I64, I64], SZ),
    "mmr_matvec_argmax_f16": ([VP, I64, I64, VP, VP, F32, VP, VP, VP, SZ, VP], C.c_int),
    "mmr_rope_table_create": ([I64, I64, F32, C.POINTER(VP)], C.c_int),
    "mmr_rope_table_destroy": ([VP], C.c_int),
    "mmr_kv_cache_create": ([I64, I64, I64, C.c_int, C.POINTER(VP)], C.c_int),
    "mmr_kv_cache_destroy": ([VP], C.c_int),
    "mmr_kv_cache_reserve": ([VP, I64], C.c_int),
    "mmr_kv_cache_reset": ([VP], C.c_int),
    "mmr_kv_cache_backed": ([VP, C.POINTER(I64), C.POINTER(U64)], C.c_int),
    "mmr_kv_cache_segment": ([VP, C.c_int, C.POINTER(VP), C.POINTER(VP), C.POINTER(I64), C.POINTER(I64)], C.c_int),
    "mmr_kv_cache_write": ([VP, I64, I64, VP, VP], C.c_int),
    "mmr_kv_cache_read": ([VP, I64, I64, VP, VP], C.c_int),
    "mmr_kv_cache_info": ([VP, C.POINTER(I64), C.POINTER(I64), C.POINTER(I64), C.POINTER(C.c_int)], C.c_int),
    "mmr_cube_matvec_available": ([], C.c_int),
    "mmr_cube_matmul_available": ([], C.c_int),
    "mmr_custom_ops_available": ([], C.c_int),
    "mmr_cube_matvec": ([VP, I64, I64, VP, VP], C.c_int),
    "mmr_cube_matmul": ([VP, I64, I64, VP, I64, VP], C.c_int),
    "mmr_cube_matvec_argmax": ([VP, I64, I64, VP, P_I32], C.c_int),
    "mmr_custom_attention": ([VP, VP, VP, I64, I64, I64, I64, VP], C.c_int),
    "mmr_custom_prefill_attention": ([VP, VP, VP, C.POINTER(VP), I64, I64, I64, I64, VP], C.c_int),
    "mmr_custom_attention_cached": ([VP, VP, VP, C.POINTER(VP), I64, I64, I64, I64, VP], C.c_int),
    "mmr_decode_qkv_postprocess": ([VP, VP, VP, VP, I64, I64, I64, I64, I64, VP, F32, VP, VP], C.c_int),
    "mmr_attention_workspace_size": ([I64, I64, I64, C.c_int], SZ),
    "mmr_attention_from_cache": ([VP, VP, I64, I64, I64, I64, VP, VP, SZ, C.c_int, VP], C.c_int),
    "mmr_attention_from_cache_noalloc": ([VP, VP, I64, I64, I64, I64, VP, C.c_int, VP], C.c_int),
    "mmr_decode_attention_fused": ([VP, VP, VP, F32, VP, VP, VP, I64, I64, I64, VP, VP, SZ, C.c_int, VP, VP],
                                   C.c_int),
    "mmr_layer_weights_create": ([C.POINTER(Config)] + [VP] * 11 + [C.POINTER(VP)], C.c_int),
    "mmr_model_layer_weights": ([VP, I64, C.POINTER(VP)], C.c_int),
    "mmr_layer_weights_destroy": ([VP], C.c_int),
    "mmr_decoder_layer_workspace_size": ([C.POINTER(Config), C.c_int], SZ),
    "mmr_decoder_layer_forward": ([VP, VP, VP, VP, VP, VP, SZ, C.c_int, VP, VP], C.c_int),
    "mmr_prefill_layer_workspace_size": ([C.POINTER(Config), I64], SZ),
    "mmr_prefill_layer_forward": ([VP, VP, VP, I64, I64, VP, VP, SZ, VP], C.c_int),
    "mmr_matmul_f16": ([VP, I64, I64, VP, I64, VP, VP, VP], C.c_int),
    "mmr_prefill_qkv_rows": ([VP, VP, VP, F32, VP, VP, I64, I64, I64, I64, I64, VP, VP], C.c_int),
    "mmr_prefill_attention": ([VP, VP, I64, I64, I64, I64, I64, VP, VP], C.c_int),
    "mmr_rms_norm_rows": ([VP, VP, F32, I64, I64, VP, VP], C.c_int),
    "mmr_add": ([VP, VP, I64, VP, VP], C.c_int),
    "mmr_swiglu_rows": ([VP, I64, I64, VP, VP], C.c_int),
    "mmr_embedding_gather": ([VP, VP, I64, I64, I64, VP, VP, VP], C.c_int),
    "mmr_default_config": ([C.POINTER(Config)], C.c_int),
    "mmr_load_config": ([C.c_char_p, C.POINTER(Config)], C.c_int),
    "mmr_has_runtime_model": ([C.c_char_p, C.POINTER(C.c_int)], C.c_int),
    "mmr_model_load": ([C.c_char_p, C.POINTER(VP)], C.c_int),
    "mmr_model_create_synthetic": ([C.POINTER(Config), U64, C.c_double, C.c_int, C.POINTER(VP)], C.c_int),
    "mmr_model_free": ([VP], C.c_int),
    "mmr_model_config": ([VP, C.POINTER(Config)], C.c_int),
    "mmr_model_weight_bytes": ([VP, C.POINTER(U64)], C.c_int),
    "mmr_write_synthetic_model": ([C.c_char_p, C.POINTER(Config), U64, C.c_double, C.c_int], C.c_int),
    "mmr_model_create_toy": ([C.POINTER(VP)], C.c_int),
    "mmr_write_toy_model": ([C.c_char_p], C.c_int),
    "mmr_synthesize_normals": ([U64, U64, U64, C.c_double, C.c_int, VP], C.c_int),
    "mmr_synthesize_prompt": ([U64, I64, I64, VP], C.c_int),
    "mmr_state_create": ([VP, I64, C.c_int, C.POINTER(VP)], C.c_int),
    "mmr_state_free": ([VP], C.c_int),
    "mmr_state_position": ([VP, C.POINTER(I64)], C.c_int),
    "mmr_state_kv_backed": ([VP, C.POINTER(I64), C.POINTER(U64)], C.c_int),
    "mmr_state_reserve": ([VP, VP, I64], C.c_int),
    "mmr_state_stream": ([VP, C.POINTER(VP)], C.c_int),
    "mmr_state_reset": ([VP, VP], C.c_int),
    "mmr_forward_token": ([VP, VP, I32, VP], C.c_int),
    "mmr_forward_next_token": ([VP, VP, I32, P_I32], C.c_int),
    "mmr_prefill_next_token": ([VP, VP, VP, I64, P_I32], C.c_int),
    "mmr_generate": ([VP, VP, I64, I64, VP, C.POINTER(I64)], C.c_int),
    "mmr_enqueue_prefill": ([VP, VP, VP, I64], C.c_int),
    "mmr_enqueue_decode": ([VP, VP, I64, I32], C.c_int),
    "mmr_state_synchronize": ([VP, VP], C.c_int),
    "mmr_read_sequence": ([VP, VP, I64, I64, VP], C.c_int),
    "mmr_read_logits": ([VP, VP, VP], C.c_int),
    "mmr_launch_step_kernel": ([VP, VP, C.c_int, I64, I64], C.c_int),
    "mmr_time_step_kernel": ([VP, VP, C.c_int, I64, I64, C.POINTER(C.c_double)], C.c_int),
    "mmr_batch_state_create": ([VP, I64, I64, C.c_int, C.POINTER(VP)], C.c_int),
    "mmr_batch_state_free": ([VP], C.c_int),
    "mmr_batch_state_info": ([VP, C.POINTER(I64), C.POINTER(I64), C.POINTER(I64)], C.c_int),
    "mmr_batch_state_stream": ([VP, C.POINTER(VP)], C.c_int),
    "mmr_batch_prefill": ([VP, VP, VP, VP, I64], C.c_int),
    "mmr_batch_decode": ([VP, VP, I64], C.c_int),
    "mmr_batch_synchronize": ([VP, VP], C.c_int),
    "mmr_batch_read_sequence": ([VP, VP, I64, I64, I64, VP], C.c_int),
    "mmr_batch_read_logits": ([VP, VP, I64, VP], C.c_int),
}

EXPORTED = sorted(_SIGS)

for _name, (_args, _res) in _SIGS.items():
    _fn = getattr(_lib, _name)
    _fn.argtypes = _args
    _fn.restype = _res


def lib() -> C.CDLL:
    return _lib


def check(code: int) -> None:
    if code != OK:
        msg = _lib.mmr_last_error().decode(errors="replace")
        raise _ERRORS.get(code, MmrError)(code, msg)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def launch_floor_us(kernels: int = 80, blocks: int = 256, load_store: bool = True, reps: int = 20) -> float:
    """Per-kernel time of a hipGraph chain of trivial kernels (mmr_launch_floor_us)."""
    us = C.c_float()
    check(_lib.mmr_launch_floor_us(kernels, blocks, int(load_store), reps, C.byref(us)))
    return float(us.value)


def device_count() -> int:
    n = C.c_int(0)
    check(_lib.mmr_device_count(C.byref(n)))
    return n.value


# ------------------------------------------------------------- plumbing ----

class DeviceArray:
    """A HIP allocation with a numpy dtype/shape for copies in and out."""

    def __init__(self, shape, dtype, zero: bool = False):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = VP()
        check(_lib.mmr_malloc(C.byref(p), max(self.nbytes, 1)))
        self.ptr = p.value
        if zero:
            self.zero()

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if a.nbytes:
            check(_lib.mmr_memcpy_h2d(d.ptr, _ptr(a), a.nbytes))
        return d

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            check(_lib.mmr_memcpy_d2h(_ptr(out), self.ptr, self.nbytes))
        return out

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        check(_lib.mmr_memcpy_h2d(self.ptr, _ptr(a), a.nbytes))

    def zero(self) -> None:
        check(_lib.mmr_memset(self.ptr, 0, max(self.nbytes, 1)))

    def copy_from(self, other: "DeviceArray", stream: "Stream | None" = None) -> None:
        """Device-to-device copy of `other` (same byte size), enqueued on `stream`."""
        assert other.nbytes == self.nbytes
        check(_lib.mmr_memcpy_d2d_async(self.ptr, other.ptr, self.nbytes, _stream_handle(stream)))

    def free(self) -> None:
        if self.ptr:
            _lib.mmr_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self, handle: int | None = None):
        self.owned = handle is None
        if handle is None:
            h = VP()
            check(_lib.mmr_stream_create(C.byref(h)))
            handle = h.value
        self.handle = handle

    def synchronize(self) -> None:
        check(_lib.mmr_stream_synchronize(self.handle))

    def __del__(self):
        if getattr(self, "owned", False) and self.handle:
            try:
                _lib.mmr_stream_destroy(self.handle)
            except Exception:
                pass


class Graph:
    """A hipGraph captured from everything enqueued on `stream` inside the
    `with` block (mmr_graph_capture_begin / _end), replayed by launch()."""

    def __init__(self, stream: Stream):
        self.stream = stream
        self.handle = None

    def __enter__(self) -> "Graph":
        check(_lib.mmr_graph_capture_begin(self.stream.handle))
        return self

    def __exit__(self, exc_type, exc, tb) -> None:
        h = VP()
        rc = _lib.mmr_graph_capture_end(self.stream.handle, C.byref(h))
        if exc_type is None:
            check(rc)
            self.handle = h.value

    def launch(self, stream: Stream | None = None) -> None:
        check(_lib.mmr_graph_launch(self.handle, (stream or self.stream).handle))

    def free(self) -> None:
        if self.handle:
            _lib.mmr_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        h = VP()
        check(_lib.mmr_event_create(C.byref(h)))
        self.handle = h.value

    def record(self, stream) -> None:
        check(_lib.mmr_event_record(self.handle, _stream_handle(stream)))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0.0)
        check(_lib.mmr_event_elapsed_ms(self.handle, end.handle, C.byref(ms)))
        return float(ms.value)

    def __del__(self):
        try:
            _lib.mmr_event_destroy(self.handle)
        except Exception:
            pass


def synchronize() -> None:
    check(_lib.mmr_device_synchronize())


def _stream_handle(stream) -> int | None:
    """A Stream, a raw hipStream_t handle (int) or None (the null stream)."""
    return stream.handle if isinstance(stream, Stream) else stream


def gemm_k_splits(m: int, n: int, k: int) -> int:
    """K splits of the prefill / batched GEMM for an m x n x k product (host arithmetic)."""
    out = C.c_int()
    check(_lib.mmr_gemm_k_splits(m, n, k, C.byref(out)))
    return out.value


def splitk_block_tile(block: int, row_blocks: int, chunks: int) -> tuple[int, int]:
    """(W row block, K chunk) that block `block` of a batched split-K GEMM launch computes (host arithmetic)."""
    rb, ch = C.c_int(), C.c_int()
    check(_lib.mmr_splitk_block_tile(block, row_blocks, chunks, C.byref(rb), C.byref(ch)))
    return rb.value, ch.value


def decode_attention_splits(n_keys: int, head_dim: int) -> int:
    """Attention splits of a single-sequence decode step over n_keys keys (host arithmetic)."""
    out = C.c_int()
    check(_lib.mmr_decode_attention_splits(n_keys, head_dim, C.byref(out)))
    return out.value


def prefill_partial_floats(cfg: Config, chunk_rows: int) -> int:
    """Floats of the prefill split-K partial buffer of a state with chunk_rows-row chunks."""
    out = C.c_int64()
    check(_lib.mmr_prefill_partial_floats(C.byref(cfg), chunk_rows, C.byref(out)))
    return out.value


def f32_to_f16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, np.uint16)
    check(_lib.mmr_f32_to_f16(_ptr(a), _ptr(out), a.size))
    return out


def f16_to_f32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, np.float32)
    check(_lib.mmr_f16_to_f32(_ptr(a), _ptr(out), a.size))
    return out


def _s(stream) -> int | None:
    if stream is None:
        return None
    return stream.handle if isinstance(stream, Stream) else stream


# ------------------------------------------------------------------ ops ----

def matvec_f16(w: DeviceArray, rows: int, cols: int, x: DeviceArray, y: DeviceArray, residual: DeviceArray | None = None,
               stream=None) -> None:
    check(_lib.mmr_matvec_f16(w.ptr, rows, cols, x.ptr, residual.ptr if residual else None, y.ptr, _s(stream)))


def matvec_f16_ex(w, rows, cols, x, y, *, norm_w=None, eps=0.0, prologue=PRO_PLAIN, epilogue=EPI_STORE,
                  residual=None, lanes_per_row=0, rows_per_group=0, stream=None) -> None:
    check(_lib.mmr_matvec_f16_ex(w.ptr, rows, cols, x.ptr, norm_w.ptr if norm_w else None, eps, prologue, epilogue,
                                 residual.ptr if residual else None, y.ptr, lanes_per_row, rows_per_group, _s(stream)))


def matvec_f16x(w: DeviceArray, rows: int, cols: int, x: DeviceArray, y: DeviceArray,
                residual: DeviceArray | None = None, stream=None) -> None:
    """mmr_matvec_f16x: x fp16 (uint16 bits) [cols]."""
    check(_lib.mmr_matvec_f16x(w.ptr, rows, cols, x.ptr, residual.ptr if residual else None, y.ptr, _s(stream)))


def matvec_argmax_f16x(w, rows, cols, x, token_out, workspace, *, logits=None, stream=None) -> None:
    """mmr_matvec_argmax_f16x: x fp16 (uint16 bits) [cols]."""
    check(_lib.mmr_matvec_argmax_f16x(w.ptr, rows, cols, x.ptr, logits.ptr if logits else None, token_out.ptr,
                                      workspace.ptr, workspace.nbytes, _s(stream)))


def matvec_argmax_workspace_size(rows: int, cols: int) -> int:
    return int(_lib.mmr_matvec_argmax_workspace_size(rows, cols))


def matvec_argmax_f16(w, rows, cols, x, token_out, workspace, *, logits=None, norm_w=None, eps=0.0,
                      stream=None) -> None:
    check(_lib.mmr_matvec_argmax_f16(w.ptr, rows, cols, x.ptr, norm_w.ptr if norm_w else None, eps,
                                     logits.ptr if logits else None, token_out.ptr, workspace.ptr, workspace.nbytes,
                                     _s(stream)))


class RopeTable:
    def __init__(self, max_positions: int, head_dim: int, theta: float):
        h = VP()
        check(_lib.mmr_rope_table_create(max_positions, head_dim, theta, C.byref(h)))
        self.handle = h.value

    def __del__(self):
        try:
            _lib.mmr_rope_table_destroy(self.handle)
        except Exception:
            pass


class KvCache:
    """One layer's KV cache (mmr_kv_cache): 64-token pages in doubling
    segments, backed on demand.  With reserve=True (the default) every
    position up to `capacity` is backed at once; with reserve=False only the
    first segment is, until reserve() / upload() back more."""

    def __init__(self, kv_heads: int, head_dim: int, capacity: int, kv_dtype: int = KV_F32, reserve: bool = True):
        h = VP()
        check(_lib.mmr_kv_cache_create(kv_heads, head_dim, capacity, kv_dtype, C.byref(h)))
        self.handle = h.value
        self.kv_heads, self.head_dim, self.capacity, self.kv_dtype = kv_heads, head_dim, capacity, kv_dtype
        self.np_dtype = np.float16 if kv_dtype == KV_F16 else np.float32
        if reserve:
            self.reserve(capacity)

    def reserve(self, tokens: int) -> None:
        check(_lib.mmr_kv_cache_reserve(self.handle, tokens))

    def reset(self) -> None:
        check(_lib.mmr_kv_cache_reset(self.handle))

    @property
    def rows(self) -> int:
        """Backed positions (from 0)."""
        n = C.c_int64(0)
        check(_lib.mmr_kv_cache_backed(self.handle, C.byref(n), None))
        return int(n.value)

    @property
    def device_bytes(self) -> int:
        b = C.c_uint64(0)
        check(_lib.mmr_kv_cache_backed(self.handle, None, C.byref(b)))
        return int(b.value)

    def segment(self, index: int) -> tuple[int, int, int, int]:
        """(keys pointer, values pointer, first position, backed positions) of one segment."""
        k, v, first, n = VP(), VP(), C.c_int64(0), C.c_int64(0)
        check(_lib.mmr_kv_cache_segment(self.handle, index, C.byref(k), C.byref(v), C.byref(first), C.byref(n)))
        return k.value or 0, v.value or 0, int(first.value), int(n.value)

    def upload(self, keys: np.ndarray, values: np.ndarray, first: int = 0) -> None:
        """keys/values [kv_heads, n, head_dim] -> rows first .. first + n - 1 (backed as needed)."""
        k = np.ascontiguousarray(keys, dtype=self.np_dtype)
        v = np.ascontiguousarray(values, dtype=self.np_dtype)
        assert k.shape == v.shape and k.shape[0] == self.kv_heads and k.shape[2] == self.head_dim
        check(_lib.mmr_kv_cache_write(self.handle, first, k.shape[1], _ptr(k), _ptr(v)))

    def download(self, count: int | None = None) -> tuple[np.ndarray, np.ndarray]:
        """Rows 0 .. count - 1 (default: every backed row) as [kv_heads, count, head_dim]."""
        n = self.rows if count is None else count
        k = np.empty((self.kv_heads, n, self.head_dim), self.np_dtype)
        v = np.empty_like(k)
        check(_lib.mmr_kv_cache_read(self.handle, 0, n, _ptr(k), _ptr(v)))
        return k, v

    def __del__(self):
        try:
            _lib.mmr_kv_cache_destroy(self.handle)
        except Exception:
            pass


def attention_workspace_size(q_heads, kv_heads, head_dim, splits=0) -> int:
    return int(_lib.mmr_attention_workspace_size(q_heads, kv_heads, head_dim, splits))


def decode_qkv_postprocess(qkv, q_norm, k_norm, cache: KvCache, tokens, q_heads, kv_heads, head_dim, position,
                           rope: RopeTable, eps, query, stream=None) -> None:
    check(_lib.mmr_decode_qkv_postprocess(qkv.ptr, q_norm.ptr, k_norm.ptr, cache.handle, tokens, q_heads, kv_heads,
                                          head_dim, position, rope.handle, eps, query.ptr, _s(stream)))


def attention_from_cache(query, cache: KvCache, tokens, q_heads, kv_heads, head_dim, out, workspace, splits=0,
                         stream=None) -> None:
    check(_lib.mmr_attention_from_cache(query.ptr, cache.handle, tokens, q_heads, kv_heads, head_dim, out.ptr,
                                        workspace.ptr, workspace.nbytes, splits, _s(stream)))


NOALLOC_SCRATCH_BYTES = 2 << 20  # MMR_NOALLOC_SCRATCH_BYTES


def attention_from_cache_noalloc(query, cache: KvCache, tokens, q_heads, kv_heads, head_dim, out, splits=0,
                                 stream=None) -> None:
    """mmr_attention_from_cache with the library's static scratch (allocates nothing)."""
    check(_lib.mmr_attention_from_cache_noalloc(query.ptr, cache.handle, tokens, q_heads, kv_heads, head_dim, out.ptr,
                                                splits, _s(stream)))


def decode_attention_fused(qkv, q_norm, k_norm, eps, rope: RopeTable, position, cache: KvCache, q_heads, kv_heads,
                           head_dim, out, workspace, splits, error, stream=None) -> None:
    check(_lib.mmr_decode_attention_fused(qkv.ptr, q_norm.ptr, k_norm.ptr, eps, rope.handle, position.ptr,
                                          cache.handle, q_heads, kv_heads, head_dim, out.ptr, workspace.ptr,
                                          workspace.nbytes, splits, error.ptr, _s(stream)))


def matmul_f16(w, rows, cols, x, batch, y, residual=None, stream=None) -> None:
    check(_lib.mmr_matmul_f16(w.ptr, rows, cols, x.ptr, batch, residual.ptr if residual else None, y.ptr, _s(stream)))


def prefill_qkv_rows(qkv, q_norm, k_norm, eps, rope: RopeTable, cache: KvCache, start_position, seq_len, q_heads,
                     kv_heads, head_dim, query, stream=None) -> None:
    check(_lib.mmr_prefill_qkv_rows(qkv.ptr, q_norm.ptr, k_norm.ptr, eps, rope.handle, cache.handle, start_position,
                                    seq_len, q_heads, kv_heads, head_dim, query.ptr, _s(stream)))


def prefill_attention(query, cache: KvCache, start_position, seq_len, q_heads, kv_heads, head_dim, out,
                      stream=None) -> None:
    check(_lib.mmr_prefill_attention(query.ptr, cache.handle, start_position, seq_len, q_heads, kv_heads, head_dim,
                                     out.ptr, _s(stream)))


def rms_norm_rows(x, w, eps, rows, cols, out, stream=None) -> None:
    check(_lib.mmr_rms_norm_rows(x.ptr, w.ptr, eps, rows, cols, out.ptr, _s(stream)))


def add(a, b, n, out, stream=None) -> None:
    check(_lib.mmr_add(a.ptr, b.ptr, n, out.ptr, _s(stream)))


def swiglu_rows(gate_up, rows, cols, out, stream=None) -> None:
    check(_lib.mmr_swiglu_rows(gate_up.ptr, rows, cols, out.ptr, _s(stream)))


def embedding_gather(table, ids, tokens, vocab, hidden, out, error=None, stream=None) -> None:
    check(_lib.mmr_embedding_gather(table.ptr, ids.ptr, tokens, vocab, hidden, out.ptr,
                                    error.ptr if error else None, _s(stream)))


class LayerWeights:
    """One decoder layer's device weights (mmr_layer_weights_create from the
    reference's DenseLayerWeights members, or a view of a model's layer)."""

    NAMES = ("input_norm", "post_attention_norm", "q_norm", "k_norm", "q_proj", "k_proj", "v_proj", "o_proj",
             "gate_proj", "up_proj", "down_proj")

    def __init__(self, handle: int, config: "Config", owner=None):
        self.handle = handle
        self.config = config
        self._owner = owner  # a Model whose weights a view shares

    @classmethod
    def create(cls, config: "Config", **arrays) -> "LayerWeights":
        host = [np.ascontiguousarray(arrays[n], dtype=np.float32) for n in cls.NAMES]
        h = VP()
        check(_lib.mmr_layer_weights_create(C.byref(config), *[_ptr(a) for a in host], C.byref(h)))
        return cls(h.value, config)

    @classmethod
    def of_model(cls, model: "Model", layer: int) -> "LayerWeights":
        h = VP()
        check(_lib.mmr_model_layer_weights(model.handle, layer, C.byref(h)))
        return cls(h.value, model.config, model)

    def workspace_size(self, splits: int) -> int:
        return int(_lib.mmr_decoder_layer_workspace_size(C.byref(self.config), splits))

    def forward(self, cache: "KvCache", hidden: DeviceArray, position: DeviceArray, out: DeviceArray,
                workspace: DeviceArray, splits: int, error: DeviceArray, stream=None) -> None:
        """mmr_decoder_layer_forward: out = layer(hidden) at device position *position."""
        check(_lib.mmr_decoder_layer_forward(self.handle, cache.handle, hidden.ptr, position.ptr, out.ptr,
                                             workspace.ptr, workspace.nbytes, splits, error.ptr, _s(stream)))

    def prefill_workspace_size(self, seq_len: int) -> int:
        return int(_lib.mmr_prefill_layer_workspace_size(C.byref(self.config), seq_len))

    def prefill(self, cache: "KvCache", hidden_seq: DeviceArray, start_position: int, seq_len: int,
                out: DeviceArray, workspace: DeviceArray, stream=None) -> None:
        """mmr_prefill_layer_forward: out = layer(hidden_seq) over seq_len rows of an empty cache."""
        check(_lib.mmr_prefill_layer_forward(self.handle, cache.handle, hidden_seq.ptr, start_position, seq_len,
                                             out.ptr, workspace.ptr, workspace.nbytes, _s(stream)))

    def free(self) -> None:
        if self.handle:
            _lib.mmr_layer_weights_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ------------------------------------------------- host-vector twins ----

def cube_matvec_available() -> bool:
    return bool(_lib.mmr_cube_matvec_available())


def cube_matmul_available() -> bool:
    return bool(_lib.mmr_cube_matmul_available())


def custom_ops_available() -> bool:
    return bool(_lib.mmr_custom_ops_available())


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def cube_matmul(matrix, inputs) -> np.ndarray:
    """inputs [batch][cols] (or [cols]) @ matrix[rows][cols]^T through mmr_cube_matmul."""
    w, x = _f32(matrix), _f32(inputs)
    rows, cols = w.shape
    batch = 1 if x.ndim == 1 else x.shape[0]
    out = np.empty((batch, rows), np.float32)
    check(_lib.mmr_cube_matmul(_ptr(w), rows, cols, _ptr(x), batch, _ptr(out)))
    return out[0] if x.ndim == 1 else out


def cube_matvec(matrix, x) -> np.ndarray:
    w, v = _f32(matrix), _f32(x)
    out = np.empty(w.shape[0], np.float32)
    check(_lib.mmr_cube_matvec(_ptr(w), w.shape[0], w.shape[1], _ptr(v), _ptr(out)))
    return out


def cube_matvec_argmax(matrix, x) -> int:
    w, v = _f32(matrix), _f32(x)
    t = C.c_int32(0)
    check(_lib.mmr_cube_matvec_argmax(_ptr(w), w.shape[0], w.shape[1], _ptr(v), C.byref(t)))
    return int(t.value)


def custom_attention(query, keys, values, tokens, q_heads, kv_heads, head_dim) -> np.ndarray:
    q, k, v = _f32(query), _f32(keys), _f32(values)
    out = np.empty(q_heads * head_dim, np.float32)
    check(_lib.mmr_custom_attention(_ptr(q), _ptr(k), _ptr(v), tokens, q_heads, kv_heads, head_dim, _ptr(out)))
    return out


class HostAttentionCache:
    """The cache handle the host-vector attention twins create, replace or grow."""

    def __init__(self):
        self.ptr = VP()

    @classmethod
    def create(cls, kv_heads: int, head_dim: int, capacity: int, kv_dtype: int) -> "HostAttentionCache":
        """A caller-made cache (e.g. fp16, the reference's device cache dtype)."""
        c = cls()
        check(_lib.mmr_kv_cache_create(kv_heads, head_dim, capacity, kv_dtype, C.byref(c.ptr)))
        return c

    def info(self) -> tuple[int, int, int, int]:
        a, b, c, d = C.c_int64(), C.c_int64(), C.c_int64(), C.c_int()
        check(_lib.mmr_kv_cache_info(self.ptr, C.byref(a), C.byref(b), C.byref(c), C.byref(d)))
        return a.value, b.value, c.value, d.value

    def __del__(self):
        try:
            if self.ptr.value:
                _lib.mmr_kv_cache_destroy(self.ptr)
        except Exception:
            pass


def custom_prefill_attention(query, keys, values, cache: HostAttentionCache, seq_len, q_heads, kv_heads,
                             head_dim) -> np.ndarray:
    q, k, v = _f32(query), _f32(keys), _f32(values)
    out = np.empty(seq_len * q_heads * head_dim, np.float32)
    check(_lib.mmr_custom_prefill_attention(_ptr(q), _ptr(k), _ptr(v), C.byref(cache.ptr), seq_len, q_heads,
                                            kv_heads, head_dim, _ptr(out)))
    return out


def custom_attention_cached(query, key, value, cache: HostAttentionCache, tokens, q_heads, kv_heads,
                            head_dim) -> np.ndarray:
    q, k, v = _f32(query), _f32(key), _f32(value)
    out = np.empty(q_heads * head_dim, np.float32)
    check(_lib.mmr_custom_attention_cached(_ptr(q), _ptr(k), _ptr(v), C.byref(cache.ptr), tokens, q_heads,
                                           kv_heads, head_dim, _ptr(out)))
    return out


# ---------------------------------------------------------------- model ----

def default_config() -> Config:
    c = Config()
    check(_lib.mmr_default_config(C.byref(c)))
    return c


def make_config(**kw) -> Config:
    c = default_config()
    for k, v in kw.items():
        if not hasattr(c, k):
            raise KeyError(k)
        setattr(c, k, v)
    return c


def load_config(path) -> Config:
    c = Config()
    check(_lib.mmr_load_config(str(path).encode(), C.byref(c)))
    return c


def has_runtime_model(model_dir) -> bool:
    out = C.c_int(0)
    check(_lib.mmr_has_runtime_model(str(model_dir).encode(), C.byref(out)))
    return bool(out.value)


def write_synthetic_model(model_dir, config: Config, seed: int, std: float = 0.02, round_fp16: bool = True) -> None:
    check(_lib.mmr_write_synthetic_model(str(model_dir).encode(), C.byref(config), seed, std, int(round_fp16)))


def write_toy_model(model_dir) -> None:
    """The toy model as a runtime directory (the oracle loads it from there)."""
    check(_lib.mmr_write_toy_model(str(model_dir).encode()))


def synthesize_normals(seed: int, first: int, count: int, std: float = 0.02, round_fp16: bool = False) -> np.ndarray:
    out = np.empty(count, np.float32)
    check(_lib.mmr_synthesize_normals(seed, first, count, std, int(round_fp16), _ptr(out)))
    return out


def synthesize_prompt(seed: int, count: int, vocab: int) -> np.ndarray:
    out = np.empty(count, np.int32)
    check(_lib.mmr_synthesize_prompt(seed, count, vocab, _ptr(out)))
    return out


class Model:
    """LanguageModel (reference language_model.h:27-49) on the GPU."""

    def __init__(self, handle: int):
        self.handle = handle
        c = Config()
        check(_lib.mmr_model_config(self.handle, C.byref(c)))
        self.config = c

    @classmethod
    def load(cls, model_dir) -> "Model":
        h = VP()
        check(_lib.mmr_model_load(str(model_dir).encode(), C.byref(h)))
        return cls(h.value)

    @classmethod
    def toy(cls) -> "Model":
        """The reference's built-in toy model (make_toy_language_model)."""
        h = VP()
        check(_lib.mmr_model_create_toy(C.byref(h)))
        return cls(h.value)

    @classmethod
    def synthetic(cls, config: Config, seed: int, std: float = 0.02, round_fp16: bool = True) -> "Model":
        h = VP()
        check(_lib.mmr_model_create_synthetic(C.byref(config), seed, std, int(round_fp16), C.byref(h)))
        return cls(h.value)

    def weight_bytes(self) -> int:
        b = C.c_uint64(0)
        check(_lib.mmr_model_weight_bytes(self.handle, C.byref(b)))
        return int(b.value)

    def make_state(self, capacity: int = 0, kv_dtype: int = KV_F32) -> "State":
        h = VP()
        check(_lib.mmr_state_create(self.handle, capacity, kv_dtype, C.byref(h)))
        return State(self, h.value)

    def make_batch_state(self, batch: int, capacity: int, kv_dtype: int = KV_F16) -> "BatchState":
        h = VP()
        check(_lib.mmr_batch_state_create(self.handle, batch, capacity, kv_dtype, C.byref(h)))
        return BatchState(self, h.value)

    def generate(self, prompt, max_new_tokens: int) -> list[int]:
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(max(int(max_new_tokens), 1), np.int32)
        n = C.c_int64(0)
        check(_lib.mmr_generate(self.handle, _ptr(p) if p.size else None, p.size, max_new_tokens, _ptr(out),
                                C.byref(n)))
        return out[: n.value].tolist()

    def free(self) -> None:
        if self.handle:
            _lib.mmr_model_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class State:
    """DecoderState (reference language_model.h:22-25) with a device KV cache."""

    def __init__(self, model: Model, handle: int):
        self.model = model
        self.handle = handle

    @property
    def position(self) -> int:
        p = C.c_int64(0)
        check(_lib.mmr_state_position(self.handle, C.byref(p)))
        return int(p.value)

    def kv_backed(self) -> tuple[int, int]:
        """(KV positions backed by device memory, the bytes they hold)."""
        n, b = C.c_int64(0), C.c_uint64(0)
        check(_lib.mmr_state_kv_backed(self.handle, C.byref(n), C.byref(b)))
        return int(n.value), int(b.value)

    def reserve(self, positions: int) -> None:
        """Back KV positions [0, positions) now (mmr_state_reserve)."""
        check(_lib.mmr_state_reserve(self.model.handle, self.handle, positions))

    @property
    def stream(self) -> int:
        s = VP()
        check(_lib.mmr_state_stream(self.handle, C.byref(s)))
        return s.value

    def reset(self) -> None:
        check(_lib.mmr_state_reset(self.model.handle, self.handle))

    def forward_token(self, token: int) -> np.ndarray:
        out = np.empty(self.model.config.vocab_size, np.float32)
        check(_lib.mmr_forward_token(self.model.handle, self.handle, token, _ptr(out)))
        return out

    def forward_next_token(self, token: int) -> int:
        n = C.c_int32(0)
        check(_lib.mmr_forward_next_token(self.model.handle, self.handle, token, C.byref(n)))
        return int(n.value)

    def prefill_next_token(self, prompt) -> int:
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        n = C.c_int32(0)
        check(_lib.mmr_prefill_next_token(self.model.handle, self.handle, _ptr(p) if p.size else None, p.size,
                                          C.byref(n)))
        return int(n.value)

    def enqueue_prefill(self, prompt) -> None:
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        check(_lib.mmr_enqueue_prefill(self.model.handle, self.handle, _ptr(p) if p.size else None, p.size))

    def enqueue_decode(self, steps: int, first_token: int = -1) -> None:
        check(_lib.mmr_enqueue_decode(self.model.handle, self.handle, steps, first_token))

    def synchronize(self) -> None:
        check(_lib.mmr_state_synchronize(self.model.handle, self.handle))

    def read_sequence(self, first: int, count: int) -> np.ndarray:
        out = np.empty(count, np.int32)
        check(_lib.mmr_read_sequence(self.model.handle, self.handle, first, count, _ptr(out) if count else None))
        return out

    def read_logits(self) -> np.ndarray:
        out = np.empty(self.model.config.vocab_size, np.float32)
        check(_lib.mmr_read_logits(self.model.handle, self.handle, _ptr(out)))
        return out

    def launch_step_kernel(self, kernel: int, layer: int, count: int) -> None:
        check(_lib.mmr_launch_step_kernel(self.model.handle, self.handle, kernel, layer, count))

    def time_step_kernel(self, kernel: int, layer: int, count: int) -> float:
        """Average us per launch of `count` back-to-back launches (mmr_time_step_kernel)."""
        us = C.c_double()
        check(_lib.mmr_time_step_kernel(self.model.handle, self.handle, kernel, layer, count, C.byref(us)))
        return float(us.value)

    def free(self) -> None:
        if self.handle:
            _lib.mmr_state_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class BatchState:
    """Batch of independent sequences decoded in lockstep over a paged KV cache."""

    def __init__(self, model: Model, handle: int):
        self.model = model
        self.handle = handle

    def _info(self):
        b, c, s = C.c_int64(0), C.c_int64(0), C.c_int64(0)
        check(_lib.mmr_batch_state_info(self.handle, C.byref(b), C.byref(c), C.byref(s)))
        return int(b.value), int(c.value), int(s.value)

    @property
    def batch(self) -> int:
        return self._info()[0]

    @property
    def capacity(self) -> int:
        return self._info()[1]

    @property
    def steps(self) -> int:
        return self._info()[2]

    @property
    def stream(self) -> int:
        s = VP()
        check(_lib.mmr_batch_state_stream(self.handle, C.byref(s)))
        return s.value

    def prefill(self, prompts) -> None:
        lengths = np.array([len(p) for p in prompts], np.int64)
        flat = np.ascontiguousarray(np.concatenate([np.asarray(p, np.int32) for p in prompts])
                                    if len(prompts) else np.zeros(0, np.int32), dtype=np.int32)
        check(_lib.mmr_batch_prefill(self.model.handle, self.handle, _ptr(flat) if flat.size else None,
                                     _ptr(lengths) if lengths.size else None, len(prompts)))

    def decode(self, steps: int) -> None:
        check(_lib.mmr_batch_decode(self.model.handle, self.handle, steps))

    def synchronize(self) -> None:
        check(_lib.mmr_batch_synchronize(self.model.handle, self.handle))

    def read_sequence(self, index: int, first: int, count: int) -> np.ndarray:
        out = np.empty(count, np.int32)
        check(_lib.mmr_batch_read_sequence(self.model.handle, self.handle, index, first, count,
                                           _ptr(out) if count else None))
        return out

    def read_logits(self, index: int) -> np.ndarray:
        out = np.empty(self.model.config.vocab_size, np.float32)
        check(_lib.mmr_batch_read_logits(self.model.handle, self.handle, index, _ptr(out)))
        return out

    def free(self) -> None:
        if self.handle:
            _lib.mmr_batch_state_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
