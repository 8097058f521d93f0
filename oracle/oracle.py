"""ctypes wrapper of oracle/build/liboracle.so (the C restatement in cpu_ref.c)
and of the reference-build driver oracle/_ref/ref_driver.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product (minimind-orangepi_amd/).
"""
from __future__ import annotations

import ctypes as C
import json
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "build" / "liboracle.so"
REF_DRIVER = HERE / "_ref" / "ref_driver"


def build() -> None:
    """Compile liboracle.so, and oracle/_ref/ref_driver where /root/reference exists."""
    subprocess.run(["make", "-C", str(HERE), "all"], check=True, capture_output=True, text=True)


class OrcConfig(C.Structure):
    """struct orc_config of cpu_ref.h."""
    _fields_ = [(n, C.c_int64) for n in ("hidden_size", "num_hidden_layers", "vocab_size", "num_attention_heads",
                                         "num_key_value_heads", "head_dim", "intermediate_size",
                                         "max_position_embeddings")] + \
               [(n, C.c_int32) for n in ("bos_token_id", "eos_token_id", "use_moe", "tie_word_embeddings")] + \
               [("rms_norm_eps", C.c_float), ("rope_theta", C.c_float)]


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        build()
    lib = C.CDLL(str(LIB_PATH))
    P = C.POINTER
    f32p, i32p = P(C.c_float), P(C.c_int32)
    sigs = {
        "orc_rms_norm_layer": ([f32p, f32p, C.c_int64, C.c_float, f32p], None),
        "orc_rms_norm_final": ([f32p, f32p, C.c_int64, C.c_float, f32p], None),
        "orc_matvec": ([f32p, C.c_int64, C.c_int64, f32p, f32p], None),
        "orc_rope_row": ([C.c_int64, C.c_int64, C.c_float, f32p, f32p], None),
        "orc_apply_rope": ([f32p, C.c_int64, C.c_int64, C.c_int64, C.c_float], None),
        "orc_silu": ([C.c_float], C.c_float),
        "orc_swiglu_from_gate_up": ([f32p, C.c_int64, f32p], None),
        "orc_attention_step": ([f32p, f32p, f32p, C.c_int64, C.c_int64, C.c_int64, C.c_int64, f32p], None),
        "orc_qk_norm_rope": ([f32p, f32p, f32p, f32p, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_float,
                              C.c_float], None),
        "orc_argmax": ([f32p, C.c_int64], C.c_int32),
        "orc_f32_to_f16": ([C.c_float], C.c_uint16),
        "orc_f16_to_f32": ([C.c_uint16], C.c_float),
        "orc_model_load": ([C.c_char_p, C.c_char_p, C.c_size_t], C.c_void_p),
        "orc_model_free": ([C.c_void_p], None),
        "orc_model_config": ([C.c_void_p], P(OrcConfig)),
        "orc_state_new": ([C.c_void_p], C.c_void_p),
        "orc_state_free": ([C.c_void_p], None),
        "orc_state_position": ([C.c_void_p], C.c_int64),
        "orc_forward_token": ([C.c_void_p, C.c_void_p, C.c_int32, f32p], C.c_int),
        "orc_forward_next_token": ([C.c_void_p, C.c_void_p, C.c_int32], C.c_int32),
        "orc_generate": ([C.c_void_p, i32p, C.c_int64, C.c_int64, i32p, P(C.c_int64), f32p], C.c_int),
        "orc_decoder_layer": ([C.c_void_p, C.c_void_p, C.c_int64, f32p, C.c_int64], C.c_int),
        "orc_state_layer_cache": ([C.c_void_p, C.c_int64, P(P(C.c_float)), P(P(C.c_float))], C.c_int64),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


_lib = _load()


def _f(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _i(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_int32))


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- primitives (each mirrors one cpu_ref.c function) -------------------------

def rms_norm_layer(x, w, eps) -> np.ndarray:
    x, w = f32(x), f32(w)
    out = np.empty_like(x)
    _lib.orc_rms_norm_layer(_f(x), _f(w), x.size, eps, _f(out))
    return out


def rms_norm_final(x, w, eps) -> np.ndarray:
    x, w = f32(x), f32(w)
    out = np.empty_like(x)
    _lib.orc_rms_norm_final(_f(x), _f(w), x.size, eps, _f(out))
    return out


def matvec(w, x) -> np.ndarray:
    w, x = f32(w), f32(x)
    rows, cols = w.shape
    out = np.empty(rows, np.float32)
    _lib.orc_matvec(_f(w), rows, cols, _f(x), _f(out))
    return out


def rope_row(position, head_dim, theta):
    c = np.empty(head_dim // 2, np.float32)
    s = np.empty(head_dim // 2, np.float32)
    _lib.orc_rope_row(position, head_dim, theta, _f(c), _f(s))
    return c, s


def apply_rope(values, heads, head_dim, position, theta) -> np.ndarray:
    v = f32(values).copy()
    _lib.orc_apply_rope(_f(v), heads, head_dim, position, theta)
    return v


def silu(v: float) -> float:
    return float(_lib.orc_silu(v))


def swiglu_from_gate_up(gu) -> np.ndarray:
    gu = f32(gu)
    F = gu.size // 2
    out = np.empty(F, np.float32)
    _lib.orc_swiglu_from_gate_up(_f(gu), F, _f(out))
    return out


def attention_step(query, keys, values, tokens, q_heads, kv_heads, head_dim) -> np.ndarray:
    """keys/values in the reference layout [token][kv_head][d]."""
    q, k, v = f32(query), f32(keys), f32(values)
    out = np.empty(q_heads * head_dim, np.float32)
    _lib.orc_attention_step(_f(q), _f(k), _f(v), tokens, q_heads, kv_heads, head_dim, _f(out))
    return out


def qk_norm_rope(query, key, q_norm, k_norm, q_heads, kv_heads, head_dim, position, eps, theta):
    q, k = f32(query).copy(), f32(key).copy()
    qn, kn = f32(q_norm), f32(k_norm)
    _lib.orc_qk_norm_rope(_f(q), _f(k), _f(qn), _f(kn), q_heads, kv_heads, head_dim, position, eps, theta)
    return q, k


def argmax(logits) -> int:
    lg = f32(logits)
    return int(_lib.orc_argmax(_f(lg), lg.size))


def f32_to_f16_bits(v: float) -> int:
    return int(_lib.orc_f32_to_f16(v))


def f16_bits_to_f32(h: int) -> float:
    return float(_lib.orc_f16_to_f32(h))


# ---- model ------------------------------------------------------------------------

class OracleModel:
    def __init__(self, model_dir):
        err = C.create_string_buffer(512)
        self.handle = _lib.orc_model_load(str(model_dir).encode(), err, 512)
        if not self.handle:
            raise RuntimeError(err.value.decode())

    def generate(self, prompt, max_new, want_logits: bool = False):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(max(max_new, 1), np.int32)
        n = C.c_int64(0)
        logits = np.empty(self.vocab, np.float32) if want_logits else None
        rc = _lib.orc_generate(self.handle, _i(p), p.size, max_new, _i(out), C.byref(n),
                               _f(logits) if want_logits else None)
        if rc != 0:
            raise ValueError("oracle generate failed")
        ids = out[: n.value].tolist()
        return (ids, logits) if want_logits else ids

    def new_state(self) -> "OracleState":
        return OracleState(self)

    @property
    def config(self) -> OrcConfig:
        return _lib.orc_model_config(self.handle).contents

    @property
    def vocab(self) -> int:
        return int(self.config.vocab_size)

    def __del__(self):
        try:
            _lib.orc_model_free(self.handle)
        except Exception:
            pass


class OracleState:
    def __init__(self, model: OracleModel):
        self.model = model
        self.handle = _lib.orc_state_new(model.handle)

    @property
    def position(self) -> int:
        return int(_lib.orc_state_position(self.handle))

    def forward_token(self, token: int) -> np.ndarray:
        out = np.empty(self.model.vocab, np.float32)
        if _lib.orc_forward_token(self.model.handle, self.handle, token, _f(out)) != 0:
            raise IndexError("token id out of vocabulary range")
        return out

    def decoder_layer(self, layer: int, hidden, position: int) -> np.ndarray:
        """One decoder layer (decoder_layer.cpp:312-407) on a copy of hidden,
        appending to this state's cache of that layer."""
        h = f32(hidden).copy()
        if _lib.orc_decoder_layer(self.model.handle, self.handle, layer, _f(h), position) != 0:
            raise IndexError("layer out of range")
        return h

    def layer_cache(self, layer: int):
        """(keys, values) of one layer, shaped [tokens][kv_heads][d]."""
        k, v = C.POINTER(C.c_float)(), C.POINTER(C.c_float)()
        n = int(_lib.orc_state_layer_cache(self.handle, layer, C.byref(k), C.byref(v)))
        c = self.model.config
        shape = (n, int(c.num_key_value_heads), int(c.head_dim))
        if n <= 0:
            return np.zeros(shape, np.float32), np.zeros(shape, np.float32)
        size = int(np.prod(shape))
        return (np.ctypeslib.as_array(k, (size,)).reshape(shape).copy(),
                np.ctypeslib.as_array(v, (size,)).reshape(shape).copy())

    def forward_next_token(self, token: int) -> int:
        nxt = int(_lib.orc_forward_next_token(self.model.handle, self.handle, token))
        if nxt < 0:
            raise IndexError("token id out of vocabulary range")
        return nxt

    def __del__(self):
        try:
            _lib.orc_state_free(self.handle)
        except Exception:
            pass


# ---- reference build (oracle/_ref) -------------------------------------------------

def ref_available() -> bool:
    return REF_DRIVER.exists()


def ref_run(mode: str, model_dir, prompt, n: int, logits_path=None, logit_steps=None, timeout=3600) -> dict:
    cmd = [str(REF_DRIVER), mode, str(model_dir), ",".join(str(int(t)) for t in prompt), str(int(n))]
    if logits_path is not None:
        cmd += [str(logits_path), ",".join(str(int(s)) for s in (logit_steps or []))]
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    if proc.returncode != 0:
        raise RuntimeError(f"ref_driver failed: {proc.stderr.strip()}")
    return json.loads(proc.stdout)
