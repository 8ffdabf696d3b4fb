"""ctypes wrapper of the CPU oracle (oracle/liboracle.so) -- TEST INFRASTRUCTURE ONLY.

The oracle restates the reference's CPU engine (metal_infrence_engine/src/cpu_inference.rs) in C.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package;
the engine itself never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

OR_OK, OR_ERR_IO, OR_ERR_FORMAT, OR_ERR_TENSOR, OR_ERR_POS, OR_ERR_ARG = range(6)


class OracleError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"oracle error {code}: {msg}")
        self.code = code


class _Cfg(ctypes.Structure):
    _fields_ = [
        ("hidden_size", ctypes.c_uint64),
        ("intermediate_size", ctypes.c_uint64),
        ("num_hidden_layers", ctypes.c_uint64),
        ("num_attention_heads", ctypes.c_uint64),
        ("num_key_value_heads", ctypes.c_uint64),
        ("head_dim", ctypes.c_uint64),
        ("vocab_size", ctypes.c_uint64),
        ("rms_norm_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float),
        ("eos_token_id", ctypes.c_uint32),
    ]


_lib = None


def build() -> str:
    """Compile liboracle.so with oracle/Makefile (strict IEEE f32 flags)."""
    res = subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + res.stdout + res.stderr)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = ctypes.CDLL(LIB_PATH)
    vp, sz, u16p, f32p = ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint16), ctypes.POINTER(ctypes.c_float)
    sig = {
        "or_load_model": (vp, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int), ctypes.c_char_p, sz]),
        "or_free_model": (None, [vp]),
        "or_get_config": (None, [vp, ctypes.POINTER(_Cfg)]),
        "or_num_tensors": (sz, [vp]),
        "or_tensor_info": (ctypes.c_int, [vp, sz, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_char_p),
                                          ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]),
        "or_kv_new": (vp, [vp]),
        "or_kv_new_bf16": (vp, [vp]),
        "or_round_bf16": (ctypes.c_float, [ctypes.c_float]),
        "or_kv_free": (None, [vp]),
        "or_kv_len": (sz, [vp]),
        "or_forward": (ctypes.c_int, [vp, ctypes.c_uint32, sz, vp, f32p]),
        "or_argmax": (ctypes.c_uint32, [f32p, sz]),
        "or_weight_bytes_per_token": (ctypes.c_uint64, [vp]),
        "or_kv_bytes_at": (ctypes.c_uint64, [ctypes.POINTER(_Cfg), ctypes.c_uint64]),
        "or_set_threads": (None, [ctypes.c_int]),
        "or_get_threads": (ctypes.c_int, []),
        "or_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "or_dot": (ctypes.c_float, [f32p, f32p, sz]),
        "or_dot_bf16": (ctypes.c_float, [u16p, f32p, sz]),
        "or_silu": (ctypes.c_float, [ctypes.c_float]),
        "or_rmsnorm": (None, [f32p, f32p, u16p, sz, ctypes.c_float]),
        "or_rmsnorm_inplace": (None, [f32p, u16p, sz, ctypes.c_float]),
        "or_rope": (None, [f32p, sz, sz, ctypes.c_float]),
        "or_softmax": (None, [f32p, sz]),
        "or_matvec": (None, [f32p, u16p, f32p, sz, sz]),
        "or_rope_table": (None, [f32p, sz, sz, ctypes.c_float]),
        "or_attention": (None, [f32p, f32p, f32p, sz, sz, sz, sz, f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def f32p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def u16p(a: np.ndarray):
    assert a.dtype == np.uint16 and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


class Model:
    """Model::load_model / forward (cpu_inference.rs:58-179)."""

    def __init__(self, path: str):
        st = ctypes.c_int(0)
        err = ctypes.create_string_buffer(1024)
        h = lib().or_load_model(os.fsencode(path), ctypes.byref(st), err, 1024)
        if not h:
            raise OracleError(st.value, err.value.decode())
        self._h = ctypes.c_void_p(h)
        c = _Cfg()
        lib().or_get_config(self._h, ctypes.byref(c))
        self._c = c
        self.config = {f: getattr(c, f) for f, _ in _Cfg._fields_}

    def tensors(self):
        out = []
        for i in range(lib().or_num_tensors(self._h)):
            n, d = ctypes.c_char_p(), ctypes.c_char_p()
            a, b = ctypes.c_int64(), ctypes.c_int64()
            lib().or_tensor_info(self._h, i, ctypes.byref(n), ctypes.byref(d), ctypes.byref(a), ctypes.byref(b))
            out.append((n.value.decode(), d.value.decode(), a.value, b.value))
        return out

    def weight_bytes_per_token(self) -> int:
        return int(lib().or_weight_bytes_per_token(self._h))

    def kv_bytes_at(self, pos: int) -> int:
        return int(lib().or_kv_bytes_at(ctypes.byref(self._c), pos))

    def new_cache(self, bf16: bool = False) -> "KVCache":
        """An f32 cache (KVCache::new), or with bf16=True one that rounds every appended K/V
        element to bf16 (nearest, ties to even) and attends with the rounded values."""
        return KVCache(self, bf16)

    def forward(self, token: int, pos: int, cache: "KVCache") -> np.ndarray:
        out = np.empty(self.config["vocab_size"], dtype=np.float32)
        rc = lib().or_forward(self._h, int(token), int(pos), cache._h, f32p(out))
        if rc != OR_OK:
            raise OracleError(rc, f"forward(token={token}, pos={pos})")
        return out

    def close(self):
        if getattr(self, "_h", None):
            lib().or_free_model(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class KVCache:
    def __init__(self, model: Model, bf16: bool = False):
        new = lib().or_kv_new_bf16 if bf16 else lib().or_kv_new
        self._h = ctypes.c_void_p(new(model._h))
        self._model = model
        self.bf16 = bool(bf16)

    def __len__(self):
        return int(lib().or_kv_len(self._h))

    def __del__(self):
        try:
            lib().or_kv_free(self._h)
        except Exception:
            pass


def argmax(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().or_argmax(f32p(x), x.size))


def round_bf16(x) -> np.ndarray:
    """Element-wise f32 -> nearest bf16 (ties to even), widened back to f32 (or_round_bf16)."""
    a = np.ascontiguousarray(x, dtype=np.float32).ravel()
    f = lib().or_round_bf16
    return np.array([f(float(v)) for v in a], dtype=np.float32).reshape(np.shape(x))


def set_threads(n: int) -> None:
    lib().or_set_threads(int(n))


def get_threads() -> int:
    return int(lib().or_get_threads())


def matvec(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = w.shape
    out = np.empty(rows, dtype=np.float32)
    lib().or_matvec(f32p(out), u16p(w), f32p(x), rows, cols)
    return out


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, n_heads: int, n_kv_heads: int, head_dim: int) -> np.ndarray:
    """q [n_heads*D]; k, v position-major [n_pos][n_kv*D] (the KVCache layout)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    n_pos = k.shape[0]
    out = np.empty(n_heads * head_dim, dtype=np.float32)
    lib().or_attention(f32p(q), f32p(k), f32p(v), n_pos, n_heads, n_kv_heads, head_dim, f32p(out))
    return out
