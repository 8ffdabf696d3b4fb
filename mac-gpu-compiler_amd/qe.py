"""Python mirror of the reference engine API over the C ABI of libqe.so (include/qe.h).

The reference crate exposes (metal_infrence_engine/src/metal_inference.rs):
    MetalModel::load_model(path)            -> Model.load_model(path)
    MetalModel::config()                    -> Model.config()
    MetalKVCache::new(&model, max_seq)      -> KVCache(model, max_seq)
    MetalModel::forward(token, pos, cache)  -> Model.forward(token, pos, cache) -> np.ndarray[V]
    MetalModel::decode(first, start_pos, steps, cache, on_token)
                                            -> Model.decode(first, start_pos, steps, cache, on_token)
Where the reference panics on a contract violation, this raises QeError with the C status.

libqe.so must be built (mac-gpu-compiler_amd/build.py); there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Callable, Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqe.so")

QE_OK = 0
QE_ERR_IO = 1
QE_ERR_FORMAT = 2
QE_ERR_TENSOR = 3
QE_ERR_POS = 4
QE_ERR_ARG = 5
QE_ERR_UNSUPPORTED = 6
QE_ERR_HIP = 7
QE_ERR_NO_DEVICE = 8
QE_ERR_KERNEL = 9
QE_DRAFT_ERROR = 0xFFFFFFFF  # a draft callback's failure return (qe_draft_fn)

QE_KV_F32 = 0
QE_KV_BF16 = 1

ERROR_NAMES = {
    QE_ERR_IO: "io", QE_ERR_FORMAT: "format", QE_ERR_TENSOR: "tensor", QE_ERR_POS: "pos",
    QE_ERR_ARG: "arg", QE_ERR_UNSUPPORTED: "unsupported", QE_ERR_HIP: "hip",
    QE_ERR_NO_DEVICE: "no_device", QE_ERR_KERNEL: "kernel",
}


class QeError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{ERROR_NAMES.get(code, code)}] {message}")
        self.code = code


class _CConfig(ctypes.Structure):
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


@dataclass(frozen=True)
class Config:
    """config.json subset (cpu_inference.rs:20-33)."""
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    vocab_size: int
    rms_norm_eps: float
    rope_theta: float
    eos_token_id: int

    def to_c(self) -> _CConfig:
        return _CConfig(*[getattr(self, f) for f, _ in _CConfig._fields_])

    @staticmethod
    def from_c(c: _CConfig) -> "Config":
        return Config(*[getattr(c, f) for f, _ in _CConfig._fields_])


# The Qwen3-0.6B architecture (28 layers, hidden 1024, 16/8 heads, head_dim 128, SwiGLU 3072,
# vocab 151936, RMSNorm eps 1e-6, RoPE theta 1e6).
QWEN3_0_6B = Config(1024, 3072, 28, 16, 8, 128, 151936, 1e-6, 1e6, 151645)

ON_TOKEN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_uint32)
# qe_draft_fn: (user, history, n, k_max, draft_out) -> draft length
DRAFT_FN = ctypes.CFUNCTYPE(ctypes.c_uint32, ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32), ctypes.c_uint64,
                            ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32))


def lookup_draft(history, ngram: int = 3, k_max: int = 4) -> list:
    """The prompt-lookup draft after `history` (qe_lookup_draft; host code, no device)."""
    h = np.ascontiguousarray(history, dtype=np.uint32)
    out = np.zeros(max(int(k_max), 1), dtype=np.uint32)
    u32p = ctypes.POINTER(ctypes.c_uint32)
    n = lib().qe_lookup_draft(h.ctypes.data_as(u32p), len(h), int(ngram), int(k_max), out.ctypes.data_as(u32p))
    return [int(t) for t in out[:n]]


class _LookupStats(ctypes.Structure):
    _fields_ = [("passes", ctypes.c_uint64), ("drafted", ctypes.c_uint64), ("accepted", ctypes.c_uint64),
                ("single_steps", ctypes.c_uint64), ("plain_steps", ctypes.c_uint64)]

_lib = None


def l2_prefetch_enabled() -> bool:
    """The engine's decode attention launch also streams the layer's gate/up and down weights
    into L2 unless QE_L2_PREFETCH=0."""
    return os.environ.get("QE_L2_PREFETCH", "1") != "0"


def l2_prefetch_max_pos(cfg: Config, kv_el: int = 4) -> int:
    """First position at which the attention launch no longer prefetches: where one layer's K/V
    history reaches half the prefetched gate/up + down bytes (the engine's rule)."""
    pf_bytes = 3 * cfg.intermediate_size * cfg.hidden_size * 2
    return int(0.5 * pf_bytes / (2 * cfg.num_key_value_heads * cfg.head_dim * kv_el))


def stage_bytes(cfg: Config, mean_pos: float, kv_el: int = 4) -> dict:
    """Algorithmic bytes per launch of each decode-step stage: a matvec moves its bf16 weights
    plus its f32 input and output once (out*in*2 + in*4 + out*4, bench.rs:106-119 counts the
    weights); the attention its K/V history at mean_pos (positions 0..mean_pos) plus the raw
    q/k/v it reads and its output. The gate/up and down weights that the attention launch also
    pulls into L2 (prefetch_bytes) are counted with the gate_up and down stages, which read them."""
    H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    QD, KD = cfg.num_attention_heads * cfg.head_dim, cfg.num_key_value_heads * cfg.head_dim
    st = {
        "embed": H * 2 + H * 4,
        "qkv": (QD + 2 * KD) * H * 2 + H * 2 + H * 4 + (QD + 2 * KD) * 4,
        "attention": 2 * KD * (mean_pos + 1) * kv_el + (QD + 2 * KD) * 4 + QD * 4,
        "o_proj": H * QD * 2 + QD * 4 + 2 * H * 4,
        "gate_up": 2 * I * H * 2 + H * 2 + H * 4 + I * 4,
        "down": H * I * 2 + I * 4 + 2 * H * 4,
        "lm_head": V * H * 2 + H * 2 + H * 4 + V * 4,
        "argmax": 8 * ((V + 15) // 16),
    }
    # the fused decode layers (QE_FUSED=1: attention block and MLP block per layer; 2: one launch
    # for all layers), counted as the stages they contain; the residual stream's partials travel
    # between launches (8 partial vectors of H floats, read with the residual)
    parts = 8 * H * 4 + H * 4
    st["attn_block"] = st["qkv"] + st["attention"] + st["o_proj"] + parts
    st["mlp_block"] = st["gate_up"] + st["down"] + parts
    st["final_reduce"] = parts + H * 4
    st["layers"] = cfg.num_hidden_layers * (st["qkv"] + st["attention"] + st["o_proj"] + st["gate_up"] + st["down"])
    return st


def prefetch_bytes(cfg: Config, mean_pos: float, kv_el: int = 4) -> int:
    """Weight bytes one decode attention launch pulls into L2 for the later stages (the layer's
    gate/up and down), or 0 at positions where the engine no longer prefetches."""
    H, I = cfg.hidden_size, cfg.intermediate_size
    return 3 * I * H * 2 if mean_pos < l2_prefetch_max_pos(cfg, kv_el) else 0


def lib() -> ctypes.CDLL:
    """Load libqe.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with mac-gpu-compiler_amd/build.py")
    # One HIP runtime per process: PyTorch links its bundled libamdhip64.so by the unversioned
    # name, libqe.so by the soname libamdhip64.so.7. Loading torch first makes libqe.so bind to
    # the copy torch already mapped (same soname) instead of mapping /opt/rocm's beside it.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = ctypes.CDLL(LIB_PATH)
    vp, u64, u32, i32, f32p = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.POINTER(ctypes.c_float)
    sig = {
        "qe_last_error": (ctypes.c_char_p, []),
        "qe_model_load": (i32, [ctypes.c_char_p, ctypes.POINTER(vp)]),
        "qe_model_free": (None, [vp]),
        "qe_model_config": (i32, [vp, ctypes.POINTER(_CConfig)]),
        "qe_weight_bytes_per_token": (u64, [vp]),
        "qe_model_fused_layers": (i32, [vp]),
        "qe_model_stream": (vp, [vp]),
        "qe_kv_bytes_at": (u64, [vp, u64, i32]),
        "qe_kv_new": (i32, [vp, u64, i32, ctypes.POINTER(vp)]),
        "qe_kv_free": (None, [vp]),
        "qe_kv_max_seq": (u64, [vp]),
        "qe_kv_len": (u64, [vp]),
        "qe_forward": (i32, [vp, u32, u64, vp, f32p]),
        "qe_prefill": (i32, [vp, ctypes.POINTER(u32), u64, u64, vp, f32p]),
        "qe_profile_step": (i32, [vp, u32, u64, vp, f32p, ctypes.POINTER(u32), ctypes.POINTER(ctypes.c_char_p),
                                  u32, ctypes.POINTER(u32)]),
        "qe_decode": (i32, [vp, u32, u64, u64, vp, ON_TOKEN, vp, f32p]),
        "qe_prefill_batch": (i32, [vp, ctypes.POINTER(u32), u64, u64, vp, u32, f32p]),
        "qe_verify": (i32, [vp, ctypes.POINTER(u32), u64, u64, vp, f32p]),
        "qe_verify_greedy": (i32, [vp, ctypes.POINTER(u32), u64, u64, vp, ctypes.POINTER(u32)]),
        "qe_lookup_draft": (u64, [ctypes.POINTER(u32), u64, u32, u32, ctypes.POINTER(u32)]),
        "qe_decode_lookup": (i32, [vp, ctypes.POINTER(u32), u64, u32, u64, u64, vp, u32, u32, ON_TOKEN, vp,
                                   ctypes.POINTER(_LookupStats)]),
        "qe_decode_drafted": (i32, [vp, ctypes.POINTER(u32), u64, u32, u64, u64, vp, u32, DRAFT_FN, vp, ctypes.c_int,
                                    ON_TOKEN, vp, ctypes.POINTER(_LookupStats)]),
        "qe_op_gemm_bf16": (i32, [vp, vp, vp, u64, u64, u64, vp]),
        "qe_write_random_checkpoint": (i32, [ctypes.c_char_p, u64, ctypes.POINTER(_CConfig)]),
        "qe_random_prompt": (None, [u64, u64, u32, ctypes.POINTER(u32)]),
        "qe_op_matvec_bf16": (i32, [vp, vp, vp, u64, u64, vp]),
        "qe_op_attention_work_bytes": (u64, [u64, u64, u64]),
        "qe_op_attention": (i32, [vp, vp, vp, vp, u64, u64, u64, u64, u32, vp, vp]),
        "qe_op_read_sum": (i32, [vp, u64, vp, u32, vp]),
        "qe_op_read_sum_nt": (i32, [vp, u64, vp, u32, vp]),
        "qe_op_argmax": (i32, [vp, u64, u64, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != QE_OK:
        raise QeError(rc, lib().qe_last_error().decode(errors="replace"))


def _fptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


class Model:
    """GPU engine handle: MetalModel (metal_inference.rs:100-113, 156-170)."""

    def __init__(self, handle: int):
        self._h = ctypes.c_void_p(handle)
        cfg = _CConfig()
        _check(lib().qe_model_config(self._h, ctypes.byref(cfg)))
        self._cfg = Config.from_c(cfg)

    @classmethod
    def load_model(cls, path: str) -> "Model":
        h = ctypes.c_void_p()
        _check(lib().qe_model_load(os.fsencode(path), ctypes.byref(h)))
        return cls(h.value)

    def config(self) -> Config:
        return self._cfg

    def weight_bytes_per_token(self) -> int:
        return int(lib().qe_weight_bytes_per_token(self._h))

    def fused_layers(self) -> int:
        """How the decode step runs its layers: 2 = one persistent launch for all of them, 1 = two
        launches per layer (attention block, MLP block; one KV head per XCD), 0 = one launch per
        stage."""
        return int(lib().qe_model_fused_layers(self._h))

    def stream_handle(self) -> int:
        """The hipStream_t all of this model's work runs on (for external timing events)."""
        return int(lib().qe_model_stream(self._h) or 0)

    def kv_bytes_at(self, pos: int, kv_dtype: int = QE_KV_F32) -> int:
        return int(lib().qe_kv_bytes_at(self._h, pos, kv_dtype))

    def forward(self, token: int, pos: int, cache: "KVCache") -> np.ndarray:
        """Logits [vocab] f32 for `token` at `pos`; appends its K/V (metal_inference.rs:284-291)."""
        out = np.empty(self._cfg.vocab_size, dtype=np.float32)
        _check(lib().qe_forward(self._h, int(token), int(pos), cache._h, _fptr(out)))
        return out

    def prefill(self, ids, start_pos: int, cache: "KVCache", want_logits: bool = True) -> Optional[np.ndarray]:
        arr = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32))
        out = np.empty(self._cfg.vocab_size, dtype=np.float32) if want_logits and arr.size else None
        _check(lib().qe_prefill(self._h, arr.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), arr.size, int(start_pos),
                                cache._h, _fptr(out) if out is not None else None))
        return out  # None for an empty prompt: there are no logits

    def profile_step(self, token: int, pos: int, cache: "KVCache"):
        """Runs `token` at `pos`, then times every stage of the step as a graph of that stage's
        launches: returns [(stage name, microseconds per launch, launches per step)]."""
        cap = 16
        us = np.empty(cap, dtype=np.float32)
        launches = (ctypes.c_uint32 * cap)()
        names = (ctypes.c_char_p * cap)()
        n = ctypes.c_uint32(0)
        _check(lib().qe_profile_step(self._h, int(token), int(pos), cache._h, _fptr(us), launches, names, cap,
                                     ctypes.byref(n)))
        return [(names[i].decode(), float(us[i]), int(launches[i])) for i in range(min(n.value, cap))]

    def prefill_batch(self, ids, start_pos: int, cache: "KVCache", chunk: int = 0, want_logits: bool = True):
        """Chunked prefill on the matrix cores (qe_prefill_batch): the last token's logits or None."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty(self.config().vocab_size, dtype=np.float32) if want_logits and len(ids) else None
        _check(lib().qe_prefill_batch(self._h, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), len(ids),
                                      int(start_pos), cache._h, int(chunk), _fptr(out) if out is not None else None))
        return out  # None for an empty prompt: there are no logits

    def verify(self, ids, start_pos: int, cache: "KVCache") -> np.ndarray:
        """k tokens in one pass (qe_verify): logits [k, vocab]."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty((len(ids), self.config().vocab_size), dtype=np.float32)
        _check(lib().qe_verify(self._h, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), len(ids),
                               int(start_pos), cache._h, _fptr(out)))
        return out

    def verify_greedy(self, ids, start_pos: int, cache: "KVCache") -> np.ndarray:
        """k tokens in one pass with the argmax on the device (qe_verify_greedy): the greedy token
        after each of them, uint32 [k]."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty(len(ids), dtype=np.uint32)
        u32p = ctypes.POINTER(ctypes.c_uint32)
        _check(lib().qe_verify_greedy(self._h, ids.ctypes.data_as(u32p), len(ids), int(start_pos), cache._h,
                                      out.ctypes.data_as(u32p)))
        return out

    def decode_lookup(self, first: int, start_pos: int, steps: int, cache: "KVCache", context=(),
                      k_max: int = 4, ngram: int = 3, on_token: Optional[Callable[[int], None]] = None):
        """Greedy decode with prompt-lookup drafts checked by verify passes (qe_decode_lookup): the
        same tokens as decode(). context: the ids before `first` (the prompt). Returns (tokens,
        stats) with stats = {passes, drafted, accepted, single_steps, plain_steps}."""
        toks = []

        def cb(_user, tok):
            toks.append(int(tok))
            if on_token is not None:
                on_token(int(tok))

        ccb = ON_TOKEN(cb)
        ctx = np.ascontiguousarray(context, dtype=np.uint32)
        st = _LookupStats()
        _check(lib().qe_decode_lookup(self._h, ctx.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), len(ctx),
                                      int(first), int(start_pos), int(steps), cache._h, int(k_max), int(ngram), ccb,
                                      None, ctypes.byref(st)))
        return toks, {f: int(getattr(st, f)) for f, _ in _LookupStats._fields_}

    def decode_drafted(self, first: int, start_pos: int, steps: int, cache: "KVCache",
                       draft: Callable[[list, int], list], context=(), k_max: int = 4, adaptive: bool = True,
                       on_token: Optional[Callable[[int], None]] = None):
        """decode_lookup with the drafts of draft(history, k_max) -> list of at most k_max tokens
        (qe_decode_drafted); adaptive: the same rule as decode_lookup's. Returns (tokens, stats)."""
        toks = []
        err = []

        def cb(_user, tok):
            toks.append(int(tok))
            if on_token is not None:
                on_token(int(tok))

        def dcb(_user, hist, n, k, out):
            try:
                d = [int(t) for t in draft(np.ctypeslib.as_array(hist, shape=(n,)).tolist(), int(k))][:int(k)]
            except Exception as e:  # an exception cannot cross the C frames: stop the decode, raise it after
                err.append(e)
                return QE_DRAFT_ERROR
            for i, t in enumerate(d):
                out[i] = t
            return len(d)

        ccb, cdraft = ON_TOKEN(cb), DRAFT_FN(dcb)
        ctx = np.ascontiguousarray(context, dtype=np.uint32)
        st = _LookupStats()
        rc = lib().qe_decode_drafted(self._h, ctx.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), len(ctx),
                                     int(first), int(start_pos), int(steps), cache._h, int(k_max), cdraft, None,
                                     int(bool(adaptive)), ccb, None, ctypes.byref(st))
        if err:
            raise err[0]
        _check(rc)
        return toks, {f: int(getattr(st, f)) for f, _ in _LookupStats._fields_}

    def decode(self, first: int, start_pos: int, steps: int, cache: "KVCache",
               on_token: Optional[Callable[[int], None]] = None, want_logits: bool = False):
        """Greedy decode (metal_inference.rs:293-316): calls on_token(token) once per finished
        step, in order. Returns (tokens, logits or None); logits is [steps, vocab]."""
        toks = []

        def cb(_user, tok):
            toks.append(int(tok))
            if on_token is not None:
                on_token(int(tok))

        ccb = ON_TOKEN(cb)
        logits = np.empty((steps, self._cfg.vocab_size), dtype=np.float32) if want_logits else None
        _check(lib().qe_decode(self._h, int(first), int(start_pos), int(steps), cache._h, ccb, None,
                               _fptr(logits) if logits is not None else None))
        return toks, logits

    def close(self) -> None:
        if self._h and self._h.value:
            lib().qe_model_free(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class KVCache:
    """MetalKVCache::new(&model, max_seq) (metal_inference.rs:115-138); kv_dtype f32 or bf16."""

    def __init__(self, model: Model, max_seq: int, kv_dtype: int = QE_KV_F32):
        h = ctypes.c_void_p()
        _check(lib().qe_kv_new(model._h, int(max_seq), int(kv_dtype), ctypes.byref(h)))
        self._h = h
        self._model = model  # the cache must not outlive its model
        self.max_seq = int(max_seq)

    def __len__(self) -> int:
        return int(lib().qe_kv_len(self._h))

    def close(self) -> None:
        if self._h and self._h.value:
            lib().qe_kv_free(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def write_random_checkpoint(directory: str, seed: int, cfg: Config = QWEN3_0_6B) -> str:
    """Seeded random-init checkpoint: <dir>/model.safetensors + config.json. Returns the path."""
    os.makedirs(directory, exist_ok=True)
    c = cfg.to_c()
    _check(lib().qe_write_random_checkpoint(os.fsencode(directory), int(seed), ctypes.byref(c)))
    return os.path.join(directory, "model.safetensors")


def random_prompt(seed: int, n: int, vocab: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    lib().qe_random_prompt(int(seed), int(n), int(vocab), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
    return out


# ---- isolated device ops on torch tensors (device memory owned by the caller) ----

def _ptr(t) -> int:
    return t.data_ptr()


def _stream_ptr(stream) -> Optional[int]:
    if stream is None:
        return None
    return int(getattr(stream, "cuda_stream", stream))


def op_matvec_bf16(w, x, out, stream=None) -> None:
    """out[r] = sum_c w[r, c] x[c]; w bf16 [rows, cols] (torch.bfloat16 or int16/uint16 view), x f32."""
    rows, cols = w.shape
    _check(lib().qe_op_matvec_bf16(_ptr(w), _ptr(x), _ptr(out), rows, cols, _stream_ptr(stream)))


def op_gemm_bf16(a, w, c, stream=None) -> None:
    """c [m, n] = a [m, k] (f32) @ w [n, k] (bf16)^T on the matrix cores."""
    m, k = a.shape
    n = w.shape[0]
    _check(lib().qe_op_gemm_bf16(_ptr(a), _ptr(w), _ptr(c), m, n, k, _stream_ptr(stream)))


def op_attention_work_bytes(n_heads: int, n_kv_heads: int, n_pos: int) -> int:
    return int(lib().qe_op_attention_work_bytes(n_heads, n_kv_heads, n_pos))


def op_attention(q, k, v, out, n_pos: int, n_heads: int, n_kv_heads: int, work, n_splits: int = 0, stream=None) -> None:
    """q [n_heads*128]; k, v [n_kv][kv_stride][128] f32; work: op_attention_work_bytes() device bytes."""
    kv_stride = k.shape[1]
    _check(lib().qe_op_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(out), n_pos, kv_stride, n_heads, n_kv_heads,
                                 n_splits, _ptr(work), _stream_ptr(stream)))


def op_argmax(logits, tokens, stream=None) -> None:
    """tokens[r] = greedy token of logits[r] (f32 [rows, n] on the device; tokens int32/uint32 [rows])."""
    rows, n = logits.shape
    _check(lib().qe_op_argmax(_ptr(logits), rows, n, _ptr(tokens), _stream_ptr(stream)))


def op_read_sum(src, partial, grid: int = 0, stream=None) -> None:
    _check(lib().qe_op_read_sum(_ptr(src), src.numel(), _ptr(partial), grid, _stream_ptr(stream)))


def op_read_sum_nt(src, partial, grid: int = 0, stream=None) -> None:
    _check(lib().qe_op_read_sum_nt(_ptr(src), src.numel(), _ptr(partial), grid, _stream_ptr(stream)))
