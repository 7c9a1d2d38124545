"""CPU oracle for the int8 attention path (numpy over ctypes).

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke check and the CPU
baseline leg of bench.py, never by the reef_amd package. ``liboracle.so`` is
the plain-C restatement of the Reef engine's arithmetic (reef_oracle.c, each
function citing the engine file:line it follows). ``_ref/libref.so``, when it
was built here from the engine's own headers (``make -C oracle ref``), wraps
the engine itself so the restatement can be compared with it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref.so")

OK, INVALID, NON_FINITE = 0, 1, 2
GRAN_TENSOR, GRAN_HEAD, GRAN_TOKEN = 0, 1, 2

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_sz = C.c_size_t
_i64 = C.c_int64


class AttnDesc(C.Structure):
    _fields_ = [
        ("batch", C.c_int64), ("q_heads", C.c_int64), ("kv_heads", C.c_int64),
        ("q_len", C.c_int64), ("kv_len", C.c_int64), ("head_dim", C.c_int64),
        ("query_start", C.c_int64), ("window", C.c_int64),
        ("softmax_scale", C.c_float),
        ("q_granularity", C.c_int32), ("kv_granularity", C.c_int32),
        ("threads", C.c_int32),
    ]


def build() -> None:
    """Compile liboracle.so (and oracle/_ref when the reference is present)."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    if os.path.isdir(os.environ.get("REEF_REFERENCE", "/root/reference/inference-engine")):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)
        if os.path.exists(os.path.join(HERE, "..", "reef_amd", "libreef_hip.so")):
            subprocess.run(["make", "-s", "-C", HERE, "dropin", "gpt_neo"], check=True)


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        build()
    lib = C.CDLL(LIB_PATH)
    sig = {
        "ro_int8_scale": (C.c_float, [C.c_float]),
        "ro_quantize_int8": (C.c_int, [C.c_float, C.c_float, C.POINTER(C.c_int8)]),
        "ro_row_max_magnitude": (C.c_float, [_f32p, _sz]),
        "ro_quantize_rows": (C.c_int, [_f32p, _sz, _sz, _i8p, _f32p]),
        "ro_quantize_per_tensor": (C.c_int, [_f32p, _sz, _i8p, _f32p]),
        "ro_quantize_per_head": (C.c_int, [_f32p, _sz, _sz, _sz, _sz, _i8p, _f32p]),
        "ro_dequantize": (None, [_i8p, _sz, _sz, _f32p, _f32p]),
        "ro_exp_nonpositive": (C.c_float, [C.c_float]),
        "ro_visible": (C.c_int, [_i64, _i64, _i64, _i64]),
        "ro_qk_i32": (None, [_i8p, _i8p, _sz, _sz, _sz, _i32p]),
        "ro_masked_softmax_row": (C.c_int, [_f32p, _u8p, _sz, _f32p]),
        "ro_attend_head_f32": (C.c_int, [_f32p, _f32p, _f32p, _sz, _sz, _sz, _i64, _i64, _f32p]),
        "ro_rounding_shift": (C.c_int32, [C.c_int32, C.c_uint]),
        "ro_saturate_int8": (C.c_int8, [C.c_int32]),
        "ro_exp_table": (None, [C.c_float, _u16p]),
        "ro_masked_softmax_int8_row": (C.c_int, [_i32p, _u8p, _sz, C.c_uint, _u16p, _u8p]),
        "ro_attend_head_int8": (C.c_int, [_i8p, _i8p, _i8p, _sz, _sz, _sz, _i64, _i64, C.c_uint,
                                          _u16p, C.c_uint, _i8p]),
        "ro_attention_int8": (C.c_int, [C.POINTER(AttnDesc), _i8p, _i8p, _i8p, _f32p, _f32p, _f32p,
                                        _f32p, C.c_void_p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# --- quantization (quant.hpp) ---------------------------------------------------------

def int8_scale(max_magnitude: float) -> np.float32:
    return np.float32(lib().ro_int8_scale(float(np.float32(max_magnitude))))


def quantize_int8(value: float, scale: float):
    """Returns the int8 code, or raises ValueError where the engine throws."""
    out = C.c_int8(0)
    rc = lib().ro_quantize_int8(float(np.float32(value)), float(np.float32(scale)), C.byref(out))
    if rc != OK:
        raise ValueError("quantize_int8 requires finite values")
    return int(out.value)


def quantize_rows(x):
    """Per-row (per-token) quantization of a [rows, width] float32 matrix."""
    x = _c(x, np.float32)
    rows, width = x.shape
    q = np.empty((rows, width), np.int8)
    s = np.empty(rows, np.float32)
    rc = lib().ro_quantize_rows(x, rows, width, q, s)
    if rc != OK:
        raise ValueError("quantize_rows requires finite values")
    return q, s


def quantize_per_tensor(x):
    x = _c(x, np.float32)
    q = np.empty(x.shape, np.int8)
    s = np.empty(1, np.float32)
    if lib().ro_quantize_per_tensor(x.reshape(-1), x.size, q.reshape(-1), s) != OK:
        raise ValueError("quantize requires finite values")
    return q, s


def quantize_per_head(x):
    """x is [B, H, S, D]; returns int8 [B, H, S, D] and scales [H]."""
    x = _c(x, np.float32)
    B, H, S, D = x.shape
    q = np.empty(x.shape, np.int8)
    s = np.empty(H, np.float32)
    if lib().ro_quantize_per_head(x.reshape(-1), B, H, S, D, q.reshape(-1), s) != OK:
        raise ValueError("quantize requires finite values")
    return q, s


def quantize_per_token(x):
    """x is [..., D]; one scale per row of D values (quantize_rows on the rows)."""
    x = _c(x, np.float32)
    q, s = quantize_rows(x.reshape(-1, x.shape[-1]))
    return q.reshape(x.shape), s.reshape(x.shape[:-1])


def dequantize(q, scales, group: int):
    """float(q[i]) * scales[i // group] for a flat int8 array (the engine's
    static_cast<float>(code) * scale, tests/test_int8.cpp:182)."""
    q = _c(q, np.int8).reshape(-1)
    scales = _c(scales, np.float32).reshape(-1)
    if group <= 0 or len(scales) < (q.size + group - 1) // group:
        raise ValueError("dequantize: group and scales do not cover the values")
    x = np.empty(q.size, np.float32)
    lib().ro_dequantize(q, q.size, group, scales, x)
    return x


# --- math / softmax / heads ---------------------------------------------------------

def exp_nonpositive(x) -> np.ndarray:
    x = np.asarray(x, np.float32).reshape(-1)
    f = lib().ro_exp_nonpositive
    return np.array([f(float(v)) for v in x], np.float32)


def visible(rows: int, keys: int, query_start: int, window: int = 0) -> np.ndarray:
    f = lib().ro_visible
    return np.array([[f(r, k, query_start, window) for k in range(keys)] for r in range(rows)],
                    np.uint8)


def qk_i32(q, k):
    q = _c(q, np.int8)
    k = _c(k, np.int8)
    out = np.empty((q.shape[0], k.shape[0]), np.int32)
    lib().ro_qk_i32(q, k, q.shape[0], k.shape[0], q.shape[1], out)
    return out


def masked_softmax(scores, vis):
    scores = _c(scores, np.float32)
    vis = _c(vis, np.uint8)
    out = np.empty_like(scores)
    for r in range(scores.shape[0]):
        row = np.empty(scores.shape[1], np.float32)
        if lib().ro_masked_softmax_row(scores[r].copy(), vis[r].copy(), scores.shape[1], row) != OK:
            raise ValueError("masked_softmax row has no visible position")
        out[r] = row
    return out


def attend_head_f32(q, k, v, query_start: int, window: int = 0):
    q, k, v = (_c(a, np.float32) for a in (q, k, v))
    out = np.empty_like(q)
    rc = lib().ro_attend_head_f32(q, k, v, q.shape[0], k.shape[0], q.shape[1], query_start,
                                  window, out)
    if rc != OK:
        raise ValueError("attend_head: a query row has no visible key")
    return out


def exp_table(step: float = 1.0 / 16.0) -> np.ndarray:
    t = np.empty(256, np.uint16)
    lib().ro_exp_table(step, t)
    return t


def attend_head_int8(q, k, v, query_start, window, score_shift, out_shift, table=None):
    q, k, v = (_c(a, np.int8) for a in (q, k, v))
    table = exp_table() if table is None else _c(table, np.uint16)
    out = np.empty_like(q)
    rc = lib().ro_attend_head_int8(q, k, v, q.shape[0], k.shape[0], q.shape[1], query_start,
                                   window, score_shift, table, out_shift, out)
    if rc != OK:
        raise ValueError("attend_head_int8: a query row has no visible key")
    return out


# --- the batched int8 attention golden ------------------------------------------------

@dataclass
class Problem:
    """Shapes and parameters of one batched int8 attention call."""
    batch: int
    q_heads: int
    kv_heads: int
    q_len: int
    kv_len: int
    head_dim: int
    query_start: int | None = None  # default kv_len - q_len (attention.hpp:415)
    window: int = 0
    softmax_scale: float = 1.0
    q_granularity: int = GRAN_HEAD
    kv_granularity: int = GRAN_HEAD

    def start(self) -> int:
        return self.kv_len - self.q_len if self.query_start is None else self.query_start


def attention_int8(p: Problem, q, k, v, q_scales, k_scales, v_scales, want_acc=False,
                   threads: int = 0):
    """Golden of the int8 kernels: int32 scores, float softmax, float P.V.

    q [B, Hq, Sq, D], k/v [B, Hkv, Skv, D] int8 (token-major). Returns out
    [B, Hq, Sq, D] float32, and the int32 scores [B, Hq, Sq, Skv] if asked.
    """
    d = AttnDesc(p.batch, p.q_heads, p.kv_heads, p.q_len, p.kv_len, p.head_dim, p.start(),
                 p.window, np.float32(p.softmax_scale), p.q_granularity, p.kv_granularity,
                 threads or os.cpu_count() or 1)
    q, k, v = (_c(a, np.int8).reshape(-1) for a in (q, k, v))
    qs, ks, vs = (_c(a, np.float32).reshape(-1) for a in (q_scales, k_scales, v_scales))
    out = np.empty((p.batch, p.q_heads, p.q_len, p.head_dim), np.float32)
    acc = np.empty((p.batch, p.q_heads, p.q_len, p.kv_len), np.int32) if want_acc else None
    rc = lib().ro_attention_int8(C.byref(d), q, k, v, qs, ks, vs, out.reshape(-1),
                                 acc.ctypes.data_as(C.c_void_p) if want_acc else None)
    if rc != OK:
        raise ValueError("attention_int8: invalid problem or a row with no visible key")
    return (out, acc) if want_acc else out


# --- the engine itself (oracle/_ref) -------------------------------------------------

_ref = None


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref() -> C.CDLL:
    """The Reef engine's own functions, compiled from its headers (tests only)."""
    global _ref
    if _ref is None:
        lib_ = C.CDLL(REF_PATH)
        sig = {
            "ref_int8_scale": (C.c_float, [C.c_float]),
            "ref_quantize_int8": (C.c_int, [C.c_float, C.c_float, C.POINTER(C.c_int8)]),
            "ref_quantize_rows": (C.c_int, [_f32p, _sz, _sz, _i8p, _f32p]),
            "ref_exp_nonpositive": (C.c_float, [C.c_float]),
            "ref_causal_visibility": (C.c_int, [_sz, _sz, _sz, _i64, _u8p]),
            "ref_qk_i32": (C.c_int, [_i8p, _i8p, _sz, _sz, _sz, _i32p]),
            "ref_masked_softmax": (C.c_int, [_f32p, _sz, _sz, _u8p, _f32p]),
            "ref_attend_head": (C.c_int, [_f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _i64, _f32p]),
            "ref_exp_table": (None, [_u16p]),
            "ref_attend_head_int8": (C.c_int, [_i8p, _i8p, _i8p, _sz, _sz, _sz, _sz, _i64,
                                               C.c_uint, C.c_uint, _i8p]),
            "ref_attention_int8_head": (C.c_int, [_i8p, _i8p, _i8p, _f32p, _f32p, _f32p, _sz, _sz,
                                                  _sz, _sz, _i64, C.c_float, _f32p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib_, name)
            fn.restype = res
            fn.argtypes = args
        _ref = lib_
    return _ref


def ref_attention_int8_head(q, k, v, q_scales, k_scales, v_scales, query_start, window,
                            softmax_scale):
    """One head through the engine's own functions; scales are per row / per key."""
    q, k, v = (_c(a, np.int8) for a in (q, k, v))
    qs, ks, vs = (_c(a, np.float32) for a in (q_scales, k_scales, v_scales))
    out = np.empty((q.shape[0], q.shape[1]), np.float32)
    rc = ref().ref_attention_int8_head(q, k, v, qs, ks, vs, q.shape[0], k.shape[0], q.shape[1],
                                       query_start, window, np.float32(softmax_scale), out)
    if rc != OK:
        raise ValueError("engine attention raised")
    return out
