"""reef_amd: int8 attention for AMD MI355X behind the reef_hip C ABI.

Host-side mirror of the Reef engine's quantization and attention operators
(inference-engine/reference/cpp/include/inference_engine/quant.hpp and
operator/attention.hpp), running on the HIP kernels of libreef_hip.so through
its C ABI (include/reef_hip/attention.h). Tensors are torch tensors on the GPU;
torch only provides device memory and the current stream. There is no CPU
fallback: without the built library every call raises.

Errors follow the engine: shape and argument errors raise InvalidArgument (a
ValueError, as the engine's std::invalid_argument), non-finite input raises
NonFiniteInput (also a ValueError, quant.hpp:72-74), cache capacity raises
CapacityError (an IndexError, the engine's std::length_error).
"""
from __future__ import annotations

import ctypes as C
import math
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libreef_hip.so")

OK, INVALID_ARGUMENT, NON_FINITE_INPUT, CAPACITY, HIP_ERROR, UNSUPPORTED, OVERFLOW = range(7)
PER_TENSOR, PER_HEAD, PER_TOKEN = 0, 1, 2
ATTN_PRECISE_PV = 0x1
# prefill schedules (reef_attention_params.flags bits 4-6)
SCHED_AUTO, SCHED_ONE_ITEM, SCHED_SPLIT, SCHED_BALANCED, SCHED_PACKED = (0x00, 0x10, 0x20,
                                                                         0x30, 0x40)
PAGE = 16

EXPORTS = [
    "reef_quantize_int8_per_tensor", "reef_quantize_int8_per_head",
    "reef_quantize_int8_per_token", "reef_dequantize_int8", "reef_read_status_word",
    "reef_attention_prefill_workspace_bytes", "reef_attention_prefill_int8", "reef_qk_scores_i32",
    "reef_qk_scores_i32_packed_workspace_bytes", "reef_qk_scores_i32_packed",
    "reef_attention_decode_workspace_bytes", "reef_attention_decode_int8",
    "reef_attention_decode_int8_paged", "reef_attention_decode_int8_paged_noalloc",
    "reef_kv_pack_v_pages", "reef_kv_append_int8",
    "reef_kv_append_int8_paged", "reef_attention_int8_integer", "reef_linear_w8a8_workspace_bytes",
    "reef_linear_w8a8", "reef_gemm_w8a8", "reef_attention_prefill_cache_workspace_bytes",
    "reef_attention_prefill_int8_cache",
]


class ReefError(RuntimeError):
    pass


class InvalidArgument(ReefError, ValueError):
    pass


class NonFiniteInput(ReefError, ValueError):
    pass


class CapacityError(ReefError, IndexError):
    pass


class HipError(ReefError):
    pass


class Unsupported(ReefError, NotImplementedError):
    pass


class Overflow(ReefError, OverflowError):
    pass


_ERRORS = {INVALID_ARGUMENT: InvalidArgument, NON_FINITE_INPUT: NonFiniteInput,
           CAPACITY: CapacityError, HIP_ERROR: HipError, UNSUPPORTED: Unsupported,
           OVERFLOW: Overflow}


class Strides(C.Structure):
    _fields_ = [("batch", C.c_int64), ("head", C.c_int64), ("token", C.c_int64)]


class AttentionParams(C.Structure):
    _fields_ = [("batch", C.c_int64), ("q_heads", C.c_int64), ("kv_heads", C.c_int64),
                ("q_len", C.c_int64), ("kv_len", C.c_int64), ("head_dim", C.c_int64),
                ("query_start", C.c_int64), ("window", C.c_int64),
                ("softmax_scale", C.c_float), ("q_granularity", C.c_int32),
                ("kv_granularity", C.c_int32), ("flags", C.c_uint32)]


class DecodeParams(C.Structure):
    _fields_ = [("batch", C.c_int64), ("q_heads", C.c_int64), ("kv_heads", C.c_int64),
                ("head_dim", C.c_int64), ("max_context", C.c_int64), ("window", C.c_int64),
                ("softmax_scale", C.c_float), ("q_granularity", C.c_int32),
                ("num_splits", C.c_int32), ("flags", C.c_uint32)]


class KvAppendParams(C.Structure):
    _fields_ = [("batch", C.c_int64), ("kv_heads", C.c_int64), ("head_dim", C.c_int64),
                ("new_tokens", C.c_int64), ("max_context", C.c_int64)]


_P = C.c_void_p
_I64 = C.c_int64
_SIGS = {
    "reef_quantize_int8_per_tensor": [_P, _I64, _P, _P, _P, _P],
    "reef_quantize_int8_per_head": [_P, _I64, _I64, _I64, _I64, C.POINTER(Strides), _P, _P, _P,
                                    _P],
    "reef_quantize_int8_per_token": [_P, _I64, _I64, _I64, _P, _P, _P, _P],
    "reef_dequantize_int8": [_P, _I64, _I64, _P, _P, _P],
    "reef_read_status_word": [_P, C.c_int, _P],
    "reef_attention_prefill_workspace_bytes": [C.POINTER(AttentionParams)],
    "reef_attention_prefill_int8": [C.POINTER(AttentionParams), _P, C.POINTER(Strides), _P,
                                    C.POINTER(Strides), _P, C.POINTER(Strides), _P, _P, _P, _P,
                                    C.POINTER(Strides), _P, C.c_size_t, _P],
    "reef_qk_scores_i32": [_P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P],
    "reef_qk_scores_i32_packed_workspace_bytes": [_I64, _I64, _I64, _I64, _I64],
    "reef_qk_scores_i32_packed": [_P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, C.c_size_t, _P],
    "reef_attention_decode_workspace_bytes": [C.POINTER(DecodeParams)],
    "reef_attention_decode_int8": [C.POINTER(DecodeParams), _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                   C.c_size_t, _P, _P],
    "reef_attention_decode_int8_paged": [C.POINTER(DecodeParams), _P, _P, _P, _P, _P, _P, _P,
                                         _I64, _I64, _P, _P, _P, C.c_size_t, _P, _P],
    "reef_attention_decode_int8_paged_noalloc": [C.POINTER(DecodeParams), _P, _P, _P, _P, _P, _P,
                                                 _P, _I64, _I64, _P, _P, _P, _P],
    "reef_kv_pack_v_pages": [_P, _I64, _I64, _P, _P],
    "reef_linear_w8a8_workspace_bytes": [_I64, _I64],
    "reef_linear_w8a8": [_P, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _I64, _P, C.c_size_t, _P,
                         _P],
    "reef_gemm_w8a8": [_P, _P, _I64, _I64, _P, _P, _P, _I64, _P, _I64, _P, _P],
    "reef_attention_int8_integer": [C.POINTER(AttentionParams), _P, C.POINTER(Strides), _P,
                                    C.POINTER(Strides), _P, C.POINTER(Strides), C.c_uint32, _P,
                                    C.c_uint32, _P, C.POINTER(Strides), _P],
    "reef_kv_append_int8": [C.POINTER(KvAppendParams), _P, C.POINTER(Strides), _P,
                            C.POINTER(Strides), _P, _P, _P, _P, _P, _P, _P, _P],
    "reef_kv_append_int8_paged": [C.POINTER(KvAppendParams), _P, C.POINTER(Strides), _P,
                                  C.POINTER(Strides), _P, _P, _I64, _I64, _P, _P, _P, _P, _P,
                                  _P, _P],
    "reef_attention_prefill_cache_workspace_bytes": [C.POINTER(AttentionParams)],
    "reef_attention_prefill_int8_cache": [C.POINTER(AttentionParams), _P, C.POINTER(Strides), _P,
                                          _P, _P, _P, _P, _I64, _P, _I64, _I64, _P,
                                          C.POINTER(Strides), _P, C.c_size_t, _P, _P],
}

_lib_handle = None


def lib() -> C.CDLL:
    """The loaded libreef_hip.so. Raises if it has not been built."""
    global _lib_handle
    if _lib_handle is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with python -m reef_amd._build")
        handle = C.CDLL(LIB_PATH)
        for name, args in _SIGS.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = C.c_size_t if name.endswith("_bytes") else C.c_int
        _lib_handle = handle
    return _lib_handle


def check(status: int, what: str) -> None:
    if status != OK:
        raise _ERRORS.get(status, ReefError)(f"{what}: reef status {status}")


# --- torch plumbing -------------------------------------------------------------------

def _torch():
    import torch
    return torch


def _stream():
    return C.c_void_p(_torch().cuda.current_stream().cuda_stream)


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _require(t, dtype, name):
    torch = _torch()
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise InvalidArgument(f"{name} must be a GPU tensor")
    if t.dtype != dtype:
        raise InvalidArgument(f"{name} must be {dtype}, got {t.dtype}")


def _strides4(t):
    """Strides of a [B, H, S, D] tensor with a contiguous last dimension."""
    if t.dim() != 4 or t.stride(3) != 1:
        raise InvalidArgument("expected [batch, heads, tokens, head_dim] with contiguous head_dim")
    return Strides(t.stride(0), t.stride(1), t.stride(2))


class StatusWord:
    """A device status word the kernels flag non-finite input and bad pages in."""

    def __init__(self, device=None):
        torch = _torch()
        self.tensor = torch.zeros(1, dtype=torch.int32, device=device or "cuda")

    @property
    def ptr(self):
        return _ptr(self.tensor)

    def check(self, what: str) -> None:
        check(lib().reef_read_status_word(self.ptr, 1, _stream()), what)


# --- quantization (quant.hpp) ---------------------------------------------------------

def quantize_per_tensor(x, status: StatusWord | None = None):
    """One scale for the whole tensor (the quant.hpp rule); returns (int8, scale[1])."""
    torch = _torch()
    _require(x, torch.float32, "x")
    x = x.contiguous()
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    s = torch.empty(1, dtype=torch.float32, device=x.device)
    own = status or StatusWord(x.device)
    check(lib().reef_quantize_int8_per_tensor(_ptr(x), x.numel(), _ptr(q), _ptr(s), own.ptr,
                                              _stream()), "quantize_per_tensor")
    if status is None:
        own.check("quantize_per_tensor requires finite values")
    return q, s


def quantize_per_head(x, status: StatusWord | None = None):
    """x [B, H, S, D] (any strides, contiguous D); one scale per head over batch and
    tokens. Returns packed int8 [B, H, S, D] and scales [H]."""
    torch = _torch()
    _require(x, torch.float32, "x")
    st = _strides4(x)
    B, H, S, D = x.shape
    q = torch.empty((B, H, S, D), dtype=torch.int8, device=x.device)
    s = torch.empty(H, dtype=torch.float32, device=x.device)
    own = status or StatusWord(x.device)
    check(lib().reef_quantize_int8_per_head(_ptr(x), B, H, S, D, C.byref(st), _ptr(q), _ptr(s),
                                            own.ptr, _stream()), "quantize_per_head")
    if status is None:
        own.check("quantize_per_head requires finite values")
    return q, s


def quantize_rows(x, status: StatusWord | None = None):
    """quantize_rows (quant.hpp:112-133) over the last dimension: one scale per row
    (per token). Returns int8 of x's shape and scales of x.shape[:-1]."""
    torch = _torch()
    _require(x, torch.float32, "x")
    width = x.shape[-1]
    x2 = x.reshape(-1, width)
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    rows = x2.shape[0]
    q = torch.empty((rows, width), dtype=torch.int8, device=x.device)
    s = torch.empty(rows, dtype=torch.float32, device=x.device)
    own = status or StatusWord(x.device)
    check(lib().reef_quantize_int8_per_token(_ptr(x2), rows, width, x2.stride(0), _ptr(q),
                                             _ptr(s), own.ptr, _stream()), "quantize_rows")
    if status is None:
        own.check("quantize_rows requires finite values")
    return q.reshape(x.shape), s.reshape(x.shape[:-1])


quantize_per_token = quantize_rows


def dequantize(q, scales, group: int):
    """x[i] = float(q[i]) * scales[i // group]."""
    torch = _torch()
    _require(q, torch.int8, "q")
    _require(scales, torch.float32, "scales")
    q = q.contiguous()
    x = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    check(lib().reef_dequantize_int8(_ptr(q), q.numel(), group, _ptr(scales.contiguous()),
                                     _ptr(x), _stream()), "dequantize")
    return x


# --- attention ------------------------------------------------------------------------

_PREFILL_WS = {}


def prefill_workspace(params: AttentionParams, device):
    """The zero-filled workspace of the balanced prefill schedule, one per (device,
    stream): every launch leaves it zero-filled, so the next launch on that stream
    reuses it."""
    torch = _torch()
    n = lib().reef_attention_prefill_workspace_bytes(C.byref(params))
    key = (torch.device(device).index, _stream().value)
    ws = _PREFILL_WS.get(key)
    if ws is None or ws.numel() < n:
        ws = torch.zeros(max(n, 256), dtype=torch.uint8, device=device)
        _PREFILL_WS[key] = ws
    return ws


def attention_prefill(q, k, v, q_scales, k_scales, v_scales, *, query_start=None, window=0,
                      softmax_scale=None, q_granularity=PER_HEAD, kv_granularity=PER_HEAD,
                      precise=False, schedule=SCHED_AUTO, out=None, workspace=None):
    """Attention::context (attention.hpp:374-432) over int8 heads in one launch.

    q [B, Hq, Sq, D], k and v [B, Hkv, Skv, D] int8 (contiguous head_dim, any other
    strides); scales by granularity. softmax_scale defaults to 1/sqrt(D); pass 1.0
    for the engine's unscaled scores. Returns fp32 [B, Hq, Sq, D]. schedule is one
    of the SCHED_* flags (SCHED_AUTO: the library's choice). workspace: None takes
    this stream's cached one (prefill_workspace), False passes none, or a
    zero-filled uint8 tensor of reef_attention_prefill_workspace_bytes bytes.
    """
    torch = _torch()
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _require(t, torch.int8, n)
    for t, n in ((q_scales, "q_scales"), (k_scales, "k_scales"), (v_scales, "v_scales")):
        _require(t, torch.float32, n)
    B, Hq, Sq, D = q.shape
    _, Hkv, Skv, _ = k.shape
    if tuple(v.shape) != tuple(k.shape) or k.shape[0] != B or k.shape[3] != D:
        raise InvalidArgument("attention_prefill shape mismatch")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    start = Skv - Sq if query_start is None else query_start
    p = AttentionParams(B, Hq, Hkv, Sq, Skv, D, start, window, softmax_scale, q_granularity,
                        kv_granularity, (ATTN_PRECISE_PV if precise else 0) | schedule)
    if out is None:
        out = torch.empty((B, Hq, Sq, D), dtype=torch.float32, device=q.device)
    qs, ks, vs, os_ = _strides4(q), _strides4(k), _strides4(v), _strides4(out)
    if workspace is None:
        workspace = prefill_workspace(p, q.device)
    ws_ptr, ws_n = (None, 0) if workspace is False else (_ptr(workspace), workspace.numel()
                                                          * workspace.element_size())
    check(lib().reef_attention_prefill_int8(
        C.byref(p), _ptr(q), C.byref(qs), _ptr(k), C.byref(ks), _ptr(v), C.byref(vs),
        _ptr(q_scales.contiguous()), _ptr(k_scales.contiguous()), _ptr(v_scales.contiguous()),
        _ptr(out), C.byref(os_), ws_ptr, ws_n, _stream()), "attention_prefill")
    return out


def attention_prefill_cache(q, q_scales, k_cache, v_cache, k_scales, v_scales, kv_len, *,
                            block_table=None, query_start=None, window=0, softmax_scale=None,
                            q_granularity=PER_HEAD, status: StatusWord | None = None, out=None):
    """A prompt chunk over the int8 cache (Attention::forward with query_len > 1 on a
    non-empty cache, attention.hpp:354-372): the cache already holds the chunk's
    keys (kv_append), kv_len tokens per sequence. Contiguous cache (block_table
    None): k_cache [B, Hkv, L, D], v_cache [B, Hkv, L/16, D, 16] (or the same bytes
    in any shape), scales [B, Hkv, L]. Paged: k_cache [P, Hkv, 16, D], v_cache
    [P, Hkv, D, 16], scales [P, Hkv, 16], block_table [B, max_blocks] int32.
    q [B, Hq, q_len, D] int8; returns fp32 [B, Hq, q_len, D]."""
    torch = _torch()
    _require(q, torch.int8, "q")
    B, Hq, Sq, D = q.shape
    Hkv = k_cache.shape[1]
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    start = kv_len - Sq if query_start is None else query_start
    p = AttentionParams(B, Hq, Hkv, Sq, kv_len, D, start, window, softmax_scale, q_granularity,
                        PER_TOKEN, 0)
    if block_table is None:
        max_context, table, max_blocks, pages = k_cache.shape[2], None, 0, 0
    else:
        max_context, table = 0, block_table.contiguous()
        max_blocks, pages = table.shape[1], k_cache.shape[0]
    n = lib().reef_attention_prefill_cache_workspace_bytes(C.byref(p))
    key = ("cache", torch.device(q.device).index, _stream().value)
    ws = _PREFILL_WS.get(key)
    if ws is None or ws.numel() < n:  # zero-filled once; every call leaves it so
        ws = torch.zeros(max(n, 256), dtype=torch.uint8, device=q.device)
        _PREFILL_WS[key] = ws
    if out is None:
        out = torch.empty((B, Hq, Sq, D), dtype=torch.float32, device=q.device)
    qs, os_ = _strides4(q), _strides4(out)
    own = status or StatusWord(q.device)
    check(lib().reef_attention_prefill_int8_cache(
        C.byref(p), _ptr(q), C.byref(qs), _ptr(q_scales.contiguous()), _ptr(k_cache.contiguous()),
        _ptr(v_cache.contiguous()), _ptr(k_scales.contiguous()), _ptr(v_scales.contiguous()),
        max_context, _ptr(table), max_blocks, pages, _ptr(out), C.byref(os_), _ptr(ws), n,
        own.ptr, _stream()), "attention_prefill_cache")
    if status is None:
        own.check("attention_prefill_cache")
    return out


def qk_scores_i32(q, k):
    """int32 q . k^T for packed q [B, Hq, Sq, D] and k [B, Hkv, Skv, D]."""
    torch = _torch()
    _require(q, torch.int8, "q")
    _require(k, torch.int8, "k")
    q = q.contiguous()
    k = k.contiguous()
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    acc = torch.empty((B, Hq, Sq, Skv), dtype=torch.int32, device=q.device)
    check(lib().reef_qk_scores_i32(_ptr(q), _ptr(k), B, Hq, Hkv, Sq, Skv, D, _ptr(acc),
                                   _stream()), "qk_scores_i32")
    return acc


def qk_scores_i32_packed(q, k):
    """int32 q . k^T for packed q [B, Hq, Sq, 128] and k [B, Hkv, Skv, 128], read from
    the packed prefill kernel's own score accumulators."""
    torch = _torch()
    _require(q, torch.int8, "q")
    _require(k, torch.int8, "k")
    q = q.contiguous()
    k = k.contiguous()
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    if D != 128:
        raise ValueError("the packed score hook takes head_dim 128")
    acc = torch.full((B, Hq, Sq, Skv), -1, dtype=torch.int32, device=q.device)
    nbytes = lib().reef_qk_scores_i32_packed_workspace_bytes(B, Hq, Hkv, Sq, Skv)
    if nbytes == 0:
        raise ValueError("qk_scores_i32_packed: invalid sizes")
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=q.device)
    check(lib().reef_qk_scores_i32_packed(_ptr(q), _ptr(k), B, Hq, Hkv, Sq, Skv, _ptr(acc),
                                          _ptr(ws), nbytes, _stream()), "qk_scores_i32_packed")
    return acc


def _decode_params(q, max_context, kv_heads, window, softmax_scale, q_granularity, num_splits):
    B, Hq, D = q.shape
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    return DecodeParams(B, Hq, kv_heads, D, max_context, window, softmax_scale, q_granularity,
                        num_splits, 0)


def decode_workspace(params: DecodeParams, device):
    """A zero-filled decode workspace (its item counters must start at zero; every
    launch leaves them so, so the workspace is reusable without refilling)."""
    torch = _torch()
    n = lib().reef_attention_decode_workspace_bytes(C.byref(params))
    return torch.zeros(max(n, 16) // 4 + 4, dtype=torch.float32, device=device)


def attention_decode(q, q_scales, k_cache, v_pages, k_scales, v_scales, context_lens=None, *,
                     window=0, softmax_scale=None, q_granularity=PER_TOKEN, num_splits=0,
                     workspace=None, status: StatusWord | None = None, out=None):
    """One decode step over a contiguous int8 cache.

    q [B, Hq, D] int8; k_cache [B, Hkv, L, D]; v_pages [B, Hkv, L/16, D, 16] (see
    pack_v_pages); k_scales, v_scales [B, Hkv, L]; context_lens [B] int32 or None.
    """
    torch = _torch()
    _require(q, torch.int8, "q")
    B, Hq, D = q.shape
    Hkv, L = k_cache.shape[1], k_cache.shape[2]
    if tuple(k_cache.shape) != (B, Hkv, L, D) or v_pages.numel() != k_cache.numel():
        raise InvalidArgument("attention_decode cache shape mismatch")
    p = _decode_params(q, L, Hkv, window, softmax_scale, q_granularity, num_splits)
    ws = workspace if workspace is not None else decode_workspace(p, q.device)
    if out is None:
        out = torch.empty((B, Hq, D), dtype=torch.float32, device=q.device)
    own = status or StatusWord(q.device)
    cl = context_lens.contiguous() if context_lens is not None else None
    check(lib().reef_attention_decode_int8(
        C.byref(p), _ptr(q.contiguous()), _ptr(q_scales.contiguous()), _ptr(k_cache.contiguous()),
        _ptr(v_pages.contiguous()), _ptr(k_scales.contiguous()), _ptr(v_scales.contiguous()),
        _ptr(cl), _ptr(out), _ptr(ws), ws.numel() * 4, own.ptr, _stream()), "attention_decode")
    if status is None:
        own.check("attention_decode")
    return out


def attention_decode_paged(q, q_scales, k_pages, v_pages, k_scale_pages, v_scale_pages,
                           block_table, context_lens, *, window=0, softmax_scale=None,
                           q_granularity=PER_TOKEN, num_splits=0, workspace=None,
                           status: StatusWord | None = None, out=None):
    """One decode step over a paged int8 cache: k_pages [P, Hkv, 16, D], v_pages
    [P, Hkv, D, 16], scale pages [P, Hkv, 16], block_table [B, max_blocks] int32,
    context_lens [B] int32."""
    torch = _torch()
    _require(q, torch.int8, "q")
    B, Hq, D = q.shape
    P, Hkv = k_pages.shape[0], k_pages.shape[1]
    max_blocks = block_table.shape[1]
    p = _decode_params(q, max_blocks * PAGE, Hkv, window, softmax_scale, q_granularity,
                       num_splits)
    ws = workspace if workspace is not None else decode_workspace(p, q.device)
    if out is None:
        out = torch.empty((B, Hq, D), dtype=torch.float32, device=q.device)
    own = status or StatusWord(q.device)
    check(lib().reef_attention_decode_int8_paged(
        C.byref(p), _ptr(q.contiguous()), _ptr(q_scales.contiguous()), _ptr(k_pages),
        _ptr(v_pages), _ptr(k_scale_pages), _ptr(v_scale_pages), _ptr(block_table.contiguous()),
        max_blocks, P, _ptr(context_lens.contiguous()), _ptr(out), _ptr(ws), ws.numel() * 4,
        own.ptr, _stream()), "attention_decode_paged")
    if status is None:
        own.check("attention_decode_paged")
    return out


def pack_v_pages(v_tokens):
    """Token-major values [..., pages * 16, D] -> transposed pages [..., pages, D, 16]."""
    torch = _torch()
    _require(v_tokens, torch.int8, "v_tokens")
    *lead, L, D = v_tokens.shape
    if L % PAGE:
        raise InvalidArgument("token count must be a multiple of 16")
    src = v_tokens.contiguous()
    pages = src.numel() // (PAGE * D)
    out = torch.empty((*lead, L // PAGE, D, PAGE), dtype=torch.int8, device=src.device)
    check(lib().reef_kv_pack_v_pages(_ptr(src), pages, D, _ptr(out), _stream()), "pack_v_pages")
    return out


# --- KV-cache append (attention.hpp:290-352) --------------------------------------------

def _append_inputs(k_new, v_new):
    torch = _torch()
    _require(k_new, torch.float32, "k_new")
    _require(v_new, torch.float32, "v_new")
    if k_new.shape != v_new.shape or k_new.dim() != 4:
        raise InvalidArgument("KV cache append shape mismatch")
    return _strides4(k_new), _strides4(v_new)


def kv_append(k_new, v_new, start_positions, k_cache, v_pages, k_scales, v_scales,
              context_lens=None, status: StatusWord | None = None):
    """Quantize fp32 rows k_new, v_new [B, Hkv, T, D] per token and write them into
    the contiguous cache (k_cache [B, Hkv, L, D], v_pages [B, Hkv, L/16, D, 16],
    scales [B, Hkv, L]) at start_positions[b] + t. context_lens, when given, is set
    to start_positions + T afterwards (it may be start_positions itself)."""
    torch = _torch()
    ks, vs = _append_inputs(k_new, v_new)
    B, H, T, D = k_new.shape
    L = k_cache.shape[2]
    if tuple(k_cache.shape) != (B, H, L, D) or v_pages.numel() != k_cache.numel():
        raise InvalidArgument("KV cache append shape mismatch")
    _require(start_positions, torch.int32, "start_positions")
    p = KvAppendParams(B, H, D, T, L)
    own = status or StatusWord(k_new.device)
    check(lib().reef_kv_append_int8(
        C.byref(p), _ptr(k_new), C.byref(ks), _ptr(v_new), C.byref(vs), _ptr(start_positions),
        _ptr(k_cache), _ptr(v_pages), _ptr(k_scales), _ptr(v_scales), _ptr(context_lens),
        own.ptr, _stream()), "kv_append")
    if status is None:
        own.check("kv_append")


def kv_append_paged(k_new, v_new, start_positions, block_table, k_pages, v_pages,
                    k_scale_pages, v_scale_pages, context_lens=None,
                    status: StatusWord | None = None, max_context=None):
    """kv_append into the paged cache (k_pages [P, Hkv, 16, D], v_pages [P, Hkv, D, 16],
    scale pages [P, Hkv, 16], block_table [B, max_blocks] int32)."""
    torch = _torch()
    ks, vs = _append_inputs(k_new, v_new)
    B, H, T, D = k_new.shape
    P = k_pages.shape[0]
    max_blocks = block_table.shape[1]
    _require(start_positions, torch.int32, "start_positions")
    _require(block_table, torch.int32, "block_table")
    p = KvAppendParams(B, H, D, T, max_context or max_blocks * PAGE)
    own = status or StatusWord(k_new.device)
    check(lib().reef_kv_append_int8_paged(
        C.byref(p), _ptr(k_new), C.byref(ks), _ptr(v_new), C.byref(vs), _ptr(start_positions),
        _ptr(block_table.contiguous()), max_blocks, P, _ptr(k_pages), _ptr(v_pages),
        _ptr(k_scale_pages), _ptr(v_scale_pages), _ptr(context_lens), own.ptr, _stream()),
        "kv_append_paged")
    if status is None:
        own.check("kv_append_paged")


# --- integer-only attention (int8.hpp:156-279) -----------------------------------------

def attention_int8_integer(q, k, v, table, *, score_shift, out_shift=8, query_start=None,
                           window=0):
    """attend_head_int8 for every (batch, head): q [B, Hq, Sq, D], k and v
    [B, Hkv, Skv, D] int8, table [256] uint16 (as int16/uint16 torch tensor) on the
    device; returns int8 [B, Hq, Sq, D], bit-identical to the engine."""
    torch = _torch()
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _require(t, torch.int8, n)
    if table.numel() != 256 or table.element_size() != 2 or not table.is_cuda:
        raise InvalidArgument("table must hold 256 16-bit entries on the GPU")
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    start = Skv - Sq if query_start is None else query_start
    p = AttentionParams(B, Hq, Hkv, Sq, Skv, D, start, window, 1.0, PER_HEAD, PER_HEAD, 0)
    out = torch.empty((B, Hq, Sq, D), dtype=torch.int8, device=q.device)
    sq, sk, sv, so = _strides4(q), _strides4(k), _strides4(v), _strides4(out)
    check(lib().reef_attention_int8_integer(
        C.byref(p), _ptr(q), C.byref(sq), _ptr(k), C.byref(sk), _ptr(v), C.byref(sv),
        score_shift, _ptr(table.contiguous()), out_shift, _ptr(out), C.byref(so), _stream()),
        "attention_int8_integer")
    return out


# --- W8A8 projection (operator/linear.hpp:106-132) ---------------------------------------

def linear_w8a8(x, weight, w_scales, bias=None, status: StatusWord | None = None):
    """y = linear(x, QuantizedWeight{weight, w_scales}, bias): x [rows, in] fp32,
    weight [out, in] int8, w_scales [out] fp32, bias [out] fp32 or None. Rows are
    quantized per row on the device; outputs are bit-identical to the engine's."""
    torch = _torch()
    _require(x, torch.float32, "x")
    _require(weight, torch.int8, "weight")
    _require(w_scales, torch.float32, "w_scales")
    if x.dim() != 2 or x.stride(1) != 1 or weight.dim() != 2 or weight.shape[1] != x.shape[1]:
        raise InvalidArgument("linear_w8a8 shapes: x [rows, in], weight [out, in]")
    rows, fin = x.shape
    fout = weight.shape[0]
    n = lib().reef_linear_w8a8_workspace_bytes(rows, fin)
    ws = torch.empty(n // 4 + 4, dtype=torch.float32, device=x.device)
    y = torch.empty((rows, fout), dtype=torch.float32, device=x.device)
    own = status or StatusWord(x.device)
    check(lib().reef_linear_w8a8(
        _ptr(x), rows, fin, x.stride(0), _ptr(weight.contiguous()), _ptr(w_scales.contiguous()),
        _ptr(bias.contiguous()) if bias is not None else None, fout, _ptr(y), fout, _ptr(ws),
        ws.numel() * 4, own.ptr, _stream()), "linear_w8a8")
    if status is None:
        own.check("linear_w8a8")
    return y
