"""The C ABI without a GPU: the library loads, exports every entry point the
public header declares, and rejects bad arguments on the host before any launch
(the engine's error paths: attention.hpp:293-327, activation.hpp:204-207)."""
import ctypes as C
import os
import re

import pytest

import reef_amd
from reef_amd import AttentionParams, DecodeParams, Strides

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "reef_hip", "attention.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:reef_status|size_t)\s+(reef_[a-z0-9_]+)\s*\(", text,
                                 re.M)))


def test_library_exports_every_declared_entry_point():
    names = declared()
    assert len(names) >= 11
    lib = reef_amd.lib()
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(reef_amd.EXPORTS) == names


def _fake(n=1):
    # Non-null, 256-byte aligned host addresses: validation never dereferences them.
    return C.c_void_p(0x10000 * n)


def _prefill(p, strides=None):
    lib = reef_amd.lib()
    s = C.byref(strides) if strides else None
    return lib.reef_attention_prefill_int8(C.byref(p), _fake(1), s, _fake(2), s, _fake(3), s,
                                           _fake(4), _fake(5), _fake(6), _fake(7), None, None, 0,
                                           None)


def good_params(**kw):
    d = dict(batch=1, q_heads=4, kv_heads=2, q_len=8, kv_len=8, head_dim=128, query_start=0,
             window=0, softmax_scale=0.1, q_granularity=1, kv_granularity=1, flags=0)
    d.update(kw)
    return AttentionParams(**d)


@pytest.mark.parametrize("change,status", [
    (dict(q_heads=3), reef_amd.INVALID_ARGUMENT),          # not a multiple of kv_heads
    (dict(query_start=1), reef_amd.INVALID_ARGUMENT),      # rows past the last key
    (dict(q_len=0), reef_amd.INVALID_ARGUMENT),
    (dict(window=-1), reef_amd.INVALID_ARGUMENT),
    (dict(q_granularity=7), reef_amd.INVALID_ARGUMENT),
    (dict(softmax_scale=float("nan")), reef_amd.INVALID_ARGUMENT),
    (dict(head_dim=96), reef_amd.UNSUPPORTED),
    (dict(kv_len=1 << 31, q_len=8), reef_amd.UNSUPPORTED),
])
def test_prefill_host_validation(change, status):
    assert _prefill(good_params(**change)) == status


def test_prefill_rejects_null_and_misaligned():
    lib = reef_amd.lib()
    p = good_params()
    assert lib.reef_attention_prefill_int8(C.byref(p), None, None, None, None, None, None, None,
                                           None, None, None, None, None, 0, None) == 1
    assert _prefill(p, Strides(0, 128, 129)) == reef_amd.INVALID_ARGUMENT  # row not 16-B aligned


def test_prefill_workspace_bytes_and_alignment():
    lib = reef_amd.lib()
    p = good_params(batch=1, q_heads=32, kv_heads=32, q_len=2048, kv_len=2048)
    n = lib.reef_attention_prefill_workspace_bytes(C.byref(p))
    # a fixed region of 65536 counters (item counters and the packed queue), then two partial slots per workgroup, two
    # workgroups per compute unit (256 without a GPU): 128 x 128 outputs plus (max,
    # sum) of 128 rows; then the packed value image: 32 tiles of 64 keys per head,
    # 16 KB each
    balanced = 65536 * 4 + 2 * 512 * (128 * 128 + 2 * 256) * 4
    image = 32 * 32 * 16384
    assert n == balanced + image
    p64 = good_params(batch=1, q_heads=32, kv_heads=32, q_len=2048, kv_len=2048, head_dim=64)
    # the same balanced region (slots sized for head_dim 128, so that every shape finds
    # its counters at the same offsets); no packed schedule at head_dim 64
    assert lib.reef_attention_prefill_workspace_bytes(C.byref(p64)) == balanced
    assert lib.reef_attention_prefill_workspace_bytes(C.byref(good_params(head_dim=96))) == 0
    assert lib.reef_attention_prefill_workspace_bytes(None) == 0
    # a workspace that is not 256-byte aligned
    assert lib.reef_attention_prefill_int8(C.byref(p), _fake(1), None, _fake(2), None, _fake(3),
                                           None, _fake(4), _fake(5), _fake(6), _fake(7), None,
                                           C.c_void_p(0x10010), n, None) == reef_amd.INVALID_ARGUMENT


def _prefill_cache(p, ws_bytes=1 << 30, max_context=64, table=None, max_blocks=0, pages=0):
    lib = reef_amd.lib()
    return lib.reef_attention_prefill_int8_cache(
        C.byref(p), _fake(1), None, _fake(2), _fake(3), _fake(4), _fake(5), _fake(6), max_context,
        table, max_blocks, pages, _fake(7), None, _fake(8), ws_bytes, None, None)


def test_prefill_cache_host_validation_and_workspace():
    """The prefill over the decode cache: gathered rows and per-token scales in the
    workspace, arguments checked before any launch."""
    lib = reef_amd.lib()
    tok = dict(kv_granularity=2, q_len=8, kv_len=40, query_start=32)
    p = good_params(**tok)
    # the prefill's balanced-schedule workspace (a fixed region of 65536 counters; two
    # part slots per workgroup, 2 x 256 workgroups without a GPU), then 1 x 2 kv heads x 40 tokens of keys and values (80 rows x 128 bytes,
    # rounded to 256) and two scale arrays (80 floats, rounded to 256)
    balanced = 65536 * 4 + 2 * 512 * (128 * 128 + 2 * 256) * 4
    assert lib.reef_attention_prefill_cache_workspace_bytes(C.byref(p)) == \
        balanced + 2 * 10240 + 2 * 512
    assert lib.reef_attention_prefill_cache_workspace_bytes(C.byref(good_params(head_dim=96))) == 0
    assert _prefill_cache(good_params(**dict(tok, kv_granularity=1))) == reef_amd.INVALID_ARGUMENT
    assert _prefill_cache(good_params(**dict(tok, query_start=33))) == reef_amd.INVALID_ARGUMENT
    assert _prefill_cache(p, max_context=32) == reef_amd.INVALID_ARGUMENT  # cache shorter than kv_len
    assert _prefill_cache(p, max_context=72) == reef_amd.INVALID_ARGUMENT  # not a multiple of 16
    assert _prefill_cache(p, ws_bytes=1000) == reef_amd.INVALID_ARGUMENT
    assert _prefill_cache(good_params(**dict(tok, head_dim=96))) == reef_amd.UNSUPPORTED
    # paged: the block table must cover kv_len and the pool must be non-empty
    assert _prefill_cache(p, table=_fake(9), max_blocks=2, pages=10) == reef_amd.INVALID_ARGUMENT
    assert _prefill_cache(p, table=_fake(9), max_blocks=3, pages=0) == reef_amd.INVALID_ARGUMENT


def test_decode_host_validation_and_workspace():
    lib = reef_amd.lib()
    p = DecodeParams(batch=64, q_heads=32, kv_heads=8, head_dim=128, max_context=4096,
                     window=0, softmax_scale=0.1, q_granularity=2, num_splits=0, flags=0)
    ws = lib.reef_attention_decode_workspace_bytes(C.byref(p))
    # a fixed region of 2048 counters (one per (sequence, kv head) of a launch that
    # deals out blocks), then two part slots (64 lanes x 17 eight-byte words) per
    # workgroup of the larger (paged) launch: 2 workgroups per compute unit (256
    # without a GPU), the 512 items' 64-key blocks dealt out among them
    slot = 17 * 64 * 8
    assert ws == 8192 + 512 * 2 * slot
    many = DecodeParams(64, 32, 8, 128, 4096, 0, 0.1, 2, 9, 0)
    # num_splits 9: 512 items x 9 / 4 waves = 1152 workgroups
    assert lib.reef_attention_decode_workspace_bytes(C.byref(many)) == 8192 + 1152 * 2 * slot
    # more items than the in-workgroup plan holds (2048): whole items per workgroup,
    # no part slots (and no counting)
    big = DecodeParams(4096, 8, 1, 128, 4096, 0, 0.1, 2, 0, 0)
    assert lib.reef_attention_decode_workspace_bytes(C.byref(big)) == 8192
    f = [_fake(i) for i in range(1, 12)]
    args = lambda pp, w: (C.byref(pp), f[0], f[1], f[2], f[3], f[4], f[5], None, f[6], f[7],  # noqa: E731
                          w, None, None)
    assert lib.reef_attention_decode_int8(*args(p, ws - 4)) == reef_amd.INVALID_ARGUMENT
    bad = DecodeParams(64, 32, 8, 128, 4100, 0, 0.1, 2, 0, 0)  # not a multiple of 16
    assert lib.reef_attention_decode_int8(*args(bad, 1 << 30)) == reef_amd.INVALID_ARGUMENT
    wide = DecodeParams(1, 32, 1, 128, 64, 0, 0.1, 2, 0, 0)  # 32 heads per kv head
    assert lib.reef_attention_decode_int8(*args(wide, 1 << 30)) == reef_amd.UNSUPPORTED
    # paged: the block table must cover max_context
    assert lib.reef_attention_decode_int8_paged(
        C.byref(p), f[0], f[1], f[2], f[3], f[4], f[5], f[6], 4096 // 16 - 1, 100, f[7], f[8],
        f[9], 1 << 30, None, None) == reef_amd.INVALID_ARGUMENT


def test_quantize_host_validation():
    lib = reef_amd.lib()
    assert lib.reef_quantize_int8_per_tensor(_fake(), 0, _fake(), _fake(), None, None) == 1
    assert lib.reef_quantize_int8_per_token(_fake(), 4, 8, 7, _fake(), _fake(), None, None) == 1
    assert lib.reef_quantize_int8_per_head(None, 1, 1, 1, 1, None, _fake(), _fake(), None,
                                           None) == 1
    assert lib.reef_read_status_word(None, 0, None) == 1


def test_integer_head_refuses_rows_beyond_65536_keys():
    """A row's uint32 weight sum (up to 65535 per key) cannot wrap within 65536
    visible keys; longer rows (kv_len, or the window when it is shorter) are refused
    before any launch."""
    lib = reef_amd.lib()
    f = [_fake(i) for i in range(1, 8)]
    for kv_len, window in ((65537, 0), (70000, 65537)):
        p = reef_amd.AttentionParams(1, 1, 1, 1, kv_len, 64, kv_len - 1, window, 1.0, 1, 1, 0)
        rc = lib.reef_attention_int8_integer(C.byref(p), f[0], None, f[1], None, f[2], None, 10,
                                             f[3], 8, f[4], None, None)
        assert rc == reef_amd.UNSUPPORTED
