"""Pins the CPU oracle (oracle/reef_oracle.c) before anything is checked against it.

Each oracle function is checked against at least one of: the engine's golden
vectors (tests/golden/*.json, written by the engine's own golden writer), the
known answers in the engine's gtests (cited file:line), the engine itself
compiled from its headers (oracle/_ref, when built here), and closed forms or
brute force chosen so that a dropped term, a wrong sign or index, or a
transposed operand fails.
"""
import json
import math
import os
import struct

import numpy as np
import pytest

import oracle

REF = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built here")


def f32(bits):
    return np.array(bits, np.uint32).view(np.float32)


def load(golden_dir, name):
    with open(os.path.join(golden_dir, name)) as f:
        return json.load(f)


# --- quant.hpp -----------------------------------------------------------------------

def test_int8_scale_known_answers():
    # test_quant.cpp:38-42
    assert oracle.int8_scale(254.0) == 2.0
    assert oracle.int8_scale(127.0) == 1.0
    assert oracle.int8_scale(0.0) == 1.0
    assert oracle.int8_scale(1.0) == np.float32(1.0) / np.float32(127.0)


def test_quantize_int8_ties_even_and_clamps():
    # test_quant.cpp:46-53
    cases = [(2.5, 2), (3.5, 4), (-2.5, -2), (2.4, 2), (500.0, 127), (-500.0, -127),
             (-0.5, 0), (1.5, 2), (126.5, 126), (127.5, 127), (-127.5, -127)]
    for value, code in cases:
        assert oracle.quantize_int8(value, 1.0) == code, value


def test_quantize_int8_rejects_non_finite():
    # test_quant.cpp:116-126
    for value, scale in [(math.nan, 1.0), (1.0, math.inf), (math.inf, 1.0), (-math.inf, 2.0)]:
        with pytest.raises(ValueError):
            oracle.quantize_int8(value, scale)
    with pytest.raises(ValueError):
        oracle.quantize_rows(np.array([[math.inf, 1.0]], np.float32))
    with pytest.raises(ValueError):
        oracle.quantize_rows(np.array([[math.nan, 1.0]], np.float32))


def test_quantize_rows_known_answer():
    # test_quant.cpp:56-74: 127/2 = 63.5 ties to the even 64; a zero row keeps scale 1.
    x = np.array([[254, 127, -127], [0, 0, 0], [1, -0.5, 0.25]], np.float32)
    q, s = oracle.quantize_rows(x)
    assert q[0].tolist() == [127, 64, -64]
    assert s[0] == 2.0 and s[1] == 1.0 and q[1].tolist() == [0, 0, 0]
    assert s[2] == np.float32(1.0) / np.float32(127.0) and q[2, 0] == 127


def test_dequantize_known_answers_and_round_trip():
    """static_cast<float>(code) * scale (test_int8.cpp:182). Pinned by the
    quantize_rows known answer of test_quant.cpp:56-74 read back ([127, 64, -64] at
    scale 2 is [254, 128, -128]), by the round-trip bound |x - deq(q(x))| <= s / 2
    on every value (a wrong scale index, a dropped scale or a sign flip breaks it),
    and by codes times powers of two, which are exact."""
    q, s = oracle.quantize_rows(np.array([[254.0, 127.0, -127.0]], np.float32))
    assert np.array_equal(oracle.dequantize(q, s, 3), np.array([254, 128, -128], np.float32))
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((37, 53)) * rng.uniform(0.01, 40.0, (37, 1))).astype(np.float32)
    x[3] = 0.0
    q, s = oracle.quantize_rows(x)
    back = oracle.dequantize(q, s, 53).reshape(37, 53)
    bound = s.astype(np.float64)[:, None] * (0.5 + 1e-6)
    assert np.all(np.abs(back.astype(np.float64) - x) <= bound)
    assert not back[3].any()
    codes = np.arange(-128, 128, dtype=np.int8)
    scales = np.float32(2.0) ** np.arange(-20, 12, dtype=np.float32)  # 32 groups of 8
    got = oracle.dequantize(codes, scales, 8)
    want = codes.astype(np.float64) * np.repeat(scales.astype(np.float64), 8)
    assert np.array_equal(got.astype(np.float64), want)
    # a tail group shorter than the others
    got = oracle.dequantize(codes[:13], np.array([0.5, 3.0], np.float32), 8)
    assert np.array_equal(got[8:], codes[8:13].astype(np.float32) * np.float32(3.0))


def test_w8a8_golden_pins_per_row_quantization(golden_dir):
    """The engine's W8A8 projection golden (linear.hpp:106-132) is reproduced bit
    for bit by oracle.quantize_rows + exact int32 sums + float(sum) * (s_row * s_col).
    A wrong rounding, scale or clamp in quantize_rows changes these outputs."""
    for c in load(golden_dir, "w8a8_linear.json")["cases"]:
        rows, fin, fout = c["rows"], c["in_features"], c["out_features"]
        x = f32(c["x_bits"]).reshape(rows, fin)
        wt = np.array(c["wt"], np.int8).reshape(fin, fout)
        ws = f32(c["w_scale_bits"])
        y = f32(c["y_bits"]).reshape(rows, fout)
        q, s = oracle.quantize_rows(x)
        acc = q.astype(np.int64) @ wt.astype(np.int64)
        got = acc.astype(np.float32) * (s[:, None] * ws[None, :])
        assert np.array_equal(got.view(np.uint32), y.view(np.uint32))


def test_per_tensor_and_per_head_are_the_row_rule_on_a_wider_row():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 3, 5, 8)).astype(np.float32)
    q, s = oracle.quantize_per_tensor(x)
    q1, s1 = oracle.quantize_rows(x.reshape(1, -1))
    assert s[0] == s1[0] and np.array_equal(q.reshape(1, -1), q1)
    qh, sh = oracle.quantize_per_head(x)
    for h in range(3):
        slab = x[:, h].reshape(1, -1)
        qr, sr = oracle.quantize_rows(slab)
        assert sh[h] == sr[0]
        assert np.array_equal(qh[:, h].reshape(1, -1), qr)
    # the largest magnitude of each head maps to +-127 exactly
    for h in range(3):
        i = np.unravel_index(np.argmax(np.abs(x[:, h])), x[:, h].shape)
        assert abs(int(qh[:, h][i])) == 127


@REF
def test_quantization_matches_engine_on_random_rows():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((64, 129)) * rng.uniform(0.01, 50, (64, 1))).astype(np.float32)
    x[3, 5] = 0.0
    x[7] = 0.0
    x[9, :4] = [63.5, -63.5, 0.5, -1.5]
    q, s = oracle.quantize_rows(x)
    qr = np.empty_like(q)
    sr = np.empty_like(s)
    assert oracle.ref().ref_quantize_rows(x, 64, 129, qr, sr) == 0
    assert np.array_equal(q, qr) and np.array_equal(s.view(np.uint32), sr.view(np.uint32))


# --- math.hpp ------------------------------------------------------------------------

def test_exp_nonpositive_engine_golden(golden_dir):
    g = load(golden_dir, "exp_nonpositive.json")
    x = f32(g["x_bits"])
    y = oracle.exp_nonpositive(x)
    assert np.array_equal(y.view(np.uint32), np.array(g["y_bits"], np.uint32))


def test_exp_nonpositive_within_one_ulp_and_edges():
    # test_math.cpp:34-60: <= 1 ulp of the correctly rounded e^x on [-87, 0].
    first = struct.unpack("<I", struct.pack("<f", -0.0))[0]
    last = struct.unpack("<I", struct.pack("<f", -87.0))[0]
    bits = np.arange(first, last + 1, 99991, dtype=np.uint32)
    x = bits.view(np.float32)
    got = oracle.exp_nonpositive(x).view(np.int32).astype(np.int64)
    exact = np.exp(x.astype(np.float64)).astype(np.float32).view(np.int32).astype(np.int64)
    assert np.max(np.abs(got - exact)) <= 1
    e = oracle.exp_nonpositive([0.0, -0.0, -87.5, -1000.0, -87.0, -1.0])
    assert e[0] == 1.0 and e[1] == 1.0 and e[2] == 0.0 and e[3] == 0.0 and e[4] > 0.0
    assert abs(e[5] - 0.36787944) < 1e-7


@REF
def test_exp_nonpositive_matches_engine_on_a_sweep():
    x = np.linspace(-90.0, 0.0, 20011, dtype=np.float32)
    got = oracle.exp_nonpositive(x)
    f = oracle.ref().ref_exp_nonpositive
    want = np.array([f(float(v)) for v in x], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# --- attention.hpp -------------------------------------------------------------------

def test_visibility_known_answers():
    # test_attention.cpp:309-333
    assert oracle.visible(1, 3, 2).tolist() == [[1, 1, 1]]
    assert oracle.visible(2, 2, 0).tolist() == [[1, 0], [1, 1]]
    assert oracle.visible(1, 4, 3, 2).tolist() == [[0, 0, 1, 1]]


@REF
def test_visibility_matches_engine():
    for rows, keys, start, window in [(5, 9, 4, 0), (4, 9, 5, 3), (7, 7, 0, 2), (1, 40, 39, 16),
                                      (3, 10, 7, 1), (6, 6, 0, 0)]:
        want = np.empty(rows * keys, np.uint8)
        assert oracle.ref().ref_causal_visibility(rows, keys, start, window, want) == 0
        assert np.array_equal(oracle.visible(rows, keys, start, window).reshape(-1), want)


def test_qk_i32_is_the_exact_integer_product():
    # test_tensor.cpp:86-95
    assert oracle.qk_i32(np.array([[100, 100]], np.int8), np.array([[100, 100]], np.int8)) \
        .tolist() == [[20000]]
    rng = np.random.default_rng(5)
    q = rng.integers(-127, 128, (9, 128), dtype=np.int8)
    k = rng.integers(-127, 128, (13, 128), dtype=np.int8)
    k[0] = -127
    q[0] = 127
    want = q.astype(np.int64) @ k.astype(np.int64).T
    assert np.array_equal(oracle.qk_i32(q, k), want)
    assert oracle.qk_i32(q, k)[0, 0] == -127 * 127 * 128


@REF
def test_qk_i32_matches_engine():
    rng = np.random.default_rng(6)
    q = rng.integers(-128, 128, (7, 64), dtype=np.int8)
    k = rng.integers(-128, 128, (11, 64), dtype=np.int8)
    want = np.empty((7, 11), np.int32)
    assert oracle.ref().ref_qk_i32(q, k, 7, 11, 64, want) == 0
    assert np.array_equal(oracle.qk_i32(q, k), want)


def test_masked_softmax_known_answers():
    # test_attention.cpp:125-142 (softmax([0, 1])) and :344-356 (renormalization)
    p = oracle.masked_softmax(np.array([[0.0, 1.0]], np.float32), np.array([[1, 1]], np.uint8))
    assert np.allclose(p, [[0.26894142, 0.73105858]], atol=1e-7)
    p = oracle.masked_softmax(np.array([[5.0, 0.0, 1.0]], np.float32),
                              np.array([[0, 1, 1]], np.uint8))
    assert p[0, 0] == 0.0
    assert np.allclose(p[0, 1:], [0.26894142, 0.73105858], atol=1e-7)
    with pytest.raises(ValueError):
        oracle.masked_softmax(np.array([[1.0, 2.0]], np.float32), np.array([[0, 0]], np.uint8))


@REF
def test_masked_softmax_matches_engine():
    rng = np.random.default_rng(7)
    s = (rng.standard_normal((6, 37)) * 4).astype(np.float32)
    vis = oracle.visible(6, 37, 31, 9)
    want = np.empty_like(s)
    assert oracle.ref().ref_masked_softmax(s, 6, 37, vis.reshape(-1).copy(), want) == 0
    assert np.array_equal(oracle.masked_softmax(s, vis).view(np.uint32), want.view(np.uint32))


def test_attend_head_engine_golden(golden_dir):
    for c in load(golden_dir, "attention_f32.json")["cases"]:
        sq, sk, d = c["query_len"], c["key_len"], c["head_dim"]
        q = f32(c["q_bits"]).reshape(sq, d)
        k = f32(c["k_bits"]).reshape(sk, d)
        v = f32(c["v_bits"]).reshape(sk, d)
        y = oracle.attend_head_f32(q, k, v, c["query_start"], c["window"])
        assert np.array_equal(y.view(np.uint32).reshape(-1), np.array(c["y_bits"], np.uint32))


def test_attend_head_against_float64_brute_force():
    rng = np.random.default_rng(8)
    q = rng.uniform(-2, 2, (4, 16)).astype(np.float32)
    k = rng.uniform(-2, 2, (9, 16)).astype(np.float32)
    v = rng.uniform(-2, 2, (9, 16)).astype(np.float32)
    y = oracle.attend_head_f32(q, k, v, 5, 3)
    vis = oracle.visible(4, 9, 5, 3).astype(bool)
    s = q.astype(np.float64) @ k.astype(np.float64).T
    s = np.where(vis, s, -np.inf)
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    assert np.allclose(y, p @ v.astype(np.float64), atol=2e-6)


# --- int8.hpp ------------------------------------------------------------------------

def test_rounding_shift_and_saturate_known_answers():
    # test_int8.cpp:37-52
    L = oracle.lib()
    for value, shift, want in [(3, 1, 2), (-3, 1, -1), (5, 2, 1), (6, 2, 2), (-6, 2, -1),
                               (-7, 2, -2), (-7, 0, -7)]:
        assert L.ro_rounding_shift(value, shift) == want
    for value, want in [(127, 127), (128, 127), (-128, -128), (-100000, -128)]:
        assert L.ro_saturate_int8(value) == want


def test_exp_table_engine_golden(golden_dir):
    t = oracle.exp_table()
    assert t.tolist() == load(golden_dir, "exp_table.json")["table"]
    assert t[0] == 32768 and t[16] == 12055 and t[255] == 0  # test_int8.cpp:117-125
    assert np.all(np.diff(t.astype(np.int64)) <= 0)


def test_int8_softmax_engine_golden(golden_dir):
    L = oracle.lib()
    table = oracle.exp_table()
    for c in load(golden_dir, "int8_softmax.json")["cases"]:
        s = np.array(c["scores"], np.int32).reshape(c["rows"], c["n"])
        want = np.array(c["probs"], np.uint8).reshape(c["rows"], c["n"])
        for r in range(c["rows"]):
            out = np.empty(c["n"], np.uint8)
            assert L.ro_masked_softmax_int8_row(s[r].copy(), np.ones(c["n"], np.uint8), c["n"],
                                                c["shift"], table, out) == 0
            assert np.array_equal(out, want[r])
    # test_int8.cpp:146-159: equal scores split the weight, masked keys get 0
    out = np.empty(4, np.uint8)
    assert L.ro_masked_softmax_int8_row(np.full(4, 5, np.int32), np.array([1, 1, 0, 0], np.uint8),
                                        4, 0, table, out) == 0
    assert out.tolist() == [128, 128, 0, 0]


def test_int8_head_engine_golden(golden_dir):
    for c in load(golden_dir, "int8_attention.json")["cases"]:
        sq, sk, d = c["query_len"], c["key_len"], c["head_dim"]
        y = oracle.attend_head_int8(np.array(c["q"], np.int8).reshape(sq, d),
                                    np.array(c["k"], np.int8).reshape(sk, d),
                                    np.array(c["v"], np.int8).reshape(sk, d),
                                    c["query_start"], c["window"], c["score_shift"],
                                    c["out_shift"])
        assert y.reshape(-1).tolist() == c["y"]


# --- the batched int8 attention golden (extension) -----------------------------------

def _random_problem(rng, p, gran_q, gran_kv):
    q = rng.integers(-127, 128, (p.batch, p.q_heads, p.q_len, p.head_dim), dtype=np.int8)
    k = rng.integers(-127, 128, (p.batch, p.kv_heads, p.kv_len, p.head_dim), dtype=np.int8)
    v = rng.integers(-127, 128, (p.batch, p.kv_heads, p.kv_len, p.head_dim), dtype=np.int8)

    def scales(gran, heads, tokens):
        n = {oracle.GRAN_TENSOR: 1, oracle.GRAN_HEAD: heads,
             oracle.GRAN_TOKEN: p.batch * heads * tokens}[gran]
        return rng.uniform(0.002, 0.03, n).astype(np.float32)

    return q, k, v, scales(gran_q, p.q_heads, p.q_len), scales(gran_kv, p.kv_heads, p.kv_len), \
        scales(gran_kv, p.kv_heads, p.kv_len)


@REF
@pytest.mark.parametrize("gran_q,gran_kv", [(0, 0), (1, 1), (2, 2), (2, 1)])
def test_attention_int8_matches_engine_composition(gran_q, gran_kv):
    """Bit-exact against the same steps done by the engine's own functions."""
    rng = np.random.default_rng(20 + gran_q * 3 + gran_kv)
    p = oracle.Problem(2, 4, 2, 5, 12, 32, window=0, softmax_scale=1 / math.sqrt(32),
                       q_granularity=gran_q, kv_granularity=gran_kv)
    q, k, v, qs, ks, vs = _random_problem(rng, p, gran_q, gran_kv)
    out = oracle.attention_int8(p, q, k, v, qs, ks, vs)

    def per_row(s, gran, b, h, heads, n):
        if gran == oracle.GRAN_TENSOR:
            return np.full(n, s[0], np.float32)
        if gran == oracle.GRAN_HEAD:
            return np.full(n, s[h], np.float32)
        return s.reshape(p.batch, heads, n)[b, h].copy()

    for b in range(p.batch):
        for h in range(p.q_heads):
            g = h // (p.q_heads // p.kv_heads)
            want = oracle.ref_attention_int8_head(
                q[b, h], k[b, g], v[b, g], per_row(qs, gran_q, b, h, p.q_heads, p.q_len),
                per_row(ks, gran_kv, b, g, p.kv_heads, p.kv_len),
                per_row(vs, gran_kv, b, g, p.kv_heads, p.kv_len), p.start(), p.window,
                p.softmax_scale)
            assert np.array_equal(out[b, h].view(np.uint32), want.view(np.uint32)), (b, h)


def test_attention_int8_with_unit_scales_is_the_float_head():
    """With scales 1 and softmax_scale 1 every int8 score is exact in float, so the
    int8 golden must equal attend_head on the same values bit for bit."""
    rng = np.random.default_rng(9)
    p = oracle.Problem(1, 1, 1, 6, 10, 16, query_start=4, window=3)
    q = rng.integers(-3, 4, (1, 1, 6, 16), dtype=np.int8)
    k = rng.integers(-3, 4, (1, 1, 10, 16), dtype=np.int8)
    v = rng.integers(-127, 128, (1, 1, 10, 16), dtype=np.int8)
    one = np.ones(1, np.float32)
    p.q_granularity = p.kv_granularity = oracle.GRAN_TENSOR
    out, acc = oracle.attention_int8(p, q, k, v, one, one, one, want_acc=True)
    y = oracle.attend_head_f32(q[0, 0].astype(np.float32), k[0, 0].astype(np.float32),
                               v[0, 0].astype(np.float32), 4, 3)
    assert np.array_equal(out[0, 0].view(np.uint32), y.view(np.uint32))
    assert np.array_equal(acc[0, 0], oracle.qk_i32(q[0, 0], k[0, 0]))


def test_attention_int8_against_float64_brute_force():
    """Independent float64 restatement: scores scaled by s_q s_k / sqrt(d), masked
    softmax, values dequantized per token. Catches a dropped or misplaced scale,
    a transposed operand or a wrong kv-head mapping."""
    rng = np.random.default_rng(10)
    p = oracle.Problem(2, 8, 2, 7, 19, 64, window=5, softmax_scale=0.125,
                       q_granularity=oracle.GRAN_TOKEN, kv_granularity=oracle.GRAN_TOKEN)
    q, k, v, qs, ks, vs = _random_problem(rng, p, p.q_granularity, p.kv_granularity)
    out = oracle.attention_int8(p, q, k, v, qs, ks, vs)
    qs = qs.reshape(2, 8, 7)
    ks = ks.reshape(2, 2, 19)
    vs = vs.reshape(2, 2, 19)
    vis = oracle.visible(7, 19, 12, 5).astype(bool)
    for b in range(2):
        for h in range(8):
            g = h // 4
            s = (q[b, h].astype(np.float64) @ k[b, g].astype(np.float64).T)
            s *= qs[b, h][:, None] * ks[b, g][None, :] * 0.125
            s = np.where(vis, s, -np.inf)
            e = np.exp(s - s.max(1, keepdims=True))
            e /= e.sum(1, keepdims=True)
            want = e @ (v[b, g].astype(np.float64) * vs[b, g][:, None])
            assert np.allclose(out[b, h], want, atol=1e-5, rtol=1e-5)


def test_attention_int8_invariants():
    rng = np.random.default_rng(12)
    # GQA == MHA with the kv heads repeated
    p = oracle.Problem(1, 4, 2, 9, 9, 32, softmax_scale=0.2)
    q, k, v, qs, ks, vs = _random_problem(rng, p, oracle.GRAN_HEAD, oracle.GRAN_HEAD)
    gqa = oracle.attention_int8(p, q, k, v, qs, ks, vs)
    p2 = oracle.Problem(1, 4, 4, 9, 9, 32, softmax_scale=0.2)
    mha = oracle.attention_int8(p2, q, np.repeat(k, 2, 1), np.repeat(v, 2, 1), qs,
                                np.repeat(ks, 2), np.repeat(vs, 2))
    assert np.array_equal(gqa, mha)
    # prefill row r == a one-row call at position r over the first r+1 keys
    for r in [0, 3, 8]:
        pd = oracle.Problem(1, 4, 2, 1, r + 1, 32, softmax_scale=0.2)
        one = oracle.attention_int8(pd, q[:, :, r:r + 1], k[:, :, :r + 1], v[:, :, :r + 1], qs,
                                    ks, vs)
        assert np.array_equal(one[:, :, 0], gqa[:, :, r])
    # batch == per-sequence calls
    p3 = oracle.Problem(3, 2, 1, 4, 6, 16, q_granularity=2, kv_granularity=2)
    q, k, v, qs, ks, vs = _random_problem(rng, p3, 2, 2)
    full = oracle.attention_int8(p3, q, k, v, qs, ks, vs)
    for b in range(3):
        pb = oracle.Problem(1, 2, 1, 4, 6, 16, q_granularity=2, kv_granularity=2)
        part = oracle.attention_int8(pb, q[b:b + 1], k[b:b + 1], v[b:b + 1],
                                     qs.reshape(3, -1)[b], ks.reshape(3, -1)[b],
                                     vs.reshape(3, -1)[b])
        assert np.array_equal(part[0], full[b])
    # the integer scores returned are q.k^T of the right kv head (h // group)
    q, k, v, qs, ks, vs = _random_problem(rng, p, 1, 1)
    _, acc = oracle.attention_int8(p, q, k, v, qs, ks, vs, want_acc=True)
    for h in range(4):
        assert np.array_equal(acc[0, h], oracle.qk_i32(q[0, h], k[0, h // 2]))


def test_attention_int8_rejects_invalid_problems():
    z2 = np.zeros((1, 1, 2, 8), np.int8)
    z4 = np.zeros((1, 1, 4, 8), np.int8)
    one = np.ones(1, np.float32)
    oracle.attention_int8(oracle.Problem(1, 1, 1, 2, 2, 8), z2, z2, z2, one, one, one)
    with pytest.raises(ValueError):  # negative query position
        oracle.attention_int8(oracle.Problem(1, 1, 1, 2, 4, 8, query_start=-1), z2, z4, z4, one,
                              one, one)
    with pytest.raises(ValueError):  # query heads not a multiple of kv heads
        oracle.attention_int8(oracle.Problem(1, 3, 2, 2, 2, 8), np.zeros((1, 3, 2, 8), np.int8),
                              np.zeros((1, 2, 2, 8), np.int8), np.zeros((1, 2, 2, 8), np.int8),
                              np.ones(3, np.float32), np.ones(2, np.float32),
                              np.ones(2, np.float32))


@pytest.mark.parametrize("n,want", [(65536, 0), (131073, 2)])
def test_int8_softmax_weight_sum_wraps_like_the_engine(n, want):
    """The engine sums a row's table weights in uint32 (int8.hpp:208-217). With the
    engine's table (first entry 32768) and n equal keys the sum is n * 32768: exact
    at 65536 keys (2^31: the reciprocal (255 << 16) / sum is 0, every probability 0),
    wrapped to 32768 at 131073 (reciprocal 510, every probability clamped to 255, so
    255 * 131073 shifted right by 24 rounds to 2). The oracle keeps the wrap, checked
    against the engine's own code where it is built. The device path refuses rows
    with more than 65536 visible keys, so past that boundary only the oracle runs."""
    d = 32
    q = np.zeros((1, d), np.int8)
    k = np.zeros((n, d), np.int8)
    v = np.ones((n, d), np.int8)
    out = oracle.attend_head_int8(q, k, v, n - 1, 0, 0, 24)
    assert (out == want).all()
    if oracle.ref_available():
        ref = np.empty((1, d), np.int8)
        assert oracle.ref().ref_attend_head_int8(q, k, v, 1, n, d, n - 1, 0, 0, 24, ref) == 0
        assert np.array_equal(out, ref)
