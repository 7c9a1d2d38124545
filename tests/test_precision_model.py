"""CPU model of how the device kernels round P for the P.V product (numpy's IEEE
fp16: round to nearest even, with subnormals), checked on the inputs that decide the
design: where one fp16 P is enough, and why the hi + lo split carries an exponent
offset. No GPU; the GPU tests run the same rows through the kernels."""
import math

import numpy as np

TOL = 1e-3


def _split(p, parts):
    """p (float64 weights, already in the kernel's fp32 range) rounded as the kernels
    round it: fp32, then one fp16 (parts=1) or fp16 hi + fp16 of the fp32 residual."""
    p32 = p.astype(np.float32)
    hi = p32.astype(np.float16)
    if parts == 1:
        return hi.astype(np.float64)
    lo = (p32 - hi.astype(np.float32)).astype(np.float16)
    return hi.astype(np.float64) + lo.astype(np.float64)


def _attend(p, v, parts, shift=0.0):
    """Output of one row from weights p and values v with P rounded as above; the row
    sum is of exactly the rounded weights (as the prefill kernels keep it)."""
    w = _split(p * 2.0 ** shift, parts)
    return float((w * v).sum() / w.sum())


def test_one_fp16_p_fails_two_keys_of_values_six():
    """Two keys of values +6 and -6 and weight ratio 0.5 + 0.9 2^-12: one fp16 P moves
    the output past 1e-3, hi + lo does not. Values of this size take hi + lo."""
    r = 0.5 + 0.9 * 2.0 ** -12
    p = np.array([1.0, r])
    v = np.array([6.0, -6.0])
    exact = float((p * v).sum() / p.sum())
    assert abs(_attend(p, v, 1) - exact) > TOL
    assert abs(_attend(p, v, 2) - exact) < 1e-6


def test_one_fp16_p_suffices_for_values_within_one():
    """At the hi-only threshold (|v| <= 1) the worst two-key ratio moves the output by
    at most 2^-11 * 2 < 1e-3, over a sweep of ratios near the fp16 rounding ties."""
    worst = 0.0
    for k in range(1, 4096):
        r = 0.5 + (k + 0.5) * 2.0 ** -12
        p = np.array([1.0, r])
        v = np.array([1.0, -1.0])
        exact = float((p * v).sum() / p.sum())
        worst = max(worst, abs(_attend(p, v, 1) - exact))
    assert worst <= 2.0 ** -11 * 2
    assert worst < TOL


def test_hi_lo_split_needs_the_exponent_offset():
    """8191 keys each of weight 1.49 2^-24 of the largest: without an offset their fp16
    hi is the subnormal 2^-24 and the lo part is zero, 2.9e-3 off over the row; with
    the offsets the kernels use (2^7 in the one-item, split and balanced kernels, 2^9
    in the packed kernel, 2^8 in decode) each part is off by at most 2^-25 against a
    row sum of at least 2^7: under 1e-4 here, and 2.9e-5 at 2^7."""
    n, r = 8192, 1.49 * 2.0 ** -24
    p = np.full(n, r)
    p[0] = 1.0
    v = np.full(n, -6.0)
    v[0] = 6.0
    exact = 6.0 * (1 - (n - 1) * r) / (1 + (n - 1) * r)
    assert abs(float((p * v).sum() / p.sum()) - exact) < 1e-12
    assert abs(_attend(p, v, 2, shift=0) - exact) > 2e-3
    for shift in (7, 8, 9):
        assert abs(_attend(p, v, 2, shift=shift) - exact) < 1e-4, shift


def test_offset_keeps_the_largest_weight_inside_fp16():
    """The lazy rescales bound the largest weight: p <= 2^(lazy + offset) with a
    rounding margin below 2^16 (fp16's largest finite value is 65504)."""
    fp16_max = float(np.finfo(np.float16).max)
    for lazy, shift, margin in ((8, 7, 0.01), (6, 9, 0.25), (6 + 1, 8, 0.0)):
        # prefill kernels (lazy 8, offset 7); packed kernel (lazy 6, offset 9, 1/4 from
        # rounding its per-row constant); decode (lazy 6 on p times at most 2 from the
        # value normalizer, offset 8)
        assert 2.0 ** (lazy + shift + margin) < fp16_max
    assert math.isfinite(float(np.float16(2.0 ** 15.25)))
