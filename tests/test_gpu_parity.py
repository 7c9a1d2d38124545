"""GPU parity: the HIP kernels, called through the C ABI, against the CPU oracle.

Integer outputs (int32 scores, int8 codes, scales) must be bit-exact; fp32
attention outputs must be within max-abs-error 1e-3 of the oracle's golden
(TOL below) on N(0, 1) data. Each case prints its name before touching the GPU.
"""
import math
import os

import numpy as np
import pytest

import oracle
from reef_amd import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

TOL = 1e-3


@pytest.fixture(scope="module")
def reef():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import reef_amd
    reef_amd.lib()  # raises if the library was not built
    return reef_amd


def case(msg):
    print(f"\n[case] {msg}", flush=True)


def gpu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rand_i8(rng, shape, low=-127):
    return rng.integers(low, 128, shape, dtype=np.int8)


# --- bit-exact integer scores ----------------------------------------------------------

@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D", [
    (1, 1, 1, 128, 128, 64), (2, 4, 2, 37, 101, 128), (1, 2, 1, 1, 33, 64),
    (1, 8, 1, 200, 96, 128), (3, 3, 3, 65, 17, 128)])
def test_qk_scores_bit_exact(reef, B, Hq, Hkv, Sq, Skv, D):
    case(f"qk_scores_i32 B{B} Hq{Hq} Hkv{Hkv} Sq{Sq} Skv{Skv} D{D}")
    rng = np.random.default_rng(B * 1000 + Sq)
    q = rand_i8(rng, (B, Hq, Sq, D), low=-128)
    k = rand_i8(rng, (B, Hkv, Skv, D), low=-128)
    k[0, 0, 0] = -128
    q[0, 0, 0] = -128
    acc = host(reef.qk_scores_i32(gpu(q), gpu(k)))
    g = Hq // Hkv
    want = np.einsum("bhqd,bhkd->bhqk", q.astype(np.int64),
                     np.repeat(k, g, axis=1).astype(np.int64))
    assert np.array_equal(acc, want)
    assert acc[0, 0, 0, 0] == 128 * 128 * D
    assert np.array_equal(acc[0, 0], oracle.qk_i32(q[0, 0], k[0, 0]))


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv", [
    (1, 1, 1, 300, 300), (2, 4, 2, 37, 101), (1, 2, 1, 1, 33), (1, 8, 1, 200, 129),
    (3, 3, 3, 65, 17), (1, 2, 2, 520, 1000)])
def test_qk_scores_packed_kernel_bit_exact(reef, B, Hq, Hkv, Sq, Skv):
    """The packed prefill kernel's own score accumulators (its LDS key order, its
    accumulators relative to the running maximum, rescales included) read back as
    int32 sums: bit-exact against the integer product, -128 * -128 included, key
    counts that are not multiples of the 64-key tile."""
    case(f"qk_scores_i32_packed B{B} Hq{Hq} Hkv{Hkv} Sq{Sq} Skv{Skv}")
    rng = np.random.default_rng(B * 1009 + Sq + Skv)
    D = 128
    q = rand_i8(rng, (B, Hq, Sq, D), low=-128)
    k = rand_i8(rng, (B, Hkv, Skv, D), low=-128)
    q[0, 0, 0] = -128
    k[0, 0, 0] = -128
    if Sq > 1 and Skv > 1:                          # a late maximum forces a rescale
        k[0, 0, Skv - 1] = 127
        q[0, 0, 1] = 127
    acc = host(reef.qk_scores_i32_packed(gpu(q), gpu(k)))
    g = Hq // Hkv
    want = np.einsum("bhqd,bhkd->bhqk", q.astype(np.int64),
                     np.repeat(k, g, axis=1).astype(np.int64))
    assert np.array_equal(acc, want)
    assert acc[0, 0, 0, 0] == 128 * 128 * D
    assert np.array_equal(acc[0, 0], oracle.qk_i32(q[0, 0], k[0, 0]))


# --- bit-exact quantization ---------------------------------------------------------------

def _ties(n):
    """Values whose scale is exactly 1 (largest magnitude 127) so x / scale is x:
    halves exercise ties-to-even in both signs."""
    x = np.linspace(-126.5, 126.5, n).astype(np.float32)
    x[: min(n, 9)] = np.array([127, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 126.5, -1.5], np.float32)[: min(n, 9)]
    return x


@pytest.mark.parametrize("n", [4, 64, 4096 * 257, 33_554_432])
def test_quantize_per_tensor_flat_bit_exact(reef, n):
    """Sizes that are multiples of 4 take the flat streaming kernels (block maxima
    in the output buffer, one reduction, quantize)."""
    case(f"quantize_per_tensor flat n={n}")
    x = (W.lcg_normal(24 + n % 97, n) * 2.5).astype(np.float32)
    x[n // 3] = -40.0
    q, s = reef.quantize_per_tensor(gpu(x))
    qo, so = oracle.quantize_per_tensor(x)
    assert host(s)[0].view(np.uint32) == so[0].view(np.uint32)
    assert np.array_equal(host(q), qo)
    z = np.zeros(n, np.float32)
    q, s = reef.quantize_per_tensor(gpu(z))
    assert host(s)[0] == 1.0 and not host(q).any()


def test_quantize_per_tensor_bit_exact(reef):
    case("quantize_per_tensor n=1000003 normal + ties")
    x = (W.lcg_normal(21, 1_000_003) * 3.7).astype(np.float32)
    q, s = reef.quantize_per_tensor(gpu(x))
    qo, so = oracle.quantize_per_tensor(x)
    assert host(s)[0].view(np.uint32) == so[0].view(np.uint32)
    assert np.array_equal(host(q), qo)
    t = _ties(1001)
    q, s = reef.quantize_per_tensor(gpu(t))
    qo, so = oracle.quantize_per_tensor(t)
    assert host(s)[0] == 1.0 and np.array_equal(host(q), qo)
    z = np.zeros(17, np.float32)
    q, s = reef.quantize_per_tensor(gpu(z))
    assert host(s)[0] == 1.0 and not host(q).any()  # an all-zero tensor keeps scale 1


def test_quantize_per_head_bit_exact_with_strides(reef):
    case("quantize_per_head [2, 6, 33, 128] from a [B, S, H, D] layout")
    x = W.lcg_normal(22, 2 * 33 * 6 * 128).reshape(2, 33, 6, 128)
    x[:, :, 3] *= 50.0
    x[:, :, 5] = 0.0
    xt = gpu(x).permute(0, 2, 1, 3)  # [B, H, S, D] view with strides
    q, s = reef.quantize_per_head(xt)
    qo, so = oracle.quantize_per_head(np.ascontiguousarray(x.transpose(0, 2, 1, 3)))
    assert np.array_equal(host(s).view(np.uint32), so.view(np.uint32))
    assert np.array_equal(host(q), qo)
    assert host(s)[5] == 1.0


@pytest.mark.parametrize("B,H,S,D", [(3, 5, 77, 128), (1, 32, 2048, 128), (2, 3, 5, 64),
                                     (1, 2, 1, 4), (600, 2, 2, 8), (3, 5, 1, 8)])
def test_quantize_per_head_contiguous_bit_exact(reef, B, H, S, D):
    """Contiguous heads take the flat streaming kernels: partial chunks, a zero head
    and a large head, bit-exact against the oracle. The last two shapes have output
    chunks shorter than a head's partial count (600 batches; 2-word chunks for 3
    partials), so their maxima are reduced by the separate scale pass."""
    case(f"quantize_per_head contiguous [{B}, {H}, {S}, {D}]")
    x = W.lcg_normal(23 + S, B * H * S * D).reshape(B, H, S, D)
    x[:, 0] *= 50.0
    x[:, H - 1] = 0.0 if H > 1 else x[:, H - 1]
    q, s = reef.quantize_per_head(gpu(x))
    qo, so = oracle.quantize_per_head(x)
    assert np.array_equal(host(s).view(np.uint32), so.view(np.uint32))
    assert np.array_equal(host(q), qo)


@pytest.mark.parametrize("rows,width", [(4096, 128), (7, 37), (300, 64), (3, 1), (33, 96),
                                        (40, 2048), (9, 5000), (17, 8192), (5, 8193)])
def test_quantize_rows_bit_exact(reef, rows, width):
    case(f"quantize_rows {rows}x{width}")
    x = W.lcg_normal(23 + width, rows * width).reshape(rows, width)
    x *= W.lcg_uniform(24, rows, 0.01, 40.0)[:, None]
    if rows > 3:
        x[1] = 0.0
        x[2, : min(width, 9)] = _ties(min(width, 9))
    q, s = reef.quantize_rows(gpu(x))
    qo, so = oracle.quantize_rows(x)
    assert np.array_equal(host(s).view(np.uint32), so.view(np.uint32))
    assert np.array_equal(host(q), qo)


def test_quantize_rows_with_row_stride(reef):
    case("quantize_rows over a strided [rows, 128] view")
    x = W.lcg_normal(25, 64 * 256).reshape(64, 256)
    view = gpu(x)[:, 64:192]
    q, s = reef.quantize_rows(view)
    qo, so = oracle.quantize_rows(np.ascontiguousarray(x[:, 64:192]))
    assert np.array_equal(host(q), qo) and np.array_equal(host(s), so)


@pytest.mark.parametrize("n,group", [(4096 * 128, 128), (1_000_003, 1_000_003), (77, 7),
                                     (3 * 8193, 8193), (4 * 61, 61), (1, 1), (10, 4)])
def test_dequantize_bit_exact(reef, n, group):
    """float(code) * scale[i / group], bit for bit: per-token rows (group = width),
    one scale over the tensor (group = n), odd sizes, groups that are not multiples
    of 4 (the scalar kernel), and a short last group."""
    case(f"dequantize n={n} group={group}")
    rng = np.random.default_rng(n + group)
    q = rand_i8(rng, (n,), low=-128)
    scales = rng.uniform(1e-4, 3.0, (n + group - 1) // group).astype(np.float32)
    x = host(reef.dequantize(gpu(q), gpu(scales), group))
    want = oracle.dequantize(q, scales, group)
    assert np.array_equal(x.view(np.uint32), want.view(np.uint32))


def test_quantize_streams_beyond_the_cache(reef):
    """537 MB of floats take the non-temporal streams (beyond the 256 MB last-level
    cache; beyond 384 MB for the two-pass scales): per head, per tensor, per token
    128 and 8192 wide, and a dequantize to 537 MB, bit-exact against the oracle."""
    import torch
    n = 4 * 32 * 8192 * 128
    g = torch.Generator(device="cuda")
    g.manual_seed(31)
    xd = torch.randn(n, generator=g, device="cuda")
    xd[::1_000_003] *= 40.0
    x = host(xd)
    case("quantize_per_head [4, 32, 8192, 128], 537 MB")
    q, s = reef.quantize_per_head(xd.view(4, 32, 8192, 128))
    qo, so = oracle.quantize_per_head(x.reshape(4, 32, 8192, 128))
    assert np.array_equal(host(s).view(np.uint32), so.view(np.uint32))
    assert np.array_equal(host(q), qo)
    case(f"quantize_per_tensor n={n}, 537 MB")
    q, s = reef.quantize_per_tensor(xd)
    qo, so = oracle.quantize_per_tensor(x)
    assert host(s)[0].view(np.uint32) == so[0].view(np.uint32)
    assert np.array_equal(host(q), qo)
    for rows, width in ((1 << 20, 128), (16384, 8192)):
        case(f"quantize_rows {rows}x{width}, 537 MB")
        q, s = reef.quantize_rows(xd.view(rows, width))
        qo, so = oracle.quantize_rows(x.reshape(rows, width))
        assert np.array_equal(host(s).view(np.uint32), so.view(np.uint32))
        assert np.array_equal(host(q), qo)
    del qo, x
    case(f"dequantize n={n} group=8192 to 537 MB")
    out = host(reef.dequantize(q.reshape(-1), s, 8192))
    want = oracle.dequantize(host(q), host(s), 8192)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))


def test_quantize_per_head_groups_beyond_the_cache(reef):
    """Per-head scales of a 436 MB stream (the two-pass kernels with non-temporal
    loads), 13 heads of 33.5 MB with a large outlier in the last value of the last
    head: bit-exact against the oracle."""
    import torch
    shape = (2, 13, 4096, 1024)
    case(f"quantize_per_head {list(shape)}, 436 MB")
    g = torch.Generator(device="cuda")
    g.manual_seed(37)
    xd = torch.randn(shape, generator=g, device="cuda")
    xd[1, 12, 4095, 1023] = 900.0
    q, s = reef.quantize_per_head(xd)
    x = host(xd)
    qo, so = oracle.quantize_per_head(x)
    assert np.array_equal(host(s).view(np.uint32), so.view(np.uint32))
    assert np.array_equal(host(q), qo)


def test_quantize_rejects_non_finite(reef):
    case("quantize non-finite -> NonFiniteInput")
    for bad in (math.nan, math.inf, -math.inf):
        x = np.ones((4, 64), np.float32)
        x[2, 5] = bad
        with pytest.raises(reef.NonFiniteInput):
            reef.quantize_rows(gpu(x))
        with pytest.raises(reef.NonFiniteInput):
            reef.quantize_per_tensor(gpu(x))
        with pytest.raises(reef.NonFiniteInput):
            reef.quantize_per_head(gpu(x.reshape(1, 2, 2, 64)))
    reef.quantize_rows(gpu(np.ones((4, 64), np.float32)))  # the status word is clean again


# --- prefill attention ----------------------------------------------------------------------

def _quantize(x, gran):
    if gran == oracle.GRAN_TENSOR:
        return oracle.quantize_per_tensor(x)
    if gran == oracle.GRAN_HEAD:
        return oracle.quantize_per_head(x)
    return oracle.quantize_per_token(x)


def _run_prefill(reef, q, k, v, p, precise=False, workspace=None, schedule=0):
    qq, qs = _quantize(q, p.q_granularity)
    kq, ks = _quantize(k, p.kv_granularity)
    vq, vs = _quantize(v, p.kv_granularity)
    out = reef.attention_prefill(gpu(qq), gpu(kq), gpu(vq), gpu(qs), gpu(ks), gpu(vs),
                                 query_start=p.start(), window=p.window,
                                 softmax_scale=p.softmax_scale, q_granularity=p.q_granularity,
                                 kv_granularity=p.kv_granularity, precise=precise,
                                 workspace=workspace, schedule=schedule)
    gold = oracle.attention_int8(p, qq, kq, vq, qs, ks, vs)
    return host(out), gold


def test_prefill_config1(reef):
    cfg = W.CONFIGS["prefill_1x1x128x64"]
    case(f"prefill {cfg.name}")
    q, k, v = W.host_prefill_inputs(cfg)
    # the kernels' quantization is bit-identical to the oracle's
    qg, sg = reef.quantize_per_tensor(gpu(q))
    qo, so = oracle.quantize_per_tensor(q)
    assert np.array_equal(host(qg), qo) and host(sg)[0] == so[0]
    p = oracle.Problem(1, 1, 1, 128, 128, 64, softmax_scale=cfg.softmax_scale,
                       q_granularity=0, kv_granularity=0)
    out, gold = _run_prefill(reef, q, k, v, p)
    err = np.abs(out - gold).max()
    print(f"max_abs_err {err:.3e}", flush=True)
    assert err <= TOL


PREFILL_CASES = [
    # B, Hq, Hkv, Sq, Skv, D, query_start, window, q_gran, kv_gran, softmax_scale
    (1, 2, 2, 256, 256, 128, None, 0, 1, 1, None),
    (2, 4, 1, 200, 200, 128, None, 0, 1, 1, None),       # GQA 4:1, ragged q tile
    (1, 8, 1, 130, 333, 128, None, 0, 1, 1, None),       # decode-like offset: query_start 203
    (1, 2, 2, 300, 300, 64, None, 40, 0, 0, None),       # sliding window 40
    (1, 2, 1, 96, 500, 128, 100, 70, 2, 2, None),        # explicit start, window, per-token
    (2, 2, 2, 77, 77, 128, None, 0, 2, 1, 1.0),          # engine's unscaled scores
    (1, 1, 1, 1, 1, 64, None, 0, 1, 1, None),            # a single token
    (1, 4, 4, 513, 513, 128, None, 0, 1, 2, None),       # per-token K/V scales
    # very large log2-domain score scales: rows dominated by one key (peaked softmax)
    (1, 2, 2, 256, 256, 128, None, 0, 1, 1, 3000.0),
    (1, 2, 1, 200, 300, 64, None, 0, 0, 0, 20000.0),
    # window past the first key tiles of a long prefix, GQA 2:1, head_dim 128
    (1, 4, 2, 300, 700, 128, 250, 90, 1, 1, None),
    # several 256-row query tiles and an odd tile count (a middle tile without a pair)
    (2, 3, 3, 1200, 1200, 128, None, 0, 1, 1, None),
    # a window shorter than a query tile on a grid of many tiles: the first fully
    # visible key tile lies past the second group's tiles of a split workgroup, whose
    # two groups must still run the same number of steps
    (1, 4, 2, 1200, 1200, 128, None, 100, 1, 1, None),
]


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D,start,window,gq,gkv,scale", PREFILL_CASES)
def test_prefill_matches_oracle(reef, B, Hq, Hkv, Sq, Skv, D, start, window, gq, gkv, scale):
    case(f"prefill B{B} Hq{Hq} Hkv{Hkv} Sq{Sq} Skv{Skv} D{D} start{start} win{window} "
         f"gq{gq} gkv{gkv} scale{scale}")
    seed = B * 7 + Sq * 3 + Skv + D + window
    q = W.lcg_normal(seed, B * Hq * Sq * D).reshape(B, Hq, Sq, D)
    k = W.lcg_normal(seed + 1, B * Hkv * Skv * D).reshape(B, Hkv, Skv, D)
    v = W.lcg_normal(seed + 2, B * Hkv * Skv * D).reshape(B, Hkv, Skv, D)
    if scale == 1.0:  # keep unscaled scores moderate
        q *= 0.1
        k *= 0.1
    p = oracle.Problem(B, Hq, Hkv, Sq, Skv, D, query_start=start, window=window,
                       softmax_scale=(1 / math.sqrt(D)) if scale is None else scale,
                       q_granularity=gq, kv_granularity=gkv)
    # both fp16 P and split P; the library's choice with and without a workspace, and
    # every schedule forced through the flags (the split schedule takes no per-token
    # K/V scales)
    runs = [(False, reef.SCHED_AUTO, None), (False, reef.SCHED_AUTO, False),
            (False, reef.SCHED_ONE_ITEM, False), (True, reef.SCHED_AUTO, None),
            (False, reef.SCHED_BALANCED, None), (True, reef.SCHED_BALANCED, None)]
    if gkv != 2:
        runs += [(False, reef.SCHED_SPLIT, False), (True, reef.SCHED_SPLIT, False)]
        if D == 128:
            runs += [(False, reef.SCHED_PACKED, None), (True, reef.SCHED_PACKED, None)]
    for precise, sched, ws in runs:
        out, gold = _run_prefill(reef, q, k, v, p, precise, workspace=ws, schedule=sched)
        err = np.abs(out - gold).max()
        print(f"precise={precise} schedule={sched:#x} workspace={ws is not False} "
              f"max_abs_err {err:.3e}", flush=True)
        assert err <= TOL, (precise, sched, ws, err)


def test_prefill_outlier_channels(reef):
    """Per-head scales with a few value channels scaled x8 (activation outliers):
    the values of those heads reach |v| ~ 30, where one fp16 P is not precise enough.
    Every schedule the library chooses by itself (balanced with a workspace, 36 tiles
    on 256 compute units; the split kernel without), the forced packed and one-item
    kernels, the forced precise one-item kernel and the forced split and balanced
    schedules (hi + lo P on the outlier heads) stay within TOL."""
    B, H, S, D = 1, 4, 1100, 128
    case(f"prefill outlier channels B{B} H{H} S{S} D{D}")
    q = W.lcg_normal(801, B * H * S * D).reshape(B, H, S, D)
    k = W.lcg_normal(802, B * H * S * D).reshape(B, H, S, D)
    v = W.lcg_normal(803, B * H * S * D).reshape(B, H, S, D)
    for h, c in ((0, 5), (1, 70), (1, 100), (3, 127)):
        for t in (q, k, v):
            t[:, h, :, c] *= 8.0
    p = oracle.Problem(B, H, H, S, S, D, softmax_scale=1 / math.sqrt(D))
    runs = [(False, reef.SCHED_AUTO, None), (False, reef.SCHED_AUTO, False),
            (False, reef.SCHED_PACKED, None), (False, reef.SCHED_ONE_ITEM, False),
            (True, reef.SCHED_ONE_ITEM, False), (False, reef.SCHED_SPLIT, False),
            (False, reef.SCHED_BALANCED, None)]
    for precise, sched, ws in runs:
        out, gold = _run_prefill(reef, q, k, v, p, precise, workspace=ws, schedule=sched)
        err = np.abs(out - gold).max()
        print(f"precise={precise} schedule={sched:#x} workspace={ws is not False} "
              f"max_abs_err {err:.3e}", flush=True)
        assert err <= TOL, (precise, sched, ws, err)


def test_prefill_two_key_rounding_of_p(reef):
    """The worst case of one fp16 P: row 1 sees two keys with values +6 and -6 in every
    channel and the weight ratio r = 0.5 + 0.9 2^-12, which fp16 rounds to 0.5; one
    fp16 P would move the output by 0.9 2^-12 * 12 / (1 + r)^2 = 1.17e-3, past the 1e-3
    of the attention tolerance. Values above 1 in magnitude take P = hi + lo in every
    schedule by default, so the library's default and REEF_ATTN_PRECISE_PV both stay
    within 1e-5 of the oracle."""
    D = 128
    case("prefill two-key row, fp16 rounding of P at its worst")
    q = np.ones((1, 1, 2, D), np.int8)
    k = np.zeros((1, 1, 2, D), np.int8)
    k[0, 0, 1] = -8                                   # s0 - s1 = 1024
    v = np.empty((1, 1, 2, D), np.int8)
    v[0, 0, 0], v[0, 0, 1] = 127, -127
    qs = np.ones(1, np.float32)
    ks = np.ones(1, np.float32)
    vs = np.full(1, 6.0 / 127.0, np.float32)
    r = 0.5 + 0.9 * 2.0 ** -12
    scale = math.log(1.0 / r) / 1024.0
    p = oracle.Problem(1, 1, 1, 2, 2, D, softmax_scale=scale, q_granularity=1,
                       kv_granularity=1)
    gold = oracle.attention_int8(p, q, k, v, qs, ks, vs)
    assert abs(gold[0, 0, 1, 0] - 6.0 * (1 - r) / (1 + r)) < 1e-5
    for precise in (True, False):
        for sched in (reef.SCHED_AUTO, reef.SCHED_ONE_ITEM, reef.SCHED_SPLIT,
                      reef.SCHED_BALANCED, reef.SCHED_PACKED):
            out = reef.attention_prefill(gpu(q), gpu(k), gpu(v), gpu(qs), gpu(ks), gpu(vs),
                                         softmax_scale=scale, precise=precise, schedule=sched)
            err = float(np.abs(host(out) - gold).max())
            print(f"precise={precise} schedule={sched:#x} max_abs_err {err:.3e}", flush=True)
            assert err <= 1e-5, (precise, sched, err)


def _many_small_keys(n, ratio, D=128):
    """One query over n keys: key 0 with value +6 in every channel and score 0, keys
    1 .. n - 1 with value -6 and weight `ratio` relative to key 0 (scores -1024 with
    the softmax scale set to give exactly that ratio). With ratio 1.49 2^-24, a p of
    an unshifted fp16 hi + lo split would be a subnormal fp16 hi (2^-24) and a zero
    lo, moving the output by about 2.9e-3 over 8191 such keys."""
    q = np.ones((1, 1, 1, D), np.int8)
    k = np.full((1, 1, n, D), -8, np.int8)
    k[0, 0, 0] = 0
    v = np.full((1, 1, n, D), -127, np.int8)
    v[0, 0, 0] = 127
    scale = math.log(1.0 / ratio) / 1024.0
    return q, k, v, scale


def test_prefill_many_small_weights_keep_their_precision(reef):
    """Thousands of keys each of weight 1.49 2^-24 of the row's largest: the P parts
    carry an exponent offset (at least 2^7 against a row sum), so every schedule, with
    and without REEF_ATTN_PRECISE_PV, stays within 1e-4 of the exact output
    6 (1 - (n-1) r) / (1 + (n-1) r); without the offset the row is 2.9e-3 off. The
    comparison is with the exact value: the oracle, which sums the weights in fp32 one
    key at a time as the engine does, is itself 1.0e-3 from it on this row (each
    8.9e-8 added to a sum near 1 rounds to a whole fp32 ulp, 1.19e-7)."""
    n, r, D = 8192, 1.49 * 2.0 ** -24, 128
    case(f"prefill {n} keys of relative weight {r:.3e}")
    q, k, v, scale = _many_small_keys(n, r, D)
    qs = np.ones(1, np.float32)
    ks = np.ones(1, np.float32)
    vs = np.full(1, 6.0 / 127.0, np.float32)
    p = oracle.Problem(1, 1, 1, 1, n, D, query_start=n - 1, softmax_scale=scale,
                       q_granularity=1, kv_granularity=1)
    gold = oracle.attention_int8(p, q, k, v, qs, ks, vs)
    exact = 6.0 * (1 - (n - 1) * r) / (1 + (n - 1) * r)
    drift = float(np.abs(gold - exact).max())
    print(f"oracle (fp32, key by key) vs exact {drift:.3e}", flush=True)
    assert 5e-4 < drift < 2e-3
    errs = {}
    for precise in (True, False):
        for sched in (reef.SCHED_AUTO, reef.SCHED_ONE_ITEM, reef.SCHED_SPLIT,
                      reef.SCHED_BALANCED, reef.SCHED_PACKED):
            out = reef.attention_prefill(gpu(q), gpu(k), gpu(v), gpu(qs), gpu(ks), gpu(vs),
                                         query_start=n - 1, softmax_scale=scale,
                                         precise=precise, schedule=sched)
            err = float(np.abs(host(out) - exact).max())
            print(f"precise={precise} schedule={sched:#x} max_abs_err vs exact {err:.3e}",
                  flush=True)
            errs[(precise, sched)] = err
    assert max(errs.values()) <= 1e-4, errs


def test_decode_many_small_weights_keep_their_precision(reef):
    """The decode form of the case above: one sequence of 8192 cached keys, per-token
    scales, key 0 carrying the weight and the other 8191 keys each 1.49 2^-24 of it;
    within 1e-4 of the exact output (the oracle drifts 1.0e-3 from it, as above)."""
    n, r, D = 8192, 1.49 * 2.0 ** -24, 128
    case(f"decode {n} keys of relative weight {r:.3e}")
    q, k, v, scale = _many_small_keys(n, r, D)
    qq = q.reshape(1, 1, D)
    qsc = np.ones((1, 1), np.float32)
    kt = k.reshape(1, 1, n, D)
    vt = v.reshape(1, 1, n, D)
    ksc = np.ones((1, 1, n), np.float32)
    vsc = np.full((1, 1, n), 6.0 / 127.0, np.float32)
    lens = np.array([n], np.int32)
    exact = 6.0 * (1 - (n - 1) * r) / (1 + (n - 1) * r)
    vp = reef.pack_v_pages(gpu(vt))
    out = reef.attention_decode(gpu(qq), gpu(qsc), gpu(kt), vp, gpu(ksc), gpu(vsc), gpu(lens),
                                softmax_scale=scale)
    err = float(np.abs(host(out)[0] - exact).max())
    print(f"max_abs_err vs exact {err:.3e}", flush=True)
    assert err <= 1e-4, err


@pytest.mark.parametrize("B,Hq,Hkv,S,D,gran", [(1, 8, 2, 300, 128, 1), (2, 4, 4, 130, 64, 0),
                                               (1, 4, 1, 77, 128, 2)])
def test_prefill_projection_layout_strides(reef, B, Hq, Hkv, S, D, gran):
    """q, k and v read in place from projection outputs [B, S, H * D] (strides
    {S H D, D, H D}, the engine's [len, heads * head_dim] rows) and the output written
    into an [B, S, Hq * D] buffer: the same result as packed heads."""
    case(f"prefill strided projection layout B{B} Hq{Hq} Hkv{Hkv} S{S} D{D} gran{gran}")
    seed = 900 + S + D
    q = W.lcg_normal(seed, B * Hq * S * D).reshape(B, Hq, S, D)
    k = W.lcg_normal(seed + 1, B * Hkv * S * D).reshape(B, Hkv, S, D)
    v = W.lcg_normal(seed + 2, B * Hkv * S * D).reshape(B, Hkv, S, D)
    qq, qs = _quantize(q, gran)
    kq, ks = _quantize(k, gran)
    vq, vs = _quantize(v, gran)
    p = oracle.Problem(B, Hq, Hkv, S, S, D, softmax_scale=1 / math.sqrt(D), q_granularity=gran,
                       kv_granularity=gran)
    gold = oracle.attention_int8(p, qq, kq, vq, qs, ks, vs)

    def proj(x):  # [B, H, S, D] -> a [B, H, S, D] view of a [B, S, H * D] buffer
        Bx, H, Sx, Dx = x.shape
        buf = gpu(np.ascontiguousarray(x.transpose(0, 2, 1, 3)).reshape(Bx, Sx, H * Dx))
        return buf.view(Bx, Sx, H, Dx).permute(0, 2, 1, 3)

    qv, kv_, vv = proj(qq), proj(kq), proj(vq)
    assert qv.stride() == (S * Hq * D, D, Hq * D, 1)
    obuf = torch.full((B, S, Hq * D), float("nan"), device="cuda")
    out = obuf.view(B, S, Hq, D).permute(0, 2, 1, 3)
    for sched in (reef.SCHED_AUTO, reef.SCHED_ONE_ITEM):
        reef.attention_prefill(qv, kv_, vv, gpu(qs), gpu(ks), gpu(vs), q_granularity=gran,
                               kv_granularity=gran, out=out, schedule=sched)
        got = host(out)
        err = np.abs(got - gold).max()
        print(f"schedule={sched:#x} max_abs_err {err:.3e}", flush=True)
        assert err <= TOL


STREAM_CASES = [
    # B, Hq, Hkv, Sq, Skv, D, query_start, window, gran
    (1, 1, 1, 2048, 2048, 128, None, 0, 1),    # 272 steps for 512 workgroups: up to 32 parts
    (1, 4, 1, 4096, 4096, 128, None, 0, 1),    # GQA, the last items in 3 parts
    (2, 3, 1, 1000, 1500, 64, None, 300, 0),   # window, query_start 500, ragged last tile
    (1, 2, 2, 700, 900, 128, 150, 0, 1),       # explicit start below kv_len - q_len
    (3, 16, 4, 384, 384, 64, None, 0, 1),      # whole items between cut ones
    # per-token K/V scales (hi + lo P): a 512-token chunk over a 4096-token prefix
    # (the prefill over the cache), and a windowed GQA case
    (1, 8, 1, 512, 4096, 128, None, 0, 2),
    (2, 4, 2, 300, 1000, 64, None, 128, 2),
]


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D,start,window,gran", STREAM_CASES)
def test_prefill_balanced_schedule(reef, B, Hq, Hkv, Sq, Skv, D, start, window, gran):
    """The balanced schedule cuts items at workgroup boundaries and merges their
    parts through the workspace: same tolerance, bit-identical on a second call
    (the merge order is fixed), and the item counters back at zero."""
    case(f"prefill balanced B{B} Hq{Hq} Hkv{Hkv} Sq{Sq} Skv{Skv} D{D} start{start} "
         f"win{window} gran{gran}")
    seed = 5 * B + Sq + 2 * Skv + D
    q = W.lcg_normal(seed, B * Hq * Sq * D).reshape(B, Hq, Sq, D)
    k = W.lcg_normal(seed + 1, B * Hkv * Skv * D).reshape(B, Hkv, Skv, D)
    v = W.lcg_normal(seed + 2, B * Hkv * Skv * D).reshape(B, Hkv, Skv, D)
    p = oracle.Problem(B, Hq, Hkv, Sq, Skv, D, query_start=start, window=window,
                       softmax_scale=1 / math.sqrt(D), q_granularity=gran, kv_granularity=gran)
    qq, qs = _quantize(q, gran)
    kq, ks = _quantize(k, gran)
    vq, vs = _quantize(v, gran)
    gold = oracle.attention_int8(p, qq, kq, vq, qs, ks, vs)
    params = reef.AttentionParams(B, Hq, Hkv, Sq, Skv, D, p.start(), window, p.softmax_scale,
                                  gran, gran, 0)
    n = reef.lib().reef_attention_prefill_workspace_bytes(reef.C.byref(params))
    ws = torch.zeros(n, dtype=torch.uint8, device="cuda")
    args = (gpu(qq), gpu(kq), gpu(vq), gpu(qs), gpu(ks), gpu(vs))
    kw = dict(query_start=p.start(), window=window, softmax_scale=p.softmax_scale,
              q_granularity=gran, kv_granularity=gran, workspace=ws,
              schedule=reef.SCHED_BALANCED)
    out1 = host(reef.attention_prefill(*args, **kw))
    out2 = host(reef.attention_prefill(*args, **kw))
    err = np.abs(out1 - gold).max()
    print(f"max_abs_err {err:.3e}", flush=True)
    assert err <= TOL
    assert np.array_equal(out1, out2)
    items = B * Hq * ((Sq + 127) // 128)
    assert not host(ws[:4 * items]).any()


@pytest.mark.parametrize("D", [64, 128])
def test_prefill_full_int8_range(reef, D):
    """Raw int8 operands over the whole range, -128 included (a caller's own
    codes, not the quantizer's): every V byte value must convert exactly."""
    case(f"prefill full int8 range D{D}")
    rng = np.random.default_rng(D)
    B, H, S = 1, 2, 192
    q = rand_i8(rng, (B, H, S, D), low=-128)
    k = rand_i8(rng, (B, H, S, D), low=-128)
    v = np.arange(B * H * S * D, dtype=np.int64).reshape(B, H, S, D)
    v = ((v * 37) % 256 - 128).astype(np.int8)  # every byte value in every tile
    qs = np.array([0.004], np.float32)
    ks = np.array([0.003], np.float32)
    vs = np.array([0.01], np.float32)
    p = oracle.Problem(B, H, H, S, S, D, softmax_scale=1 / math.sqrt(D),
                       q_granularity=0, kv_granularity=0)
    gold = oracle.attention_int8(p, q, k, v, qs, ks, vs)
    for precise in (False, True):
        out = host(reef.attention_prefill(gpu(q), gpu(k), gpu(v), gpu(qs), gpu(ks), gpu(vs),
                                          q_granularity=0, kv_granularity=0, precise=precise))
        err = np.abs(out - gold).max()
        print(f"precise={precise} max_abs_err {err:.3e}", flush=True)
        assert err <= TOL


def test_prefill_rejects_bad_arguments(reef):
    case("prefill argument errors")
    z = torch.zeros((1, 1, 8, 128), dtype=torch.int8, device="cuda")
    s = torch.ones(1, dtype=torch.float32, device="cuda")
    with pytest.raises(reef.InvalidArgument):  # query rows past the keys
        reef.attention_prefill(z, z, z, s, s, s, query_start=4)
    with pytest.raises(reef.Unsupported):
        zz = torch.zeros((1, 1, 8, 96), dtype=torch.int8, device="cuda")
        reef.attention_prefill(zz, zz, zz, s, s, s)


def test_prefill_auto_falls_back_outside_packed_limits(reef):
    """2048 sequences x 32 heads of 128 tokens: 65536 (batch, kv head) pairs, one past
    the packed schedule's 16-bit launch dimension. The library's choice (the packed
    schedule for a grid this large) falls back to the one-item kernel and matches the
    oracle; forcing the packed schedule reports REEF_UNSUPPORTED."""
    B, H, S, D = 2048, 32, 128, 128
    case(f"prefill B{B} H{H} S{S}: past the packed schedule's grid limits")
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    q, k, v = (torch.randint(-127, 128, (B, H, S, D), dtype=torch.int8, device="cuda",
                             generator=g) for _ in range(3))
    sc = torch.full((H,), 0.02, dtype=torch.float32, device="cuda")
    out = reef.attention_prefill(q, k, v, sc, sc, sc)
    with pytest.raises(reef.Unsupported):
        reef.attention_prefill(q, k, v, sc, sc, sc, schedule=reef.SCHED_PACKED)
    p = oracle.Problem(1, 1, 1, S, S, D, softmax_scale=1 / math.sqrt(D), q_granularity=1,
                       kv_granularity=1)
    one = np.full(1, 0.02, np.float32)
    for b, h in ((0, 0), (1023, 17), (2047, 31)):
        sl = lambda t: host(t[b:b + 1, h:h + 1])  # noqa: E731
        gold = oracle.attention_int8(p, sl(q), sl(k), sl(v), one, one, one)
        err = float(np.abs(host(out[b:b + 1, h:h + 1]) - gold).max())
        print(f"b{b} h{h} max_abs_err {err:.3e}", flush=True)
        assert err <= TOL, (b, h, err)


# --- decode ----------------------------------------------------------------------------------

def _decode_problem(B, Hq, Hkv, D, lens, seed, max_ctx):
    """fp32 draws quantized per token, as the cache stores them."""
    q = W.lcg_normal(seed, B * Hq * D).reshape(B, Hq, D)
    kf = W.lcg_normal(seed + 1, B * Hkv * max_ctx * D).reshape(B, Hkv, max_ctx, D)
    vf = W.lcg_normal(seed + 2, B * Hkv * max_ctx * D).reshape(B, Hkv, max_ctx, D)
    qq, qs = oracle.quantize_rows(q.reshape(B * Hq, D))
    kq, ks = oracle.quantize_per_token(kf)
    vq, vs = oracle.quantize_per_token(vf)
    return qq.reshape(B, Hq, D), qs.reshape(B, Hq), kq, ks, vq, vs


def _decode_gold(qq, qs, kq, ks, vq, vs, lens, window, scale):
    B, Hq, D = qq.shape
    Hkv = kq.shape[1]
    out = np.zeros((B, Hq, D), np.float32)
    for b in range(B):
        L = int(lens[b])
        p = oracle.Problem(1, Hq, Hkv, 1, L, D, window=window, softmax_scale=scale,
                           q_granularity=2, kv_granularity=2)
        out[b] = oracle.attention_int8(p, qq[b:b + 1, :, None], kq[b:b + 1, :, :L],
                                       vq[b:b + 1, :, :L], qs[b], ks[b, :, :L], vs[b, :, :L])[0, :, 0]
    return out


@pytest.mark.parametrize("B,Hq,Hkv,D,lens,window,splits", [
    (3, 8, 2, 128, [256, 100, 17], 0, 0),
    (2, 32, 8, 128, [1024, 1024], 0, 0),
    (4, 4, 4, 64, [64, 1, 300, 129], 0, 3),
    (2, 16, 1, 128, [700, 333], 50, 0),
])
def test_decode_contiguous_matches_oracle(reef, B, Hq, Hkv, D, lens, window, splits):
    max_ctx = ((max(lens) + 15) // 16) * 16
    case(f"decode contiguous B{B} Hq{Hq} Hkv{Hkv} D{D} lens{lens} win{window} splits{splits}")
    qq, qs, kq, ks, vq, vs = _decode_problem(B, Hq, Hkv, D, lens, 31 + B + D, max_ctx)
    scale = 1 / math.sqrt(D)
    v_pages = reef.pack_v_pages(gpu(vq))
    assert np.array_equal(host(v_pages),
                          vq.reshape(B, Hkv, max_ctx // 16, 16, D).transpose(0, 1, 2, 4, 3))
    out = reef.attention_decode(gpu(qq), gpu(qs), gpu(kq), v_pages, gpu(ks), gpu(vs),
                                gpu(np.array(lens, np.int32)), window=window,
                                softmax_scale=scale, num_splits=splits)
    gold = _decode_gold(qq, qs, kq, ks, vq, vs, lens, window, scale)
    err = np.abs(host(out) - gold).max()
    print(f"max_abs_err {err:.3e}", flush=True)
    assert err <= TOL


def test_decode_per_head_query_scales(reef):
    """q quantized with one scale per query head over the whole batch (PER_HEAD), the
    setting of the B64 32q/8kv decode workload, against the oracle with the same
    per-head scales."""
    B, Hq, Hkv, D, lens = 6, 32, 8, 128, [640, 1, 333, 640, 129, 17]
    max_ctx = 640
    case(f"decode per-head q scales B{B} Hq{Hq} Hkv{Hkv} lens{lens}")
    _, _, kq, ks, vq, vs = _decode_problem(B, Hq, Hkv, D, lens, 71, max_ctx)
    qf = W.lcg_normal(72, B * Hq * D).reshape(B, Hq, 1, D)
    qf[:, 5] *= 9.0
    qq, qs_head = oracle.quantize_per_head(qf)
    qq = qq.reshape(B, Hq, D)
    scale = 1 / math.sqrt(D)
    out = reef.attention_decode(gpu(qq), gpu(qs_head), gpu(kq), reef.pack_v_pages(gpu(vq)),
                                gpu(ks), gpu(vs), gpu(np.array(lens, np.int32)),
                                softmax_scale=scale, q_granularity=reef.PER_HEAD)
    gold = _decode_gold(qq, np.broadcast_to(qs_head, (B, Hq)), kq, ks, vq, vs, lens, 0, scale)
    err = np.abs(host(out) - gold).max()
    print(f"max_abs_err {err:.3e}", flush=True)
    assert err <= TOL


def _paged(kq, ks, vq, vs, lens, seed, slack=1.5):
    """Scatter each sequence's pages into a pool at seeded positions."""
    B, Hkv, Lmax, D = kq.shape
    npages = [(int(L) + 15) // 16 for L in lens]
    pool = int(sum(npages) * slack) + 1
    order = np.argsort(W.lcg_states(seed, pool), kind="stable").astype(np.int32)
    k_pages = np.zeros((pool, Hkv, 16, D), np.int8)
    v_pages = np.zeros((pool, Hkv, D, 16), np.int8)
    ks_pages = np.zeros((pool, Hkv, 16), np.float32)
    vs_pages = np.zeros((pool, Hkv, 16), np.float32)
    max_blocks = Lmax // 16
    table = np.full((B, max_blocks), -7, np.int32)  # unused entries hold junk
    nxt = 0
    for b in range(B):
        for i in range(npages[b]):
            pg = order[nxt]
            nxt += 1
            table[b, i] = pg
            k_pages[pg] = kq[b, :, 16 * i:16 * i + 16]
            v_pages[pg] = vq[b, :, 16 * i:16 * i + 16].transpose(0, 2, 1)
            ks_pages[pg] = ks[b, :, 16 * i:16 * i + 16]
            vs_pages[pg] = vs[b, :, 16 * i:16 * i + 16]
    return k_pages, v_pages, ks_pages, vs_pages, table


@pytest.mark.parametrize("B,Hq,Hkv,D,lens,window", [
    (5, 8, 1, 128, [512, 37, 1000, 16, 777], 0),
    (3, 4, 2, 64, [200, 64, 129], 0),
    (2, 8, 1, 128, [900, 650], 100),
])
def test_decode_paged_matches_oracle(reef, B, Hq, Hkv, D, lens, window):
    max_ctx = ((max(lens) + 63) // 64) * 64
    case(f"decode paged B{B} Hq{Hq} Hkv{Hkv} D{D} lens{lens} win{window}")
    qq, qs, kq, ks, vq, vs = _decode_problem(B, Hq, Hkv, D, lens, 41 + B, max_ctx)
    kp, vp, ksp, vsp, table = _paged(kq, ks, vq, vs, lens, 43 + B)
    scale = 1 / math.sqrt(D)
    out = reef.attention_decode_paged(gpu(qq), gpu(qs), gpu(kp), gpu(vp), gpu(ksp), gpu(vsp),
                                      gpu(table), gpu(np.array(lens, np.int32)), window=window,
                                      softmax_scale=scale)
    gold = _decode_gold(qq, qs, kq, ks, vq, vs, lens, window, scale)
    err = np.abs(host(out) - gold).max()
    print(f"max_abs_err {err:.3e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("paged,B,Hq,Hkv,D,window,max_len", [
    (False, 300, 4, 2, 128, 0, 1500),   # 300 sequences x 2 kv heads
    (True, 130, 8, 1, 128, 0, 1500),    # ragged pool, 8:1 grouping
    (True, 40, 16, 2, 64, 300, 1500),   # window
    (True, 24, 8, 1, 128, 0, 8192),     # lengths up to 8192: items over many workgroups
    (False, 2100, 2, 1, 64, 0, 64),     # more items than the block plan holds: whole items
])
def test_decode_ragged_merge_in_launch(reef, paged, B, Hq, Hkv, D, window, max_len):
    """Sequences whose keys are dealt out over several workgroups are merged by the
    last of them in the same launch: oracle tolerance, bit-identical on a second
    call (fixed merge order), item counters back at zero, and another split count
    agrees."""
    rng = np.random.default_rng(B + D)
    lens = [int(x) for x in rng.integers(1, max_len, B)]
    lens[0], lens[-1] = 1, max_len
    max_ctx = ((max(lens) + 63) // 64) * 64
    case(f"decode ragged paged={paged} B{B} Hq{Hq} Hkv{Hkv} D{D} win{window} max_len{max_len}")
    qq, qs, kq, ks, vq, vs = _decode_problem(B, Hq, Hkv, D, lens, 61 + B, max_ctx)
    scale = 1 / math.sqrt(D)
    glens = gpu(np.array(lens, np.int32))
    if paged:
        kp, vp, ksp, vsp, table = _paged(kq, ks, vq, vs, lens, 63 + B)
        args = (gpu(qq), gpu(qs), gpu(kp), gpu(vp), gpu(ksp), gpu(vsp), gpu(table), glens)
        fn = reef.attention_decode_paged
    else:
        args = (gpu(qq), gpu(qs), gpu(kq), reef.pack_v_pages(gpu(vq)), gpu(ks), gpu(vs), glens)
        fn = reef.attention_decode
    p = reef._decode_params(gpu(qq), max_ctx, Hkv, window, scale, reef.PER_TOKEN, 0)
    ws = reef.decode_workspace(p, "cuda")
    out1 = host(fn(*args, window=window, softmax_scale=scale, workspace=ws))
    out2 = host(fn(*args, window=window, softmax_scale=scale, workspace=ws))
    fixed = host(fn(*args, window=window, softmax_scale=scale, num_splits=9))
    gold = _decode_gold(qq, qs, kq, ks, vq, vs, lens, window, scale)
    err = np.abs(out1 - gold).max()
    print(f"max_abs_err {err:.3e} vs 9 splits {np.abs(out1 - fixed).max():.3e}", flush=True)
    assert err <= TOL
    assert np.abs(fixed - gold).max() <= TOL
    assert np.array_equal(out1, out2)
    assert not host(ws[:B * Hkv]).any()  # the counters lead the workspace


def test_decode_paged_flags_bad_pages_and_lengths(reef):
    case("decode paged: out-of-range page and length are reported")
    B, Hq, Hkv, D, lens = 2, 4, 1, 64, [40, 30]
    qq, qs, kq, ks, vq, vs = _decode_problem(B, Hq, Hkv, D, lens, 51, 64)
    kp, vp, ksp, vsp, table = _paged(kq, ks, vq, vs, lens, 52)
    bad = table.copy()
    bad[1, 0] = 10_000
    with pytest.raises(reef.InvalidArgument):
        reef.attention_decode_paged(gpu(qq), gpu(qs), gpu(kp), gpu(vp), gpu(ksp), gpu(vsp),
                                    gpu(bad), gpu(np.array(lens, np.int32)))
    with pytest.raises(reef.InvalidArgument):
        reef.attention_decode_paged(gpu(qq), gpu(qs), gpu(kp), gpu(vp), gpu(ksp), gpu(vsp),
                                    gpu(table), gpu(np.array([40, 0], np.int32)))


def test_workspaces_serve_calls_of_any_shape(reef):
    """One zero-filled workspace reused by calls of different shapes: the balanced
    prefill with 48 items and then 96 (a layout with a per-call number of counters
    made the second call read the first call's part slots as counters), the packed
    prefill (whose item queue sits in the last words of the same counter region)
    between them, and decode with 8 items and then 80. The counters sit at fixed
    offsets and every call leaves them zero, so every call matches the oracle."""
    big = reef.AttentionParams(2, 16, 4, 300, 1000, 128, 700, 0, 0.125, 1, 1, 0)
    ws = torch.zeros(reef.lib().reef_attention_prefill_workspace_bytes(reef.C.byref(big)),
                     dtype=torch.uint8, device="cuda")
    counters = 65536 * 4
    for B, D, sched in ((1, 64, "BALANCED"), (2, 128, "PACKED"), (2, 64, "BALANCED"),
                        (1, 128, "PACKED"), (1, 64, "BALANCED"), (2, 64, "BALANCED")):
        case(f"prefill {sched.lower()} B{B} Hq16 Hkv4 Sq300 Skv1000 D{D}, one workspace")
        seed = 400 + B + D
        q = W.lcg_normal(seed, B * 16 * 300 * D).reshape(B, 16, 300, D)
        k = W.lcg_normal(seed + 1, B * 4 * 1000 * D).reshape(B, 4, 1000, D)
        v = W.lcg_normal(seed + 2, B * 4 * 1000 * D).reshape(B, 4, 1000, D)
        p = oracle.Problem(B, 16, 4, 300, 1000, D, softmax_scale=0.125)
        out, gold = _run_prefill(reef, q, k, v, p, workspace=ws,
                                 schedule=getattr(reef, "SCHED_" + sched))
        err = np.abs(out - gold).max()
        print(f"max_abs_err {err:.3e}", flush=True)
        assert err <= TOL
        assert not ws[:counters].any(), "a call left counters behind"
    D, Hq, Hkv = 128, 8, 2
    dbig = reef.DecodeParams(40, Hq, Hkv, D, 640, 0, 1 / math.sqrt(D), reef.PER_TOKEN, 0, 0)
    dws = reef.decode_workspace(dbig, "cuda")
    for B in (4, 40, 4, 40):
        lens = [int(x) for x in (np.arange(B) * 97 % 630 + 1)]
        case(f"decode B{B} Hq{Hq} Hkv{Hkv}, one workspace")
        qq, qs, kq, ks, vq, vs = _decode_problem(B, Hq, Hkv, D, lens, 500 + B, 640)
        out = reef.attention_decode(gpu(qq), gpu(qs), gpu(kq), reef.pack_v_pages(gpu(vq)),
                                    gpu(ks), gpu(vs), gpu(np.array(lens, np.int32)),
                                    softmax_scale=1 / math.sqrt(D), workspace=dws)
        gold = _decode_gold(qq, qs, kq, ks, vq, vs, lens, 0, 1 / math.sqrt(D))
        err = np.abs(host(out) - gold).max()
        print(f"max_abs_err {err:.3e}", flush=True)
        assert err <= TOL
