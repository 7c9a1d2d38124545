"""GPU parity at the benchmark workloads, full size, on the launches bench.py times.

Each test builds its workload with bench.py's own setup function (inputs drawn on
the GPU, quantized by the library, the same parameters, workspace and grid), runs
that launch, reads the int8 inputs back and checks a fixed sample of output rows
against the CPU oracle: the first and last rows, rows on both sides of query-tile
boundaries, and rows at seeded random positions, over several batches and heads
(for the 4x32x8192x128 workload, heads with and without the x8 outlier channels).
Decode checks every query head of a sample of sequences, the longest and the
shortest included. fp32 outputs must be within max-abs-error 1e-3 of the oracle
(TOL); each case prints its error.
"""
import math

import numpy as np
import pytest

import bench
import oracle
from reef_amd import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

TOL = 1e-3
THREADS = 16  # oracle worker threads: the GPU box's CPU share


@pytest.fixture(scope="module")
def reef():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import reef_amd
    reef_amd.lib()
    return reef_amd


def case(msg):
    print(f"\n[case] {msg}", flush=True)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def row_blocks(S, seed, width=16, randoms=4):
    """Starts of `width`-row blocks: first rows, last rows, blocks straddling the
    128-row tile boundaries near the start, middle and end, and seeded random ones."""
    starts = {0, S - width}
    for t in (1, S // 256, S // 128 - 1):
        if 0 < t * 128 < S:
            starts.add(max(0, min(S - width, t * 128 - width // 2)))
    rng = np.random.default_rng(seed)
    starts.update(int(x) for x in rng.integers(0, S - width + 1, randoms))
    return sorted(starts)


def prefill_heads(name, cfg):
    """(batch, q head) pairs to check."""
    if name == "prefill_4x32x8192x128":
        heads = sorted(set(int(c) // cfg.head_dim for c in W.outlier_channels(cfg)))
        clean = [h for h in range(cfg.q_heads) if h not in heads]
        return [(0, heads[0]), (3, heads[-1]), (1, clean[0]), (2, 31 if 31 in heads else heads[1])]
    if name == "prefill_1x8x4096x128_gqa":
        return [(0, 0), (0, 3), (0, 7)]
    if name == "prefill_1x32x2048x128":
        return [(0, 0), (0, 17), (0, 31)]
    return [(0, 0)]


PREFILL = ["prefill_1x1x128x64", "prefill_1x32x2048x128", "prefill_1x8x4096x128_gqa",
           "prefill_4x32x8192x128"]


@pytest.mark.parametrize("name", PREFILL)
def test_prefill_workload_full_size(reef, name):
    cfg = W.CONFIGS[name]
    case(f"{cfg.name}: bench launch, sampled rows vs oracle")
    cfg, fp32_inputs, (q, k, v, qs, ks, vs), out, launch = bench.prefill_setup(torch, reef, W,
                                                                              name)
    del fp32_inputs
    launch()
    first = out.clone()
    launch()  # a second launch writes the same bits
    torch.cuda.synchronize()
    assert torch.equal(first, out), "two launches differ"
    del first
    S, D = cfg.seq, cfg.head_dim
    group = cfg.q_heads // cfg.kv_heads
    qs_h, ks_h, vs_h = host(qs), host(ks), host(vs)
    if name == "prefill_4x32x8192x128":
        # the seeded outlier channels make the quantized values of their heads 8x wider
        out_heads = set(int(c) // D for c in W.outlier_channels(cfg))
        assert min(vs_h[list(out_heads)]) > 4 * max(np.delete(vs_h, list(out_heads)))
    worst = 0.0
    for b, h in prefill_heads(name, cfg):
        kvh = h // group
        qh = host(q[b, h])
        kh = host(k[b, kvh])
        vh = host(v[b, kvh])
        oh = host(out[b, h])
        gs = lambda s, i: s[i if s.size > 1 else 0: (i if s.size > 1 else 0) + 1]  # noqa: E731
        for r0 in row_blocks(S, 1000 * b + h):
            w = min(16, S - r0)
            p = oracle.Problem(1, 1, 1, w, r0 + w, D, query_start=r0,
                               softmax_scale=cfg.softmax_scale, q_granularity=cfg.granularity,
                               kv_granularity=cfg.granularity)
            gold = oracle.attention_int8(p, qh[r0:r0 + w], kh[:r0 + w], vh[:r0 + w], gs(qs_h, h),
                                         gs(ks_h, kvh), gs(vs_h, kvh), threads=THREADS)
            err = float(np.abs(oh[r0:r0 + w] - gold[0, 0]).max())
            worst = max(worst, err)
            assert err <= TOL, (b, h, r0, err)
    print(f"{name}: max_abs_err {worst:.3e}", flush=True)


def _fp64_attention_rows(q, k, v, qs, ks, vs, b, h, kvh, scale, gran, r0, r1):
    """Rows r0 .. r1 - 1 of causal attention for (batch b, q head h) in float64 on the
    GPU over the dequantized int8 inputs: float(q) s_q . float(k) s_k * scale, softmax,
    times float(v) s_v. A second opinion beside the oracle's sampled rows, fast enough
    to cover every row of a workload."""
    sq = qs[h] if gran == 1 else qs[0]
    sk = ks[kvh] if gran == 1 else ks[0]
    sv = vs[kvh] if gran == 1 else vs[0]
    qf = q[b, h, r0:r1].to(torch.float64) * sq.to(torch.float64)
    kf = k[b, kvh, :r1].to(torch.float64).contiguous() * sk.to(torch.float64)
    vf = v[b, kvh, :r1].to(torch.float64).contiguous() * sv.to(torch.float64)
    s = torch.matmul(qf, kf.t().contiguous()) * scale
    rows = torch.arange(r0, r1, device=s.device)[:, None]
    keys = torch.arange(r1, device=s.device)[None, :]
    s = s.masked_fill(keys > rows, float("-inf"))
    pr = torch.softmax(s, dim=1)
    return torch.matmul(pr, vf)


@pytest.mark.parametrize("name", ["prefill_1x32x2048x128", "prefill_1x8x4096x128_gqa",
                                  "prefill_4x32x8192x128"])
def test_prefill_workload_every_row(reef, name):
    """Every output row of the benchmark workload from the bench's launch (the library's
    default precision) against float64 attention on the GPU, within TOL."""
    cfg = W.CONFIGS[name]
    case(f"{cfg.name}: bench launch, every row vs float64 attention")
    cfg, fp32_inputs, (q, k, v, qs, ks, vs), out, launch = bench.prefill_setup(torch, reef, W,
                                                                              name)
    del fp32_inputs
    launch()
    torch.cuda.synchronize()
    S = cfg.seq
    group = cfg.q_heads // cfg.kv_heads
    chunk = 2048
    worst = 0.0
    for b in range(cfg.batch):
        for h in range(cfg.q_heads):
            for r0 in range(0, S, chunk):
                r1 = min(S, r0 + chunk)
                ref = _fp64_attention_rows(q, k, v, qs, ks, vs, b, h, h // group,
                                           cfg.softmax_scale, cfg.granularity, r0, r1)
                err = float((out[b, h, r0:r1].to(torch.float64) - ref).abs().max())
                worst = max(worst, err)
                assert err <= TOL, (b, h, r0, err)
    print(f"{name}: every row, max_abs_err {worst:.3e}", flush=True)


def _decode_gold(qq, qs, k_tok, v_tok, ks, vs, L, scale):
    """One sequence: qq [Hq, D] int8 with per-head scales qs [Hq]; k_tok, v_tok
    [Hkv, >= L, D] int8; ks, vs [Hkv, >= L] per-token scales."""
    Hq, D = qq.shape
    Hkv = k_tok.shape[0]
    p = oracle.Problem(1, Hq, Hkv, 1, L, D, query_start=L - 1, softmax_scale=scale,
                       q_granularity=oracle.GRAN_HEAD, kv_granularity=oracle.GRAN_TOKEN)
    return oracle.attention_int8(p, qq[None, :, None], k_tok[None, :, :L], v_tok[None, :, :L],
                                 qs, np.ascontiguousarray(ks[:, :L]),
                                 np.ascontiguousarray(vs[:, :L]), threads=THREADS)[0, :, 0]


def test_decode_b64_l4096_full_size(reef):
    cfg = W.CONFIGS["decode_b64_l4096"]
    case(f"{cfg.name}: bench launch, sampled sequences vs oracle")
    cfg, launch, (q, qsc, k, vp, ksc, vsc, out) = bench.decode_contiguous_setup(torch, reef, W)
    launch()
    launch.check()
    got = host(out)
    B, Hkv, L, D = k.shape
    qq, qs_h = host(q), host(qsc)
    worst = 0.0
    for b in (0, 1, 31, 42, 63):
        v_tok = vp[b].permute(0, 1, 3, 2).reshape(Hkv, L, D)
        gold = _decode_gold(qq[b], qs_h, host(k[b]), host(v_tok), host(ksc[b]), host(vsc[b]), L,
                            1 / math.sqrt(D))
        err = float(np.abs(got[b] - gold).max())
        worst = max(worst, err)
        assert err <= TOL, (b, err)
    print(f"decode_b64_l4096: max_abs_err {worst:.3e}", flush=True)


def test_decode_paged_b128_ragged_full_size(reef):
    cfg = W.CONFIGS["decode_paged_b128_ragged"]
    case(f"{cfg.name}: bench launch on every page pool, sampled sequences vs oracle")
    cfg, lens, launch, setups, (q, qsc, out) = bench.decode_paged_setup(torch, reef, W)
    assert lens.min() >= 512 and lens.max() <= 8192
    qq, qs_h = host(q), host(qsc)
    D = cfg.head_dim
    order = np.argsort(lens)
    rng = np.random.default_rng(6)
    sample = sorted({int(order[0]), int(order[-1]), *(int(x) for x in rng.integers(0, len(lens), 6))})
    worst = 0.0
    for pool, (kp, vp, ksp, vsp, table) in enumerate(setups):
        launch(pool)
        launch.check()
        got = host(out)
        for b in sample:
            L = int(lens[b])
            n = (L + 15) // 16
            pages = table[b, :n].long()
            Hkv = kp.shape[1]
            k_tok = kp[pages].permute(1, 0, 2, 3).reshape(Hkv, n * 16, D)
            v_tok = vp[pages].permute(1, 0, 3, 2).reshape(Hkv, n * 16, D)
            ks_tok = ksp[pages].permute(1, 0, 2).reshape(Hkv, n * 16)
            vs_tok = vsp[pages].permute(1, 0, 2).reshape(Hkv, n * 16)
            gold = _decode_gold(qq[b], qs_h, host(k_tok), host(v_tok), host(ks_tok), host(vs_tok),
                                L, 1 / math.sqrt(D))
            err = float(np.abs(got[b] - gold).max())
            worst = max(worst, err)
            assert err <= TOL, (pool, b, L, err)
    print(f"decode_paged_b128_ragged: max_abs_err {worst:.3e} over sequences {sample}", flush=True)
