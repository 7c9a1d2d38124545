"""Prefill over the int8 decode cache (chunked and multi-turn prompts): a chunk of
queries attends over every cached key (Attention::forward with query_len > 1 on a
non-empty cache, attention.hpp:354-372, query_start = key_len - query_len :415).

The cache holds per-token codes and scales (quantize_rows, quant.hpp:112-133),
contiguous or paged. Each case checks the call against the oracle's attention over
the same token-major codes (max |diff| <= 1e-3), and against the prefill entry
point run on those token-major codes directly: the gather must hand the prefill
exactly the cached rows, so the two outputs are bit-identical."""
import math

import numpy as np
import pytest

import oracle
from reef_amd import workloads as W

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def reef():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import reef_amd
    reef_amd.lib()
    return reef_amd


def case(msg):
    print(f"\n[case] {msg}", flush=True)


def gpu(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def _problem(B, Hq, Hkv, D, kv_len, q_len, max_ctx, seed, q_gran):
    q = W.lcg_normal(seed, B * Hq * q_len * D).reshape(B, Hq, q_len, D)
    kf = W.lcg_normal(seed + 1, B * Hkv * max_ctx * D).reshape(B, Hkv, max_ctx, D)
    vf = W.lcg_normal(seed + 2, B * Hkv * max_ctx * D).reshape(B, Hkv, max_ctx, D)
    vf[:, :, :, 3] *= 8.0  # an activation-outlier channel
    qq, qs = (oracle.quantize_per_head(q) if q_gran == oracle.GRAN_HEAD
              else oracle.quantize_per_token(q))
    kq, ks = oracle.quantize_per_token(kf)
    vq, vs = oracle.quantize_per_token(vf)
    return qq, qs, kq, ks, vq, vs


def _paged(kq, ks, vq, vs, kv_len, seed):
    """Scatter every sequence's pages into a pool at seeded positions."""
    B, Hkv, Lmax, D = kq.shape
    npg = (kv_len + 15) // 16
    pool = B * npg * 2 + 1
    order = np.argsort(W.lcg_states(seed, pool), kind="stable").astype(np.int32)
    k_pages = np.zeros((pool, Hkv, 16, D), np.int8)
    v_pages = np.zeros((pool, Hkv, D, 16), np.int8)
    ks_pages = np.zeros((pool, Hkv, 16), np.float32)
    vs_pages = np.zeros((pool, Hkv, 16), np.float32)
    table = np.full((B, Lmax // 16), -3, np.int32)
    at = 0
    for b in range(B):
        for i in range(npg):
            pg = order[at]
            at += 1
            table[b, i] = pg
            k_pages[pg] = kq[b, :, 16 * i:16 * i + 16]
            v_pages[pg] = vq[b, :, 16 * i:16 * i + 16].transpose(0, 2, 1)
            ks_pages[pg] = ks[b, :, 16 * i:16 * i + 16]
            vs_pages[pg] = vs[b, :, 16 * i:16 * i + 16]
    return k_pages, v_pages, ks_pages, vs_pages, table


@pytest.mark.parametrize("paged,B,Hq,Hkv,D,kv_len,q_len,window,q_gran", [
    (False, 2, 8, 2, 128, 700, 100, 0, oracle.GRAN_HEAD),
    (False, 1, 4, 4, 64, 96, 96, 24, oracle.GRAN_TOKEN),   # a whole prompt, local layer
    (True, 3, 8, 1, 128, 333, 17, 0, oracle.GRAN_TOKEN),
    (True, 2, 16, 4, 64, 1000, 300, 128, oracle.GRAN_HEAD),
    (True, 1, 8, 1, 128, 4096, 512, 0, oracle.GRAN_HEAD),  # a 512-token turn on a 4k cache
])
def test_prefill_over_cache(reef, paged, B, Hq, Hkv, D, kv_len, q_len, window, q_gran):
    max_ctx = ((kv_len + 63) // 64) * 64
    start = kv_len - q_len
    case(f"prefill over {'paged' if paged else 'contiguous'} cache B{B} Hq{Hq} Hkv{Hkv} D{D} "
         f"kv_len{kv_len} q_len{q_len} win{window}")
    qq, qs, kq, ks, vq, vs = _problem(B, Hq, Hkv, D, kv_len, q_len, max_ctx, 90 + kv_len, q_gran)
    scale = 1 / math.sqrt(D)
    if paged:
        kp, vp, ksp, vsp, table = _paged(kq, ks, vq, vs, kv_len, 7 + B)
        out = reef.attention_prefill_cache(gpu(qq), gpu(qs), gpu(kp), gpu(vp), gpu(ksp), gpu(vsp),
                                           kv_len, block_table=gpu(table), window=window,
                                           softmax_scale=scale, q_granularity=q_gran)
    else:
        v_pages = reef.pack_v_pages(gpu(vq))
        out = reef.attention_prefill_cache(gpu(qq), gpu(qs), gpu(kq), v_pages, gpu(ks), gpu(vs),
                                           kv_len, window=window, softmax_scale=scale,
                                           q_granularity=q_gran)
    out = host(out)
    # the same codes, token-major, through the prefill entry point
    kt, vt = kq[:, :, :kv_len], vq[:, :, :kv_len]
    kst, vst = ks[:, :, :kv_len], vs[:, :, :kv_len]
    direct = host(reef.attention_prefill(gpu(qq), gpu(kt), gpu(vt), gpu(qs), gpu(kst), gpu(vst),
                                         query_start=start, window=window, softmax_scale=scale,
                                         q_granularity=q_gran, kv_granularity=reef.PER_TOKEN))
    assert np.array_equal(out.view(np.uint32), direct.view(np.uint32))
    # the oracle on sampled query rows (one-row problems at query_start + r)
    rows = sorted({0, q_len - 1, q_len // 2, min(q_len - 1, 63), min(q_len - 1, 64)})
    err = 0.0
    for r in rows:
        p = oracle.Problem(B, Hq, Hkv, 1, kv_len, D, query_start=start + r, window=window,
                           softmax_scale=scale, q_granularity=q_gran,
                           kv_granularity=oracle.GRAN_TOKEN)
        qsr = qs if q_gran == oracle.GRAN_HEAD else np.ascontiguousarray(qs[:, :, r:r + 1])
        gold = oracle.attention_int8(p, np.ascontiguousarray(qq[:, :, r:r + 1]), kt, vt, qsr,
                                     kst, vst)
        err = max(err, float(np.abs(out[:, :, r:r + 1] - gold).max()))
    print(f"max_abs_err {err:.3e} over rows {rows}", flush=True)
    assert err <= TOL


def test_chunked_prompt_matches_whole_prompt(reef):
    """A 600-token prompt in three chunks (each chunk's keys appended to the cache
    with kv_append, then its queries over the cache) against the whole prompt in
    one prefill: every row within the tolerance."""
    import torch
    B, Hq, Hkv, D, S = 1, 8, 2, 128, 600
    chunks = [200, 1, 399]
    case(f"chunked prompt {chunks} vs one prefill, B{B} Hq{Hq} Hkv{Hkv} D{D}")
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    qf = torch.randn((B, Hq, S, D), generator=g, device="cuda")
    kf = torch.randn((B, Hkv, S, D), generator=g, device="cuda")
    vf = torch.randn((B, Hkv, S, D), generator=g, device="cuda")
    L = 640
    k_cache = torch.zeros((B, Hkv, L, D), dtype=torch.int8, device="cuda")
    v_cache = torch.zeros((B, Hkv, L // 16, D, 16), dtype=torch.int8, device="cuda")
    k_scales = torch.zeros((B, Hkv, L), device="cuda")
    v_scales = torch.zeros((B, Hkv, L), device="cuda")
    scale = 1 / math.sqrt(D)
    parts = []
    at = 0
    for n in chunks:
        starts = torch.full((B,), at, dtype=torch.int32, device="cuda")
        reef.kv_append(kf[:, :, at:at + n], vf[:, :, at:at + n], starts, k_cache, v_cache,
                       k_scales, v_scales)
        qq, qs = reef.quantize_rows(qf[:, :, at:at + n].reshape(B * Hq * n, D))
        parts.append(reef.attention_prefill_cache(
            qq.reshape(B, Hq, n, D), qs.reshape(B, Hq, n), k_cache, v_cache, k_scales, v_scales,
            at + n, softmax_scale=scale, q_granularity=reef.PER_TOKEN))
        at += n
    chunked = torch.cat(parts, dim=2)
    qq, qs = reef.quantize_rows(qf.reshape(B * Hq * S, D))
    kq, ks = reef.quantize_rows(kf.reshape(B * Hkv * S, D))
    vq, vs = reef.quantize_rows(vf.reshape(B * Hkv * S, D))
    whole = reef.attention_prefill(qq.reshape(B, Hq, S, D), kq.reshape(B, Hkv, S, D),
                                   vq.reshape(B, Hkv, S, D), qs.reshape(B, Hq, S),
                                   ks.reshape(B, Hkv, S), vs.reshape(B, Hkv, S),
                                   softmax_scale=scale, q_granularity=reef.PER_TOKEN,
                                   kv_granularity=reef.PER_TOKEN)
    err = float((chunked - whole).abs().max())
    print(f"max_abs_err {err:.3e}", flush=True)
    assert err <= TOL


def test_prefill_over_cache_flags_bad_page(reef):
    """A block-table entry outside the pool sets BAD_PAGE (InvalidArgument)."""
    B, Hq, Hkv, D, kv_len, q_len = 1, 4, 1, 64, 64, 8
    case("prefill over paged cache with a bad page number")
    qq, qs, kq, ks, vq, vs = _problem(B, Hq, Hkv, D, kv_len, q_len, 64, 3, oracle.GRAN_HEAD)
    kp, vp, ksp, vsp, table = _paged(kq, ks, vq, vs, kv_len, 4)
    table[0, 2] = kp.shape[0] + 5
    with pytest.raises(reef.InvalidArgument):
        reef.attention_prefill_cache(gpu(qq), gpu(qs), gpu(kp), gpu(vp), gpu(ksp), gpu(vsp),
                                     kv_len, block_table=gpu(table), q_granularity=reef.PER_HEAD)
