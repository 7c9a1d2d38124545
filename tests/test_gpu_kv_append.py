"""GPU parity of the KV-cache append (Attention::append_kv_cache,
attention.hpp:290-352) on the int8 cache: the codes and scales it writes must be
bit-identical to quantize_rows (quant.hpp:112-133) of the same fp32 rows, in the
layout the decode kernels read, and nothing outside the appended positions may
change. Each case prints its name before touching the GPU."""
import numpy as np
import pytest

import oracle
from reef_amd import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SENTINEL = 0x55


@pytest.fixture(scope="module")
def reef():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import reef_amd
    reef_amd.lib()
    return reef_amd


def case(msg):
    print(f"\n[case] {msg}", flush=True)


def gpu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def empty_cache(B, H, L, D):
    k = np.full((B, H, L, D), SENTINEL, np.int8)
    v = np.full((B, H, L // 16, D, 16), SENTINEL, np.int8)
    ks = np.full((B, H, L), -1.0, np.float32)
    vs = np.full((B, H, L), -1.0, np.float32)
    return k, v, ks, vs


def expect_rows(k, v, ks, vs, b, pos, kf, vf):
    """Write the expected quantized rows kf, vf [H, T, D] at positions pos.. of b."""
    kq, ksc = oracle.quantize_per_token(kf)
    vq, vsc = oracle.quantize_per_token(vf)
    T = kf.shape[1]
    for t in range(T):
        p = pos + t
        k[b, :, p] = kq[:, t]
        v[b, :, p // 16, :, p % 16] = vq[:, t]
        ks[b, :, p] = ksc[:, t]
        vs[b, :, p] = vsc[:, t]


@pytest.mark.parametrize("D", [128, 64])
def test_append_prompt_then_tokens(reef, D):
    case(f"kv_append contiguous D{D}: prompt of 37 tokens, then 3 single tokens")
    B, H, L = 3, 2, 64
    k, v, ks, vs = empty_cache(B, H, L, D)
    dk, dv, dks, dvs = gpu(k), gpu(v), gpu(ks), gpu(vs)
    lens = gpu(np.zeros(B, np.int32))
    steps = [37, 1, 1, 1]
    pos = 0
    for i, T in enumerate(steps):
        kf = W.lcg_normal(100 + i, B * H * T * D).reshape(B, H, T, D)
        vf = W.lcg_normal(200 + i, B * H * T * D).reshape(B, H, T, D)
        kf[:, :, :, 5] *= 8.0  # an outlier channel
        reef.kv_append(gpu(kf), gpu(vf), lens, dk, dv, dks, dvs, context_lens=lens)
        for b in range(B):
            expect_rows(k, v, ks, vs, b, pos, kf[b], vf[b])
        pos += T
        assert np.array_equal(host(lens), np.full(B, pos, np.int32))
    assert np.array_equal(host(dk), k)
    assert np.array_equal(host(dv), v)
    assert np.array_equal(host(dks).view(np.uint32), ks.view(np.uint32))
    assert np.array_equal(host(dvs).view(np.uint32), vs.view(np.uint32))


def test_append_from_projection_layout_and_ragged_starts(reef):
    case("kv_append contiguous: [T, H*D] projection rows, different start per sequence")
    B, H, L, D, T = 2, 4, 48, 128, 5
    k, v, ks, vs = empty_cache(B, H, L, D)
    dk, dv, dks, dvs = gpu(k), gpu(v), gpu(ks), gpu(vs)
    starts = np.array([0, 29], np.int32)
    proj_k = W.lcg_normal(7, B * T * H * D).reshape(B, T, H * D)
    proj_v = W.lcg_normal(8, B * T * H * D).reshape(B, T, H * D)
    # [B, T, H*D] viewed as [B, H, T, D]: strides {T*H*D, D, H*D}
    tk = gpu(proj_k).view(B, T, H, D).permute(0, 2, 1, 3)
    tv = gpu(proj_v).view(B, T, H, D).permute(0, 2, 1, 3)
    reef.kv_append(tk, tv, gpu(starts), dk, dv, dks, dvs)
    for b in range(B):
        kf = proj_k[b].reshape(T, H, D).transpose(1, 0, 2)
        vf = proj_v[b].reshape(T, H, D).transpose(1, 0, 2)
        expect_rows(k, v, ks, vs, b, int(starts[b]), kf, vf)
    assert np.array_equal(host(dk), k)
    assert np.array_equal(host(dv), v)
    assert np.array_equal(host(dks).view(np.uint32), ks.view(np.uint32))


@pytest.mark.parametrize("D,offset", [(128, 0), (128, 1), (64, 1)])
def test_append_ties_and_unaligned_rows(reef, D, offset):
    """Rows whose scale is exactly 1 (largest magnitude 127) with half-integer values:
    x / scale is a tie, so the kernel's reciprocal product lands on the half-integer
    and the wave redoes the row with IEEE divisions (ties to even). offset 1 shifts
    the rows by one float, so they are not 16-byte aligned (scalar loads)."""
    case(f"kv_append ties D{D} offset{offset}")
    B, H, L, T = 2, 2, 48, 20
    k, v, ks, vs = empty_cache(B, H, L, D)
    dk, dv, dks, dvs = gpu(k), gpu(v), gpu(ks), gpu(vs)
    rng = np.random.default_rng(D + offset)
    kf = (rng.integers(-254, 255, (B, H, T, D)) / 2.0).astype(np.float32)
    kf[:, :, :, 0] = 127.0
    vf = W.lcg_normal(9, B * H * T * D).reshape(B, H, T, D)
    vf[:, :, ::2, 3] = -127.0
    vf[:, :, ::2, 4:12] = np.array([2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 126.5, -1.5], np.float32)
    starts = np.array([5, 16], np.int32)

    def shifted(a):
        flat = torch.zeros(a.size + offset, dtype=torch.float32, device="cuda")
        flat[offset:] = torch.from_numpy(a.ravel()).cuda()
        return flat[offset:].view(a.shape)
    reef.kv_append(shifted(kf), shifted(vf), gpu(starts), dk, dv, dks, dvs)
    for b in range(B):
        expect_rows(k, v, ks, vs, b, int(starts[b]), kf[b], vf[b])
    assert np.array_equal(host(dk), k)
    assert np.array_equal(host(dv), v)
    assert np.array_equal(host(dks).view(np.uint32), ks.view(np.uint32))
    assert np.array_equal(host(dvs).view(np.uint32), vs.view(np.uint32))


def test_append_capacity_and_non_finite(reef):
    case("kv_append: capacity exceeded for one sequence; non-finite rows")
    B, H, L, D, T = 2, 1, 32, 64, 4
    k, v, ks, vs = empty_cache(B, H, L, D)
    dk, dv, dks, dvs = gpu(k), gpu(v), gpu(ks), gpu(vs)
    kf = W.lcg_normal(9, B * H * T * D).reshape(B, H, T, D)
    vf = W.lcg_normal(10, B * H * T * D).reshape(B, H, T, D)
    starts = gpu(np.array([2, 30], np.int32))  # sequence 1 would end at 34 > 32
    lens = gpu(np.array([2, 30], np.int32))
    with pytest.raises(reef.CapacityError):
        reef.kv_append(gpu(kf), gpu(vf), starts, dk, dv, dks, dvs, context_lens=lens)
    expect_rows(k, v, ks, vs, 0, 2, kf[0], vf[0])
    assert np.array_equal(host(dk), k)  # sequence 1 untouched
    assert np.array_equal(host(dv), v)
    assert np.array_equal(host(lens), np.array([6, 30], np.int32))
    with pytest.raises(reef.CapacityError):  # longer than the whole cache: host check
        big = gpu(np.zeros((B, H, 40, D), np.float32))
        reef.kv_append(big, big, starts, dk, dv, dks, dvs)
    bad = kf.copy()
    bad[0, 0, 1, 3] = np.nan
    with pytest.raises(reef.NonFiniteInput):
        reef.kv_append(gpu(bad), gpu(vf), gpu(np.array([8, 8], np.int32)), dk, dv, dks, dvs)


@pytest.mark.parametrize("D", [128, 64])
def test_append_paged_then_decode(reef, D):
    case(f"kv_append paged D{D}: ragged starts into a permuted pool, then decode")
    B, Hq, H, T = 3, 8, 1, 3
    max_blocks = 8
    L = max_blocks * 16
    starts = np.array([0, 17, 60], np.int32)
    pool = 40
    order = np.argsort(W.lcg_states(61, pool), kind="stable").astype(np.int32)
    table = order[:B * max_blocks].reshape(B, max_blocks).copy()
    # the sequences' earlier tokens, quantized by the oracle into the pages
    full_k = W.lcg_normal(62, B * H * L * D).reshape(B, H, L, D)
    full_v = W.lcg_normal(63, B * H * L * D).reshape(B, H, L, D)
    kq, ksc = oracle.quantize_per_token(full_k)
    vq, vsc = oracle.quantize_per_token(full_v)
    kp = np.full((pool, H, 16, D), SENTINEL, np.int8)
    vp = np.full((pool, H, D, 16), SENTINEL, np.int8)
    ksp = np.full((pool, H, 16), -1.0, np.float32)
    vsp = np.full((pool, H, 16), -1.0, np.float32)

    def place(b, p):
        pg, s = table[b, p // 16], p % 16
        kp[pg, :, s] = kq[b, :, p]
        vp[pg, :, :, s] = vq[b, :, p]
        ksp[pg, :, s] = ksc[b, :, p]
        vsp[pg, :, s] = vsc[b, :, p]
    for b in range(B):
        for p in range(starts[b]):
            place(b, p)
    dkp, dvp, dksp, dvsp = gpu(kp), gpu(vp), gpu(ksp), gpu(vsp)
    lens = gpu(starts)
    new_k = np.stack([full_k[b, :, starts[b]:starts[b] + T] for b in range(B)])
    new_v = np.stack([full_v[b, :, starts[b]:starts[b] + T] for b in range(B)])
    reef.kv_append_paged(gpu(new_k), gpu(new_v), lens, gpu(table), dkp, dvp, dksp, dvsp,
                         context_lens=lens)
    for b in range(B):
        for p in range(starts[b], starts[b] + T):
            place(b, p)
    assert np.array_equal(host(lens), starts + T)
    assert np.array_equal(host(dkp), kp)
    assert np.array_equal(host(dvp), vp)
    assert np.array_equal(host(dksp).view(np.uint32), ksp.view(np.uint32))
    assert np.array_equal(host(dvsp).view(np.uint32), vsp.view(np.uint32))
    # decode over the appended cache equals decode over the oracle-built one
    q = W.lcg_normal(64, B * Hq * D).reshape(B * Hq, D)
    qq, qs = oracle.quantize_rows(q)
    args = (gpu(qq.reshape(B, Hq, D)), gpu(qs.reshape(B, Hq)))
    out_a = reef.attention_decode_paged(*args, dkp, dvp, dksp, dvsp, gpu(table), lens)
    out_b = reef.attention_decode_paged(*args, gpu(kp), gpu(vp), gpu(ksp), gpu(vsp), gpu(table),
                                        lens)
    assert np.array_equal(host(out_a), host(out_b))
