"""The allocation-free paged decode (reef_attention_decode_int8_paged_noalloc)
against the paged decode with a caller workspace: bit-identical outputs on two
calls in a row (the second smaller, so the scratch array holds the first call's
counters and slots when it starts), both with sequences whose keys are dealt out
over several workgroups so that the part slots and counters in the scratch array
are used."""
import ctypes as C
import math

import numpy as np
import pytest

from reef_amd import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def reef():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import reef_amd
    lib = reef_amd.lib()
    fn = lib.reef_attention_decode_int8_paged_noalloc
    P = C.c_void_p
    fn.argtypes = [C.POINTER(reef_amd.DecodeParams), P, P, P, P, P, P, P, C.c_int64, C.c_int64, P,
                   P, P, P]
    fn.restype = C.c_int
    return reef_amd


def _problem(seed, B, Hq, Hkv, D, lens, pool_slack=1.3):
    """Random int8 paged cache with per-token scales, q per head."""
    rng = np.random.default_rng(seed)
    npages = [(L + 15) // 16 for L in lens]
    pool = int(sum(npages) * pool_slack) + 1
    max_blocks = max(npages)
    kp = rng.integers(-127, 128, (pool, Hkv, 16, D), dtype=np.int8)
    vp = rng.integers(-127, 128, (pool, Hkv, D, 16), dtype=np.int8)
    ksp = rng.uniform(0.005, 0.04, (pool, Hkv, 16)).astype(np.float32)
    vsp = rng.uniform(0.005, 0.04, (pool, Hkv, 16)).astype(np.float32)
    order = rng.permutation(pool).astype(np.int32)
    table = np.zeros((B, max_blocks), np.int32)
    at = 0
    for b, n in enumerate(npages):
        table[b, :n] = order[at:at + n]
        at += n
    q = rng.integers(-127, 128, (B, Hq, D), dtype=np.int8)
    qs = rng.uniform(0.01, 0.05, Hq).astype(np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    return dict(q=t(q), qs=t(qs), kp=t(kp), vp=t(vp), ksp=t(ksp), vsp=t(vsp), table=t(table),
                lens=t(np.array(lens, np.int32)), max_blocks=max_blocks, pool=pool)


def _run(reef, x, B, Hq, Hkv, D, noalloc, num_splits=0):
    lib = reef.lib()
    p = reef.DecodeParams(B, Hq, Hkv, D, x["max_blocks"] * 16, 0, 1 / math.sqrt(D), reef.PER_HEAD,
                          num_splits, 0)
    out = torch.full((B, Hq, D), float("nan"), device="cuda")
    status = reef.StatusWord()
    ptr = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    common = (C.byref(p), ptr(x["q"]), ptr(x["qs"]), ptr(x["kp"]), ptr(x["vp"]), ptr(x["ksp"]),
              ptr(x["vsp"]), ptr(x["table"]), x["max_blocks"], x["pool"], ptr(x["lens"]),
              ptr(out))
    if noalloc:
        rc = lib.reef_attention_decode_int8_paged_noalloc(*common, status.ptr, stream)
    else:
        n = lib.reef_attention_decode_workspace_bytes(C.byref(p))
        ws = torch.zeros(max(n, 256) // 4, dtype=torch.int32, device="cuda")
        rc = lib.reef_attention_decode_int8_paged(*common, ptr(ws), ws.numel() * 4, status.ptr,
                                                  stream)
    assert rc == reef.OK, rc
    status.check("decode paged")
    torch.cuda.synchronize()
    return out.cpu().numpy(), p


def test_noalloc_matches_workspace_entry_point_on_two_calls(reef):
    D = 128
    # first call: 40 sequences x 2 kv heads, lengths up to 1500 (their 64-key blocks
    # dealt out over 120 workgroups: the long sequences merge through the scratch slots)
    lens1 = [int(x) for x in np.random.default_rng(1).integers(1, 1500, 40)]
    lens1[0], lens1[-1] = 1500, 1
    x1 = _problem(11, 40, 8, 2, D, lens1)
    print("\n[case] noalloc decode call 1: B40 8q/2kv", flush=True)
    a1, p1 = _run(reef, x1, 40, 8, 2, D, noalloc=True)
    r1, _ = _run(reef, x1, 40, 8, 2, D, noalloc=False)
    # part slots beyond the 80 counters: the merge goes through the scratch array
    assert reef.lib().reef_attention_decode_workspace_bytes(C.byref(p1)) > 80 * 2 * 17 * 64 * 8
    assert np.isfinite(a1).all()
    assert np.array_equal(a1.view(np.uint32), r1.view(np.uint32))
    # second call, smaller: 7 sequences, 1 kv head, num_splits 9 (16 workgroups)
    lens2 = [900, 17, 1024, 3, 640, 511, 1000]
    x2 = _problem(12, 7, 8, 1, D, lens2)
    print("[case] noalloc decode call 2: B7 8q/1kv, 9 splits", flush=True)
    a2, _ = _run(reef, x2, 7, 8, 1, D, noalloc=True, num_splits=9)
    r2, _ = _run(reef, x2, 7, 8, 1, D, noalloc=False, num_splits=9)
    assert np.isfinite(a2).all()
    assert np.array_equal(a2.view(np.uint32), r2.view(np.uint32))
    # and the first shape again after the smaller one
    a3, _ = _run(reef, x1, 40, 8, 2, D, noalloc=True)
    assert np.array_equal(a3.view(np.uint32), r1.view(np.uint32))


def test_noalloc_rejects_workspace_beyond_scratch(reef):
    """A shape whose split-merge workspace exceeds the 16 MiB scratch array is
    refused before any launch."""
    lib = reef.lib()
    p = reef.DecodeParams(2048, 8, 1, 128, 8192, 0, 0.1, reef.PER_HEAD, 64, 0)
    assert lib.reef_attention_decode_workspace_bytes(C.byref(p)) > 16 << 20
    f = lambda n: C.c_void_p(0x10000 * n)  # noqa: E731
    rc = lib.reef_attention_decode_int8_paged_noalloc(C.byref(p), f(1), f(2), f(3), f(4), f(5), f(6),
                                                      f(7), 512, 100, f(8), f(9), None, None)
    assert rc == reef.UNSUPPORTED
