"""GPU parity of the integer-only attention (attend_head_int8, int8.hpp:250-279):
bit-identical int8 outputs against the engine's golden vectors and the oracle's
restatement, over causal and windowed masks, grouped heads and head sizes. Each
case prints its name before touching the GPU."""
import json
import os

import numpy as np
import pytest

import oracle
from reef_amd import workloads as W

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


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


def table_gpu(step=1.0 / 16.0):
    return gpu(oracle.exp_table(step).view(np.int16))


def test_integer_head_engine_golden(reef):
    cases = json.load(open(os.path.join(GOLDEN, "int8_attention.json")))["cases"]
    for c in cases:
        sq, sk, d = c["query_len"], c["key_len"], c["head_dim"]
        case(f"integer head golden sq{sq} sk{sk} d{d} start{c['query_start']} win{c['window']}")
        dp = 32 if d <= 32 else (64 if d <= 64 else 128)  # zero channels change no score
        pad = lambda a, rows: np.pad(np.array(a, np.int8).reshape(rows, d),  # noqa: E731
                                     ((0, 0), (0, dp - d)))[None, None]
        out = reef.attention_int8_integer(gpu(pad(c["q"], sq)), gpu(pad(c["k"], sk)),
                                          gpu(pad(c["v"], sk)), table_gpu(),
                                          score_shift=c["score_shift"],
                                          out_shift=c["out_shift"],
                                          query_start=c["query_start"], window=c["window"])
        got = host(out)[0, 0, :, :d].reshape(-1)
        assert got.tolist() == c["y"]


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D,start,window,score_shift,out_shift", [
    (1, 2, 2, 200, 200, 128, None, 0, 10, 8),
    (2, 4, 1, 130, 333, 64, None, 0, 9, 8),     # GQA 4:1, decode-like offset
    (1, 2, 1, 96, 500, 128, 100, 70, 11, 8),    # explicit start and window
    (1, 1, 1, 1, 1, 32, None, 0, 6, 8),         # a single token
    (1, 3, 3, 257, 257, 32, None, 33, 8, 7),    # window, odd out_shift
])
def test_integer_head_matches_oracle(reef, B, Hq, Hkv, Sq, Skv, D, start, window, score_shift,
                                     out_shift):
    case(f"integer head B{B} Hq{Hq} Hkv{Hkv} Sq{Sq} Skv{Skv} D{D} start{start} win{window}")
    rng = np.random.default_rng(B * 31 + Sq + Skv + D)
    q = rng.integers(-127, 128, (B, Hq, Sq, D), dtype=np.int8)
    k = rng.integers(-127, 128, (B, Hkv, Skv, D), dtype=np.int8)
    v = rng.integers(-127, 128, (B, Hkv, Skv, D), dtype=np.int8)
    qs = Skv - Sq if start is None else start
    out = host(reef.attention_int8_integer(gpu(q), gpu(k), gpu(v), table_gpu(),
                                           score_shift=score_shift, out_shift=out_shift,
                                           query_start=start, window=window))
    group = Hq // Hkv
    for b in range(B):
        for h in range(Hq):
            gold = oracle.attend_head_int8(q[b, h], k[b, h // group], v[b, h // group], qs,
                                           window, score_shift, out_shift)
            assert np.array_equal(out[b, h], gold), (b, h)


def test_integer_head_long_sequence(reef):
    case("integer head 1x1x2048x128 causal, quantized normal data")
    S, D = 2048, 128
    x = [W.lcg_normal(70 + i, S * D).reshape(1, 1, S, D) for i in range(3)]
    q, k, v = (oracle.quantize_per_tensor(t)[0] for t in x)
    out = host(reef.attention_int8_integer(gpu(q), gpu(k), gpu(v), table_gpu(),
                                           score_shift=10, out_shift=8))
    gold = oracle.attend_head_int8(q[0, 0], k[0, 0], v[0, 0], 0, 0, 10, 8)
    assert np.array_equal(out[0, 0], gold)


def test_integer_head_random_shapes(reef):
    """Twelve seeded shapes: query offsets, windows that start mid-tile, GQA, head
    dims 32/64/128, lengths that are not multiples of the 64-key tile (staged K and
    V tiles partly past kv_len, waves with no rows). Bit-exact against the oracle."""
    rng = np.random.default_rng(2024)
    for i in range(12):
        D = int(rng.choice([32, 64, 128]))
        Hkv = int(rng.integers(1, 3))
        Hq = Hkv * int(rng.choice([1, 2, 4]))
        Sq = int(rng.integers(1, 300))
        Skv = Sq + int(rng.integers(0, 200))
        start = Skv - Sq if rng.random() < 0.5 else int(rng.integers(0, Skv - Sq + 1))
        window = 0 if rng.random() < 0.5 else int(rng.integers(1, 150))
        shift = int(rng.integers(6, 12))
        case(f"integer head random {i}: Hq{Hq} Hkv{Hkv} Sq{Sq} Skv{Skv} D{D} start{start} "
             f"win{window} shift{shift}")
        q = rng.integers(-127, 128, (1, Hq, Sq, D), dtype=np.int8)
        k = rng.integers(-127, 128, (1, Hkv, Skv, D), dtype=np.int8)
        v = rng.integers(-127, 128, (1, Hkv, Skv, D), dtype=np.int8)
        out = host(reef.attention_int8_integer(gpu(q), gpu(k), gpu(v), table_gpu(),
                                               score_shift=shift, out_shift=8,
                                               query_start=start, window=window))
        group = Hq // Hkv
        for h in range(Hq):
            gold = oracle.attend_head_int8(q[0, h], k[0, h // group], v[0, h // group], start,
                                           window, shift, 8)
            assert np.array_equal(out[0, h], gold), (i, h)
