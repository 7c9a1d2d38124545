"""GPU parity of the W8A8 projection (linear() with a QuantizedWeight,
operator/linear.hpp:106-132): outputs bit-identical to the engine's golden
vectors and to the oracle's restatement (quantize_rows, exact int32 sums,
float(sum) * (s_row * s_col) + bias in float32, one rounding per step). Each
case prints its name before touching the GPU."""
import json
import os

import numpy as np
import pytest

import oracle

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


def f32(bits):
    return np.array(bits, np.uint32).view(np.float32)


def oracle_linear(x, w, ws, bias=None):
    q, s = oracle.quantize_rows(x)
    acc = q.astype(np.int64) @ w.astype(np.int64).T
    y = acc.astype(np.float32) * (s[:, None] * ws[None, :])
    if bias is not None:
        y = y + bias[None, :]
    return y.astype(np.float32)


def test_linear_engine_golden(reef):
    for c in json.load(open(os.path.join(GOLDEN, "w8a8_linear.json")))["cases"]:
        rows, fin, fout = c["rows"], c["in_features"], c["out_features"]
        case(f"w8a8 golden rows{rows} in{fin} out{fout}")
        x = f32(c["x_bits"]).reshape(rows, fin)
        w = np.array(c["wt"], np.int8).reshape(fin, fout).T
        ws = f32(c["w_scale_bits"])
        # zero input features change neither a row's scale nor any sum
        pad = (-fin) % 16
        xp = np.pad(x, ((0, 0), (0, pad)))
        wp = np.pad(w, ((0, 0), (0, pad)))
        y = host(reef.linear_w8a8(gpu(xp), gpu(wp), gpu(ws)))
        assert np.array_equal(y.view(np.uint32), f32(c["y_bits"]).reshape(rows, fout).view(np.uint32))


@pytest.mark.parametrize("rows,fin,fout,bias", [
    (1, 64, 48, False), (37, 160, 129, True), (300, 1024, 1000, True), (129, 4096, 256, False),
])
def test_linear_matches_oracle(reef, rows, fin, fout, bias):
    case(f"w8a8 rows{rows} in{fin} out{fout} bias{bias}")
    rng = np.random.default_rng(rows + fin + fout)
    x = rng.standard_normal((rows, fin)).astype(np.float32)
    x[:, 3] *= 20.0  # an outlier feature
    w = rng.integers(-127, 128, (fout, fin), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, fout).astype(np.float32)
    b = rng.standard_normal(fout).astype(np.float32) if bias else None
    y = host(reef.linear_w8a8(gpu(x), gpu(w), gpu(ws), gpu(b) if bias else None))
    gold = oracle_linear(x, w, ws, b)
    assert np.array_equal(y.view(np.uint32), gold.view(np.uint32))


def test_linear_errors(reef):
    case("w8a8 errors: non-finite input, overflowing output, unsupported width")
    x = np.ones((4, 32), np.float32)
    w = np.ones((8, 32), np.int8)
    ws = np.ones(8, np.float32)
    bad = x.copy()
    bad[2, 5] = np.inf
    with pytest.raises(reef.NonFiniteInput):
        reef.linear_w8a8(gpu(bad), gpu(w), gpu(ws))
    with pytest.raises(reef.Overflow):
        reef.linear_w8a8(gpu(x), gpu(w), gpu(np.full(8, 3e38, np.float32)))
    with pytest.raises(reef.Unsupported):
        reef.linear_w8a8(gpu(np.ones((4, 30), np.float32)), gpu(np.ones((8, 30), np.int8)), gpu(ws))
    y = host(reef.linear_w8a8(gpu(x), gpu(w), gpu(ws)))  # the status word is clean again
    assert np.all(np.isfinite(y))


@pytest.mark.parametrize("rows,fout", [(2000, 2500), (2000, 2980)])
@pytest.mark.parametrize("quadrants", ["1", "0"])
def test_linear_quadrant_tiles(reef, rows, fout, quadrants, monkeypatch):
    """2000 x 256 -> 2500: 16 x 20 = 320 output tiles of 128 x 128, a quarter more
    than the 256 compute units, so the tiles past the first 256 run as four 64 x 64
    quadrants each; -> 2980: 16 x 24 = 384 tiles, cut into two 128 x 64 halves. The
    pieces include the ragged last row and column of tiles. Bit-exact against the
    oracle with the pieces and with whole tiles only."""
    monkeypatch.setenv("REEF_GEMM_QUADRANTS", quadrants)
    fin = 256
    case(f"w8a8 rows{rows} in{fin} out{fout} pieces={quadrants}")
    rng = np.random.default_rng(77 + fout)
    x = rng.standard_normal((rows, fin)).astype(np.float32)
    w = rng.integers(-127, 128, (fout, fin), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, fout).astype(np.float32)
    b = rng.standard_normal(fout).astype(np.float32)
    y = host(reef.linear_w8a8(gpu(x), gpu(w), gpu(ws), gpu(b)))
    gold = oracle_linear(x, w, ws, b)
    assert np.array_equal(y.view(np.uint32), gold.view(np.uint32))
