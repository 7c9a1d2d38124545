"""The CPU-baseline helpers of bench.py, on the oracle restatement (no GPU).

The sample's ops count must be the algorithmic work of exactly the rows it ran:
checked against a brute-force count of the visible pairs of a causal mask."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
import oracle  # noqa: E402
from reef_amd import workloads as W  # noqa: E402


def test_causal_pairs_brute_force():
    for S in (1, 7, 64, 130):
        vis = np.tril(np.ones((S, S), dtype=np.int64))
        for r0, rows in ((0, S), (0, 1), (S - 1, 1), (S // 3, S - S // 3), (S // 2, S // 4 or 1)):
            assert bench.causal_pairs(r0, rows) == int(vis[r0:r0 + rows].sum())


@pytest.fixture(scope="module")
def small_host():
    cfg = W.CONFIGS["prefill_1x1x128x64"]
    qf, kf, vf = W.host_prefill_inputs(cfg)
    q, qs = oracle.quantize_per_tensor(qf)
    k, ks = oracle.quantize_per_tensor(kf)
    v, vs = oracle.quantize_per_tensor(vf)
    one = lambda s: np.full(cfg.q_heads, np.float32(s[0]), np.float32)  # noqa: E731
    return cfg, (q, k, v, one(qs), one(ks), one(vs))


def test_prefill_rows_match_whole_head(small_host):
    """Rows run in slices through the sample path give the whole head's ops."""
    cfg, host = small_host
    S = cfg.seq
    total = sum(bench.cpu_prefill_rows(oracle, "port", cfg, host, 0, 0, r0, 32)
                for r0 in range(0, S, 32))
    assert total == 4 * cfg.head_dim * S * (S + 1) // 2 == cfg.algorithmic_ops()


def test_prefill_sample_record(small_host):
    cfg, host = small_host
    rec = bench.cpu_prefill_sample(oracle, "port", cfg, host, 2, 0.05)
    assert rec["cores"] == 2 and rec["kind"] == "port" and rec["value"] > 0
    assert rec["single_thread"]["cores"] == 1 and rec["single_thread"]["value"] > 0
    assert rec["seconds_full_workload_extrapolated"] > 0


def test_run_jobs_threads():
    total, t = bench.run_jobs([lambda i=i: i for i in range(10)], 3)
    assert total == 45 and t >= 0
