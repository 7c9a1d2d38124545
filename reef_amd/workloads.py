"""Synthetic workloads of the int8 attention path: seeded inputs and the sizes of
the five benchmark configurations.

Uniform draws use the Reef golden writer's generator (coral/host/gen_golden.cpp:48-86,
the same LCG as weights.hpp:237-247): state = state * 1664525 + 1013904223 (mod
2^32), value = (state >> 8) * 2^-24. It is evaluated here in closed form, state_n =
a^n seed + c (a^(n-1) + ... + 1), so a whole stream is one vectorised pass. Normal
draws pair uniforms by Box-Muller (new here; the engine draws only uniforms).

Small problems are generated on the host with this generator. Full-size problems
(hundreds of millions of values) are drawn on the GPU with torch's seeded
generator; every check of those reads the same device data back.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

LCG_A = np.uint32(1664525)
LCG_C = np.uint32(1013904223)


def lcg_states(seed: int, n: int) -> np.ndarray:
    """The first n states after `seed` (gen_golden.cpp:80-83)."""
    a_pow = np.multiply.accumulate(np.full(n, LCG_A, np.uint32), dtype=np.uint32)  # a^1 .. a^n
    prev = np.empty(n, np.uint32)
    prev[0] = 1
    prev[1:] = a_pow[:-1]                                          # a^0 .. a^(n-1)
    geo = np.cumsum(prev, dtype=np.uint32)                         # 1 + a + .. + a^(k-1)
    with np.errstate(over="ignore"):
        return a_pow * np.uint32(seed) + LCG_C * geo


def lcg_fraction(seed: int, n: int) -> np.ndarray:
    """Uniform float32 in [0, 1): the top 24 bits of each state times 2^-24."""
    return (lcg_states(seed, n) >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)


def lcg_uniform(seed: int, n: int, low: float, high: float) -> np.ndarray:
    """Rng::uniform(low, high): low + (high - low) * fraction, in float32."""
    f = lcg_fraction(seed, n)
    return np.float32(low) + (np.float32(high) - np.float32(low)) * f


def lcg_normal(seed: int, n: int) -> np.ndarray:
    """N(0, 1) float32 by Box-Muller over consecutive uniform pairs."""
    m = (n + 1) // 2
    u = lcg_fraction(seed, 2 * m).astype(np.float64)
    r = np.sqrt(-2.0 * np.log1p(-u[0::2]))  # 1 - u1 lies in (0, 1]
    th = 2.0 * math.pi * u[1::2]
    z = np.empty(2 * m, np.float64)
    z[0::2] = r * np.cos(th)
    z[1::2] = r * np.sin(th)
    return z[:n].astype(np.float32)


@dataclass
class PrefillConfig:
    name: str
    batch: int
    q_heads: int
    kv_heads: int
    seq: int
    head_dim: int
    granularity: int           # 0 per-tensor, 1 per-head
    seed: int
    outlier_fraction: float = 0.0   # fraction of the H*D channels scaled by outlier_gain
    outlier_gain: float = 8.0
    causal: bool = True

    @property
    def softmax_scale(self) -> float:
        return 1.0 / math.sqrt(self.head_dim)

    def visible_pairs(self) -> int:
        return self.batch * self.q_heads * self.seq * (self.seq + 1) // 2

    def algorithmic_ops(self) -> int:
        """4 d per visible (query, key) pair: QK^T and P.V, 2 ops per multiply-add."""
        return 4 * self.head_dim * self.visible_pairs()

    def io_bytes(self) -> int:
        D = self.head_dim
        return (self.batch * (self.q_heads + 2 * self.kv_heads) * self.seq * D   # int8 in
                + self.batch * self.q_heads * self.seq * D * 4)                    # fp32 out


@dataclass
class DecodeConfig:
    name: str
    batch: int
    q_heads: int
    kv_heads: int
    head_dim: int
    context: int               # fixed length, or the maximum of a ragged draw
    min_context: int = 0       # > 0: lengths uniform in [min_context, context]
    paged: bool = False
    seed: int = 0
    pool_slack: float = 1.25   # paged pool holds this many times the pages in use

    def lengths(self) -> np.ndarray:
        if self.min_context <= 0:
            return np.full(self.batch, self.context, np.int32)
        span = self.context - self.min_context + 1
        draws = lcg_states(self.seed + 101, self.batch) >> np.uint32(8)
        return (self.min_context + (draws % np.uint32(span)).astype(np.int64)).astype(np.int32)

    def kv_bytes(self, lengths=None) -> int:
        """Algorithmic bytes of one decode step: every int8 K/V byte and K/V scale of
        the visible keys, q and its scales, the fp32 output, and block-table words."""
        L = self.lengths() if lengths is None else lengths
        tokens = int(np.sum(L)) * self.kv_heads
        D = self.head_dim
        b = tokens * (2 * D + 2 * 4)
        b += self.batch * self.q_heads * D + self.q_heads * 4   # q int8 + per-head scales
        b += self.batch * self.q_heads * D * 4                  # fp32 out
        if self.paged:
            b += 4 * int(np.sum((L + 15) // 16))
        return b


CONFIGS = {
    "prefill_1x1x128x64": PrefillConfig("causal prefill 1x1x128x64, per-tensor", 1, 1, 1, 128, 64, 0, seed=1),
    "prefill_1x32x2048x128": PrefillConfig("causal prefill 1x32x2048x128, per-head", 1, 32, 32, 2048, 128, 1,
                        seed=2),
    "decode_b64_l4096": DecodeConfig("decode B64 32q/8kv L4096 d128, per-token KV", 64, 32, 8, 128, 4096,
                       seed=3),
    "prefill_4x32x8192x128": PrefillConfig("causal prefill 4x32x8192x128, per-head, 1% x8 outliers", 4, 32, 32,
                        8192, 128, 1, seed=4, outlier_fraction=0.01),
    "prefill_1x8x4096x128_gqa": PrefillConfig("causal prefill 1x8q/1kv x4096x128, per-head", 1, 8, 1, 4096, 128, 1,
                         seed=5),
    "decode_paged_b128_ragged": DecodeConfig("ragged paged decode B128 8q/1kv L~U[512,8192] d128, page 16", 128, 8,
                        1, 128, 8192, min_context=512, paged=True, seed=6),
}


def outlier_channels(cfg: PrefillConfig) -> np.ndarray:
    """Seeded choice of round(fraction * H * D) distinct channels of the H*D hidden width."""
    width = cfg.q_heads * cfg.head_dim
    count = int(round(cfg.outlier_fraction * width))
    if count == 0:
        return np.zeros(0, np.int64)
    keys = lcg_states(cfg.seed + 77, width)
    return np.sort(np.argsort(keys, kind="stable")[:count])


def host_prefill_inputs(cfg: PrefillConfig):
    """fp32 q [B, Hq, S, D], k and v [B, Hkv, S, D] from the LCG normal stream."""
    B, Hq, Hkv, S, D = cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.seq, cfg.head_dim
    nq, nk = B * Hq * S * D, B * Hkv * S * D
    z = lcg_normal(cfg.seed, nq + 2 * nk)
    q = z[:nq].reshape(B, Hq, S, D)
    k = z[nq:nq + nk].reshape(B, Hkv, S, D)
    v = z[nq + nk:].reshape(B, Hkv, S, D)
    ch = outlier_channels(cfg)
    for c in ch:
        h, d = divmod(int(c), D)
        q[:, h, :, d] *= cfg.outlier_gain
        if h < Hkv:
            k[:, h, :, d] *= cfg.outlier_gain
            v[:, h, :, d] *= cfg.outlier_gain
    return q, k, v


def device_prefill_inputs(cfg: PrefillConfig, device="cuda"):
    """The same shapes drawn on the GPU with torch's seeded generator."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(cfg.seed)
    B, Hq, Hkv, S, D = cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.seq, cfg.head_dim
    q = torch.randn((B, Hq, S, D), generator=g, device=device, dtype=torch.float32)
    k = torch.randn((B, Hkv, S, D), generator=g, device=device, dtype=torch.float32)
    v = torch.randn((B, Hkv, S, D), generator=g, device=device, dtype=torch.float32)
    ch = outlier_channels(cfg)
    if len(ch):
        for t, heads in ((q, Hq), (k, Hkv), (v, Hkv)):
            hh = torch.as_tensor(ch // D, device=device)
            dd = torch.as_tensor(ch % D, device=device)
            keep = hh < heads
            t[:, hh[keep], :, dd[keep]] *= cfg.outlier_gain
    return q, k, v
