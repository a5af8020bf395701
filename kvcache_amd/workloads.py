"""Workload generators for the decode benchmarks.

Reference generators (bit-exact restatements, uint32 LCG s = s*1103515245 + 12345,
r = (s >> 9) / 2^23 in float32):
  * ref_lengths  -- bench_throughput.cu:50-57, L = 16 + (int)((LMAX-16)*r*r), seed 12345
  * ref_trace    -- bench_continuous.cu:38-50, prompt 16+(int)(240*rp*rp),
                    gen 8+(int)(504*rg*rg), Poisson gaps -log(u)/rate*1e6 drawn only
                    when rate > 0 (so the online trace differs from the offline one)
  * hval         -- bench_throughput.cu:21-25 deterministic K/V values in [-1, 1)
  * shuffle_perm -- main_paged.cu:28-37 seeded block-table shuffle
BASELINE distributions (seeded numpy PCG64; no reference counterpart):
  * loguniform_lengths -- lengths log-uniform in [lo, hi]
  * baseline_trace     -- prompts uniform [1, 256], generation geometric (mean
                          190) capped at 512, arrivals offline or Poisson.
"""
from __future__ import annotations

import math

import numpy as np

_A = 1103515245
_C = 12345
_M = 0xFFFFFFFF


def _lcg01(seed: int) -> tuple[int, np.float32]:
    seed = (seed * _A + _C) & _M
    return seed, np.float32(seed >> 9) / np.float32(8388608.0)


def ref_lengths(n: int = 128, lmax: int = 2048, seed: int = 12345) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    s = seed
    span = np.float32(lmax - 16)
    for i in range(n):
        s, r = _lcg01(s)
        out[i] = 16 + int(span * r * r)
    return out


def ref_trace(nreq: int = 256, prompt_max: int = 256, gen_max: int = 512, rate: float = 0.0,
              seed: int = 2024) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    prompt = np.empty(nreq, dtype=np.int32)
    gen = np.empty(nreq, dtype=np.int32)
    arrival = np.zeros(nreq, dtype=np.float64)
    s = seed
    t = 0.0
    ps, gs = np.float32(prompt_max - 16), np.float32(gen_max - 8)
    for i in range(nreq):
        s, rp = _lcg01(s)
        s, rg = _lcg01(s)
        prompt[i] = 16 + int(ps * rp * rp)
        gen[i] = 8 + int(gs * rg * rg)
        if rate > 0:
            s, u = _lcg01(s)
            u = float(u)
            if u < 1e-9:
                u = 1e-9
            t += -math.log(u) / rate * 1e6
            arrival[i] = t
    return prompt, gen, arrival


def hval(s, h, pos, d, salt) -> np.ndarray:
    """Vectorised bench_throughput.cu:21-25 (uint32 arithmetic)."""
    u = np.uint64
    x = ((((u(s) * u(131) + u(h)) * u(131) + u(pos)) * u(131) + u(d)) + u(salt) * u(2654435761)) & u(_M)
    x = x ^ (x >> u(13))
    x = (x * u(0x9E3779B1)) & u(_M)
    x = x ^ (x >> u(16))
    return (np.asarray(x >> u(9)).astype(np.float32) / np.float32(8388608.0)) * np.float32(2.0) - np.float32(1.0)


def shuffle_perm(nb: int, seed: int = 42) -> np.ndarray:
    perm = list(range(nb))
    s = seed
    for i in range(nb - 1, 0, -1):
        s = (s * _A + _C) & _M
        j = s % (i + 1)
        perm[i], perm[j] = perm[j], perm[i]
    return np.asarray(perm, dtype=np.int32)


def loguniform_lengths(n: int = 128, lo: int = 16, hi: int = 2048, seed: int = 7) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = np.exp(rng.uniform(math.log(lo), math.log(hi + 1), size=n))
    return np.clip(np.floor(x), lo, hi).astype(np.int32)


def baseline_trace(nreq: int = 256, rate: float = 0.0, seed: int = 11, prompt_max: int = 256,
                   gen_mean: float = 190.0, gen_cap: int = 512) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    rng = np.random.default_rng(seed)
    prompt = rng.integers(1, prompt_max + 1, size=nreq).astype(np.int32)
    gen = np.minimum(rng.geometric(1.0 / gen_mean, size=nreq), gen_cap).astype(np.int32)
    if rate > 0:
        arrival = np.cumsum(rng.exponential(1e6 / rate, size=nreq))
    else:
        arrival = np.zeros(nreq)
    return prompt, gen, arrival.astype(np.float64)


def build_tables(lengths, block: int, allocator) -> tuple[np.ndarray, np.ndarray]:
    """Concatenated block tables + offsets, blocks taken from `allocator` in order
    (bench_throughput.cu:62-71 layout)."""
    tab_off = np.zeros(len(lengths) + 1, dtype=np.int32)
    table = []
    for s, L in enumerate(lengths):
        tab_off[s] = len(table)
        for _ in range((int(L) + block - 1) // block):
            b = allocator.alloc()
            if b < 0:
                raise RuntimeError("pool exhausted while building tables")
            table.append(b)
    tab_off[len(lengths)] = len(table)
    return np.asarray(table, dtype=np.int32), tab_off
