"""Workload generators for the decode benchmarks.

Reference generators (bit-exact restatements, uint32 LCG s = s*1103515245 + 12345,
r = (s >> 9) / 2^23 in float32):
  * ref_lengths  -- bench_throughput.cu:50-57, L = 16 + (int)((LMAX-16)*r*r), seed 12345
  * ref_trace    -- bench_continuous.cu:38-50, prompt 16+(int)(240*rp*rp),
                    gen 8+(int)(504*rg*rg), Poisson gaps -log(u)/rate*1e6 drawn only
                    when rate > 0 (so the online trace differs from the offline one)
  * fill_rand    -- bench_paged.cu:19-24, values 2r - 1 in [-1, 1) from the same LCG
  * hval         -- bench_throughput.cu:21-25 deterministic K/V values in [-1, 1)
  * shuffle_perm -- main_paged.cu:28-37 seeded block-table shuffle
  * demo_trace   -- demo_engine.cu:18-28, prompt 8 + rand() % 120 then gen
                    16 + rand() % 200 after srand(123), with glibc's rand()
                    (GlibcRand: the TYPE_3 additive feedback generator)
These are input generators: every parity check holds for whatever inputs they
produce (outputs are compared with the CPU oracle on the same inputs).
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


def fill_rand(n: int, seed: int) -> np.ndarray:
    """bench_paged.cu:19-24: x = r * 2 - 1 per element, r from the LCG above (float32)."""
    out = np.empty(n, dtype=np.float32)
    s = seed
    for i in range(n):
        s, r = _lcg01(s)
        out[i] = r * np.float32(2.0) - np.float32(1.0)
    return out


class GlibcRand:
    """glibc's rand() (random() with the default 128-byte TYPE_3 state): an additive
    lagged-Fibonacci generator r[i] = r[i-3] + r[i-31] (mod 2^32) seeded through the
    Park-Miller recurrence r[i] = 16807 r[i-1] mod (2^31 - 1) for i < 31, r[i] =
    r[i-31] for 31 <= i < 34, with the first 310 outputs discarded; rand() returns
    r[i] >> 1.  (Published description of glibc's random_r.c; demo_engine.cu draws
    its trace with srand/rand.)"""

    def __init__(self, seed: int = 1):
        seed &= _M
        if seed == 0:
            seed = 1
        r = [0] * 34
        r[0] = seed
        for i in range(1, 31):
            hi, lo = divmod(r[i - 1] if r[i - 1] < 2**31 else r[i - 1] - 2**32, 127773)
            # C division truncates toward zero
            if r[i - 1] >= 2**31 and lo != 0:
                hi, lo = hi + 1, lo - 127773
            word = 16807 * lo - 2836 * hi
            if word < 0:
                word += 2147483647
            r[i] = word & _M
        for i in range(31, 34):
            r[i] = r[i - 31]
        self._r = r
        for _ in range(310):
            self._next()

    def _next(self) -> int:
        r = self._r
        v = (r[-3] + r[-31]) & _M
        r.append(v)
        del r[0]
        return v

    def rand(self) -> int:
        return self._next() >> 1


def demo_trace(nreq: int = 256, seed: int = 123) -> tuple[np.ndarray, np.ndarray]:
    """demo_engine.cu:18-28: srand(seed); per request prompt = 8 + rand() % 120,
    then gen = 16 + rand() % 200."""
    g = GlibcRand(seed)
    prompt = np.empty(nreq, dtype=np.int32)
    gen = np.empty(nreq, dtype=np.int32)
    for i in range(nreq):
        prompt[i] = 8 + g.rand() % 120
        gen[i] = 16 + g.rand() % 200
    return prompt, gen


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
