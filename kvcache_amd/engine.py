"""Python handles over the C++ serving loop (include/kvc/engine.h, scheduler.h,
block_alloc.h) through the C ABI.

Mirrors the reference's host API (src/include/engine.h:24-149,
src/include/scheduler.h:24-89, src/include/block_alloc.h:10-43): BlockAllocator
{alloc, free_blocks, reset, free_count, used_count}, Engine {add_request, step,
run, reset} and run_static(reqs, engine, max_batch).  The decisions are made by
the same C++ code a C++ caller compiles.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from ._native import KVC_F32, EngineConfigC, EngineStatsC, RequestC, check, lib


class BlockAllocator:
    def __init__(self, total_blocks: int):
        h = C.c_void_p()
        check(lib().kvc_block_allocator_create(total_blocks, C.byref(h)))
        self._h = h.value
        self.total_blocks = total_blocks

    def alloc(self) -> int:
        return lib().kvc_block_allocator_alloc(self._h)

    def free_blocks(self, blocks) -> None:
        a = np.ascontiguousarray(np.asarray(blocks, dtype=np.int32))
        lib().kvc_block_allocator_free(self._h, a.ctypes.data, int(a.size))

    def reset(self) -> None:
        lib().kvc_block_allocator_reset(self._h)

    def shuffle(self, seed: int) -> None:
        lib().kvc_block_allocator_shuffle(self._h, seed)

    def free_count(self) -> int:
        return lib().kvc_block_allocator_free_count(self._h)

    def used_count(self) -> int:
        return lib().kvc_block_allocator_used_count(self._h)

    def __del__(self):
        try:
            if self._h:
                lib().kvc_block_allocator_destroy(self._h)
                self._h = None
        except Exception:
            pass


def blocks_needed(seq_len: int, block: int) -> int:
    return lib().kvc_blocks_needed(seq_len, block)


@dataclass
class EngineConfig:
    n_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    max_batch: int
    n_kv_heads: int = 0
    n_layers: int = 1
    dtype: int = KVC_F32
    kv_write: bool = False
    clock_mode: int = 0          # 0 measured GPU step time, 1 virtual c0 + c1*N + c2*sum(len)
    virt_c0: float = 0.0
    virt_c1: float = 0.0
    virt_c2: float = 0.0
    device: bool = True
    split_tokens: int = 0
    decode_path: int = 0         # 0 host-planned decode, 1 device-lengths path with split_tokens
    prefill: bool = False        # admitted prompts run K/V writes + causal attention (measured clock)
    seed: int = 0
    graph: bool = False          # planned decode steps replay one captured HIP graph

    def to_c(self) -> EngineConfigC:
        return EngineConfigC(self.n_heads, self.n_kv_heads, self.head_dim, self.block_size, self.num_blocks,
                             self.max_batch, self.n_layers, self.dtype, int(self.kv_write), self.clock_mode,
                             self.virt_c0, self.virt_c1, self.virt_c2, int(self.device), self.split_tokens,
                             self.decode_path, int(self.prefill), self.seed, int(self.graph))


@dataclass
class EngineStats:
    name: str = ""
    iters: int = 0
    tokens: int = 0
    gpu_us: float = 0.0
    wall_us: float = 0.0
    slot_steps: int = 0
    useful_steps: int = 0
    peak_blocks: int = 0
    finished: int = 0
    avg_latency_us: float = 0.0
    p50_latency_us: float = 0.0
    p99_latency_us: float = 0.0
    step_digest: int = 0
    host_wall_us: float = 0.0
    prefill_us: float = 0.0
    extra: dict = field(default_factory=dict)

    @classmethod
    def from_c(cls, name: str, s: EngineStatsC) -> "EngineStats":
        return cls(name, s.iters, s.tokens, s.gpu_us, s.wall_us, s.slot_steps, s.useful_steps, s.peak_blocks,
                   s.finished, s.avg_latency_us, s.p50_latency_us, s.p99_latency_us, s.step_digest,
                   s.host_wall_us, s.prefill_us)

    @property
    def slot_util(self) -> float:
        return self.useful_steps / self.slot_steps if self.slot_steps else 0.0

    @property
    def avg_batch(self) -> float:
        return self.slot_steps / self.iters if self.iters else 0.0


class Engine:
    def __init__(self, cfg: EngineConfig):
        self.cfg = cfg
        h = C.c_void_p()
        c = cfg.to_c()
        check(lib().kvc_engine_create(C.byref(c), C.byref(h)))
        self._h = h.value

    def add_request(self, prompt_len: int, max_new_tokens: int, arrival_us: float = 0.0) -> None:
        check(lib().kvc_engine_add_request(self._h, int(prompt_len), int(max_new_tokens), float(arrival_us)))

    def step(self) -> bool:
        more = C.c_int(0)
        check(lib().kvc_engine_step(self._h, C.byref(more)))
        return bool(more.value)

    def run(self) -> EngineStats:
        s = EngineStatsC()
        check(lib().kvc_engine_run(self._h, C.byref(s)))
        return EngineStats.from_c("continuous", s)

    def last_step(self) -> dict:
        """The last decode step's batch (kvc_engine_last_step): lens, tab_off, table, wpos,
        slots (host arrays) and the device addresses of the runner's q / new K / new V /
        out buffers and of the K / V pools."""
        import numpy as np
        n = C.c_int(0)
        cap = 1 << 16
        lens, off = np.zeros(cap, np.int32), np.zeros(cap + 1, np.int32)
        table, wpos, slots = np.zeros(cap, np.int32), np.zeros(cap, np.int32), np.zeros(cap, np.int32)
        dev = (C.c_void_p * 6)()
        check(lib().kvc_engine_last_step(self._h, C.byref(n), lens.ctypes.data_as(C.POINTER(C.c_int)),
                                         off.ctypes.data_as(C.POINTER(C.c_int)),
                                         table.ctypes.data_as(C.POINTER(C.c_int)), cap,
                                         wpos.ctypes.data_as(C.POINTER(C.c_int)),
                                         slots.ctypes.data_as(C.POINTER(C.c_int)), dev))
        m = n.value
        T = int(off[m]) if m else 0
        return {"n": m, "lens": lens[:m].copy(), "tab_off": off[:m + 1].copy(), "table": table[:T].copy(),
                "wpos": wpos[:m].copy(), "slots": slots[:m].copy(),
                "dev": {k: dev[i] for i, k in enumerate(["q", "k_new", "v_new", "out", "k_pool", "v_pool"])}}

    def stats(self) -> EngineStats:
        s = EngineStatsC()
        check(lib().kvc_engine_stats_get(self._h, C.byref(s)))
        return EngineStats.from_c("continuous", s)

    def reset(self) -> None:
        check(lib().kvc_engine_reset(self._h))

    def close(self) -> None:
        if self._h:
            lib().kvc_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def run_static(prompt, gen, arrival, engine: Engine, max_batch: int) -> EngineStats:
    """Static batching (scheduler.h:33-89) over the engine's pool and runner."""
    n = len(prompt)
    arr = (RequestC * n)()
    for i in range(n):
        arr[i] = RequestC(i, float(arrival[i]), int(prompt[i]), int(gen[i]))
    s = EngineStatsC()
    check(lib().kvc_run_static(engine._h, arr, n, max_batch, C.byref(s)))
    return EngineStats.from_c("static", s)


def run_continuous(prompt, gen, arrival, engine: Engine) -> EngineStats:
    engine.reset()
    for p, g, a in zip(prompt, gen, arrival):
        engine.add_request(int(p), int(g), float(a))
    return engine.run()
