"""ctypes binding of the CPU oracle (oracle/oracle.cpp).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by
bench.py's cpu_baseline leg, always as the checker -- never by kvcache_amd/.
Every function restates a reference function (file:line in oracle.cpp).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"
REF_DRIVER = HERE / "_ref" / "ref_alloc_driver"

vp, i32, f64, u32 = C.c_void_p, C.c_int, C.c_double, C.c_uint


class OStats(C.Structure):
    _fields_ = [("iters", i32), ("tokens", C.c_longlong), ("gpu_us", f64), ("wall_us", f64),
                ("slot_steps", C.c_longlong), ("useful_steps", C.c_longlong), ("peak_blocks", i32),
                ("finished", i32), ("avg_latency_us", f64), ("p50_latency_us", f64), ("p99_latency_us", f64),
                ("digest", C.c_uint64)]

    def as_dict(self) -> dict:
        return {k: getattr(self, k) for k, _ in self._fields_}


_SIGS = {
    "orc_batched_paged": (None, [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, f64, i32, i32]),
    "orc_batched_contig": (None, [vp, vp, vp, vp, vp, i32, i32, i32, i32, C.c_longlong, f64, i32, i32]),
    "orc_flash_split": (None, [vp, vp, vp, vp, vp, vp, i32, i32, C.c_longlong, i32, f64, i32, i32]),
    "orc_flash_merge": (None, [vp, vp, vp, vp, i32, i32, i32]),
    "orc_flash_decode": (None, [vp, vp, vp, vp, i32, i32, i32, C.c_longlong, f64, i32, i32]),
    "orc_ref_lengths": (None, [i32, i32, u32, vp]),
    "orc_ref_trace": (None, [i32, i32, i32, f64, u32, vp, vp, vp]),
    "orc_kvm_new": (vp, [i32, i32, i32, i32]),
    "orc_kvm_delete": (None, [vp]),
    "orc_kvm_free_blocks": (i32, [vp]),
    "orc_kvm_allocate_prompt": (i32, [vp, i32, i32]),
    "orc_kvm_append_token": (i32, [vp, i32]),
    "orc_kvm_free": (None, [vp, i32]),
    "orc_kvm_slack": (i32, [vp, i32]),
    "orc_kvm_cur_len": (i32, [vp, i32]),
    "orc_kvm_table": (i32, [vp, i32, vp, i32]),
    "orc_kvm_slot_offset": (C.c_longlong, [vp, i32, i32, i32]),
    "orc_alloc_script": (None, [i32, vp, vp, i32, vp]),
    "orc_sim_engine": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, f64, f64, f64, C.POINTER(OStats)]),
    "orc_sim_static": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, f64, f64, f64, C.POINTER(OStats), vp]),
}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data


def _f(a, dtype):
    """Contiguous input array; fp16 stays fp16 (decoded exactly by the oracle)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        return a, 1
    return np.ascontiguousarray(a, dtype=np.float32), 0


# ---- attention ---------------------------------------------------------------
def batched_paged(q, k_pool, v_pool, table_all, tab_off, cur_len, Hkv, BLOCK, scale, nthreads=1):
    q, dt = _f(q, None)
    k_pool, _ = _f(k_pool.astype(q.dtype, copy=False), None)
    v_pool, _ = _f(v_pool.astype(q.dtype, copy=False), None)
    N, Hq, D = q.shape
    out = np.zeros((N, Hq, D), dtype=np.float64)
    t = np.ascontiguousarray(table_all, dtype=np.int32)
    o = np.ascontiguousarray(tab_off, dtype=np.int32)
    l = np.ascontiguousarray(cur_len, dtype=np.int32)
    lib().orc_batched_paged(_p(q), _p(k_pool), _p(v_pool), _p(t), _p(o), _p(l), _p(out), N, Hq, Hkv, D, BLOCK,
                            scale, dt, nthreads)
    return out


def batched_contig(q, k, v, cur_len, scale, nthreads=1):
    """k, v: [N, Hkv, MAXS, D]."""
    q, dt = _f(q, None)
    k, _ = _f(k.astype(q.dtype, copy=False), None)
    v, _ = _f(v.astype(q.dtype, copy=False), None)
    N, Hq, D = q.shape
    Hkv, MAXS = k.shape[1], k.shape[2]
    out = np.zeros((N, Hq, D), dtype=np.float64)
    l = np.ascontiguousarray(cur_len, dtype=np.int32)
    lib().orc_batched_contig(_p(q), _p(k), _p(v), _p(l), _p(out), N, Hq, Hkv, D, MAXS, scale, dt, nthreads)
    return out


def flash_decode(q, k, v, cur_len, scale, num_splits):
    """Single sequence, q [H, D], k/v [H, S, D]."""
    q, dt = _f(q, None)
    k, _ = _f(k.astype(q.dtype, copy=False), None)
    v, _ = _f(v.astype(q.dtype, copy=False), None)
    H, D = q.shape
    S = k.shape[1]
    out = np.zeros((H, D), dtype=np.float64)
    lib().orc_flash_decode(_p(q), _p(k), _p(v), _p(out), cur_len, H, D, S, scale, num_splits, dt)
    return out


def flash_split(q, k, v, cur_len, scale, num_splits):
    q, dt = _f(q, None)
    k, _ = _f(k.astype(q.dtype, copy=False), None)
    v, _ = _f(v.astype(q.dtype, copy=False), None)
    H, D = q.shape
    S = k.shape[1]
    pa = np.zeros((H, num_splits, D)); pm = np.zeros((H, num_splits)); pl = np.zeros((H, num_splits))
    lib().orc_flash_split(_p(q), _p(k), _p(v), _p(pa), _p(pm), _p(pl), H, D, S, cur_len, scale, num_splits, dt)
    return pa, pm, pl


# ---- workloads -----------------------------------------------------------------
def ref_lengths(n=128, lmax=2048, seed=12345):
    out = np.zeros(n, dtype=np.int32)
    lib().orc_ref_lengths(n, lmax, seed, _p(out))
    return out


def ref_trace(nreq=256, prompt_max=256, gen_max=512, rate=0.0, seed=2024):
    p = np.zeros(nreq, np.int32); g = np.zeros(nreq, np.int32); a = np.zeros(nreq, np.float64)
    lib().orc_ref_trace(nreq, prompt_max, gen_max, rate, seed, _p(p), _p(g), _p(a))
    return p, g, a


# ---- scheduling ------------------------------------------------------------------
def sim_engine(prompt, gen, arrival, block, num_blocks, max_batch, kv_write=False, c=(1.0, 0.0, 0.0)):
    p = np.ascontiguousarray(prompt, np.int32); g = np.ascontiguousarray(gen, np.int32)
    a = np.ascontiguousarray(arrival, np.float64)
    st = OStats()
    rc = lib().orc_sim_engine(_p(p), _p(g), _p(a), len(p), block, num_blocks, max_batch, int(kv_write), c[0], c[1],
                              c[2], C.byref(st))
    return rc, st


def sim_static(prompt, gen, arrival, block, num_blocks, max_batch, kv_write=False, c=(1.0, 0.0, 0.0)):
    p = np.ascontiguousarray(prompt, np.int32); g = np.ascontiguousarray(gen, np.int32)
    a = np.ascontiguousarray(arrival, np.float64)
    st = OStats()
    order = np.zeros(len(p), np.int32)
    rc = lib().orc_sim_static(_p(p), _p(g), _p(a), len(p), block, num_blocks, max_batch, int(kv_write), c[0], c[1],
                              c[2], C.byref(st), _p(order))
    return rc, st, order


def alloc_script(total, ops, args):
    o = np.ascontiguousarray(ops, np.int32); a = np.ascontiguousarray(args, np.int32)
    out = np.zeros(len(o), np.int32)
    lib().orc_alloc_script(total, _p(o), _p(a), len(o), _p(out))
    return out


class Kvm:
    """Handle over the oracle's KV block accounting (kv_cache_manager.h:56-91)."""

    def __init__(self, nb, bs, hkv, d):
        self.h = lib().orc_kvm_new(nb, bs, hkv, d)

    def __del__(self):
        try:
            lib().orc_kvm_delete(self.h)
        except Exception:
            pass

    def free_blocks(self): return lib().orc_kvm_free_blocks(self.h)
    def allocate_prompt(self, sid, plen): return bool(lib().orc_kvm_allocate_prompt(self.h, sid, plen))
    def append_token(self, sid): return bool(lib().orc_kvm_append_token(self.h, sid))
    def free(self, sid): lib().orc_kvm_free(self.h, sid)
    def slack(self, sid): return lib().orc_kvm_slack(self.h, sid)
    def cur_len(self, sid): return lib().orc_kvm_cur_len(self.h, sid)
    def slot_offset(self, phys, kvh, inb): return lib().orc_kvm_slot_offset(self.h, phys, kvh, inb)

    def table(self, sid):
        buf = np.zeros(4096, np.int32)
        n = lib().orc_kvm_table(self.h, sid, _p(buf), 4096)
        return buf[:n].tolist()


def ref_driver_available() -> bool:
    return REF_DRIVER.exists()


def run_ref_alloc_driver(script: str) -> list[int]:
    """Runs the reference's own BlockAllocator/Sequence (oracle/_ref) over a script."""
    r = subprocess.run([str(REF_DRIVER)], input=script, capture_output=True, text=True, check=True)
    return [int(x) for x in r.stdout.split()]


def paged_causal(q, k_pool, v_pool, block_table, q_pos_base, Hkv, BLOCK, scale, nthreads=1):
    """Prompt attention of one sequence (qwen_kernels.cu:146-181): query i at position
    q_pos_base + i over positions 0..q_pos_base + i.  Each query is the batched paged
    decode of a sequence of that length over the same table (batched.cu:91-130 with
    the causal length of qwen_kernels.cu:151)."""
    import numpy as np
    n = q.shape[0]
    lens = np.arange(q_pos_base + 1, q_pos_base + n + 1, dtype=np.int32)
    tab_off = np.zeros(n + 1, dtype=np.int32)
    return batched_paged(q, k_pool, v_pool, np.asarray(block_table, np.int32), tab_off, lens, Hkv, BLOCK, scale,
                         nthreads=nthreads)
