"""Headline benchmark: batched ragged paged decode on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10]

Workload (config 2 of the path's spec, `config.workload` in the JSON line):
N = 128 sequences, lengths from the reference generator (bench_throughput.cu:50-57,
seed 12345: sum 83,212, max 2,022), H = 8 query = KV heads, D = 64, BLOCK = 16,
fp16 K/V in a shared pool sized to actual use, blocks handed out by the
free-list in a seeded random order, q/K/V ~ N(0,1), fp32 accumulation.
A step is one decode pass over the whole batch (one kernel launch).
Inputs are resident in HBM; the timed loop rotates over --rotate pool copies
(4 x 172 MB > the 256 MB Infinity Cache) so every step streams from HBM.

value = algorithmic bytes per step / mean kernel time (GB/s); algorithmic bytes
= sum_i L_i * Hkv * D * 2 (K,V) * 2 B + q + out + block tables + lengths/offsets.
The output is checked against the CPU oracle before timing.

Extras in the same line: config 3 (long-context split-K, Qwen2.5-0.5B attention
shape) and config 4 (256-request continuous vs static batching trace, 24 layers
of append + GQA decode per step), each measured the same way.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

# kernel arguments in device memory (also for the C++ child process): see kvcache_amd/_native.py
os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "1")

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "paged decode KV GB/s (% of HBM peak) @N=128 ragged; continuous tokens/s"
# Measured HBM traffic of the headline kernel: a rocprofv3 --pmc summary (FETCH_SIZE and
# WRITE_SIZE per dispatch, scaled by the same counters read for a plain copy of known size).
TRAFFIC_SUMMARY = ROOT / "profiles" / "split_kernel_planned_c2_traffic.txt"


def measured_traffic():
    """(bytes per launch, kernel symbol) from the committed --pmc summary, or (None, None)."""
    try:
        text = TRAFFIC_SUMMARY.read_text()
    except OSError:
        return None, None
    vals = dict(line.split(":", 1) for line in text.splitlines() if ":" in line and not line.startswith(" "))
    try:
        return int(vals["traffic_bytes_per_launch"].split()[0]), vals.get("kernel", "").strip()
    except (KeyError, ValueError):
        return None, None


STATS_SUMMARY = ROOT / "profiles" / "split_kernel_planned_c2_stats.txt"
PROFILES = ROOT / "profiles"


def profile_sources():
    """key -> (value, file) for the `key: number` lines of the committed rocprofv3
    summaries under profiles/ (mean kernel durations in us of each workload's timed
    dispatches; each summary names the command that made it)."""
    out = {}
    for f in sorted(PROFILES.glob("*.txt")):
        try:
            text = f.read_text()
        except OSError:
            continue
        for line in text.splitlines():
            k, sep, v = line.partition(":")
            if sep and k and not k.startswith((" ", "#")) and " " not in k:
                try:
                    out[k] = (float(v), f)
                except ValueError:
                    pass
    return out


def profile_values():
    return {k: v for k, (v, _) in profile_sources().items()}


def profiled_launch_us():
    """Mean duration (us) of the headline kernel's timed dispatches in the committed
    rocprofv3 kernel-trace summary of the default command, or None."""
    return profile_values().get("headline_timed_mean_us")


def roofline_block(alg_bytes, us, kernel, profile_keys=()):
    """An HBM roofline entry for an extra workload: algorithmic bytes over the measured
    time, and the same over the profiled kernel time (sum of profile_keys) when the
    committed summary has it."""
    gbs = alg_bytes / (us * 1e-6) / 1e9
    out = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(gbs / HBM_PEAK_GBS, 4), "kernel": kernel, "algorithmic_bytes_per_launch": alg_bytes}
    src = profile_sources()
    if profile_keys and all(k in src for k in profile_keys):
        kus = sum(src[k][0] for k in profile_keys)
        out["profile"] = {"file": str(src[profile_keys[0]][1].relative_to(ROOT)), "kernel_us": round(kus, 3),
                          "keys": list(profile_keys),
                          "frac": round(alg_bytes / (kus * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    return out


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def set_tuning(key: str, value: int) -> None:
    from kvcache_amd._native import check, lib
    check(lib().kvc_set_tuning(key.encode(), int(value)))


def build_c2(lens, Hq, Hkv, D, B, rotate, seed, shuffle=True, dtype=None):
    from kvcache_amd import KVC_F16
    from kvcache_amd.device import DeviceBuffer, fill_normal
    from kvcache_amd.engine import BlockAllocator
    from kvcache_amd.workloads import build_tables

    dtype = KVC_F16 if dtype is None else dtype
    esz = 2 if dtype == KVC_F16 else 4
    nb = int(sum((int(x) + B - 1) // B for x in lens))
    alloc = BlockAllocator(nb)           # pool sized to actual use
    if shuffle:
        alloc.shuffle(seed)              # blocks come out in a seeded random physical order
    table, tab_off = build_tables(lens, B, alloc)
    N = len(lens)
    elems = nb * Hkv * B * D
    pools = []
    for r in range(rotate):
        k, v = DeviceBuffer(elems * esz), DeviceBuffer(elems * esz)
        fill_normal(k, elems, dtype, seed * 1000 + 2 * r + 1)
        fill_normal(v, elems, dtype, seed * 1000 + 2 * r + 2)
        pools.append((k, v))
    q = DeviceBuffer(N * Hq * D * esz)
    fill_normal(q, N * Hq * D, dtype, seed * 1000 + 999)
    meta = dict(table=DeviceBuffer.from_numpy(table), tab_off=DeviceBuffer.from_numpy(tab_off),
                lens=DeviceBuffer.from_numpy(np.asarray(lens, np.int32)), out=DeviceBuffer(N * Hq * D * esz))
    return dict(nb=nb, table_host=table, tab_off_host=tab_off, pools=pools, q=q, dtype=dtype, **meta)


def alg_bytes(lens, Hq, Hkv, D, B, esz=2):
    kv = int(np.sum(lens, dtype=np.int64)) * Hkv * D * 2 * esz
    n = len(lens)
    other = 2 * n * Hq * D * esz + 4 * int(sum((int(x) + B - 1) // B for x in lens)) + 4 * (2 * n + 1)
    return kv, kv + other


def time_decode(W, lens, Hq, Hkv, D, B, split, steps, warmup, stream=None, per_launch=False):
    """Runs warmup + steps back-to-back launches (rotating pools).  Returns (mean ms per
    launch over the timed region bracketed by one event pair, per-launch event
    intervals when per_launch -- those markers add inter-kernel gaps)."""
    from kvcache_amd import KVC_F16, ops
    from kvcache_amd.device import Event, synchronize

    cap = int(max(lens))
    N = len(lens)
    scale = 1.0 / np.sqrt(D)

    def launch(i):
        k, v = W["pools"][i % len(W["pools"])]
        ops.launch_batched_paged(W["q"], k, v, W["table"], W["tab_off"], W["lens"], W["out"], N, Hq, D, B, cap,
                                 scale, Hkv=Hkv, dtype=W.get("dtype", KVC_F16), split=split, stream=stream)

    for i in range(warmup):
        launch(i)
    synchronize()
    if per_launch:
        evs = [Event() for _ in range(steps + 1)]
        evs[0].record(stream)
        for i in range(steps):
            launch(i)
            evs[i + 1].record(stream)
        synchronize()
        return evs[0].elapsed_ms(evs[-1]) / steps, np.array([evs[i].elapsed_ms(evs[i + 1]) for i in range(steps)])
    e0, e1 = Event(), Event()
    e0.record(stream)
    for i in range(steps):
        launch(i)
    e1.record(stream)
    synchronize()
    return e0.elapsed_ms(e1) / steps, None


def time_planned(W, lens, Hq, Hkv, D, B, steps, warmup, target=0, rotate=None):
    """The planned path: the host plan (built once from the host lengths, as the
    scheduler does every step) is resident on the device; launches back to back."""
    from kvcache_amd import KVC_F16, ops
    from kvcache_amd.device import DeviceBuffer, Event, synchronize

    work, nu, nr = ops.decode_plan(lens, Hq, Hkv, D, B, tab_off=W["tab_off_host"], table=W["table_host"],
                                   dtype=KVC_F16, target_tokens=target)
    wdev = DeviceBuffer.from_numpy(work)
    ws = DeviceBuffer(max(ops.planned_workspace_size(Hq, Hkv, D, nr, BLOCK=B, dtype=KVC_F16), 256))
    pools = W["pools"] if rotate is None else W["pools"][:rotate]
    N = len(lens)

    def launch(i):
        k, v = pools[i % len(pools)]
        ops.launch_batched_paged_planned(W["q"], k, v, W["table"], len(W["table_host"]), W["out"], N, Hq, Hkv, D,
                                         B, 1.0 / np.sqrt(D), wdev, nu, nr, dtype=KVC_F16, workspace=ws)

    for i in range(warmup):
        launch(i)
    synchronize()
    e0, e1 = Event(), Event()
    e0.record()
    for i in range(steps):
        launch(i)
    e1.record()
    synchronize()
    return e0.elapsed_ms(e1) / steps, nu, nr, launch


def practical_ceiling(W, lens, Hq, Hkv, D, B, steps, warmup, target=0):
    """The read-only probe (kvc_read_probe_planned) over the planned decode's own work list:
    the same units in the same grid order, the same loads, the same rotating pools, and no
    arithmetic.  Its time is the floor of the access pattern.  Returns (us per launch, units)."""
    from kvcache_amd import KVC_F16, ops
    from kvcache_amd._native import check, lib
    from kvcache_amd.device import DeviceBuffer, Event, synchronize

    dtype = W.get("dtype", KVC_F16)
    work, nu, _ = ops.decode_plan(lens, Hq, Hkv, D, B, tab_off=W["tab_off_host"], table=W["table_host"],
                                  dtype=dtype, target_tokens=target)
    wdev = DeviceBuffer.from_numpy(work)
    sink = DeviceBuffer(max(nu, 1) * 4)
    tl = len(W["table_host"])

    def launch(i):
        k, v = W["pools"][i % len(W["pools"])]
        check(lib().kvc_read_probe_planned(k.ptr, v.ptr, W["table"].ptr, tl, wdev.ptr, nu, Hq, Hkv, D, B, dtype,
                                           sink.ptr, None))

    for i in range(warmup):
        launch(i)
    synchronize()
    e0, e1 = Event(), Event()
    e0.record()
    for i in range(steps):
        launch(i)
    e1.record()
    synchronize()
    return e0.elapsed_ms(e1) / steps * 1e3, nu


def launch_floor(steps, warmup):
    """us per launch of an empty kernel (kvc_empty_launch) back to back, with 1 and with 1024
    one-wave workgroups: the cost every decode launch pays before any work."""
    from kvcache_amd._native import check, lib
    from kvcache_amd.device import Event, synchronize
    out = {}
    for blocks in (1, 1024):
        for _ in range(warmup):
            check(lib().kvc_empty_launch(blocks, None))
        synchronize()
        e0, e1 = Event(), Event()
        e0.record()
        for _ in range(steps):
            check(lib().kvc_empty_launch(blocks, None))
        e1.record()
        synchronize()
        out[f"{blocks}_workgroups_us"] = round(e0.elapsed_ms(e1) / steps * 1e3, 3)
    return out


def bench_c2_contiguous(steps, warmup, rotate):
    """The reference's bench_throughput comparison (bench_throughput.cu:120-132): the config-2 batch
    (reference lengths) as contiguous caches [N, H, LMAX=2048, D] (launch_batched_decode) and as the
    paged pool (launch_batched_paged), both from device lengths, in fp16 (config 2) and in the
    reference's fp32.  The reference publishes 1340 us contiguous / 1454 us paged in fp32 on its GPU
    (README.md:76-77)."""
    from kvcache_amd import KVC_F16, KVC_F32, ops
    from kvcache_amd import workloads as Wl
    from kvcache_amd.device import DeviceBuffer, Event, fill_normal, synchronize

    lens = Wl.ref_lengths()
    N, H, D, B, LMAX = 128, 8, 64, 16, 2048
    scale = float(1.0 / np.sqrt(D))
    res = {"workload": "C2 batch (reference lengths, N=128, H=8, D=64): contiguous [N,H,2048,D] caches vs the "
                       "paged pool (BLOCK 16, shuffled free list), device-lengths path, rotating copies",
           "reference_published_us": {"contiguous": 1340.0, "paged": 1454.0, "dtype": "f32",
                                      "source": "README.md:76-77"}}
    for dtype, name in ((KVC_F16, "f16"), (KVC_F32, "f32")):
        esz = 2 if dtype == KVC_F16 else 4
        _, total = alg_bytes(lens, H, H, D, B, esz)
        W = build_c2(lens, H, H, D, B, rotate, seed=12345, dtype=dtype)
        t_paged, _ = time_decode(W, lens, H, H, D, B, 0, steps, warmup)
        del W["pools"]
        elems = N * H * LMAX * D
        caches = []
        for r in range(rotate):
            k, v = DeviceBuffer(elems * esz), DeviceBuffer(elems * esz)
            fill_normal(k, elems, dtype, 4242 + 2 * r)
            fill_normal(v, elems, dtype, 4243 + 2 * r)
            caches.append((k, v))
        cap = int(max(lens))

        def launch(i):
            k, v = caches[i % len(caches)]
            ops.launch_batched_decode(W["q"], k, v, W["lens"], W["out"], N, H, D, LMAX, cap, scale, Hkv=H,
                                      dtype=dtype)

        for i in range(warmup):
            launch(i)
        synchronize()
        e0, e1 = Event(), Event()
        e0.record()
        for i in range(steps):
            launch(i)
        e1.record()
        synchronize()
        t_contig = e0.elapsed_ms(e1) / steps
        del caches
        res[name] = {"contiguous_us": round(t_contig * 1e3, 3), "paged_us": round(t_paged * 1e3, 3),
                     "paged_over_contiguous": round(t_paged / t_contig, 4),
                     "contiguous_GBps": round(total / (t_contig * 1e-3) / 1e9, 1),
                     "paged_GBps": round(total / (t_paged * 1e-3) / 1e9, 1), "algorithmic_bytes": total}
    res["reference_paged_over_contiguous"] = round(1454.0 / 1340.0, 4)
    return res


def bench_single_seq(iters=300, warmup=30):
    """The reference's single-sequence latency sweep (bench_paged.cu:40-108): H=8, D=64, fp32, one query,
    S = 128 ... 4096, contiguous [H,S,D] (launch_decode) vs paged [NB,H,16,D] with the identity block table
    (launch_paged); back-to-back launches between two events; the two outputs must agree bit for bit.
    The reference publishes 21.9/27.2, 139.6/222.3 and 507.6/881.1 us at S = 128, 1024, 4096
    (README.md:62-66) on its GPU."""
    from kvcache_amd import KVC_F32, ops
    from kvcache_amd.device import DeviceBuffer, Event, synchronize

    H, D, B = 8, 64, 16
    scale = float(1.0 / np.sqrt(D))
    published = {128: (21.9, 27.2), 1024: (139.6, 222.3), 4096: (507.6, 881.1)}
    rng = np.random.default_rng(64)
    rows = []
    for S in (128, 256, 512, 1024, 2048, 4096):
        q = rng.standard_normal((H, D)).astype(np.float32)
        K = rng.standard_normal((H, S, D)).astype(np.float32)
        V = rng.standard_normal((H, S, D)).astype(np.float32)
        nb = (S + B - 1) // B
        kp = np.zeros((nb, H, B, D), np.float32)
        vp = np.zeros_like(kp)
        for b in range(nb):                      # identity table: logical block b is physical block b
            t1 = min((b + 1) * B, S)
            kp[b, :, : t1 - b * B] = K[:, b * B:t1]
            vp[b, :, : t1 - b * B] = V[:, b * B:t1]
        dq, dK, dV = (DeviceBuffer.from_numpy(x) for x in (q, K, V))
        dkp, dvp = DeviceBuffer.from_numpy(kp), DeviceBuffer.from_numpy(vp)
        dtab = DeviceBuffer.from_numpy(np.arange(nb, dtype=np.int32))
        oc, op = DeviceBuffer(H * D * 4), DeviceBuffer(H * D * 4)
        runs = {"contiguous": lambda: ops.launch_decode(dq, dK, dV, oc, S, H, D, S, scale, dtype=KVC_F32),
                "paged": lambda: ops.launch_paged(dq, dkp, dvp, dtab, op, S, H, D, B, scale, dtype=KVC_F32)}
        t = {}
        for name, run in runs.items():
            for _ in range(warmup):
                run()
            synchronize()
            e0, e1 = Event(), Event()
            e0.record()
            for _ in range(iters):
                run()
            e1.record()
            synchronize()
            t[name] = e0.elapsed_ms(e1) / iters * 1e3
        diff = float(np.abs(oc.to_numpy(np.float32, (H, D)) - op.to_numpy(np.float32, (H, D))).max())
        row = {"S": S, "contiguous_us": round(t["contiguous"], 2), "paged_us": round(t["paged"], 2),
               "paged_overhead_pct": round(100 * (t["paged"] / t["contiguous"] - 1), 1),
               "max_abs_diff": diff}
        if S in published:
            row["reference_us"] = {"contiguous": published[S][0], "paged": published[S][1]}
        rows.append(row)
    return {"workload": "single sequence, H=8, D=64, fp32, one query; identity block table, BLOCK 16",
            "rows": rows, "source": "bench_paged.cu:40-108, README.md:62-66"}


def check_c2(W, lens, Hq, Hkv, D, B, split):
    """One launch on pool copy 0, compared with the CPU oracle (max abs <= 2e-3)."""
    import oracle
    from kvcache_amd import KVC_F16, ops
    from kvcache_amd.device import synchronize

    N = len(lens)
    k, v = W["pools"][0]
    ops.launch_batched_paged(W["q"], k, v, W["table"], W["tab_off"], W["lens"], W["out"], N, Hq, D, B,
                             int(max(lens)), 1.0 / np.sqrt(D), Hkv=Hkv, dtype=KVC_F16, split=split)
    synchronize()
    shape = (W["nb"], Hkv, B, D)
    kp, vp = k.to_numpy(np.float16, shape), v.to_numpy(np.float16, shape)
    q = W["q"].to_numpy(np.float16, (N, Hq, D))
    got = W["out"].to_numpy(np.float16, (N, Hq, D)).astype(np.float64)
    ref = oracle.batched_paged(q, kp, vp, W["table_host"], W["tab_off_host"], lens, Hkv, B, 1.0 / np.sqrt(D),
                               nthreads=min(os.cpu_count() or 1, 16))
    return float(np.abs(got - ref).max()), (q, kp, vp)


def check_planned(W, launch, lens, Hq, Hkv, D, B, host_data):
    """The planned path's output on pool copy 0 against the oracle's."""
    import oracle
    from kvcache_amd.device import synchronize
    launch(0)
    synchronize()
    q, kp, vp = host_data
    got = W["out"].to_numpy(np.float16, (len(lens), Hq, D)).astype(np.float64)
    ref = oracle.batched_paged(q, kp, vp, W["table_host"], W["tab_off_host"], lens, Hkv, B, 1.0 / np.sqrt(D),
                               nthreads=min(os.cpu_count() or 1, 16))
    return float(np.abs(got - ref).max())


def cpu_baseline(host_data, W, lens, Hkv, B, D, budget_s, kv_bytes):
    """The oracle (C++ restatement, double accumulation) on the host cores: full
    passes over the same workload repeated until ~budget_s of wall time."""
    import oracle

    q, kp, vp = host_data
    threads = min(os.cpu_count() or 1, 16)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.batched_paged(q, kp, vp, W["table_host"], W["tab_off_host"], lens, Hkv, B, 1.0 / np.sqrt(D),
                             nthreads=threads)
        reps += 1
        if time.perf_counter() - t0 >= budget_s or reps >= 2000:
            break
    dt = (time.perf_counter() - t0) / reps
    t1 = time.perf_counter()
    oracle.batched_paged(q, kp, vp, W["table_host"], W["tab_off_host"], lens, Hkv, B, 1.0 / np.sqrt(D), nthreads=1)
    dt1 = time.perf_counter() - t1
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(kv_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{reps} full passes of the N=128 ragged batch (oracle/oracle.cpp, double accumulation over "
                      f"the same fp16 pool), {threads} threads, {reps * dt:.1f} s",
            "single_thread_GBps": round(kv_bytes / dt1 / 1e9, 3), "cpu_model": cpu_model,
            "host_cpus": os.cpu_count()}


def host_plan_cost(W, lens, Hq, Hkv, D, B, reps=500):
    """Mean host time of one kvc_decode_plan (size query + fill, through ctypes) for this
    batch, the work list's bytes (what the step's upload carries) and the chunk target."""
    import ctypes as C

    from kvcache_amd import KVC_F16, ops
    from kvcache_amd._native import lib
    L = lib()
    lens = np.ascontiguousarray(lens, np.int32)
    toff, tab = W["tab_off_host"], W["table_host"]
    nu, nr = C.c_int(0), C.c_int(0)
    ipu = int(L.kvc_decode_plan_entry_ints(Hq, Hkv, D, B, KVC_F16))
    L.kvc_decode_plan(lens.ctypes.data, toff.ctypes.data, tab.ctypes.data, len(tab), len(lens), Hq, Hkv, D, B,
                      KVC_F16, 0, None, 0, C.byref(nu), C.byref(nr))
    work = np.zeros((nu.value, ipu), np.int32)
    t0 = time.perf_counter()
    for _ in range(reps):
        L.kvc_decode_plan(lens.ctypes.data, toff.ctypes.data, tab.ctypes.data, len(tab), len(lens), Hq, Hkv, D, B,
                          KVC_F16, 0, None, 0, C.byref(nu), C.byref(nr))
        L.kvc_decode_plan(lens.ctypes.data, toff.ctypes.data, tab.ctypes.data, len(tab), len(lens), Hq, Hkv, D, B,
                          KVC_F16, 0, work.ctypes.data, nu.value, C.byref(nu), C.byref(nr))
    us = (time.perf_counter() - t0) / reps * 1e6
    return {"us_per_plan": round(us, 2), "work_list_bytes": int(work.nbytes), "units": nu.value,
            "chunk_tokens": ops.decode_plan_chunk(lens, Hq, Hkv, D, B)}


def host_plan_pipelined(W, lens, Hq, Hkv, D, B, steps, warmup, mode=0):
    """The planned path as a serving loop runs it, in C++ over the C ABI
    (tests/cpp/plan_pipeline.cpp, a child process): the host plans EVERY step
    (kvc_decode_plan into a ring of 4 pinned buffers) and uploads the work list on a
    copy stream while the GPU runs the previous step's kernel.  Returns the program's
    JSON: compute-stream event time per step (host planning, uploads and kernels all
    inside it) and the host's own time per step; the last step's output must equal a
    plain planned launch's bit for bit."""
    import json
    import subprocess
    import tempfile

    exe = ROOT / "kvcache_amd" / "_build" / "bin" / "plan_pipeline"
    if not exe.exists():
        raise FileNotFoundError(f"{exe} (python -m kvcache_amd.build)")
    lens = np.ascontiguousarray(lens, np.int32)
    toff, tab = np.asarray(W["tab_off_host"], np.int32), np.asarray(W["table_host"], np.int32)
    with tempfile.NamedTemporaryFile(suffix=".bin", delete=False) as f:
        np.concatenate([np.array([len(lens), Hq, Hkv, D, B, len(tab)], np.int32), lens, toff, tab]).tofile(f)
        path = f.name
    try:
        r = subprocess.run([str(exe), path, str(steps), str(warmup), str(mode)], stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                           text=True, timeout=120)
    finally:
        os.unlink(path)
    if r.returncode != 0:
        raise RuntimeError(f"plan_pipeline exit {r.returncode}: {r.stderr.strip()[-300:]}")
    return json.loads(r.stdout.strip().splitlines()[-1])


def c2_variant(lens, steps, warmup, rotate):
    """A C2 batch of other lengths: planned and self-planned (device-lengths) paths."""
    N, Hq, Hkv, D, B = len(lens), 8, 8, 64, 16
    W = build_c2(lens, Hq, Hkv, D, B, rotate, seed=777)
    err, _ = check_c2(W, lens, Hq, Hkv, D, B, 0)
    kv, total = alg_bytes(lens, Hq, Hkv, D, B)
    t_self, _ = time_decode(W, lens, Hq, Hkv, D, B, 0, steps, warmup)
    t_plan, nu, _, launch = time_planned(W, lens, Hq, Hkv, D, B, steps, warmup)
    t_probe, _ = practical_ceiling(W, lens, Hq, Hkv, D, B, steps, warmup)
    return {"sum_len": int(np.sum(lens)), "algorithmic_bytes": total, "parity_max_abs_err": err,
            "practical_ceiling_us": round(t_probe, 3),
            "practical_ceiling_frac": round(total / (t_probe * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "planned": {"us_per_step": round(t_plan * 1e3, 3), "GBps": round(total / (t_plan * 1e-3) / 1e9, 1),
                        "frac_hbm_peak": round(total / (t_plan * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "units": nu},
            "device_lengths_self_planned": {"us_per_step": round(t_self * 1e3, 3),
                                            "GBps": round(total / (t_self * 1e-3) / 1e9, 1),
                                            "frac_hbm_peak": round(total / (t_self * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}}


def bench_c4_layer(steps, warmup):
    """The config-4 per-layer kernel at the trace's typical step: 32 running sequences of
    the BASELINE trace halfway through their generation (prompt + gen/2 tokens), one
    planned grouped-query launch with the new token's K/V appended (14q/2kv, D 64, fp16)."""
    from kvcache_amd import KVC_F16, ops
    from kvcache_amd import workloads as Wl
    from kvcache_amd.device import DeviceBuffer, Event, fill_normal, synchronize
    p, g, _ = Wl.baseline_trace(256, 0.0, 11)
    lens = (p[:32] + g[:32] // 2).astype(np.int32)
    Hq, Hkv, D, B = 14, 2, 64, 16
    W = build_c2(lens, Hq, Hkv, D, B, rotate=8, seed=44)
    N = len(lens)
    kv, total = alg_bytes(lens, Hq, Hkv, D, B)
    work, nu, nr = ops.decode_plan(lens, Hq, Hkv, D, B, tab_off=W["tab_off_host"], table=W["table_host"])
    wdev = DeviceBuffer.from_numpy(work)
    ws = DeviceBuffer(max(ops.planned_workspace_size(Hq, Hkv, D, nr, BLOCK=B, dtype=KVC_F16), 256))
    knew, vnew = DeviceBuffer(N * Hkv * D * 2), DeviceBuffer(N * Hkv * D * 2)
    fill_normal(knew, N * Hkv * D, KVC_F16, 45)
    fill_normal(vnew, N * Hkv * D, KVC_F16, 46)
    wpos = DeviceBuffer.from_numpy(lens - 1)

    def launch(i):
        k, v = W["pools"][i % len(W["pools"])]
        ops.launch_batched_paged_append_planned(W["q"], knew, vnew, wpos, k, v, W["table"], len(W["table_host"]),
                                                W["out"], N, Hq, Hkv, D, B, 1.0 / np.sqrt(D), wdev, nu, nr,
                                                dtype=KVC_F16, workspace=ws)
    for i in range(warmup):
        launch(i)
    synchronize()
    e0, e1 = Event(), Event()
    e0.record()
    for i in range(steps):
        launch(i)
    e1.record()
    synchronize()
    t = e0.elapsed_ms(e1) / steps
    return {"workload": "config-4 layer step: 32 sequences of the BASELINE trace at prompt + gen/2 tokens "
                        f"(sum {int(lens.sum())}), planned grouped-query decode with fused append",
            "units": nu, "algorithmic_bytes": total, "us_per_launch": round(t * 1e3, 3),
            "GBps": round(total / (t * 1e-3) / 1e9, 1), "frac_hbm_peak": round(total / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "roofline": roofline_block(total, t * 1e3, "gqa_mfma_kernel<64, kPlannedUniform, 8> (one launch per "
                                       "layer step; latency-bound: ~25k token-heads)", ("c4_layer_timed_mean_us",))}


def bench_c3(steps, warmup, plan_sweep=()):
    """Config 3: Hq 14 / Hkv 2, D 64, lengths {8192,16384,32768,32768}: 512-token splits on the
    device-lengths path (the configuration as stated) and the planned path (host-chosen chunks)."""
    lens = np.array([8192, 16384, 32768, 32768], np.int32)
    Hq, Hkv, D, B = 14, 2, 64, 16
    W = build_c2(lens, Hq, Hkv, D, B, rotate=8, seed=3)   # 8 x 46 MB rotate past the Infinity Cache
    t, _ = time_decode(W, lens, Hq, Hkv, D, B, 512, steps, warmup)
    kv, total = alg_bytes(lens, Hq, Hkv, D, B)
    res = {"workload": "C3 long-context split-K 14q/2kv D64 ctx {8k,16k,32k,32k} fp16 split 512",
           "us_per_step": round(t * 1e3, 2), "GBps": round(total / (t * 1e-3) / 1e9, 1),
           "frac_hbm_peak": round(total / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "kv_bytes": kv,
           "algorithmic_bytes": total,
           "roofline": roofline_block(total, t * 1e3, "gqa_mfma_kernel<64, kPagedUniform, 4> + merge_kernel<f16, 64> "
                                      "(split 512; per step: both kernels and the gap between them)",
                                      ("c3_split512_split_kernel_mean_us", "c3_split512_merge_kernel_mean_us"))}
    # the read-only probe over 512-token units of every (sequence, KV head): the same bytes in
    # the split kernel's units (a host plan cut at 512 tokens)
    set_tuning("mfma_min_chunk", 512)
    try:
        t_probe, nu_probe = practical_ceiling(W, lens, Hq, Hkv, D, B, steps, warmup, target=512)
    finally:
        set_tuning("mfma_min_chunk", 1024)
    res["roofline"]["practical_ceiling_us"] = round(t_probe, 3)
    res["roofline"]["practical_ceiling"] = {
        "what": "kvc_read_probe_planned over 512-token units of every (sequence, KV head): the split kernel's "
                "bytes and units, no arithmetic, one launch", "units": nu_probe, "us": round(t_probe, 3),
        "frac": round(total / (t_probe * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    t2, _ = time_decode(W, lens, Hq, Hkv, D, B, 1024, steps, warmup)
    res["split_1024"] = {"us_per_step": round(t2 * 1e3, 2), "GBps": round(total / (t2 * 1e-3) / 1e9, 1),
                         "frac_hbm_peak": round(total / (t2 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    ts, _ = time_decode(W, lens, Hq, Hkv, D, B, 0, steps, warmup)
    res["device_lengths_self_planned"] = {"us_per_step": round(ts * 1e3, 2),
                                          "GBps": round(total / (ts * 1e-3) / 1e9, 1),
                                          "frac_hbm_peak": round(total / (ts * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    for tgt in plan_sweep:
        tp, nu, nr, _ = time_planned(W, lens, Hq, Hkv, D, B, 30, 5, target=tgt)
        log(f"C3 sweep planned target={tgt}: {tp * 1e3:.2f} us ({nu} units, {nr} records)")
    tp, nu, _, _ = time_planned(W, lens, Hq, Hkv, D, B, steps, warmup)
    res["planned"] = {"us_per_step": round(tp * 1e3, 2), "GBps": round(total / (tp * 1e-3) / 1e9, 1),
                      "frac_hbm_peak": round(total / (tp * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "units": nu}
    return res


def bench_prefill(steps, warmup):
    """Prompt attention (qk_paged_causal_attn) of one sequence, Qwen attention shape
    (14q/2kv, D 64, fp16, BLOCK 16), prompts of 256 and 2048 tokens at position 0."""
    from kvcache_amd import KVC_F16, ops
    from kvcache_amd.device import DeviceBuffer, Event, fill_normal, synchronize
    Hq, Hkv, D, B = 14, 2, 64, 16
    res = {"workload": "prefill attention, one sequence, 14q/2kv D64 fp16 BLOCK 16, causal from position 0"}
    for P in (256, 2048):
        nb = (P + B - 1) // B
        table = np.random.default_rng(P).permutation(nb).astype(np.int32)
        kp, vp = DeviceBuffer(nb * Hkv * B * D * 2), DeviceBuffer(nb * Hkv * B * D * 2)
        q, out = DeviceBuffer(P * Hq * D * 2), DeviceBuffer(P * Hq * D * 2)
        for i, buf in enumerate((kp, vp, q)):
            fill_normal(buf, buf.nbytes // 2, KVC_F16, seed=70 + i)
        dt = DeviceBuffer.from_numpy(table)
        ws = DeviceBuffer(max(int(lib_call("kvc_paged_causal_attn_workspace_size", 0, P, Hq, Hkv, D, B, KVC_F16)), 256))

        def launch():
            ops.qk_paged_causal_attn(q, out, kp, vp, dt, 0, P, Hq, Hkv, D, B, 1.0 / np.sqrt(D), workspace=ws)
        for _ in range(warmup):
            launch()
        synchronize()
        e0, e1 = Event(), Event()
        e0.record()
        for _ in range(steps):
            launch()
        e1.record()
        synchronize()
        us = e0.elapsed_ms(e1) / steps * 1e3
        kv_once = P * Hkv * D * 2 * 2
        kv_per_query = (P * (P + 1) // 2) * Hkv * D * 2 * 2
        res[f"P{P}"] = {"us": round(us, 2), "kv_bytes_once": kv_once, "kv_bytes_read": kv_per_query,
                        "GBps_read": round(kv_per_query / (us * 1e-6) / 1e9, 1)}
    return res


def bench_c5(n_req=64, gen=64, seed=5, graph=False, chain=0):
    """Config 5: the Qwen2-shaped decoder (24 layers, hidden 896, 14q/2kv, D 64, SwiGLU 4864, vocab 151936,
    random N(0, 0.02) fp16 weights) serving n_req requests greedily with continuous batching at batch 32;
    prompts of 16..256 random tokens, gen tokens each.  Throughput on the host clock around the whole run
    (each step ends with the sampled tokens on the host, as serving needs them).  chain=1: the linear layers
    between two attention launches as one launch (kvc_rows_chain)."""
    from kvcache_amd.model import QwenConfig, QwenModel
    rng = np.random.default_rng(seed)
    cfg = QwenConfig(max_batch=32, max_rows=256, seed=seed, graph=int(graph), chain=int(chain))
    m = QwenModel(cfg)
    try:
        prompts = [rng.integers(0, cfg.vocab, int(n)) for n in rng.integers(16, 257, n_req)]
        m.serve(prompts[:4], [4] * 4)  # warm-up (library loading, GEMM kernel selection)
        out, st = m.serve(prompts, [gen] * n_req)
    finally:
        m.close()
    # algorithmic bytes of the decode steps: each step reads every layer's weights and the (tied)
    # lm_head once for the whole batch, and each running sequence's K/V once per layer; a
    # sequence's decode step t = 1 .. gen-1 attends over its prompt + t keys
    L, H, I, V, Hq, Hkv, Dh = cfg.layers, cfg.hidden, cfg.inter, cfg.vocab, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    qkv = (Hq + 2 * Hkv) * Dh
    layer_w = 2 * (H * qkv + qkv + Hq * Dh * H + H * 2 * I + I * H + 2 * H)
    head_w = 2 * (V * H + H)
    kv_keys = sum(len(p) * (gen - 1) + gen * (gen - 1) // 2 for p in prompts)
    kv_bytes = kv_keys * L * 2 * Hkv * Dh * 2
    step_bytes = st["steps"] * (L * layer_w + head_w) + kv_bytes
    dec_s = st["decode_us"] * 1e-6
    roof = {"bound": "hbm", "achieved": round(step_bytes / dec_s / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(step_bytes / dec_s / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "whole decode step: 24 x (q|k|v rows kernel, attention with fused append, o_proj, gate|up, "
                      "down) + lm_head + argmax",
            "algorithmic_bytes_per_step": round(step_bytes / max(st["steps"], 1)),
            "weights_bytes_per_step": L * layer_w + head_w, "kv_bytes_all_steps": kv_bytes,
            "floor_us_per_step": round(step_bytes / max(st["steps"], 1) / (HBM_PEAK_GBS * 1e9) * 1e6, 1)}
    return {"workload": f"C5 Qwen2-shaped decoder, {n_req} requests, prompts 16-256 tokens, {gen} generated each, "
                        "greedy, continuous batching width 32, random fp16 weights",
            "roofline": roof,
            "graph_replay": bool(graph), "graph_steps": st["graph_steps"],
            "layer_chain": bool(chain), "chain_launches": st["chain_launches"],
            "tokens": st["tokens"], "prompt_tokens": st["prompt_tokens"], "steps": st["steps"],
            "tokens_per_s": round(st["tokens"] / (st["wall_us"] * 1e-6), 1),
            "wall_ms": round(st["wall_us"] / 1e3, 2), "prefill_ms": round(st["prefill_us"] / 1e3, 2),
            "decode_ms": round(st["decode_us"] / 1e3, 2),
            "ms_per_decode_step": round(st["decode_us"] / 1e3 / max(st["steps"], 1), 3)}


def memory_accounting(lens, H, D, B, lmax=2048):
    """The memory report of bench_throughput.cu:73-80,135-139 for this batch: KV bytes
    actually used, the paged pool (blocks + table ints) and the contiguous max-length
    reservation, for the fp16 layout measured here and the reference's fp32 one (whose
    numbers are the README's 325.0 / 328.7 / 1024 MB)."""
    MB = 1048576.0
    blocks = int(sum((int(x) + B - 1) // B for x in lens))
    out = {"sequences": len(lens), "tokens": int(np.sum(lens)), "blocks": blocks, "lmax_reserved": lmax,
           "table_bytes": blocks * 4}
    for name, es in (("fp16", 2), ("fp32_reference_layout", 4)):
        used = float(np.sum(lens)) * H * D * es * 2 / MB
        paged = (blocks * H * B * D * es * 2 + blocks * 4) / MB
        reserved = len(lens) * H * lmax * D * es * 2 / MB
        budget = 4096 * MB
        out[name] = {"used_mb": round(used, 1), "paged_mb": round(paged, 1), "contiguous_reserved_mb": round(reserved, 1),
                     "contiguous_util_pct": round(100 * used / reserved, 1),
                     "paged_overhead_pct": round(100 * (paged - used) / used, 2),
                     "seqs_in_4096mb_contiguous": int(budget / (H * lmax * D * es * 2)),
                     "seqs_in_4096mb_paged": int(budget / (((int(np.mean(lens)) + B - 1) // B) * H * B * D * es * 2))}
    return out


def lib_call(name, *args):
    from kvcache_amd._native import lib
    return getattr(lib(), name)(*args)


def bench_c4(graph=False):
    """Config 4: 256 requests, width 32, 2048 MB pool, 24 layers of write + GQA decode
    per step (14q/2kv, D 64, fp16); continuous vs static, offline and Poisson 400/s."""
    from kvcache_amd import KVC_F16
    from kvcache_amd import workloads as Wl
    from kvcache_amd.engine import Engine, EngineConfig, run_continuous, run_static

    num_blocks = (2048 * 1024 * 1024) // (24 * 2 * 16 * 64 * 2 * 2)
    cfg = EngineConfig(n_heads=14, n_kv_heads=2, head_dim=64, block_size=16, num_blocks=num_blocks, max_batch=32,
                       n_layers=24, dtype=KVC_F16, kv_write=True, clock_mode=0)
    eng = Engine(cfg)
    import dataclasses
    # --graph: the 24 launches of a step also replayed as one HIP graph (measured equal to
    # eager launches; off by default so the default command profiles cleanly)
    eng_g = Engine(dataclasses.replace(cfg, graph=True)) if graph else None
    out = {"workload": "C4 256 requests, width 32, 2048 MB pool, 24 layers write+decode, 14q/2kv D64 fp16",
           "num_blocks": num_blocks}
    for name, trace in (("offline", Wl.baseline_trace(256, 0.0, 11)), ("poisson400", Wl.baseline_trace(256, 400.0, 11)),
                        ("ref_offline", Wl.ref_trace())):
        p, g, a = trace
        res = {}
        pols = [("continuous", lambda: run_continuous(p, g, a, eng))]
        if eng_g is not None:
            pols.append(("continuous_graph", lambda: run_continuous(p, g, a, eng_g)))
        pols.append(("static", lambda: run_static(p, g, a, eng, 32)))
        for pol, fn in pols:
            st = fn()
            res[pol] = {"iters": st.iters, "tokens": st.tokens,
                        "tokens_per_s": round(st.tokens / (st.wall_us * 1e-6), 1) if st.wall_us else 0.0,
                        "host_tokens_per_s": round(st.tokens / (st.host_wall_us * 1e-6), 1),
                        "slot_util": round(st.slot_util, 4), "avg_batch": round(st.avg_batch, 2),
                        "peak_blocks": st.peak_blocks, "p50_ms": round(st.p50_latency_us / 1e3, 3),
                        "p99_ms": round(st.p99_latency_us / 1e3, 3), "avg_ms": round(st.avg_latency_us / 1e3, 3),
                        "gpu_ms": round(st.gpu_us / 1e3, 2), "makespan_ms": round(st.wall_us / 1e3, 2)}
        out[name] = res
    # the same offline trace with each admitted prompt processed (K/V writes + causal
    # attention for all 24 layers) on the measured clock
    eng_pf = Engine(EngineConfig(n_heads=14, n_kv_heads=2, head_dim=64, block_size=16, num_blocks=num_blocks,
                                 max_batch=32, n_layers=24, dtype=KVC_F16, kv_write=True, clock_mode=0, prefill=True))
    p, g, a = Wl.baseline_trace(256, 0.0, 11)
    res = {}
    for pol, fn in (("continuous", lambda: run_continuous(p, g, a, eng_pf)),
                    ("static", lambda: run_static(p, g, a, eng_pf, 32))):
        st = fn()
        res[pol] = {"iters": st.iters, "tokens": st.tokens,
                    "tokens_per_s": round(st.tokens / (st.wall_us * 1e-6), 1) if st.wall_us else 0.0,
                    "prefill_ms": round(st.prefill_us / 1e3, 2), "gpu_ms": round(st.gpu_us / 1e3, 2),
                    "slot_util": round(st.slot_util, 4), "p50_ms": round(st.p50_latency_us / 1e3, 3),
                    "p99_ms": round(st.p99_latency_us / 1e3, 3)}
    out["offline_with_prefill"] = res
    return out


def copy_calibration(mib: int) -> int:
    """A plain copy of known size: under rocprofv3 --pmc its FETCH_SIZE / WRITE_SIZE per
    dispatch against mib MiB gives the scale factor applied to the decode counters."""
    from kvcache_amd._native import check, lib
    from kvcache_amd.device import DeviceBuffer, Event, synchronize
    n = mib << 20
    a, b = DeviceBuffer(n), DeviceBuffer(n)
    a.zero(); b.zero()
    synchronize()
    e0, e1 = Event(), Event()
    e0.record()
    for _ in range(10):
        check(lib().kvc_memcpy_d2d(b.ptr, a.ptr, n, None))
    e1.record()
    ms = e0.elapsed_ms(e1) / 10
    print(json.dumps({"copy_MiB": mib, "ms_per_copy": round(ms, 4), "GBps_read_plus_write": round(2 * n / ms / 1e6, 1)}))
    return 0


def summarize_rocprof(root: Path, patterns) -> None:
    """Summary of rocprofv3 CSV output (what profiles/*.txt hold): the kernel stats table;
    for kernels whose name contains one of `patterns`, the runs of consecutive dispatches
    (dispatch-id gaps of at most 8) with their mean duration and the mean of their last
    50 dispatches (a timed loop's); for --pmc output, each counter's mean per dispatch
    over the same runs."""
    import csv
    import glob
    import re
    from collections import defaultdict

    def short(name):
        n = re.sub(r"_ZN3kvc12_GLOBAL__N_112split_kernelIDF16_Li(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)EEEvPKiiNS_12DecodeParamsE",
                   r"split_kernel<f16, D\1, G\2, mode\3, WPB\4, U\5>", name)
        n = re.sub(r"_ZN3kvc12_GLOBAL__N_115gqa_mfma_kernelILi(\d+)ELi(\d+)ELi(\d+)EEEvPKiiNS_12DecodeParamsE",
                   r"gqa_mfma_kernel<D\1, mode\2, WPB\3>", n)
        n = re.sub(r"_ZN3kvc12_GLOBAL__N_112merge_kernelIDF16_Li(\d+)EEEvNS_12DecodeParamsE", r"merge_kernel<f16, D\1>", n)
        n = re.sub(r"_ZN3kvc12_GLOBAL__N_117read_probe_kernelEPKiiNS_11ProbeParamsE", "read_probe_kernel", n)
        return n[:72]

    def runs_of(rows):
        rows.sort()
        out, cur = [], [rows[0]]
        for r in rows[1:]:
            if r[0] - cur[-1][0] > 8:
                out.append(cur)
                cur = []
            cur.append(r)
        out.append(cur)
        return out

    for f in sorted(glob.glob(str(root / "**" / "*kernel_stats.csv"), recursive=True)):
        rows = sorted(csv.DictReader(open(f)), key=lambda r: -float(r["TotalDurationNs"]))
        print(f"# {Path(f).name}: kernels by total time")
        print(f"{'kernel':72s} {'calls':>8s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'pct':>6s}")
        for r in rows[:24]:
            print(f"{short(r['Name']):72s} {int(r['Calls']):8d} {float(r['AverageNs']) / 1e3:9.3f} "
                  f"{float(r['MinNs']) / 1e3:9.3f} {float(r['MaxNs']) / 1e3:9.3f} {float(r['Percentage']):6.2f}")
    for f in sorted(glob.glob(str(root / "**" / "*kernel_trace.csv"), recursive=True)):
        by = defaultdict(list)
        with open(f) as fh:
            for r in csv.DictReader(fh):
                if any(pt in r["Kernel_Name"] for pt in patterns):
                    by[r["Kernel_Name"]].append((int(r["Dispatch_Id"]), int(r["Start_Timestamp"]),
                                                 int(r["End_Timestamp"])))
        print(f"# {Path(f).name}: runs of consecutive dispatches (us)")
        for name, rows in sorted(by.items(), key=lambda kv: min(x[0] for x in kv[1])):
            print(short(name))
            for i, run in enumerate(runs_of(rows)):
                dur = [(e - s) / 1e3 for _, s, e in run]
                last = dur[-50:]
                print(f"  run {i:3d} dispatches {run[0][0]:>8d}-{run[-1][0]:<8d} n={len(run):6d} "
                      f"mean {sum(dur) / len(dur):9.3f} last50 {sum(last) / len(last):9.3f}")
    for f in sorted(glob.glob(str(root / "**" / "*counter_collection.csv"), recursive=True)):
        by = defaultdict(lambda: defaultdict(list))
        with open(f) as fh:
            for r in csv.DictReader(fh):
                if any(pt in r["Kernel_Name"] for pt in patterns):
                    by[r["Kernel_Name"]][r["Counter_Name"]].append((int(r["Dispatch_Id"]), float(r["Counter_Value"])))
        print(f"# {Path(f).name}: counters per dispatch")
        for name, ctrs in by.items():
            print(short(name))
            for c, rows in ctrs.items():
                for i, run in enumerate(runs_of([(d, v, 0) for d, v in rows])):
                    vals = [v for _, v, _ in run][-50:]
                    print(f"  {c:22s} run {i:3d} n={len(run):5d} last50 mean {sum(vals) / len(vals):14.1f} "
                          f"min {min(vals):14.1f} max {max(vals):14.1f}")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--split", type=int, default=0, help="decode split size in tokens (0 = automatic)")
    ap.add_argument("--rotate", type=int, default=4, help="pool copies cycled by the timed loop")
    ap.add_argument("--lengths", choices=["reference", "loguniform", "uniform"], default="reference",
                    help="reference generator, log-uniform variant, or every sequence at the reference mean")
    ap.add_argument("--no-shuffle", action="store_true", help="hand out pool blocks in order (diagnostic)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip configs 3 and 4")
    ap.add_argument("--sweep", type=str, default="",
                    help="comma list of split[:waves_per_block[:fused_merge]] to time (diagnostic)")
    ap.add_argument("--wpb", type=int, default=0, help="waves per workgroup (0 automatic, 4, 8)")
    ap.add_argument("--batch", type=int, default=4, help="wave-loads per batch (2, 4, 8)")
    ap.add_argument("--plan-target", type=int, default=0, help="planned path: tokens per unit (0 automatic)")
    ap.add_argument("--plan-sweep", type=str, default="", help="comma list of planned targets to time")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="only run 10 device-to-device copies of MIB MiB (HBM counter calibration) and exit")
    ap.add_argument("--chain", type=int, default=0, choices=[0, 1],
                    help="--only c5: 1 runs the linear layers between two attention launches as one launch")
    ap.add_argument("--only", choices=["c3", "c4", "c4_layer", "c5", "prefill"], default=None,
                    help="run only one extra workload and print its result (profiling)")
    ap.add_argument("--summarize-rocprof", metavar="DIR", default=None,
                    help="print a summary of the rocprofv3 CSV output under DIR (kernel stats, runs of "
                         "consecutive dispatches per kernel, --pmc counter means) and exit")
    ap.add_argument("--kernels", default="split_kernel,gqa_mfma_kernel,merge_kernel,read_probe_kernel",
                    help="with --summarize-rocprof: comma list of kernel-name substrings whose runs are listed")
    ap.add_argument("--warm", action="store_true",
                    help="also time the planned path on one pool copy (Infinity-Cache resident)")
    ap.add_argument("--graph", action="store_true",
                    help="configs 4 and 5: replay each decode step as a captured HIP graph (default: eager launches)")
    ap.add_argument("--tune", action="append", default=[], metavar="KEY=VALUE",
                    help="set a library tuning knob (kvc_set_tuning), e.g. wg_per_cu=4")
    ap.add_argument("--fused", type=int, default=-1,
                    help="merge mode: -1 automatic, 0 merge kernel, 1 fused with fences, 2 fused coherent")
    a = ap.parse_args()
    if a.summarize_rocprof:  # host-only: reads rocprofv3's CSV files
        summarize_rocprof(Path(a.summarize_rocprof), [k for k in a.kernels.split(",") if k])
        return 0
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {a.gpus} is not supported (the path shards by "
              "sequence with no exchange, so a single GPU's share at its real shape is what is measured)",
              file=sys.stderr)
        return 2

    from kvcache_amd import ops
    from kvcache_amd.device import has_device
    from kvcache_amd import workloads as Wl

    if not has_device():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    set_tuning("waves_per_block", a.wpb)
    set_tuning("fused_merge", a.fused)
    set_tuning("batch", a.batch)
    for kv in a.tune:
        key, val = kv.split("=", 1)
        set_tuning(key, int(val))
    if a.copy_calib:
        return copy_calibration(a.copy_calib)
    sweep_targets = [int(x) for x in a.plan_sweep.split(",") if x]
    if a.only:
        res = (bench_c3(a.steps, a.warmup, sweep_targets) if a.only == "c3" else
               bench_prefill(a.steps, a.warmup) if a.only == "prefill" else
               bench_c4_layer(a.steps, a.warmup) if a.only == "c4_layer" else
               bench_c5(graph=a.graph, chain=a.chain) if a.only == "c5" else bench_c4(graph=a.graph))
        print(json.dumps(res), flush=True)
        return 0
    if a.lengths == "reference":
        lens = Wl.ref_lengths()
    elif a.lengths == "loguniform":
        lens = Wl.loguniform_lengths(128, 16, 2048, 7)
    else:
        lens = np.full(128, int(round(Wl.ref_lengths().mean())), np.int32)
    N, Hq, Hkv, D, B = 128, 8, 8, 64, 16
    # device-lengths path: split 0 = the kernel plans its own chunks from the device lengths
    split = a.split
    log(f"C2: N={N} sum_len={int(lens.sum())} max={int(lens.max())} split={split} rotate={a.rotate}")
    W = build_c2(lens, Hq, Hkv, D, B, a.rotate, seed=12345, shuffle=not a.no_shuffle)
    err, host_data = check_c2(W, lens, Hq, Hkv, D, B, split)
    log(f"parity vs oracle: max abs err {err:.3e} (bar 2e-3)")
    if not err <= 2e-3:
        print(json.dumps({"metric": METRIC, "error": f"parity failure: max abs err {err}"}))
        return 1
    kv, total = alg_bytes(lens, Hq, Hkv, D, B)

    sweep = {}
    knobs = [("waves_per_block", 0), ("fused_merge", -1), ("batch", 4), ("last_chunk_first", 1)]
    for spec in [x for x in a.sweep.split(",") if x]:
        # split[:waves_per_block[:fused_merge[:batch[:last_chunk_first]]]]
        parts = [int(v) for v in spec.split(":")]
        for (key, dflt), val in zip(knobs, parts[1:] + [None] * len(knobs)):
            set_tuning(key, dflt if val is None else val)
        t, _ = time_decode(W, lens, Hq, Hkv, D, B, parts[0], 30, 5)
        sweep[spec] = round(t * 1e3, 2)
        log(f"sweep split:wpb:merge:batch:order={spec}: {sweep[spec]} us")
    set_tuning("waves_per_block", a.wpb)
    set_tuning("fused_merge", a.fused)
    set_tuning("batch", a.batch)
    set_tuning("last_chunk_first", 1)

    t_raw, _ = time_decode(W, lens, Hq, Hkv, D, B, split, a.steps, a.warmup)   # ms per launch
    raw = total / (t_raw * 1e-3) / 1e9
    log(f"C2 cold, device-lengths path ({'self-planned' if split == 0 else f'split {split}'}): "
        f"{t_raw * 1e3:.2f} us/launch, {raw:.1f} GB/s")
    for tgt in [int(x) for x in a.plan_sweep.split(",") if x]:
        tp, nu, nr, _ = time_planned(W, lens, Hq, Hkv, D, B, 30, 5, target=tgt)
        sweep[f"plan{tgt}"] = round(tp * 1e3, 2)
        log(f"sweep planned target={tgt}: {tp * 1e3:.2f} us ({nu} units, {nr} records)")
    t_launch, n_units, n_records, launch = time_planned(W, lens, Hq, Hkv, D, B, a.steps, a.warmup, target=a.plan_target)
    err_planned = check_planned(W, launch, lens, Hq, Hkv, D, B, host_data)
    log(f"planned parity vs oracle: max abs err {err_planned:.3e}")
    if not err_planned <= 2e-3:
        print(json.dumps({"metric": METRIC, "error": f"planned parity failure: max abs err {err_planned}"}))
        return 1
    ms_per_step = t_launch
    t_probe, _ = practical_ceiling(W, lens, Hq, Hkv, D, B, a.steps, a.warmup, target=a.plan_target)
    log(f"C2 read-only probe over the same plan: {t_probe:.2f} us/launch")
    floor = launch_floor(200, 20)
    log(f"launch floor (empty kernels back to back): {floor}")
    traffic, sym = measured_traffic()
    prof_us = profiled_launch_us()
    traffic_src = (f"rocprofv3 --pmc FETCH_SIZE x2.0 + WRITE_SIZE x1.0 per dispatch of {sym} "
                   f"({TRAFFIC_SUMMARY.relative_to(ROOT)})") if traffic else None
    achieved = total / (t_launch * 1e-3) / 1e9
    log(f"C2 cold, planned path ({n_units} units): {t_launch * 1e3:.2f} us/launch, {achieved:.1f} GB/s")
    warm = None
    if a.warm:
        t_warm, _, _, _ = time_planned(W, lens, Hq, Hkv, D, B, a.steps, a.warmup, target=a.plan_target, rotate=1)
        warm = round(total / (t_warm * 1e-3) / 1e9, 1)
        log(f"C2 warm (one pool, Infinity-Cache resident): {t_warm * 1e3:.2f} us, {warm} GB/s")

    plan_cost = host_plan_cost(W, lens, Hq, Hkv, D, B)
    plan_cost["plan_plus_kernel_us"] = round(plan_cost["us_per_plan"] + t_launch * 1e3, 2)
    plan_cost["plan_plus_kernel_frac"] = round(total / ((plan_cost["us_per_plan"] + t_launch * 1e3) * 1e-6) / 1e9 /
                                               HBM_PEAK_GBS, 4)
    try:
        for mode, key in ((1, "pipelined"), (0, "pipelined_copy_stream")):
            pp = host_plan_pipelined(W, lens, Hq, Hkv, D, B, a.steps, a.warmup, mode)
            pp["what"] = ("C++ serving loop (tests/cpp/plan_pipeline.cpp): the host plans every step while the "
                          "previous step's kernel runs; compute-stream events around the steps")
            pp["frac_hbm_peak"] = round(total / (pp["us_per_step"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
            plan_cost[key] = pp
    except Exception as e:  # noqa: BLE001 -- reported, not fatal to the headline
        plan_cost["pipelined"] = {"error": repr(e)}
    plan_cost["per_step_on_device"] = ("a serving loop that re-plans every step can instead pass the lengths in "
                                       "device memory: device_lengths_path plans each launch on the GPU")
    log(f"host plan: {plan_cost}")

    extras = {}
    if not a.no_extras:
        del W["pools"]
        try:
            extras["c2_loguniform"] = c2_variant(Wl.loguniform_lengths(128, 16, 2048, 7), a.steps, a.warmup, a.rotate)
            log(f"C2 log-uniform: {extras['c2_loguniform']}")
        except Exception as e:  # noqa: BLE001 -- extras never hide the headline
            extras["c2_loguniform"] = {"error": repr(e)}
        try:
            extras["c2_contiguous_vs_paged"] = bench_c2_contiguous(a.steps, a.warmup, a.rotate)
            log(f"C2 contiguous vs paged: {extras['c2_contiguous_vs_paged']}")
        except Exception as e:  # noqa: BLE001 -- extras never hide the headline
            extras["c2_contiguous_vs_paged"] = {"error": repr(e)}
        try:
            extras["single_seq"] = bench_single_seq()
            log(f"single sequence sweep: {extras['single_seq']}")
        except Exception as e:  # noqa: BLE001
            extras["single_seq"] = {"error": repr(e)}
        try:
            extras["c4_layer"] = bench_c4_layer(a.steps, a.warmup)
            log(f"C4 layer kernel: {extras['c4_layer']}")
        except Exception as e:  # noqa: BLE001
            extras["c4_layer"] = {"error": repr(e)}
        try:
            extras["c3"] = bench_c3(a.steps, a.warmup)
            log(f"C3: {extras['c3']}")
        except Exception as e:  # noqa: BLE001 -- extras never hide the headline
            extras["c3"] = {"error": repr(e)}
        try:
            extras["prefill"] = bench_prefill(a.steps, a.warmup)
            log(f"prefill: {extras['prefill']}")
        except Exception as e:  # noqa: BLE001
            extras["prefill"] = {"error": repr(e)}
        try:
            extras["c5"] = bench_c5(graph=a.graph)
            log(f"C5: {extras['c5']}")
            ch = bench_c5(chain=1)
            extras["c5"]["with_layer_chain"] = {k: ch[k] for k in ("ms_per_decode_step", "tokens_per_s", "decode_ms",
                                                                    "chain_launches")}
            log(f"C5 with the layer chain: {extras['c5']['with_layer_chain']}")
        except Exception as e:  # noqa: BLE001
            extras["c5"] = {"error": repr(e)}
        try:
            extras["c4"] = bench_c4(graph=a.graph)
            log(f"C4: {json.dumps(extras['c4'])}")
        except Exception as e:  # noqa: BLE001
            extras["c4"] = {"error": repr(e)}

    cpu = None
    if not a.no_cpu_baseline:
        cpu = cpu_baseline(host_data, W, lens, Hkv, B, D, a.cpu_seconds, total)
        log(f"CPU baseline: {cpu}")

    line = {
        "metric": METRIC, "value": round(achieved, 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": "C2 batched ragged paged decode: N=128, reference lengths (seed 12345, sum 83212, "
                               "max 2022), H=8 (MHA), D=64, BLOCK=16, fp16 KV, fp32 accumulate, shuffled free list",
                   "lengths": a.lengths, "path": "planned (host plan resident, one kernel per step)",
                   "planned_units": n_units, "rotating_pool_copies": a.rotate, "parallelism": "single GPU"},
        "device_lengths_path": {"path": "self-planned (launch_batched_paged: the kernel plans from the device "
                                        "lengths, no host plan)" if split == 0 else f"split {split}",
                                "us_per_step": round(t_raw * 1e3, 3), "GBps": round(raw, 1),
                                "frac_hbm_peak": round(raw / HBM_PEAK_GBS, 4),
                                "profile_mean_launch_us": profile_values().get("device_lengths_timed_mean_us")},
        "host_plan": plan_cost,
        "pct_hbm_peak": round(100 * achieved / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": "split_kernel<_Float16, D=64, G=1, kPlannedUniform, ...> (planned paged decode, "
                               "fused LSE merge)",
                     "algorithmic_bytes_per_launch": total, "kv_bytes_per_launch": kv,
                     "mean_launch_us": round(t_launch * 1e3, 3),
                     "practical_ceiling_us": round(t_probe, 3),
                     "practical_ceiling": {"what": "kvc_read_probe_planned: the same work list, grid order, loads "
                                                   "and rotating pools, no arithmetic (the access pattern's floor)",
                                           "us": round(t_probe, 3),
                                           "GBps": round(total / (t_probe * 1e-6) / 1e9, 1),
                                           "frac": round(total / (t_probe * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                           "decode_over_probe": round(t_launch * 1e3 / t_probe, 4)},
                     "launch_floor": dict(floor, what="kvc_empty_launch back to back: the per-launch cost before "
                                                      "any work"),
                     "profile": ({"file": str(STATS_SUMMARY.relative_to(ROOT)), "mean_launch_us": prof_us,
                                  "frac": round(total / (prof_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                  "note": "rocprofv3 kernel trace of the headline command (bench.py --no-extras "
                                          "--no-cpu-baseline) on an earlier box; achieved/frac above come from "
                                          "this run's HIP events",
                                  "across_boxes_us": "33.2-34.4 (HIP events of the planned step on the boxes "
                                                     "measured; the profile is one of them)"}
                                 if prof_us else None)},
        "warm_GBps": warm,
        "memory": memory_accounting(lens, Hkv, D, B),
        "parity_max_abs_err": err,
        "cpu_baseline": cpu,
        "extras": extras,
    }
    if sweep:
        line["split_sweep_us"] = sweep
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
