"""ctypes binding of libkvcache_amd.so (the C ABI in include/kvc_abi.h).

The library is loaded from this package directory only.  If it is missing the
import of any op fails loudly: there is no CPU fallback for the hot path.
"""
from __future__ import annotations

import ctypes as C
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libkvcache_amd.so"

KVC_OK = 0
KVC_ERR_ARG = 1
KVC_ERR_UNSUPPORTED = 2
KVC_ERR_HIP = 3
KVC_ERR_NOMEM = 4
KVC_ERR_WORKSPACE = 5
KVC_ERR_STATE = 6
KVC_F32 = 0
KVC_F16 = 1
KVC_DECODE_PLANNED = 0
KVC_DECODE_DEVICE_LENGTHS = 1

vp = C.c_void_p
i32 = C.c_int
f32 = C.c_float
f64 = C.c_double
sz = C.c_size_t
u64 = C.c_uint64
ip = C.POINTER(C.c_int)


class KvcError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"kvc status {status}: {msg}")
        self.status = status


class EngineConfigC(C.Structure):
    _fields_ = [
        ("n_heads", i32), ("n_kv_heads", i32), ("head_dim", i32), ("block_size", i32),
        ("num_blocks", i32), ("max_batch", i32), ("n_layers", i32), ("dtype", i32),
        ("kv_write", i32), ("clock_mode", i32), ("virt_c0", f64), ("virt_c1", f64),
        ("virt_c2", f64), ("device", i32), ("split_tokens", i32), ("decode_path", i32), ("prefill", i32), ("seed", u64),
        ("graph", i32),
    ]


class QwenConfigC(C.Structure):
    _fields_ = [
        ("layers", i32), ("hidden", i32), ("n_heads", i32), ("n_kv_heads", i32), ("head_dim", i32),
        ("inter", i32), ("vocab", i32), ("eps", C.c_float), ("theta", C.c_float), ("init_std", C.c_float),
        ("block_size", i32), ("num_blocks", i32), ("max_batch", i32), ("max_rows", i32), ("seed", u64),
        ("step_path", i32), ("graph", i32), ("prefill_rows", i32), ("chain", i32),
    ]


class QwenStatsC(C.Structure):
    _fields_ = [
        ("steps", i32), ("finished", i32), ("tokens", C.c_longlong), ("prompt_tokens", C.c_longlong),
        ("wall_us", f64), ("prefill_us", f64), ("decode_us", f64), ("graph_steps", C.c_longlong),
        ("graph_captures", C.c_longlong), ("chain_launches", C.c_longlong),
    ]


class LayerChainC(C.Structure):
    """kvc_layer_chain (include/kvc_abi.h)."""
    _fields_ = [
        ("M", i32), ("H", i32), ("Hq", i32), ("Hkv", i32), ("D", i32), ("I", i32), ("eps", C.c_float),
        ("theta", C.c_float), ("x", C.c_void_p), ("att", C.c_void_p), ("w_o", C.c_void_p), ("ln2", C.c_void_p),
        ("w_gate_up", C.c_void_p), ("act", C.c_void_p), ("w_down", C.c_void_p), ("q", C.c_void_p),
        ("k", C.c_void_p), ("v", C.c_void_p), ("ln1", C.c_void_p), ("w_qkv", C.c_void_p), ("b_qkv", C.c_void_p),
        ("pos", C.c_void_p),
    ]


class EngineStatsC(C.Structure):
    _fields_ = [
        ("iters", i32), ("tokens", C.c_longlong), ("gpu_us", f64), ("wall_us", f64),
        ("slot_steps", C.c_longlong), ("useful_steps", C.c_longlong), ("peak_blocks", i32),
        ("finished", i32), ("avg_latency_us", f64), ("p50_latency_us", f64),
        ("p99_latency_us", f64), ("step_digest", u64), ("host_wall_us", f64), ("prefill_us", f64),
    ]


class RequestC(C.Structure):
    _fields_ = [("id", i32), ("arrival_us", f64), ("prompt_len", i32), ("gen_len", i32)]


# name -> (restype, argtypes)
_SIGS = {
    "kvc_version": (i32, []),
    "kvc_status_string": (C.c_char_p, [i32]),
    "kvc_last_error": (C.c_char_p, []),
    "kvc_device_count": (i32, [ip]),
    "kvc_set_tuning": (i32, [C.c_char_p, i32]),
    "kvc_get_tuning": (i32, [C.c_char_p, ip]),
    "kvc_malloc": (i32, [C.POINTER(vp), sz]),
    "kvc_free": (i32, [vp]),
    "kvc_host_alloc": (i32, [C.POINTER(vp), sz]),
    "kvc_host_free": (i32, [vp]),
    "kvc_memcpy_h2d": (i32, [vp, vp, sz, vp]),
    "kvc_memcpy_d2h": (i32, [vp, vp, sz, vp]),
    "kvc_memcpy_d2d": (i32, [vp, vp, sz, vp]),
    "kvc_memset": (i32, [vp, i32, sz, vp]),
    "kvc_stream_create": (i32, [C.POINTER(vp)]),
    "kvc_stream_destroy": (i32, [vp]),
    "kvc_stream_synchronize": (i32, [vp]),
    "kvc_device_synchronize": (i32, []),
    "kvc_event_create": (i32, [C.POINTER(vp)]),
    "kvc_event_destroy": (i32, [vp]),
    "kvc_event_record": (i32, [vp, vp]),
    "kvc_event_synchronize": (i32, [vp]),
    "kvc_stream_wait_event": (i32, [vp, vp]),
    "kvc_event_elapsed_ms": (i32, [C.POINTER(f32), vp, vp]),
    "kvc_step_upload": (i32, [vp, vp, sz, vp]),
    "kvc_fill_normal": (i32, [vp, sz, i32, u64, f32, vp]),
    "kvc_append": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, i32, vp]),
    "kvc_write_kv": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp]),
    "kvc_write_kv_dev": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp]),
    "kvc_batched_write_kv": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp]),
    "kvc_write_kv_slots": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp]),
    "kvc_decode": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, f32, i32, vp]),
    "kvc_paged_decode": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, f32, i32, vp]),
    "kvc_batched_decode": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32, i32, vp, sz, vp]),
    "kvc_batched_decode_split": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32, i32, i32, vp, sz, vp]),
    "kvc_batched_paged_decode": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32, i32, vp, sz, vp]),
    "kvc_batched_paged_decode_split": (
        i32, [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32, i32, i32, vp, sz, vp]),
    "kvc_decode_workspace_size": (sz, [i32, i32, i32, i32, i32, i32, i32, i32]),
    "kvc_decode_auto_split": (i32, [i32, i32, i32, i32, i32, i32, i32]),
    "kvc_decode_plan_entry_ints": (i32, [i32, i32, i32, i32, i32]),
    "kvc_decode_plan": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32, vp, i32, ip, ip]),
    "kvc_decode_planned_workspace_size": (sz, [i32, i32, i32, i32, i32, i32]),
    "kvc_batched_paged_decode_planned": (
        i32, [vp, vp, vp, vp, i32, vp, i32, i32, i32, i32, i32, f32, i32, vp, i32, i32, vp, sz, vp]),
    "kvc_batched_paged_append_decode_planned": (
        i32, [vp, vp, vp, vp, vp, vp, vp, i32, vp, i32, i32, i32, i32, i32, f32, i32, vp, i32, i32, vp, sz, vp]),
    "kvc_paged_causal_attn": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32, i32, vp, sz, vp]),
    "kvc_paged_causal_attn_workspace_size": (sz, [i32, i32, i32, i32, i32, i32, i32]),
    "kvc_paged_causal_attn_dev": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, f32, i32, vp, sz, vp]),
    "kvc_paged_causal_attn_dev_workspace_size": (sz, [i32, i32, i32, i32, i32, i32]),
    "kvc_paged_causal_attn_dev_noalloc": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, f32, i32, vp]),
    "kvc_embed_gather": (i32, [vp, vp, vp, i32, i32, i32, vp]),
    "kvc_rmsnorm": (i32, [vp, vp, vp, i32, i32, f32, vp]),
    "kvc_add_bias": (i32, [vp, vp, i32, i32, vp]),
    "kvc_add_residual": (i32, [vp, vp, sz, vp]),
    "kvc_silu_mul": (i32, [vp, vp, vp, sz, vp]),
    "kvc_rope": (i32, [vp, vp, i32, i32, i32, i32, f32, vp]),
    "kvc_rope_dev": (i32, [vp, vp, i32, i32, i32, f32, vp]),
    "kvc_argmax": (i32, [vp, i32, i32, vp, vp]),
    "kvc_linear": (i32, [vp, vp, vp, i32, i32, i32, i32, vp]),
    "kvc_rows_workspace_size": (sz, [i32, i32]),
    "kvc_rows_linear": (i32, [vp, vp, vp, i32, i32, i32, vp, f32, i32, vp, vp, sz, vp]),
    "kvc_rows_qkv": (i32, [vp, vp, vp, vp, vp, f32, vp, vp, vp, i32, i32, i32, i32, i32, f32, vp, vp]),
    "kvc_rows_swiglu": (i32, [vp, vp, vp, f32, vp, i32, i32, i32, vp, vp]),
    "kvc_rows_lm_head": (i32, [vp, vp, vp, vp, f32, vp, i32, i32, i32, vp, vp, sz, vp]),
    "kvc_embed_gather_dev": (i32, [vp, vp, vp, vp, i32, i32, i32, vp]),
    "kvc_batched_paged_decode_planned_dev": (
        i32, [vp, vp, vp, vp, vp, vp, vp, i32, vp, i32, i32, i32, i32, i32, f32, i32, vp, i32, i32, vp, vp, sz, vp]),
    "kvc_decode_plan_capacity": (i32, [i32, C.c_longlong, i32, i32, i32, i32, i32, ip]),
    "kvc_decode_plan_chunk": (i32, [vp, i32, i32, i32, i32, i32, i32, i32, ip]),
    "kvc_read_probe_planned": (i32, [vp, vp, vp, i32, vp, i32, i32, i32, i32, i32, i32, vp, vp]),
    "kvc_empty_launch": (i32, [i32, vp]),
    "kvc_stream_is_capturing": (i32, [vp, ip]),
    "kvc_check_device_errors": (i32, [vp]),
    "kvc_graph_begin": (i32, [vp]),
    "kvc_graph_end": (i32, [vp, C.POINTER(vp)]),
    "kvc_graph_launch": (i32, [vp, vp]),
    "kvc_graph_destroy": (i32, [vp]),
    "kvc_rows_set_tuning": (i32, [i32, i32, i32]),
    "kvc_rows_chain_workspace_size": (sz, [i32, i32]),
    "kvc_rows_chain": (i32, [vp, vp, sz, vp]),
    "kvc_flash_decode": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, f32, i32, i32, vp, sz, vp]),
    "kvc_flash_decode_workspace_size": (sz, [i32, i32, i32]),
    "kvc_block_allocator_create": (i32, [i32, C.POINTER(vp)]),
    "kvc_block_allocator_destroy": (None, [vp]),
    "kvc_block_allocator_alloc": (i32, [vp]),
    "kvc_block_allocator_free": (None, [vp, vp, i32]),
    "kvc_block_allocator_reset": (None, [vp]),
    "kvc_block_allocator_free_count": (i32, [vp]),
    "kvc_block_allocator_used_count": (i32, [vp]),
    "kvc_block_allocator_shuffle": (None, [vp, u64]),
    "kvc_blocks_needed": (i32, [i32, i32]),
    "kvc_engine_create": (i32, [C.POINTER(EngineConfigC), C.POINTER(vp)]),
    "kvc_qwen_create": (i32, [C.POINTER(QwenConfigC), C.POINTER(vp)]),
    "kvc_qwen_destroy": (None, [vp]),
    "kvc_qwen_tensor": (i32, [vp, C.c_char_p, i32, C.POINTER(vp), C.POINTER(sz)]),
    "kvc_qwen_serve": (i32, [vp, i32, vp, vp, vp, vp, C.POINTER(QwenStatsC)]),
    "kvc_qwen_prefill_logits": (i32, [vp, vp, i32, vp, vp]),
    "kvc_qwen_load_weights": (i32, [vp, C.c_char_p]),
    "kvc_qwen_save_weights": (i32, [vp, C.c_char_p]),
    "kvc_engine_destroy": (None, [vp]),
    "kvc_engine_reset": (i32, [vp]),
    "kvc_engine_add_request": (i32, [vp, i32, i32, f64]),
    "kvc_engine_step": (i32, [vp, ip]),
    "kvc_engine_run": (i32, [vp, C.POINTER(EngineStatsC)]),
    "kvc_engine_stats_get": (i32, [vp, C.POINTER(EngineStatsC)]),
    "kvc_engine_last_step": (i32, [vp, ip, ip, ip, ip, i32, ip, ip, C.POINTER(vp)]),
    "kvc_run_static": (i32, [vp, C.POINTER(RequestC), i32, i32, C.POINTER(EngineStatsC)]),
}

_lib = None
_lock = threading.Lock()


def lib() -> C.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"{LIB_PATH} is missing: build it with `python -m kvcache_amd.build` "
                        "(there is no CPU fallback for the decode path)")
                # kernel arguments in device memory (unless the caller chose otherwise): every
                # decode workgroup reads its parameter block from the kernel-argument segment,
                # and where the HIP runtime's default puts that segment in host memory each
                # read crosses PCIe (MI355X, same box: config 2 37.4 vs 33.5 us per launch,
                # one config-4 layer 8.0 vs 6.0 us).  HIP reads it when it initialises, which
                # the library's first call does.
                os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "1")
                L = C.CDLL(str(LIB_PATH))
                for name, (res, args) in _SIGS.items():
                    fn = getattr(L, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != KVC_OK:
        L = lib()
        raise KvcError(rc, f"{L.kvc_status_string(rc).decode()}: {L.kvc_last_error().decode()}")


def exported_names() -> list[str]:
    return sorted(_SIGS)
