"""Python mirror of the reference's kernel launchers (src/include/kv_cache.h:2-34,
src/include/qwen_kernels.h:15-37), over the C ABI.

Same names and argument order as the reference; every pointer argument may be a
DeviceBuffer or a raw device address (int).  Extra keyword arguments carry what
the MI355X boundary adds: dtype (KVC_F32 default, as the reference), Hkv for
GQA, split size, workspace and stream.  Failures raise KvcError (the reference
printed and exited).  Parity tests call these exactly as the reference's
drivers call the CUDA launchers.
"""
from __future__ import annotations

from ._native import KVC_ERR_ARG, KVC_F16, KVC_F32, KvcError, check, lib
from .device import DeviceBuffer

__all__ = [
    "launch_append", "launch_decode", "launch_paged", "launch_batched_decode", "launch_batched_paged",
    "launch_batched_paged_flash", "launch_flash_decode", "qk_write_kv", "qk_batched_write_kv",
    "qk_batched_paged_decode_attn", "write_kv_slots", "decode_workspace_size", "decode_auto_split",
    "decode_plan", "planned_workspace_size", "launch_batched_paged_planned", "launch_batched_paged_append_planned",
    "flash_decode_workspace_size", "qk_paged_causal_attn", "qkcuda_paged_causal_attn", "qkcuda_write_kv",
    "qkcuda_rope", "check_device_errors", "stream_is_capturing", "KVC_F16", "KVC_F32",
]


def _p(x):
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)


def _ws(workspace):
    if workspace is None:
        return None, 0
    if isinstance(workspace, DeviceBuffer):
        return workspace.ptr, workspace.nbytes
    ptr, nbytes = workspace
    return int(ptr), int(nbytes)


def launch_append(k_new, v_new, k_cache, v_cache, pos, H, D, S, *, dtype=KVC_F32, stream=None):
    check(lib().kvc_append(_p(k_new), _p(v_new), _p(k_cache), _p(v_cache), pos, H, D, S, dtype, stream))


def launch_decode(q, k_cache, v_cache, out, cur_len, H, D, S, scale, *, dtype=KVC_F32, stream=None):
    check(lib().kvc_decode(_p(q), _p(k_cache), _p(v_cache), _p(out), cur_len, H, D, S, scale, dtype, stream))


def launch_paged(q, k_pool, v_pool, block_table, out, cur_len, H, D, BLOCK, scale, *, dtype=KVC_F32, stream=None):
    check(lib().kvc_paged_decode(_p(q), _p(k_pool), _p(v_pool), _p(block_table), _p(out), cur_len, H, D, BLOCK,
                                 scale, dtype, stream))


def launch_batched_decode(q, k_cache, v_cache, cur_len, out, N, H, D, MAXS, cap, scale, *, Hkv=None,
                          dtype=KVC_F32, split=0, workspace=None, stream=None):
    ws, wsb = _ws(workspace)
    check(lib().kvc_batched_decode_split(_p(q), _p(k_cache), _p(v_cache), _p(cur_len), _p(out), N, H,
                                         Hkv or H, D, MAXS, cap, scale, dtype, split, ws, wsb, stream))


def launch_batched_paged(q, k_pool, v_pool, table_all, tab_off, cur_len, out, N, H, D, BLOCK, cap, scale, *,
                         Hkv=None, dtype=KVC_F32, split=0, workspace=None, stream=None):
    ws, wsb = _ws(workspace)
    check(lib().kvc_batched_paged_decode_split(_p(q), _p(k_pool), _p(v_pool), _p(table_all), _p(tab_off),
                                               _p(cur_len), _p(out), N, H, Hkv or H, D, BLOCK, cap, scale, dtype,
                                               split, ws, wsb, stream))


# Same kernel as launch_batched_paged (online softmax is the only implementation).
launch_batched_paged_flash = launch_batched_paged


def launch_flash_decode(q, k_cache, v_cache, out, cur_len, H, D, S, scale, num_splits, *, dtype=KVC_F32,
                        workspace=None, stream=None):
    ws, wsb = _ws(workspace)
    check(lib().kvc_flash_decode(_p(q), _p(k_cache), _p(v_cache), _p(out), cur_len, H, D, S, scale, num_splits,
                                 dtype, ws, wsb, stream))


def qk_write_kv(k, v, k_pool, v_pool, block_table_dev, start_pos, L, Hkv, D, BLOCK, *, dtype=KVC_F16, stream=None):
    check(lib().kvc_write_kv(_p(k), _p(v), _p(k_pool), _p(v_pool), _p(block_table_dev), start_pos, L, Hkv, D, BLOCK,
                             dtype, stream))


def qk_batched_write_kv(k, v, k_pool, v_pool, table_all, tab_off, wpos, N, Hkv, D, BLOCK, *, dtype=KVC_F16,
                        stream=None):
    check(lib().kvc_batched_write_kv(_p(k), _p(v), _p(k_pool), _p(v_pool), _p(table_all), _p(tab_off), _p(wpos), N,
                                     Hkv, D, BLOCK, dtype, stream))


def qk_batched_paged_decode_attn(q, out, k_pool, v_pool, table_all, tab_off, cur_len, N, Hq, Hkv, D, BLOCK, scale,
                                 *, cap=0, dtype=KVC_F16, split=0, workspace=None, stream=None):
    """qwen_kernels.h:35-37: no length bound is needed (cap = 0: the kernel plans its
    own chunks from the device lengths; larger batches run as consecutive launches;
    shapes without a self-planned path read the longest length from the device); a
    cap > 0 raises the planning budget."""
    ws, wsb = _ws(workspace)
    check(lib().kvc_batched_paged_decode_split(_p(q), _p(k_pool), _p(v_pool), _p(table_all), _p(tab_off),
                                               _p(cur_len), _p(out), N, Hq, Hkv, D, BLOCK, cap, scale, dtype, split,
                                               ws, wsb, stream))


def decode_plan(lens, Hq, Hkv, D, BLOCK, *, tab_off=None, table=None, dtype=KVC_F16, target_tokens=0):
    """Host-side plan of a batched paged decode (kvc_decode_plan): returns
    (work [units, entry_ints] int32, n_units, n_records).  `table` (the host copy of
    table_all) lets grouped-query plans carry each unit's block ids."""
    import ctypes as C

    import numpy as np
    lens = np.ascontiguousarray(np.asarray(lens, dtype=np.int32))
    toff = None if tab_off is None else np.ascontiguousarray(np.asarray(tab_off, dtype=np.int32))
    tab = None if table is None else np.ascontiguousarray(np.asarray(table, dtype=np.int32))
    tp = None if toff is None else toff.ctypes.data
    tbp, tbl = (None, 0) if tab is None else (tab.ctypes.data, len(tab))
    nu, nr = C.c_int(0), C.c_int(0)
    L = lib()
    ipu = int(L.kvc_decode_plan_entry_ints(Hq, Hkv, D, BLOCK, dtype))
    if ipu <= 0:
        raise KvcError(KVC_ERR_ARG, f"no plan for Hq={Hq} Hkv={Hkv} D={D} BLOCK={BLOCK} dtype={dtype}")
    check(L.kvc_decode_plan(lens.ctypes.data, tp, tbp, tbl, len(lens), Hq, Hkv, D, BLOCK, dtype, target_tokens, None,
                            0, C.byref(nu), C.byref(nr)))
    work = np.zeros((max(nu.value, 1), ipu), dtype=np.int32)
    check(L.kvc_decode_plan(lens.ctypes.data, tp, tbp, tbl, len(lens), Hq, Hkv, D, BLOCK, dtype, target_tokens,
                            work.ctypes.data, nu.value, C.byref(nu), C.byref(nr)))
    return work[: nu.value], nu.value, nr.value


def decode_plan_chunk(lens, Hq, Hkv, D, BLOCK, *, dtype=KVC_F16, target_tokens=0) -> int:
    """The chunk target (tokens) kvc_decode_plan uses for these lengths."""
    import ctypes as C

    import numpy as np
    lens = np.ascontiguousarray(np.asarray(lens, dtype=np.int32))
    out = C.c_int(0)
    check(lib().kvc_decode_plan_chunk(lens.ctypes.data, len(lens), Hq, Hkv, D, BLOCK, dtype, target_tokens,
                                      C.byref(out)))
    return out.value


def planned_workspace_size(Hq, Hkv, D, n_records, *, BLOCK=16, dtype=KVC_F16) -> int:
    return int(lib().kvc_decode_planned_workspace_size(Hq, Hkv, D, BLOCK, dtype, n_records))


def launch_batched_paged_planned(q, k_pool, v_pool, table_all, table_len, out, N, Hq, Hkv, D, BLOCK, scale,
                                 work_dev, n_units, n_records, *, dtype=KVC_F16, workspace=None, stream=None):
    ws, wsb = _ws(workspace)
    check(lib().kvc_batched_paged_decode_planned(_p(q), _p(k_pool), _p(v_pool), _p(table_all), int(table_len),
                                                 _p(out), N, Hq, Hkv, D, BLOCK, scale, dtype, _p(work_dev), n_units,
                                                 n_records, ws, wsb, stream))


def launch_batched_paged_append_planned(q, k_new, v_new, wpos, k_pool, v_pool, table_all, table_len, out, N, Hq,
                                        Hkv, D, BLOCK, scale, work_dev, n_units, n_records, *, dtype=KVC_F16,
                                        workspace=None, stream=None):
    """qk_batched_write_kv followed by qk_batched_paged_decode_attn as one planned launch."""
    ws, wsb = _ws(workspace)
    check(lib().kvc_batched_paged_append_decode_planned(_p(q), _p(k_new), _p(v_new), _p(wpos), _p(k_pool), _p(v_pool),
                                                        _p(table_all), int(table_len), _p(out), N, Hq, Hkv, D, BLOCK,
                                                        scale, dtype, _p(work_dev), n_units, n_records, ws, wsb,
                                                        stream))


def qk_paged_causal_attn(q, out, k_pool, v_pool, block_table, q_pos_base, Nq, Hq, Hkv, D, BLOCK, scale, *,
                         dtype=KVC_F16, workspace=None, stream=None):
    """Prompt attention of one sequence (qwen_kernels.h:19-21): query i at position
    q_pos_base + i attends causally over the paged pools through block_table."""
    ws, wsb = _ws(workspace)
    check(lib().kvc_paged_causal_attn(_p(q), _p(out), _p(k_pool), _p(v_pool), _p(block_table), q_pos_base, Nq, Hq,
                                      Hkv, D, BLOCK, scale, dtype, ws, wsb, stream))


def qkcuda_paged_causal_attn(q, out, k_pool, v_pool, block_table, dev_q_pos_base, Nq, Hq, Hkv, D, BLOCK, scale, *,
                             dtype=KVC_F16, workspace=None, stream=None):
    """qwen_kernels.h:45-47: qk_paged_causal_attn with q_pos_base in device memory."""
    ws, wsb = _ws(workspace)
    check(lib().kvc_paged_causal_attn_dev(_p(q), _p(out), _p(k_pool), _p(v_pool), _p(block_table),
                                          _p(dev_q_pos_base), Nq, Hq, Hkv, D, BLOCK, scale, dtype, ws, wsb, stream))


def qkcuda_write_kv(k, v, k_pool, v_pool, block_table_dev, dev_start_pos, L, Hkv, D, BLOCK, *, dtype=KVC_F16,
                    stream=None):
    """qwen_kernels.h:43-44: qk_write_kv with start_pos in device memory."""
    check(lib().kvc_write_kv_dev(_p(k), _p(v), _p(k_pool), _p(v_pool), _p(block_table_dev), _p(dev_start_pos), L,
                                 Hkv, D, BLOCK, dtype, stream))


def qkcuda_rope(x, L, n_heads, D, dev_pos_base, theta, *, stream=None):
    """qwen_kernels.h:42: qk_rope with pos_base in device memory."""
    check(lib().kvc_rope_dev(_p(x), _p(dev_pos_base), L, n_heads, D, theta, stream))


# ---- decoder-step operations (qwen_kernels.h:7-13,22-24) -----------------------------
def qk_embed_gather(out, embed, ids, L, H, V, *, stream=None):
    check(lib().kvc_embed_gather(_p(out), _p(embed), _p(ids), L, H, V, stream))


def qk_rmsnorm(out, x, w, L, H, eps, *, stream=None):
    check(lib().kvc_rmsnorm(_p(out), _p(x), _p(w), L, H, eps, stream))


def qk_add_bias(x, bias, L, N, *, stream=None):
    check(lib().kvc_add_bias(_p(x), _p(bias), L, N, stream))


def qk_add_residual(x, y, n, *, stream=None):
    check(lib().kvc_add_residual(_p(x), _p(y), n, stream))


def qk_silu_mul(out, gate, up, n, *, stream=None):
    check(lib().kvc_silu_mul(_p(out), _p(gate), _p(up), n, stream))


def qk_rope(x, L, n_heads, D, pos_base, theta, *, stream=None):
    check(lib().kvc_rope(_p(x), None, pos_base, L, n_heads, D, theta, stream))


def qk_rope_pos(x, n_rows, n_heads, D, pos, theta, *, stream=None):
    check(lib().kvc_rope(_p(x), _p(pos), 0, n_rows, n_heads, D, theta, stream))


def qk_argmax(logits, L, V, out, *, stream=None):
    check(lib().kvc_argmax(_p(logits), L, V, _p(out), stream))


def linear(y, x, w, M, N, K, *, out_dtype=KVC_F16, stream=None):
    """y[M,N] = x[M,K] w[N,K]^T (fp16 inputs, fp32 accumulation)."""
    check(lib().kvc_linear(_p(y), _p(x), _p(w), M, N, K, out_dtype, stream))


# ---- decode-step linear layers over at most 32 rows (fused matrix-core kernels) ----------
def rows_workspace_size(N, K) -> int:
    return int(lib().kvc_rows_workspace_size(N, K))


def rows_linear(y, x, w, M, N, K, *, norm_w=None, eps=1e-6, residual=False, dev_rows=None, workspace=None,
                stream=None):
    """y[M,N] = A w^T, or y += A w^T (residual), A = x or RMSNorm(x) * norm_w."""
    ws, wsb = _ws(workspace)
    check(lib().kvc_rows_linear(_p(y), _p(x), _p(w), M, N, K, _p(norm_w), eps, int(residual), _p(dev_rows), ws, wsb,
                                stream))


def rows_qkv(q, k, v, x, w_qkv, b_qkv, pos, M, H, Hq, Hkv, D, theta, *, norm_w=None, eps=1e-6, dev_rows=None,
             stream=None):
    """q|k|v = RMSNorm(x) [wq;wk;wv]^T + bias, rotary on q and k at pos[r]."""
    check(lib().kvc_rows_qkv(_p(q), _p(k), _p(v), _p(x), _p(norm_w), eps, _p(w_qkv), _p(b_qkv), _p(pos), M, H, Hq,
                             Hkv, D, theta, _p(dev_rows), stream))


def rows_swiglu(act, x, w_gate_up, M, I, H, *, norm_w=None, eps=1e-6, dev_rows=None, stream=None):
    """act = silu(A wg^T) * (A wu^T), w_gate_up = [wg; wu]."""
    check(lib().kvc_rows_swiglu(_p(act), _p(x), _p(norm_w), eps, _p(w_gate_up), M, I, H, _p(dev_rows), stream))


def rows_lm_head(logits, tokens, x, w, M, V, H, *, norm_w=None, eps=1e-6, dev_rows=None, workspace=None,
                 stream=None):
    """fp32 logits (or None) and the greedy token of each row."""
    ws, wsb = _ws(workspace)
    check(lib().kvc_rows_lm_head(_p(logits), _p(tokens), _p(x), _p(norm_w), eps, _p(w), M, V, H, _p(dev_rows), ws,
                                 wsb, stream))


def rows_chain_workspace_size(H, I) -> int:
    return int(lib().kvc_rows_chain_workspace_size(H, I))


def rows_chain(x, M, H, Hq, Hkv, D, I, *, eps=1e-6, theta=1e6, tail=None, head=None, workspace=None, stream=None):
    """The linear layers between two attention launches as one launch (kvc_rows_chain).
    tail: dict(att, w_o, ln2, w_gate_up, act, w_down) -- o_proj + residual, norm + gate|up
    + SwiGLU, down_proj + residual; head: dict(q, k, v, ln1, w_qkv, b_qkv, pos) -- norm +
    q|k|v + bias + rotary.  Returns the status (KVC_ERR_UNSUPPORTED / KVC_ERR_STATE are
    returned, not raised)."""
    import ctypes as C

    from ._native import LayerChainC
    t, h = tail or {}, head or {}
    c = LayerChainC(M, H, Hq, Hkv, D, I, eps, theta, _p(x), _p(t.get("att")), _p(t.get("w_o")), _p(t.get("ln2")),
                    _p(t.get("w_gate_up")), _p(t.get("act")), _p(t.get("w_down")), _p(h.get("q")), _p(h.get("k")),
                    _p(h.get("v")), _p(h.get("ln1")), _p(h.get("w_qkv")), _p(h.get("b_qkv")), _p(h.get("pos")))
    ws, wsb = _ws(workspace)
    return int(lib().kvc_rows_chain(C.byref(c), ws, wsb, stream))


def rows_set_tuning(splits: int = -1, groups_per_wg: int = -1, shape: int = -1) -> None:
    """Overrides of the rows kernels' launch shape (-1: automatic)."""
    check(lib().kvc_rows_set_tuning(int(splits), int(groups_per_wg), int(shape)))


def write_kv_slots(k, v, k_pool, v_pool, slot_map, rows, Hkv, D, BLOCK, *, dtype=KVC_F16, stream=None):
    check(lib().kvc_write_kv_slots(_p(k), _p(v), _p(k_pool), _p(v_pool), _p(slot_map), rows, Hkv, D, BLOCK, dtype,
                                   stream))


def decode_workspace_size(N, Hq, Hkv, D, BLOCK, cap, split=0, dtype=KVC_F16) -> int:
    return int(lib().kvc_decode_workspace_size(N, Hq, Hkv, D, BLOCK, cap, split, dtype))


def decode_auto_split(N, Hq, Hkv, D, BLOCK, cap, dtype=KVC_F16) -> int:
    return int(lib().kvc_decode_auto_split(N, Hq, Hkv, D, BLOCK, cap, dtype))


def flash_decode_workspace_size(H, D, num_splits) -> int:
    return int(lib().kvc_flash_decode_workspace_size(H, D, num_splits))


def check_device_errors(stream=None) -> None:
    """kvc_check_device_errors: synchronizes `stream`; raises KvcError when an earlier
    launch on this device reported a failure, and clears the report: KVC_ERR_ARG for a
    device-length decode launch with a sequence it could not attend whole (its rows were
    written as NaN), KVC_ERR_STATE for a layer-chain launch whose grid barrier gave up."""
    check(lib().kvc_check_device_errors(stream))


def stream_is_capturing(stream) -> bool:
    import ctypes as C
    flag = C.c_int(0)
    check(lib().kvc_stream_is_capturing(stream, C.byref(flag)))
    return bool(flag.value)
