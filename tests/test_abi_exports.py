"""The C ABI library loads, exports every symbol include/kvc_abi.h declares, and
rejects bad shapes with a status (no GPU needed: validation precedes any HIP call)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from kvcache_amd import _native as N
from kvcache_amd import ops

HEADER = Path(__file__).resolve().parents[1] / "include" / "kvc_abi.h"


def declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(kvc_\w+)\s*\(", text, flags=re.M))


def test_header_declares_functions():
    names = declared_functions()
    assert len(names) > 40 and "kvc_batched_paged_decode" in names and "kvc_engine_run" in names


def test_library_exports_every_declared_symbol():
    L = N.lib()
    missing = [n for n in sorted(declared_functions()) if not hasattr(L, n)]
    assert not missing, missing


def test_python_bindings_cover_header():
    assert declared_functions() == set(N.exported_names())


def test_version_and_status_strings():
    L = N.lib()
    assert L.kvc_version() >= 100
    assert L.kvc_status_string(N.KVC_ERR_WORKSPACE) == b"workspace too small"


def _fake(n=16):
    return 0x10000  # 16-byte aligned non-null address; never dereferenced on the error paths below


@pytest.mark.parametrize("D,status", [(48, N.KVC_ERR_UNSUPPORTED), (512, N.KVC_ERR_UNSUPPORTED)])
def test_unsupported_head_dim(D, status):
    p = _fake()
    with pytest.raises(N.KvcError) as e:
        ops.launch_batched_paged(p, p, p, p, p, p, p, 4, 8, D, 16, 100, 0.1, dtype=N.KVC_F16)
    assert e.value.status == status and "head_dim" in str(e.value)


def test_batch_beyond_descriptor_range_rejected():
    # lengths and table offsets are read through 32-bit byte-sized descriptors
    p = _fake()
    with pytest.raises(N.KvcError) as e:
        ops.launch_batched_paged(p, p, p, p, p, p, p, 1 << 28, 8, 64, 16, 100, 0.1, dtype=N.KVC_F16)
    assert e.value.status == N.KVC_ERR_UNSUPPORTED and "2^28" in str(e.value)


def test_bad_arguments_rejected():
    p = _fake()
    with pytest.raises(N.KvcError) as e:  # Hq not a multiple of Hkv
        ops.launch_batched_paged(p, p, p, p, p, p, p, 4, 7, 64, 16, 100, 0.1, Hkv=2, dtype=N.KVC_F16)
    assert e.value.status == N.KVC_ERR_ARG
    with pytest.raises(N.KvcError) as e:  # misaligned q
        ops.launch_batched_paged(p + 2, p, p, p, p, p, p, 4, 8, 64, 16, 100, 0.1, dtype=N.KVC_F16)
    assert e.value.status == N.KVC_ERR_ARG and "aligned" in str(e.value)
    with pytest.raises(N.KvcError) as e:  # split not a multiple of BLOCK
        ops.launch_batched_paged(p, p, p, p, p, p, p, 4, 8, 64, 16, 100, 0.1, dtype=N.KVC_F16, split=24)
    assert e.value.status == N.KVC_ERR_ARG
    with pytest.raises(N.KvcError) as e:  # caller workspace too small
        ops.launch_batched_paged(p, p, p, p, p, p, p, 4, 8, 64, 16, 5000, 0.1, dtype=N.KVC_F16, split=128,
                                 workspace=(p, 64))
    assert e.value.status == N.KVC_ERR_WORKSPACE
    with pytest.raises(N.KvcError) as e:
        ops.launch_decode(p, p, p, p, 10, 8, 64, 5, 0.1)  # cur_len > S
    assert e.value.status == N.KVC_ERR_ARG
    with pytest.raises(N.KvcError) as e:
        ops.launch_append(p, p, p, p, 7, 8, 64, 7)  # pos >= S
    assert e.value.status == N.KVC_ERR_ARG


def test_empty_batch_is_a_noop():
    ops.launch_batched_paged(None, None, None, None, None, None, None, 0, 8, 64, 16, 0, 0.1, dtype=N.KVC_F16)


def test_workspace_size_and_auto_split():
    # ragged C2 shape: auto split is a power of two, multiple of BLOCK, and sizes the partials
    sp = ops.decode_auto_split(128, 8, 8, 64, 16, 2022)
    assert sp >= 16 and sp % 16 == 0 and (sp & (sp - 1)) == 0
    ws = ops.decode_workspace_size(128, 8, 8, 64, 16, 2022)
    chunks = -(-2022 // sp)
    assert ws >= 128 * chunks * 8 * (64 + 2) * 4
    assert ops.decode_workspace_size(4, 14, 2, 64, 16, 32768, 512) >= 4 * 64 * 14 * 66 * 4
    assert ops.decode_workspace_size(4, 8, 8, 64, 16, 100, 128) == 0  # single chunk: no partials
    assert ops.flash_decode_workspace_size(8, 64, 1) == 0
    assert ops.flash_decode_workspace_size(8, 64, 7) >= 8 * 7 * 66 * 4


# ---- planned / prefill entry points: validation before any HIP call -------------------
def test_plan_entry_sizes():
    L = N.lib()
    assert L.kvc_decode_plan_entry_ints(8, 8, 64, 16, N.KVC_F16) == 16    # VALU, uniform paging: 8 inline ids
    assert L.kvc_decode_plan_entry_ints(14, 2, 64, 16, N.KVC_F16) == 64   # matrix cores: up to 56 inline ids
    assert L.kvc_decode_plan_entry_ints(8, 8, 64, 4, N.KVC_F16) == 8      # per-lane paging: header only
    assert L.kvc_decode_plan_entry_ints(8, 3, 64, 16, N.KVC_F16) == 0     # bad shape


def test_plan_argument_errors():
    import numpy as np
    L = N.lib()
    lens = np.array([5, 100], np.int32)
    nu, nr = C.c_int(0), C.c_int(0)
    assert L.kvc_decode_plan(lens.ctypes.data, None, None, 0, 2, 8, 8, 64, 16, N.KVC_F16, 0, None, 0, None,
                             C.byref(nr)) == N.KVC_ERR_ARG
    assert L.kvc_decode_plan(lens.ctypes.data, None, None, 0, 2, 8, 3, 64, 16, N.KVC_F16, 0, None, 0, C.byref(nu),
                             C.byref(nr)) == N.KVC_ERR_ARG
    assert L.kvc_decode_plan(lens.ctypes.data, None, None, -1, 2, 8, 8, 64, 16, N.KVC_F16, 0, None, 0,
                             C.byref(nu), C.byref(nr)) == N.KVC_OK          # no table: length ignored
    tab = np.zeros(4, np.int32)
    assert L.kvc_decode_plan(lens.ctypes.data, None, tab.ctypes.data, -1, 2, 8, 8, 64, 16, N.KVC_F16, 0, None, 0,
                             C.byref(nu), C.byref(nr)) == N.KVC_ERR_ARG
    assert nu.value > 0
    work = np.zeros((1, 16), np.int32)
    assert L.kvc_decode_plan(lens.ctypes.data, None, None, 0, 2, 8, 8, 64, 16, N.KVC_F16, 0, work.ctypes.data,
                             0, C.byref(nu), C.byref(nr)) == N.KVC_ERR_WORKSPACE
    with pytest.raises(N.KvcError):
        ops.decode_plan(lens, 8, 3, 64, 16)


def test_planned_and_prefill_argument_errors():
    L = N.lib()
    fake = C.c_void_p(16)  # never dereferenced: validation fails first
    assert L.kvc_batched_paged_append_decode_planned(fake, None, None, None, fake, fake, fake, 4, fake, 2, 8, 8, 64,
                                                     16, 0.125, N.KVC_F16, fake, 2, 0, None, 0,
                                                     None) == N.KVC_ERR_ARG
    assert L.kvc_batched_paged_decode_planned(fake, fake, fake, None, 0, fake, 2, 8, 8, 64, 16, 0.125, N.KVC_F16,
                                              None, 2, 0, None, 0, None) == N.KVC_ERR_ARG
    assert L.kvc_paged_causal_attn(fake, fake, fake, fake, fake, -1, 4, 8, 8, 64, 16, 0.125, N.KVC_F16, None, 0,
                                   None) == N.KVC_ERR_ARG
    assert L.kvc_paged_causal_attn(fake, fake, fake, fake, fake, 0, 0, 8, 8, 64, 16, 0.125, N.KVC_F16, None, 0,
                                   None) == N.KVC_OK                        # empty prompt: nothing to do
    assert L.kvc_paged_causal_attn_workspace_size(0, 4, 8, 3, 64, 16, N.KVC_F16) == 0


def test_tuning_round_trip_and_rejects():
    L = N.lib()
    v = C.c_int(0)
    for key in (b"mfma", b"wg_per_cu", b"split_first", b"fused_merge", b"waves_per_block", b"self_prefetch_xcd",
                b"self_lead_tokens", b"chain_spin"):
        assert L.kvc_get_tuning(key, C.byref(v)) == N.KVC_OK
        old = v.value
        assert L.kvc_set_tuning(key, old) == N.KVC_OK
    assert L.kvc_set_tuning(b"mfma", 7) == N.KVC_ERR_ARG
    assert L.kvc_set_tuning(b"no_such_knob", 1) == N.KVC_ERR_ARG
    assert L.kvc_set_tuning(b"self_lead_tokens", -1) == N.KVC_ERR_ARG
    assert L.kvc_empty_launch(0, None) == N.KVC_ERR_ARG and L.kvc_empty_launch(65536, None) == N.KVC_ERR_ARG
    # the layer chain: argument checks before any device call
    assert L.kvc_rows_chain(None, None, 0, None) == N.KVC_ERR_ARG
    assert L.kvc_rows_chain_workspace_size(896, 4864) > L.kvc_rows_workspace_size(896, 4864) > 0
    assert L.kvc_rows_chain_workspace_size(896, 100) == 0
    assert L.kvc_get_tuning(b"self_lead_tokens", C.byref(v)) == N.KVC_OK and v.value == 320
    assert L.kvc_get_tuning(b"chain_spin", C.byref(v)) == N.KVC_OK and v.value == 1 << 20
    assert L.kvc_set_tuning(b"chain_spin", -1) == N.KVC_ERR_ARG
