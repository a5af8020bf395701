"""C++ programs written against the drop-in headers (include/kvc/*.h), built by
kvcache_amd.build into kvcache_amd/_build/bin.  Host-only variants run here; the
device variants need the GPU."""
import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parents[1] / "kvcache_amd" / "_build" / "bin"


def run(name, *args):
    exe = BIN / name
    if not exe.exists():
        pytest.fail(f"{exe} not built: run python -m kvcache_amd.build")
    r = subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:])
    return r


def test_kv_manager_scenario_host():
    assert run("kv_manager_scenario", "--host").returncode == 0


def test_demo_engine_host():
    assert run("demo_engine", "--host").returncode == 0


@pytest.mark.gpu
def test_kv_manager_scenario_device():
    assert run("kv_manager_scenario").returncode == 0


@pytest.mark.gpu
def test_reference_kv_manager_test_unchanged_against_dropin_headers():
    """The reference's tests/test_kv_manager.cu, source unchanged, compiled against
    include/kvc by kvcache_amd.build (only where the reference tree was present at build
    time; the binary travels with the built library)."""
    if not (BIN / "ref_test_kv_manager").exists():
        pytest.skip("reference test program not built (reference tree absent at build time)")
    r = run("ref_test_kv_manager")
    assert r.returncode == 0 and "[FAIL]" not in r.stdout


@pytest.mark.gpu
def test_qwen_graph_recaptured_after_workspace_growth():
    assert run("test_qwen_graph_regrow").returncode == 0


@pytest.mark.gpu
def test_demo_engine_device():
    assert run("demo_engine").returncode == 0


@pytest.mark.gpu
def test_paged_flash_device():
    assert run("test_paged_flash").returncode == 0


@pytest.mark.gpu
def test_dropin_device_position_causal_attention_in_and_out_of_capture():
    r = run("test_dropin_causal")
    assert r.returncode == 0 and "PASS" in r.stdout


@pytest.mark.gpu
def test_runner_planned_and_device_length_paths_agree():
    assert run("test_runner_paths").returncode == 0


@pytest.mark.gpu
@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (14, 2)])
@pytest.mark.parametrize("mode", [0, 1], ids=["copy_stream", "pinned_host_list"])
def test_plan_pipeline_serving_loop_output(tmp_path, Hq, Hkv, mode):
    """tests/cpp/plan_pipeline.cpp, the serving loop over the C ABI: the host plans every
    step (kvc_decode_plan) while the previous step's kernel runs, the work list reaching
    the kernel through a copy stream (mode 0) or from pinned host memory (mode 1); the
    last step's output equals a plain planned launch's bit for bit."""
    import json

    import numpy as np
    rng = np.random.default_rng(17 + mode + Hq)
    N, D, B = 48, 64, 16
    lens = rng.integers(1, 1500, N).astype(np.int32)
    nb = (lens + B - 1) // B
    tab_off = np.concatenate([[0], np.cumsum(nb)]).astype(np.int32)
    table = rng.permutation(int(tab_off[-1]) + 7)[: tab_off[-1]].astype(np.int32)
    path = tmp_path / "batch.bin"
    np.concatenate([np.array([N, Hq, Hkv, D, B, len(table)], np.int32), lens, tab_off, table]).tofile(path)
    r = run("plan_pipeline", str(path), "8", "2", str(mode))
    assert r.returncode == 0
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["units"] > 0 and res["steps"] == 8
    assert res["output_equals_plain_planned_launch"] is True
