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
def test_runner_planned_and_device_length_paths_agree():
    assert run("test_runner_paths").returncode == 0
