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


def test_kv_manager_host():
    assert run("test_kv_manager", "--host").returncode == 0


def test_demo_engine_host():
    assert run("demo_engine", "--host").returncode == 0


@pytest.mark.gpu
def test_kv_manager_device():
    assert run("test_kv_manager").returncode == 0


@pytest.mark.gpu
def test_demo_engine_device():
    assert run("demo_engine").returncode == 0


@pytest.mark.gpu
def test_paged_flash_device():
    assert run("test_paged_flash").returncode == 0


@pytest.mark.gpu
def test_runner_planned_and_device_length_paths_agree():
    assert run("test_runner_paths").returncode == 0
