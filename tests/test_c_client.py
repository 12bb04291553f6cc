"""include/palladium_hip.h is valid C and libpalladium_hip.so is usable
from C alone (no Python): tests/c_client/ph_client.c built with gcc."""

import subprocess
from pathlib import Path

import pytest

from palladium_amd import runtime as rt

ROOT = Path(__file__).resolve().parents[1]
CLIENT = ROOT / "tests" / "c_client" / "ph_client.c"


def _build(tmp_path: Path) -> Path:
    lib = rt.library_path()
    exe = tmp_path / "ph_client"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-O1", f"-I{ROOT / 'include'}", str(CLIENT), "-o", str(exe),
                    f"-L{lib.parent}", "-lpalladium_hip", f"-Wl,-rpath,{lib.parent}"], check=True)
    return exe


def test_c_client_compiles_a_kernel_without_a_gpu(tmp_path):
    out = subprocess.run([str(_build(tmp_path)), "compile"], capture_output=True, text=True, check=True).stdout
    assert "compiled" in out and "ELF=1" in out
    assert "bad math mode -> 1" in out and "math_mode out of range" in out


@pytest.mark.gpu
def test_c_client_dispatches_on_the_gpu(tmp_path):
    r = subprocess.run([str(_build(tmp_path)), "dispatch"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ph_dispatch ok" in r.stdout and "ph_dispatch_device ok" in r.stdout
    assert "ph_dispatch_noalloc ok" in r.stdout and "oversized -> 1" in r.stdout
