"""Exhaustive CPU check of the byte-lane helpers shared by the image kernels."""
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_swar_helpers_exhaustive(tmp_path):
    exe = tmp_path / "swar_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", str(ROOT / "strict_amd" / "csrc"),
                    str(ROOT / "tests" / "cpp" / "swar_check.cpp"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "failures=0" in r.stdout
