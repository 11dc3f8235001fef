"""The scratch pool's ownership rules, checked on the CPU against a model of
streams and events (tests/scratch_pool_model.cpp drives the same header the
library builds, torchvulkan_amd/csrc/scratch_pool.h)."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_scratch_pool_model(tmp_path):
    exe = tmp_path / "scratch_pool_model"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-pthread", f"-I{ROOT / 'torchvulkan_amd' / 'csrc'}",
                    str(ROOT / "tests" / "scratch_pool_model.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "ok"
