"""The decode kernels' balanced token partition (csrc/cq_plan.h), checked on
the host: tests/plan_check.cpp walks every workgroup's range as the kernels
do, over the benchmark shapes and 12,000 random batches (uniform, ragged,
empty sequences, lengths at unit edges; 1 to 300 workgroups)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_balanced_partition(tmp_path):
    exe = tmp_path / "plan_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", "-o", str(exe),
                    os.path.join(HERE, "plan_check.cpp")], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0 and res.stdout.startswith("ok"), res.stdout + res.stderr
