"""The persistent launch schedule of the matrix-core GEMV and Q6_K kernels
(modgrad_amd/csrc/q4k_launch.hpp: persistent_plan, sched_count, sched_group),
compiled for the host and checked over ~3,600 shapes: every row group is
streamed by exactly one (work-group, round), work-group b starts with row
group b (the GEMV issues that stage's loads before computing the schedule),
and no work-group takes more rounds than its result buffer holds."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not os.path.exists(HIPCC) and shutil.which("hipcc") is None,
                    reason="hipcc not available")
def test_persistent_schedule_partitions_row_groups(tmp_path):
    exe = tmp_path / "sched_check"
    src = os.path.join(HERE, "native", "sched_check.cpp")
    hipcc = HIPCC if os.path.exists(HIPCC) else shutil.which("hipcc")
    subprocess.run([hipcc, "-O2", "-std=c++17", "-x", "hip", "--offload-arch=gfx950",
                    "-o", str(exe), src], check=True, capture_output=True, timeout=300)
    env = dict(os.environ, HIP_VISIBLE_DEVICES="")  # the schedule needs no device
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok")
