"""CPU: the list arithmetic shared by the attention kernels, compiled for the host and run
(tests/list_slice_check.hip): the planned pass's per-split slice of the block list built from the
chunk masks by a team of threads (every split of random masks, split 0 included) and the bounds of the statistics
writes between list entries (exact for valid entries, inside the head for any entry value)."""

import os
import subprocess

import pytest

HIPCC = "/opt/rocm/bin/hipcc"
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc absent")
def test_list_slice_and_gap_arithmetic(tmp_path):
    exe = tmp_path / "list_slice_check"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", f"-I{ROOT}/include", "-Xclang",
                    "-target-feature", "-Xclang", "-packed-fp32-ops", os.path.join(ROOT, "tests", "list_slice_check.hip"),
                    "-o", str(exe)], check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout[-2000:]
