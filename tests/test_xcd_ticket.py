"""The XCD-local split-K ticket arithmetic (metalops_amd/csrc/q4_common.h), run
on the host: tests/xcd_ticket_check.cpp is compiled with hipcc (host code only,
no GPU call) and checks the arrival count and the per-split placement mask for
every split count and seeded mixed placements."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_ticket_arithmetic_mixed_placements(tmp_path):
    hipcc = "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    exe = str(tmp_path / "xcd_ticket_check")
    subprocess.run([hipcc, "-O1", "-std=c++17", "--offload-arch=gfx950",
                    "-I", os.path.join(ROOT, "metalops_amd", "csrc"), "-I", os.path.join(ROOT, "include"),
                    "-x", "hip", os.path.join(HERE, "xcd_ticket_check.cpp"), "-o", exe],
                   check=True, capture_output=True)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout + out.stderr
