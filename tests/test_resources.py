"""No gfx950 kernel of the library spills registers or uses scratch memory:
the compiler's resource-usage remarks for gemm.hip, attention.hip,
rowops.hip and few.hip (edgebert_amd/csrc/resource_report.py).  CPU only (hipcc
cross-compiles); skipped where hipcc is absent."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPORT = os.path.join(ROOT, "edgebert_amd", "csrc", "resource_report.py")


@pytest.mark.skipif(not os.path.exists(os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")), reason="no hipcc")
def test_no_kernel_spills_or_uses_scratch():
    r = subprocess.run([sys.executable, REPORT, "--fail-on-scratch"], capture_output=True, text=True, timeout=600)
    assert "kernels with spills or scratch: 0" in r.stdout, r.stdout[-3000:] + r.stderr[-2000:]
    assert r.returncode == 0
