"""The drop-in, proven in mensurflow's own tree (CPU container only): the reference sources are
copied, rocm_wiring.patch is applied, the ROCm backend (mensurflow_amd/host/src/backends/rocm/
backend.cpp + include/mfr_rocm.h) is compiled against the reference's real core headers and
linked to libmfr_rocm.so, and every test the reference's CMakeLists registers must pass. Without
a GPU the backend reports no device and the registry drops it, so this checks that the wiring
compiles, links and leaves mensurflow's CPU behaviour unchanged. Skipped where the reference
sources are absent (the GPU box)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCRIPT = os.path.join(ROOT, "mensurflow_amd", "host", "integration", "check_in_reference.py")
REFERENCE = os.environ.get("MFR_REFERENCE", "/root/reference")


@pytest.mark.skipif(not os.path.isdir(os.path.join(REFERENCE, "src")),
                    reason="the reference sources are not present")
def test_reference_suite_passes_with_rocm_backend_wired_in():
    if not os.path.exists(os.path.join(ROOT, "mensurflow_amd", "_lib", "libmfr_rocm.so")):
        pytest.skip("libmfr_rocm.so is not built")
    proc = subprocess.run([sys.executable, SCRIPT, "--reference", REFERENCE], capture_output=True,
                          text=True, timeout=1500)
    out = proc.stdout + proc.stderr
    print(out)
    assert proc.returncode == 0, out[-4000:]
    assert "reference tests passed with the ROCm backend wired in" in out
    assert "warnings in src/backends/rocm" not in out
