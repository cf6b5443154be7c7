"""Host-side AddressSanitizer run (CPU only): the C oracle and the product library's host code
(validation, workspace layout, size queries, error paths) built with -fsanitize=address and
driven by tests/asan/*.c[pp]; any memory error aborts the driver and fails this test."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(not (shutil.which("gcc") and os.path.exists("/opt/rocm/bin/hipcc")),
                    reason="needs gcc and hipcc")
def test_host_code_under_asan(tmp_path):
    r = subprocess.run(["make", "-s", "-C", os.path.join(HERE, "asan"), "check",
                        f"OUT={tmp_path}"], capture_output=True, text=True, timeout=900)
    print(r.stdout[-2000:], r.stderr[-4000:])
    assert r.returncode == 0
    assert "oracle_check:" in r.stdout and "abi_check:" in r.stdout
