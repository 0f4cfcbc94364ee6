"""CPU: host code under AddressSanitizer + UndefinedBehaviorSanitizer.

* the library's host side (volta_amd/csrc/host_check.hip, linked with every
  source of libvolta_hip.so, the sanitizers on the host pass only): shape
  validation, algorithm selection and the workspace sizing of every conv
  backward plan over a grid of shapes, dtypes and algorithms -- no GPU call;
* the CPU oracle (oracle/asan_check.c): every or_* function on small and edge
  shapes with exact-size buffers, plus agreement of its forward forms.

Either binary exits non-zero on the first sanitizer report."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _make(path, target, timeout):
    r = subprocess.run(["make", "-s", "-C", path, "-j8", target], capture_output=True, text=True,
                       timeout=timeout)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    return r.stdout


@pytest.mark.skipif(shutil.which("gcc") is None and shutil.which("cc") is None, reason="no C compiler")
def test_oracle_under_asan_ubsan():
    out = _make(os.path.join(ROOT, "oracle"), "asan-check", 300)
    assert "0 failures" in out, out


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not installed")
def test_library_host_logic_under_asan_ubsan():
    out = _make(os.path.join(ROOT, "volta_amd", "csrc"), "host-check", 900)
    assert "0 failures" in out, out
