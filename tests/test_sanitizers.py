"""The host runtime under ThreadSanitizer and under AddressSanitizer + UBSan
(the reference's CI runs its no-GPU suite under Clang ASan + UBSan,
.github/workflows/ci.yml:420-470; the session queue is where threads meet, so
TSan too). tests/sanitize/Makefile links the C-ABI
stress driver (several caller threads on one session: GEMMs with cancels,
transactions, prefetches, telemetry readers) with the runtime sources and the
host-memory device simulation; both binaries must finish their checks with no
sanitizer report. CPU only."""
import os
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize")


@pytest.fixture(scope="module")
def binaries():
    proc = subprocess.run(["make", "-s", "-j4", "-C", HERE], capture_output=True, text=True,
                          timeout=600)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    return os.path.join(HERE, "_build")


@pytest.mark.parametrize("name,marker", [("stress_tsan", "WARNING: ThreadSanitizer"),
                                         ("stress_asan", "ERROR: AddressSanitizer")])
def test_stress_under_sanitizer(binaries, name, marker):
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1", ASAN_OPTIONS="detect_leaks=1")
    proc = subprocess.run([os.path.join(binaries, name)], capture_output=True, text=True,
                          timeout=300, env=env)
    out = proc.stdout + proc.stderr
    print(out[-2000:])
    assert marker not in out and "runtime error:" not in out
    assert proc.returncode == 0, out[-4000:]
    assert "failures 0" in proc.stdout
