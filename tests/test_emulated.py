"""The product's kernels, compiled for the host against tests/cpu_emu's
emulation of the device features they use, run under AddressSanitizer on the
parity cases (tests/cpu_emu/run_cases.py): bounds and results checked on the
CPU, before any GPU run."""
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "cpu_emu"))


@pytest.mark.timeout(900)
def test_kernels_in_bounds_and_correct_on_the_cpu():
    import build_emu
    lib = build_emu.build()
    assert os.path.exists(lib)
    env = dict(os.environ, LD_PRELOAD=build_emu.asan_runtime(),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1")
    r = subprocess.run([sys.executable, os.path.join(HERE, "cpu_emu", "run_cases.py"), "quick"],
                       env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=800)
    assert r.returncode == 0, r.stdout[-4000:]
    assert "failed: 0" in r.stdout
