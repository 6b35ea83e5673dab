"""The C++ host mirror (include/biv_hip.hpp: Engine, Moe, DeviceMoe::ffn as
Model::ffn, DeviceDense, Error as Error::Backend) on the GPU against the CPU
oracle: tests/probes/host_mirror.cpp, built with the library."""
import os
import subprocess

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

EXE = os.path.join(ROOT, "tests", "probes", "host_mirror")


def test_host_mirror():
    if not os.path.exists(EXE):
        pytest.fail("tests/probes/host_mirror is not built (python -m biv_amd.build)")
    print("case C++ host mirror", flush=True)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert "host mirror: 0 failures" in r.stdout, r.stdout + r.stderr
    assert r.stdout.count(": ok") >= 20, r.stdout
    assert r.returncode == 0, r.stdout + r.stderr
