"""Runs the C++ drop-in test program (tests/cpp/test_dropin.cpp, built by
`python -m ccinfer_amd.build`): validation paths on the CPU, full paths on the GPU."""
import subprocess

import pytest

from ccinfer_amd import build


def _run(mode):
    exe = build.CPP_TEST
    assert exe.exists(), f"{exe} missing: run `python -m ccinfer_amd.build`"
    res = subprocess.run([str(exe), mode], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr


def test_dropin_validation_cpu():
    _run("cpu")


@pytest.mark.gpu
def test_dropin_backend_and_launchers_gpu(gpu):
    _run("gpu")
