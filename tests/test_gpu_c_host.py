"""The plain C host of libqdc_hip.so (tests/c_host/qdc_c_host.c, built by
``__graft_entry__.build()``): device buffers from hipMalloc, the entry points
called with raw pointers, results checked in C against double-precision loops
(fp32 RMSNorm and SwiGLU within 1e-5, the bf16 residual norm within 1e-2, the
split output within 1e-5, the residual and the widening gather bit-exact).  It
runs as a child process; this test checks its exit status and report."""
import os
import subprocess

import pytest
import torch

from conftest import ROOT

pytestmark = pytest.mark.gpu

EXE = os.path.join(ROOT, "tests", "c_host", "qdc_c_host")


def test_c_host_program():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert os.path.exists(EXE), "tests/c_host/qdc_c_host is built by __graft_entry__.build()"
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout
    assert r.stdout.count("ok  ") >= 20
