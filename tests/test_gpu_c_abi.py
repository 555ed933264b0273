"""The C ABI from plain C: tests/c_abi_caller.c (built by
__graft_entry__.build() into tests/_build/c_abi_caller) creates plans, runs
C2C forward on the NULL stream, C2C inverse through mfft_execute_ws with its
own workspace and stream, and an R2C -> C2R round trip, and checks each
against a direct DFT in double precision (relative L2 <= 1e-5).  It runs as
a child process with only the HIP runtime and libmfft.so loaded."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_build", "c_abi_caller")


def test_plain_c_caller(gpu):
    assert os.path.exists(EXE), f"{EXE} missing: run __graft_entry__.build() first"
    res = subprocess.run([EXE], capture_output=True, text=True, timeout=90)
    print(res.stdout)
    assert res.returncode == 0, f"rc={res.returncode}\n{res.stdout}\n{res.stderr}"
    assert res.stdout.strip().endswith("OK")
    assert res.stdout.count("rel L2") == 6

