"""The C ABI driven with no torch in the process: tests/capi/capi_check (built by
tests/capi/build.py, which __graft_entry__.build() runs) allocates with hipMalloc, calls
co_alibi_fwd / co_alibi_bwd / co_alibi_decode on a stream and compares against the plain-C
oracle in double precision (fp32 1e-4, fp16 2e-2), then checks the error codes and
messages.  It runs as a child process so that its HIP context is its own."""
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "capi", "capi_check")


@pytest.mark.gpu
def test_c_abi_without_torch():
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built: run `python tests/capi/build.py` (or __graft_entry__.build())")
    print(f"running {BIN}", flush=True)
    res = subprocess.run([BIN], capture_output=True, text=True, timeout=90)
    sys.stdout.write(res.stdout)
    sys.stdout.write(res.stderr)
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-2000:]
    assert "PASSED: 0 failure(s)" in res.stdout
