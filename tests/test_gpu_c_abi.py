"""The op through libglif's C ABI from a plain C host program (tests/c/abi_from_c.c, built by
__graft_entry__.build()): no Python or torch between the caller and the library, as a
TensorFlow custom op would bind it.  The program checks the pre_ind_table against a stable
counting sort, the deterministic forward bit for bit against the reference's accumulation
order, the event forward and the custom gradient (dz, dW) within 1e-5 of each element's sum of
absolute terms + 1e-6 of float64 sums, and three refusals (NULL table, B = 0, short workspace)."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c", "abi_from_c")


def test_op_from_a_c_host():
    assert os.path.exists(EXE), "tests/c/abi_from_c is not built: run __graft_entry__.build()"
    out = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    print(out.stdout, out.stderr)
    assert out.returncode == 0 and out.stdout.startswith("PASS"), out.stdout + out.stderr
