"""libglif's C ABI from plain C host programs (tests/c, built by __graft_entry__.build()): no
Python or torch between the caller and the library, as a TensorFlow custom op would bind it.

* abi_from_c (the op): the pre_ind_table against a stable counting sort, the deterministic
  forward bit for bit against the reference's accumulation order written out in C, the event
  forward and the custom gradient (dz, dW) within 1e-5 of each element's sum of absolute terms
  + 1e-6 of float64 sums, and three refusals (NULL table, B = 0, short workspace);
* cell_from_c (the cell): a network built in C run for 40 ticks, spike trains, voltages and
  final state bit-exact with the C oracle compiled into the program, the BPTT weight gradients
  within 1e-5 of the largest |dW| + 1e-6."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c")


@pytest.mark.parametrize("prog", ["abi_from_c", "cell_from_c"])
def test_from_a_c_host(prog):
    exe = os.path.join(HERE, prog)
    assert os.path.exists(exe), f"tests/c/{prog} is not built: run __graft_entry__.build()"
    out = subprocess.run([exe], capture_output=True, text=True, timeout=120,
                         env=dict(os.environ, OMP_NUM_THREADS="4"))
    print(out.stdout, out.stderr)
    assert out.returncode == 0 and out.stdout.startswith("PASS"), out.stdout + out.stderr
