"""bench.py's command-line contract on the host: more than one GPU is refused with a JSON
error and exit code 2, an op-level batch outside [1, 32] is refused before any work, and
without a GPU the run stops with the library's error instead of timing anything on the CPU."""
import json
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args, timeout=600):
    return subprocess.run([sys.executable, os.path.join(HERE, "bench.py"), *args], cwd=HERE,
                          capture_output=True, text=True, timeout=timeout)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]


@pytest.mark.parametrize("batch", ["0", "33"])
def test_op_batch_out_of_range_is_refused(batch):
    r = _run("--op", "--op-batch", batch, timeout=120)
    assert r.returncode != 0
    assert "--op-batch must be in [1, 32]" in r.stderr


def test_no_gpu_fails_loudly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    r = _run("--steps", "1", "--warmup", "0", "--cpu-steps", "0")
    assert r.returncode != 0
    assert "no CPU fallback" in r.stderr
