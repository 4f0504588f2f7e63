"""The C-ABI library loads and exports every entry point include/glif.h declares
(no compute calls: this runs without a GPU), and the host-side pieces work on CPU."""
import os
import re

import numpy as np
import pytest

from oracle import dense

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "glif.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(glif_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    from v1_glif_model_amd import _lib
    L = _lib.lib()
    names = _declared()
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert L.glif_version() >= 1


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_host_pre_ind_table_bit_exact(seed):
    from v1_glif_model_amd.ops import make_pre_ind_table
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 2000))
    cols = rng.integers(0, n, int(rng.integers(0, 20000)))
    ind = np.stack([np.zeros_like(cols), cols], -1)
    t = make_pre_ind_table(ind, n_source_neurons=n)
    eo, er = dense.csr_build_numpy(cols, n)
    assert t.values.dtype == np.int32 and t.row_splits.dtype == np.int32
    np.testing.assert_array_equal(t.values, eo)
    np.testing.assert_array_equal(t.row_splits, er)


def test_host_pre_ind_table_errors_match_reference():
    from v1_glif_model_amd.ops import make_pre_ind_table
    with pytest.raises(ValueError, match="must be > 0"):
        make_pre_ind_table(np.zeros((1, 2), np.int64), n_source_neurons=0)
    with pytest.raises(ValueError, match="must have shape"):
        make_pre_ind_table(np.zeros((3,), np.int64), n_source_neurons=4)
    with pytest.raises(ValueError, match=r"Presynaptic index 9 is out of bounds for `n_source_neurons=4`"):
        make_pre_ind_table(np.array([[0, 1], [0, 9]]), n_source_neurons=4)
    t = make_pre_ind_table(np.zeros((0, 2), np.int64), n_source_neurons=3)
    assert t.values.size == 0 and t.row_splits.tolist() == [0, 0, 0, 0]


def test_product_path_has_no_cpu_fallback():
    """The package never imports the oracle and refuses to run without a GPU."""
    import torch
    pkg = os.path.join(ROOT, "v1_glif_model_amd")
    for f in os.listdir(pkg):
        if f.endswith(".py"):
            assert "oracle" not in re.sub(r'""".*?"""', "", open(os.path.join(pkg, f)).read(), flags=re.S), f
    if not torch.cuda.is_available():
        from v1_glif_model_amd.ops import SynapseTable
        with pytest.raises(RuntimeError, match="no CPU fallback"):
            SynapseTable(np.zeros((1, 2), np.int64), np.zeros(1, np.uint8), (1, 1), np.eye(1, dtype=np.float32))
