"""glif_syn_fwd_noalloc, the op forward whose scratch is a static device array (for callers
that cannot allocate), against glif_syn_fwd with a workspace, called through the C ABI.

Two calls in a row per mode, the second on a smaller input (fewer batch entries, another
spike pattern), so leftovers of the first call in the shared array would show.  Bars:
deterministic mode bit-exact; event mode (fp32 atomics) within 1e-5 of each element's sum of
absolute terms + 1e-6.  A table whose forward needs more than the array holds is refused with
GLIF_ENOMEM before any launch.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import dense
from tests.helpers import network, tiny_config

pytestmark = pytest.mark.gpu


def _table(seed=0):
    from v1_glif_model_amd.ops import SynapseTable
    cfg = tiny_config(n=3000, fanin=60, delays=4, rs=1.0)
    _, tb = network(cfg, seed=seed, dense_basis=True)
    t = SynapseTable(tb.rec.indices, tb.rec.syn_id, (tb.n_neurons, tb.rec.n_cols), tb.basis,
                     n_delay_slots=tb.max_delay)
    t.set_weights(torch.tensor(tb.rec.weight, device="cuda"))
    return t, tb


def _fwd_ws(t, z, mode):
    from v1_glif_model_amd import _lib
    return t.forward(z, mode=mode)


def _fwd_noalloc(t, z, mode, counts=False):
    from v1_glif_model_amd import _lib
    from v1_glif_model_amd.ops import MODES
    B = z.shape[0]
    I = torch.full((B * t.n_post, t.n_basis), float("nan"), dtype=torch.float32, device="cuda")
    _lib.check(_lib.lib().glif_syn_fwd_noalloc(t.handle, _lib.ptr(z), B, int(counts), MODES[mode], _lib.ptr(I),
                                               _lib.stream_ptr()))
    return I


@pytest.mark.parametrize("mode", ["deterministic", "event"])
def test_noalloc_forward_matches_workspace_forward(mode):
    t, tb = _table()
    rng = np.random.default_rng(1)
    inputs = [(rng.uniform(size=(5, tb.rec.n_cols)) < 0.02).astype(np.float32),
              (rng.uniform(size=(2, tb.rec.n_cols)) < 0.05).astype(np.float32)]
    for z_np in inputs:   # the second call: smaller batch, denser spikes
        z = torch.tensor(z_np, device="cuda")
        a = _fwd_noalloc(t, z, mode).cpu().numpy()
        e = _fwd_ws(t, z, mode).cpu().numpy()
        assert np.all(np.isfinite(a))
        if mode == "deterministic":
            np.testing.assert_array_equal(a.view(np.uint32), e.view(np.uint32))
        else:
            scale = dense.syn_fwd_abs(tb.rec, z_np, tb.basis)
            assert np.all(np.abs(a - e) <= 1e-5 * scale + 1e-6)
            ref = dense.syn_fwd_f64(tb.rec, z_np, tb.basis)
            assert np.all(np.abs(a - ref) <= 1e-5 * scale + 1e-6)


def test_noalloc_refuses_oversized_tables():
    """A table of 10M columns needs ~41 MiB of scratch (over the 32 MiB array): GLIF_ENOMEM
    with a message, checked on the host before anything is launched."""
    from v1_glif_model_amd import _lib
    from v1_glif_model_amd.ops import SynapseTable
    n_post, D = 2_500_000, 4
    rng = np.random.default_rng(2)
    post = np.sort(rng.integers(0, n_post, 2000))
    col = rng.integers(0, D * n_post, 2000)
    t = SynapseTable(np.stack([post, col], -1), np.zeros(2000, np.uint8), (n_post, D * n_post),
                     np.eye(1, 1, dtype=np.float32), n_delay_slots=D)
    z = torch.zeros((1, D * n_post), dtype=torch.float32, device="cuda")
    I = torch.empty((n_post, 1), dtype=torch.float32, device="cuda")
    rc = _lib.lib().glif_syn_fwd_noalloc(t.handle, _lib.ptr(z), 1, 0, 0, _lib.ptr(I), _lib.stream_ptr())
    assert rc == _lib.GLIF_ENOMEM
    assert b"static array" in _lib.lib().glif_last_error()
