"""GPU parity of the op-level entry points (glif_syn_fwd / glif_syn_bwd through
ops.SynapseTable) over a seeded random draw of recurrent tables: 5-300 neurons, 1-7 delay
slots, 1-8 receptors, 1-12 types with a dense basis (with few types per post the table's own
compact G rows serve the backward), fan-ins 1-9, batch 1-20, spike or Poisson-count inputs at
0.5-30 % density.  Per draw, against the C oracle: the deterministic forward bit for bit; the
event forward, dz and dW within 1e-5 of each element's sum of absolute terms + 1e-6
(oracle.dense's float64 sums)."""
import dataclasses

import numpy as np
import pytest
import torch

from oracle import cpu as orc
from oracle import dense
from tests.helpers import network, tiny_config

pytestmark = pytest.mark.gpu


def _draw(n_cases=40, seed=4048):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n_cases:
        N = int(rng.choice([5, 63, 64, 65, 127, 129, 257, 300]))
        nb, nt, D = int(rng.integers(1, 9)), int(rng.integers(1, 13)), int(rng.integers(1, 8))
        fan, B = int(rng.integers(1, 10)), int(rng.integers(1, 21))
        p, counts = float(rng.choice([0.005, 0.05, 0.3])), bool(rng.integers(0, 2))
        if fan >= N:
            continue
        cases.append((N, fan, D, nb, nt, B, p, counts))
    return cases


CASES = _draw()


@pytest.mark.parametrize("i", range(len(CASES)))
def test_random_op(i):
    from v1_glif_model_amd.ops import SynapseTable
    N, fan, D, nb, nt, B, p, counts = CASES[i]
    print("case", CASES[i], flush=True)
    cfg = dataclasses.replace(tiny_config(n=N, fanin=fan, delays=D), n_basis=nb, n_syn_types=nt, fanin_mean=fan,
                              fanin_sigma=None)
    _, tb = network(cfg, seed=800 + i, dense_basis=True)
    t = SynapseTable(tb.rec.indices, tb.rec.syn_id, (tb.n_neurons, tb.rec.n_cols), tb.basis,
                     n_delay_slots=tb.max_delay)
    t.set_weights(torch.tensor(tb.rec.weight, device="cuda"))
    rng = np.random.default_rng(900 + i)
    z = (rng.random((B, tb.rec.n_cols)) < p).astype(np.float32)
    if counts:
        z *= rng.integers(1, 4, z.shape).astype(np.float32)
    zt = torch.tensor(z, device="cuda")
    ref = orc.syn_fwd(tb.rec, z, tb.basis, use_count=counts)
    scale = dense.syn_fwd_abs(tb.rec, z, tb.basis, use_count=counts)
    det = t.forward(zt, counts=counts, mode="deterministic").cpu().numpy()
    np.testing.assert_array_equal(det.view(np.uint32), ref.view(np.uint32))
    ev = t.forward(zt, counts=counts, mode="event").cpu().numpy()
    assert np.max(np.abs(ev - ref) - 1e-5 * scale) <= 1e-6
    dy = rng.normal(0, 1, (B * tb.n_neurons, tb.n_basis)).astype(np.float32)
    dz, dw = t.backward(zt, torch.tensor(dy, device="cuda"), counts=counts)
    rdz, rdw = orc.syn_bwd(tb.rec, z, tb.basis, dy, use_count=counts)
    _, _, dz_abs, dw_abs = dense.syn_bwd_f64(tb.rec, z, tb.basis, dy, use_count=counts)
    assert np.max(np.abs(dz.cpu().numpy() - rdz) - 1e-5 * dz_abs) <= 1e-6
    assert np.max(np.abs(dw.cpu().numpy() - rdw) - 1e-5 * dw_abs) <= 1e-6
