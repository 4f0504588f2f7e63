"""GPU parity over a seeded random draw of network shapes, beside the hand-picked sweep of
test_gpu_shapes.py: neurons 5-300 (around the 64-lane wave), delay slots 1-7, receptors 1-8,
synapse types 1-12 (dense basis), batch 1-16 (the resident chunk pull, the half-wave pull
when B * nb > 64, both backward walks), fan-ins 1-9, 6-19 ticks, both surrogates.  Per shape,
against the C oracle on the same inputs: the deterministic forward (spikes, voltages, final
state) bit for bit, BPTT within 1e-5 of each element's sum of absolute terms + 1e-6, and the
event forward from the oracle's state every other tick, three ticks on, with equal spike
trains and voltages within 1e-5 relative / 1e-6 absolute."""
import dataclasses

import numpy as np
import pytest
import torch

from oracle.cpu import OracleCell, bptt_abs_scale
from tests.helpers import assert_grads_per_element, tiny_config
from tests.test_gpu_shapes import _state_np
from v1_glif_model_amd import synthetic as sy
from v1_glif_model_amd.tables import build_cell_tables

pytestmark = pytest.mark.gpu


def _draw(n_cases=40, seed=2026):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n_cases:
        N = int(rng.choice([5, 63, 64, 65, 127, 129, 257, 300]))
        nb, nt, D = int(rng.integers(1, 9)), int(rng.integers(1, 13)), int(rng.integers(1, 8))
        B = int(rng.choice([1, 2, 3, 4, 5, 6, 8, 11, 13, 16]))
        fan, nl, lf = int(rng.integers(1, 10)), int(rng.integers(3, 60)), int(rng.integers(1, 6))
        T, pg = int(rng.integers(6, 20)), bool(rng.integers(0, 2))
        ins = float(rng.choice([20.0, 40.0, 80.0, 150.0]))
        if fan >= N or lf >= nl:
            continue
        cases.append((N, fan, D, nb, nt, B, T, nl, lf, pg, ins))
    return cases


CASES = _draw()


@pytest.mark.parametrize("i", range(len(CASES)))
def test_random_shape(i):
    from tests.test_gpu_params import _state_dev
    from v1_glif_model_amd.models import V1Column
    N, fan, D, nb, nt, B, T, nl, lf, pg, ins = CASES[i]
    print("case", CASES[i], flush=True)
    cfg = dataclasses.replace(tiny_config(n=N, fanin=fan, delays=D, n_lgn=nl, lgn_fanin=lf, n_bkg=6,
                                          bkg_fanin=3, rs=3.0, ins=ins, lgn_p=0.08),
                              n_basis=nb, n_syn_types=nt, fanin_mean=fan, fanin_sigma=None)
    net = sy.make_network(cfg, seed=500 + i, dense_basis=True)
    lgn, bkg = sy.make_inputs(cfg, seed=600 + i, seq_len=T, batch=B)
    tb = build_cell_tables(net)
    okw = dict(gauss_std=0.3, damp=0.3, rd=0.2, vgd=0.4, pseudo_gauss=pg)
    ckw = dict(gauss_std=0.3, dampening_factor=0.3, recurrent_dampening_factor=0.2,
               voltage_gradient_dampening=0.4, pseudo_gauss=pg)
    oc = OracleCell(tb, **okw)
    oz, ov, oref, ost = oc.forward(lgn, bkg)
    cell = V1Column(net, mode="deterministic", **ckw)
    z, v, st = cell.rollout(lgn, bkg)
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    for k, a in _state_np(st).items():
        e = ost[k]
        np.testing.assert_array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                                      e.view(np.uint32) if e.dtype == np.float32 else e, err_msg=k)
    gz = np.random.default_rng(700 + i).normal(0, 1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"))
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz)
    sc = bptt_abs_scale(tb, lgn, bkg, oz, oref, ov, gz_loss=gz, **okw)
    for k in ("rec", "lgn", "bkg"):
        assert_grads_per_element(g[k].cpu().numpy(), og[k], sc[k], what=k)
    ev = V1Column(net, mode="event", **ckw)
    K = 3
    ws = ev.workspace(B, K)
    s = oc.zero_state(B)
    for t0 in range(0, T - K + 1, 2):
        ze, ve, _ = ev.rollout(lgn[t0:t0 + K], bkg[t0:t0 + K], state=_state_dev(ev, s), ws=ws)
        oz3, ov3, _, _ = oc.forward(lgn[t0:t0 + K], bkg[t0:t0 + K], state=s)
        np.testing.assert_array_equal(ze.cpu().numpy().astype(np.uint8), oz3, err_msg=f"tick {t0}")
        err = np.abs(ve.cpu().numpy().astype(np.float64) - ov3)
        assert np.all(err <= 1e-5 * np.abs(ov3) + 1e-6), (t0, float(err.max()))
        _, _, _, s = oc.forward(lgn[t0:t0 + 2], bkg[t0:t0 + 2], state=s)
    print("spikes", int(oz.sum()), flush=True)
