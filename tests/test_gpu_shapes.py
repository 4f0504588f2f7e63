"""GPU parity over a seeded sweep of small, irregular shapes.

The other GPU tests fix a few network shapes; this sweep varies what the kernels' index
arithmetic and launch shapes depend on: neuron counts around the 64-lane wave (1, 37, 64, 65,
130, 200), delay slots 1-9, receptors 1-8, synapse types 1-20 (dense basis), batch 1-32
(every G row length and backward window width), sparse tables with empty columns, and both
surrogates; cases 4 and 5 receive few of their types per neuron, so they run with compact G rows
(grouped walk at B = 3, type-phased at B = 7) and the event push into per-type slots; the last
case fills all 64 accumulator lanes of the deterministic chunk pull (B = 8, nb = 8).  Per case,
against the C oracle on the same inputs:

* deterministic forward: spikes, voltages and the final state bit-exact;
* event forward: from the oracle's state at every tick, three ticks on, spike trains equal and
  voltages within 1e-5 relative / 1e-6 absolute;
* BPTT after the deterministic forward: every weight gradient within 1e-5 of its element's
  sum of absolute terms + 1e-6 (oracle.cpu.bptt_abs_scale).
"""
import dataclasses

import numpy as np
import pytest
import torch

from oracle.cpu import OracleCell, bptt_abs_scale
from tests.helpers import assert_grads_per_element, tiny_config
from v1_glif_model_amd import synthetic as sy
from v1_glif_model_amd.tables import build_cell_tables

pytestmark = pytest.mark.gpu

# (N, fan-in, D, nb, n_types, B, T, n_lgn, lgn fan-in, pseudo_gauss, input weight scale: set so
# that 3-7 % of the (tick, batch, neuron) entries spike)
CASES = [
    (1, 1, 1, 1, 1, 1, 20, 5, 2, True, 150.0),
    (37, 3, 2, 2, 3, 2, 24, 11, 3, False, 60.0),
    (64, 8, 4, 3, 7, 4, 20, 30, 4, True, 60.0),
    (65, 5, 9, 5, 5, 5, 24, 17, 5, True, 25.0),
    (130, 6, 8, 8, 20, 3, 18, 40, 6, False, 25.0),
    (130, 2, 3, 4, 12, 7, 18, 9, 2, True, 150.0),
    (200, 12, 5, 6, 2, 12, 16, 50, 8, True, 60.0),
    (65, 4, 2, 1, 4, 17, 14, 20, 3, False, 400.0),
    (64, 6, 6, 4, 9, 32, 12, 25, 4, True, 150.0),
    (200, 10, 1, 5, 5, 9, 16, 60, 5, False, 60.0),
    (130, 5, 3, 8, 8, 8, 16, 20, 4, True, 30.0),   # B * nb = 64: every lane of the chunk pull adds
]


def _case(i):
    N, fan, D, nb, nt, B, T, nl, lf, pg, ins = CASES[i]
    cfg = dataclasses.replace(tiny_config(n=N, fanin=fan, delays=D, n_lgn=nl, lgn_fanin=lf, n_bkg=6,
                                          bkg_fanin=3, rs=3.0, ins=ins, lgn_p=0.08),
                              n_basis=nb, n_syn_types=nt, fanin_mean=fan, fanin_sigma=None)
    net = sy.make_network(cfg, seed=100 + i, dense_basis=True)
    lgn, bkg = sy.make_inputs(cfg, seed=200 + i, seq_len=T, batch=B)
    kw = dict(gauss_std=0.3, damp=0.3, rd=0.2, vgd=0.4, pseudo_gauss=pg)
    ckw = dict(gauss_std=0.3, dampening_factor=0.3, recurrent_dampening_factor=0.2,
               voltage_gradient_dampening=0.4, pseudo_gauss=pg)
    return net, build_cell_tables(net), lgn, bkg, kw, ckw


def _state_np(st):
    return dict(zbuf=st[0].cpu().numpy(), v=st[1].cpu().numpy(), r=st[2].cpu().numpy().astype(np.int32),
                asc=st[3].cpu().numpy(), psc_rise=st[4].cpu().numpy(), psc=st[5].cpu().numpy())


@pytest.mark.parametrize("i", range(len(CASES)))
def test_shape_sweep(i):
    from tests.test_gpu_params import _state_dev
    from v1_glif_model_amd.models import V1Column
    net, tb, lgn, bkg, okw, ckw = _case(i)
    T, B = lgn.shape[0], lgn.shape[1]
    print("case", CASES[i], "synapses", tb.rec.n_syn, flush=True)
    oc = OracleCell(tb, **okw)
    oz, ov, oref, ost = oc.forward(lgn, bkg)
    # deterministic forward + BPTT
    cell = V1Column(net, mode="deterministic", **ckw)
    z, v, st = cell.rollout(lgn, bkg)
    assert oz.sum() > 0
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    for k, a in _state_np(st).items():
        e = ost[k]
        np.testing.assert_array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                                      e.view(np.uint32) if e.dtype == np.float32 else e, err_msg=k)
    gz = np.random.default_rng(300 + i).normal(0, 1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"))
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz)
    sc = bptt_abs_scale(tb, lgn, bkg, oz, oref, ov, gz_loss=gz, **okw)
    for k in ("rec", "lgn", "bkg"):
        assert_grads_per_element(g[k].cpu().numpy(), og[k], sc[k], what=k)
    # event forward, three ticks at a time from the oracle's state
    ev = V1Column(net, mode="event", **ckw)
    K = 3
    ws = ev.workspace(B, K)
    s = oc.zero_state(B)
    for t0 in range(T - K + 1):
        ze, ve, _ = ev.rollout(lgn[t0:t0 + K], bkg[t0:t0 + K], state=_state_dev(ev, s), ws=ws)
        oz3, ov3, _, _ = oc.forward(lgn[t0:t0 + K], bkg[t0:t0 + K], state=s)
        np.testing.assert_array_equal(ze.cpu().numpy().astype(np.uint8), oz3, err_msg=f"tick {t0}")
        err = np.abs(ve.cpu().numpy().astype(np.float64) - ov3)
        assert np.all(err <= 1e-5 * np.abs(ov3) + 1e-6), (t0, float(err.max()))
        _, _, _, s = oc.forward(lgn[t0:t0 + 1], bkg[t0:t0 + 1], state=s)
    print("spikes", int(oz.sum()), flush=True)
