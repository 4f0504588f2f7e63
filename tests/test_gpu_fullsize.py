"""Parity at the benchmark's full size: config 2 (66k GLIF_3 neurons, 16.5M recurrent synapses,
delays 1-5, 5 receptor types, 17.4k LGN units, batch 5).

* deterministic forward: spike trains and voltages bit-exact with the C oracle over the first
  200 ms (the network is silent until ~70 ms, then ramps to ~1000 spikes per ms);
* event forward over the full 500 ms against the deterministic one: spike trains identical over
  the first 50 ms and per-(batch, neuron) spike-count agreement of at least 99.9 % over the run;
* BPTT of a 100 ms deterministic rollout (the grouped row-sliced walk on the full table, 33
  backward windows) against the oracle's, within 1e-5 of the gradient's scale.

The oracle runs its OpenMP loops, which give the same bits as one thread."""
import os

import numpy as np
import pytest
import torch

from oracle import cpu as orc
from v1_glif_model_amd import synthetic as sy
from v1_glif_model_amd.tables import build_cell_tables

pytestmark = pytest.mark.gpu

CELL_KW = dict(gauss_std=0.5, dampening_factor=0.5, recurrent_dampening_factor=0.5,
               voltage_gradient_dampening=0.5, pseudo_gauss=True)
ORC_KW = dict(vgd=0.5, rd=0.5, gauss_std=0.5, damp=0.5, pseudo_gauss=True)


@pytest.fixture(scope="module")
def config2():
    cfg = sy.config(2)
    net = sy.make_network(cfg, seed=0)
    tb = build_cell_tables(net)
    orc.set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    return cfg, net, tb


def test_config2_forward_deterministic_and_event(config2):
    from v1_glif_model_amd.models import V1Column
    cfg, net, tb = config2
    T, B, To = 500, cfg.batch, 200
    lgn, bkg = sy.make_inputs(cfg, seed=1, seq_len=T, batch=B)
    cell = V1Column(net, mode="deterministic", **CELL_KW)
    zd, vd, _ = cell.rollout(lgn, bkg)
    ze, _, _ = cell.rollout(lgn, bkg, mode="event")
    zd = zd.cpu().numpy().astype(np.uint8)
    vd = vd.cpu().numpy()
    ze = ze.cpu().numpy().astype(np.uint8)
    del cell
    oz, ov, _, _ = orc.OracleCell(tb, **ORC_KW).forward(lgn[:To], bkg[:To])
    print("oracle spikes over", To, "ms:", int(oz.sum()), "; GPU spikes over", T, "ms:", int(zd.sum()), flush=True)
    assert oz.sum() > 10000
    np.testing.assert_array_equal(zd[:To], oz)
    np.testing.assert_array_equal(vd[:To].view(np.uint32), ov.view(np.uint32))
    differ = np.flatnonzero((ze != zd).any(axis=(1, 2)))
    agree = float(np.mean(ze.sum(0) == zd.sum(0)))
    print("event vs deterministic: first differing ms", differ[0] if differ.size else None,
          "count agreement", agree, flush=True)
    assert np.array_equal(ze[:50], zd[:50])
    assert agree >= 0.999


def test_config2_bptt(config2):
    from v1_glif_model_amd.models import V1Column
    cfg, net, tb = config2
    T, B = 100, cfg.batch
    lgn, bkg = sy.make_inputs(cfg, seed=1, seq_len=T, batch=B)
    cell = V1Column(net, mode="deterministic", **CELL_KW)
    z, v, _ = cell.rollout(lgn, bkg)
    oc = orc.OracleCell(tb, **ORC_KW)
    oz, ov, oref, _ = oc.forward(lgn, bkg)
    assert oz.sum() > 100
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    gz = np.random.default_rng(11).normal(0, 1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"))
    g = {k: t.cpu().numpy() for k, t in g.items()}
    del cell
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz)
    for k in ("rec", "lgn", "bkg"):
        a, e = g[k], og[k]
        scale = np.max(np.abs(e))
        err = np.max(np.abs(a - e))
        print(k, "max|dW|", scale, "max err", err, "nonzero", int(np.count_nonzero(e)), flush=True)
        assert scale > 0, k
        assert err <= 1e-5 * scale + 1e-6, k
