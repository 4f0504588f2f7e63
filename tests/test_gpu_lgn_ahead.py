"""GPU parity of the LGN currents computed ahead of the T loop.

For batch sizes up to 8 the cell computes the LGN currents of 64 ticks at a time (k_lgn_rows)
into a ring of 130 current slots, the first segment before the loop and each later one on the
cell's side stream beside the previous segment's ticks; the deterministic step
adds a slot to the pulled recurrent currents, the event push (from batch 3) adds the recurrent
events onto it.  These tests run rollouts long enough to cross segment boundaries and wrap the
ring (T = 64, 65 and 200: segments of 64, 1 and 8 ticks at the end), at batch sizes on both sides
of the thresholds (1, 2: event mode pushes the LGN events; 3, 5, 8: the pass in both modes; 9:
neither, the per-tick LGN push and pull), against the C oracle on the same inputs:

* deterministic forward over all T: spikes, voltages and the final state bit-exact;
* event forward with zero recurrent weights, at the batch sizes where event mode runs the pass
  (3, 5, 8): the currents are then the LGN pass's (in the reference's order) plus the
  background, so the event forward too is bit-exact over all T (below batch 3 and above 8 the
  LGN events are pushed with atomics, in no fixed order);
* event forward of the full network: per-neuron spike-count agreement >= 99.9 %, spike trains
  identical and voltages within 1e-5 relative / 1e-6 absolute up to the first tick whose trains
  differ (the recurrent atomics' order is free);
* a deterministic rollout split at tick 70 (the second half starts its own segments from the
  carried state) equals the one-piece rollout bit for bit;
* rollouts enqueued on torch streams other than the default one (the side stream's events
  order its passes against whichever stream the caller uses).
"""
import dataclasses

import numpy as np
import pytest
import torch

from oracle.cpu import OracleCell
from tests.helpers import tiny_config
from v1_glif_model_amd import synthetic as sy
from v1_glif_model_amd.tables import build_cell_tables

pytestmark = pytest.mark.gpu

BATCHES = [1, 2, 3, 5, 8, 9]
KW = dict(gauss_std=0.3, damp=0.3, rd=0.2, vgd=0.4, pseudo_gauss=True)
CKW = dict(gauss_std=0.3, dampening_factor=0.3, recurrent_dampening_factor=0.2,
           voltage_gradient_dampening=0.4, pseudo_gauss=True)


def _net(rs, seed, ins=2.0):
    cfg = dataclasses.replace(tiny_config(n=130, fanin=6, delays=3, n_lgn=40, lgn_fanin=6, n_bkg=6,
                                          bkg_fanin=3, rs=rs, ins=ins, lgn_p=0.08),
                              n_basis=3, n_syn_types=4, fanin_mean=6, fanin_sigma=None)
    return cfg, sy.make_network(cfg, seed=seed, dense_basis=True)


def _inputs(cfg, B, T, seed):
    return sy.make_inputs(cfg, seed=seed, seq_len=T, batch=B)


def _state_np(st):
    return dict(zbuf=st[0].cpu().numpy(), v=st[1].cpu().numpy(), r=st[2].cpu().numpy().astype(np.int32),
                asc=st[3].cpu().numpy(), psc_rise=st[4].cpu().numpy(), psc=st[5].cpu().numpy())


def _assert_bit_exact(z, v, st, oz, ov, ost, what):
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz, err_msg=f"{what}: spikes")
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32), err_msg=f"{what}: voltages")
    for k, a in _state_np(st).items():
        e = ost[k]
        np.testing.assert_array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                                      e.view(np.uint32) if e.dtype == np.float32 else e, err_msg=f"{what}: {k}")


@pytest.mark.parametrize("B", BATCHES)
def test_deterministic_forward_across_segments(B):
    from v1_glif_model_amd.models import V1Column
    cfg, net = _net(3.0, 11)
    lgn, bkg = _inputs(cfg, B, 200, 21 + B)
    print("B", B, "T", 200, flush=True)
    oz, ov, _, ost = OracleCell(build_cell_tables(net), **KW).forward(lgn, bkg)
    assert oz.mean() > 0.01
    z, v, st = V1Column(net, mode="deterministic", **CKW).rollout(lgn, bkg)
    _assert_bit_exact(z, v, st, oz, ov, ost, f"deterministic B={B}")


@pytest.mark.parametrize("T", [64, 65, 200])
@pytest.mark.parametrize("B", [3, 5, 8])
def test_event_forward_input_currents_bit_exact(B, T):
    from v1_glif_model_amd.models import V1Column
    cfg, net = _net(0.0, 12, ins=5.0)
    assert not np.any(net["network"]["synapses"]["weights"])
    lgn, bkg = _inputs(cfg, B, T, 31 + B)
    print("B", B, "T", T, flush=True)
    oz, ov, _, ost = OracleCell(build_cell_tables(net), **KW).forward(lgn, bkg)
    assert oz.mean() > 0.01
    z, v, st = V1Column(net, mode="event", **CKW).rollout(lgn, bkg)
    _assert_bit_exact(z, v, st, oz, ov, ost, f"event, zero recurrent weights, B={B}")


@pytest.mark.parametrize("B", BATCHES)
def test_event_forward_across_segments(B):
    from v1_glif_model_amd.models import V1Column
    cfg, net = _net(3.0, 13)
    T = 200
    lgn, bkg = _inputs(cfg, B, T, 41 + B)
    print("B", B, "T", T, flush=True)
    oz, ov, _, _ = OracleCell(build_cell_tables(net), **KW).forward(lgn, bkg)
    z, v, _ = V1Column(net, mode="event", **CKW).rollout(lgn, bkg)
    z = z.cpu().numpy().astype(np.uint8)
    v = v.cpu().numpy().astype(np.float64)
    cg, co = z.sum(0).astype(np.int64), oz.sum(0).astype(np.int64)
    agree = 1.0 - np.abs(cg - co).sum() / max(co.sum(), 1)
    assert agree >= 0.999, agree
    diff = np.nonzero(np.any(z != oz, axis=(1, 2)))[0]
    t_end = int(diff[0]) if diff.size else T
    err = np.abs(v[:t_end] - ov[:t_end])
    assert np.all(err <= 1e-5 * np.abs(ov[:t_end]) + 1e-6), float(err.max())
    print("ticks compared", t_end, "spikes", int(co.sum()), flush=True)


@pytest.mark.parametrize("B", [3, 5])
def test_deterministic_split_rollout_equals_one_piece(B):
    from v1_glif_model_amd.models import V1Column
    cfg, net = _net(3.0, 14)
    lgn, bkg = _inputs(cfg, B, 200, 51 + B)
    cell = V1Column(net, mode="deterministic", **CKW)
    z, v, st = cell.rollout(lgn, bkg)
    z1, v1, st1 = cell.rollout(lgn[:70], bkg[:70])
    z2, v2, st2 = cell.rollout(lgn[70:], bkg[70:], state=st1)
    np.testing.assert_array_equal(torch.cat([z1, z2]).cpu().numpy(), z.cpu().numpy())
    np.testing.assert_array_equal(torch.cat([v1, v2]).cpu().numpy().view(np.uint32), v.cpu().numpy().view(np.uint32))
    for a, b in zip(st2, st):
        np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy())


def test_forward_on_non_default_streams():
    """The side stream's LGN passes are ordered against the caller's stream by events: a
    deterministic rollout over 200 ticks enqueued on a fresh torch stream (inputs copied there
    first) equals the oracle bit for bit, and event rollouts on two different streams one after
    the other each agree with the oracle's per-neuron spike counts to 99.9 %."""
    from v1_glif_model_amd.models import V1Column
    cfg, net = _net(3.0, 15)
    B, T = 5, 200
    lgn, bkg = _inputs(cfg, B, T, 61)
    oz, ov, _, ost = OracleCell(build_cell_tables(net), **KW).forward(lgn, bkg)
    cell = V1Column(net, mode="deterministic", **CKW)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(s1):
        lg, bk = torch.tensor(lgn, device="cuda"), torch.tensor(bkg, device="cuda")
        z, v, st = cell.rollout(lg, bk)
    s1.synchronize()
    _assert_bit_exact(z, v, st, oz, ov, ost, "deterministic on a side torch stream")
    ev = V1Column(net, mode="event", **CKW)
    out = []
    for s in (s1, s2):
        with torch.cuda.stream(s):
            lg, bk = torch.tensor(lgn, device="cuda"), torch.tensor(bkg, device="cuda")
            ze, _, _ = ev.rollout(lg, bk)
        s.synchronize()
        out.append(ze.cpu().numpy())
    co = oz.sum(0).astype(np.int64)
    for ze in out:
        cg = ze.sum(0).astype(np.int64)
        assert 1.0 - np.abs(cg - co).sum() / max(co.sum(), 1) >= 0.999
