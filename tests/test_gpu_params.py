"""GPU parity away from the symmetric point 0.5 of the surrogate and dampening parameters.

At rd = vgd = gauss_std = dampening_factor = 0.5 a swapped rd / 1 - rd, vgd / 1 - vgd or
Gaussian width / amplitude gives the same numbers; these tests run the cell at
(rd 0.2, vgd 0.3, dampening 0.3, width 0.7) and at the reference's training defaults
(rd 0.1, vgd 0.5, dampening 0.1, width 0.3; multi_training.py:1071-1074, 1155), for both
surrogates (models.py:17-28) with and without hard reset (models.py:1020-1023).

Bars: the deterministic forward is bit-exact (vgd != 0.5 makes the straight-through
re-sum v * (1 - vgd) + v * vgd differ from v by rounding, models.py:284-296, so this also
checks that the forward keeps the reference's two products); weight gradients per element
within 1e-5 of the element's sum of absolute terms + 1e-6 (oracle.cpu.bptt_abs_scale);
event mode: spike trains equal and voltages, three ticks on from an identical state, within
1e-5 relative / 1e-6 absolute.
"""
import numpy as np
import pytest
import torch

from oracle.cpu import OracleCell, bptt_abs_scale
from tests.helpers import assert_grads_per_element, error_summary, network, tiny_config
from tests.test_pins import PSETS
from v1_glif_model_amd import synthetic as sy

pytestmark = pytest.mark.gpu


def _kw(pset, pseudo_gauss, hard_reset):
    p = PSETS[pset]
    cell = dict(gauss_std=p["gauss_std"], dampening_factor=p["damp"], recurrent_dampening_factor=p["rd"],
                voltage_gradient_dampening=p["vgd"], pseudo_gauss=pseudo_gauss, hard_reset=hard_reset)
    orc = dict(vgd=p["vgd"], rd=p["rd"], gauss_std=p["gauss_std"], damp=p["damp"], pseudo_gauss=pseudo_gauss,
               hard_reset=hard_reset)
    return cell, orc


def _state_np(st):
    return dict(zbuf=st[0].cpu().numpy(), v=st[1].cpu().numpy(), r=st[2].cpu().numpy().astype(np.int32),
                asc=st[3].cpu().numpy(), psc_rise=st[4].cpu().numpy(), psc=st[5].cpu().numpy())


def _state_dev(cell, d):
    B = d["v"].shape[0]
    st = list(cell.zero_state(B))
    for i, k in enumerate(("zbuf", "v", "r", "asc", "psc_rise", "psc")):
        st[i] = torch.tensor(d[k].astype(np.int16) if k == "r" else d[k], device="cuda")
    return st


@pytest.mark.parametrize("hard_reset", [False, True])
@pytest.mark.parametrize("pseudo_gauss", [True, False])
@pytest.mark.parametrize("pset", list(PSETS))
@pytest.mark.parametrize("B", [2, 5])
def test_forward_and_bptt_asymmetric(B, pset, pseudo_gauss, hard_reset):
    """B = 2 takes the type-phased recurrent backward (8-float G rows), B = 5 the grouped
    row-sliced walk (16-float rows)."""
    from v1_glif_model_amd.models import V1Column
    ckw, okw = _kw(pset, pseudo_gauss, hard_reset)
    cfg = tiny_config(rs=2.0, ins=3.0)
    net, tb = network(cfg, seed=21 + B, dense_basis=True)
    T = 40
    lgn, bkg = sy.make_inputs(cfg, seed=22, seq_len=T, batch=B)
    cell = V1Column(net, mode="deterministic", **ckw)
    z, v, st = cell.rollout(lgn, bkg)
    oc = OracleCell(tb, **okw)
    oz, ov, oref, ost = oc.forward(lgn, bkg)
    assert oz.sum() > 0 and (not hard_reset or oref.sum() > 0)
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    for k, a in _state_np(st).items():
        np.testing.assert_array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                                      ost[k].view(np.uint32) if ost[k].dtype == np.float32 else ost[k], err_msg=k)
    rng = np.random.default_rng(B * 7 + len(pset))
    gz = rng.normal(0, 1, oz.shape).astype(np.float32)
    gv = rng.normal(0, 0.1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"), gv=torch.tensor(gv, device="cuda"))
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz, gv_loss=gv)
    sc = bptt_abs_scale(tb, lgn, bkg, oz, oref, ov, gz_loss=gz, gv_loss=gv, **okw)
    for k in ("rec", "lgn", "bkg"):
        a = g[k].cpu().numpy()
        assert np.max(np.abs(og[k])) > 0, k
        worst = assert_grads_per_element(a, og[k], sc[k], what=k)
        print(k, error_summary(a, og[k], sc[k]), "worst", worst)


@pytest.mark.parametrize("pset", list(PSETS))
def test_event_mode_asymmetric(pset):
    """Event (atomic) mode: spike trains equal the oracle's over the run, voltages within
    1e-5 relative / 1e-6 absolute over three ticks from the oracle's state at every tick, and
    the BPTT after the event rollout within the per-element bar."""
    from v1_glif_model_amd.models import V1Column
    ckw, okw = _kw(pset, True, False)
    cfg = tiny_config(rs=2.0, ins=3.0)
    net, tb = network(cfg, seed=31, dense_basis=True)
    T, B, K = 40, 3, 3
    lgn, bkg = sy.make_inputs(cfg, seed=32, seq_len=T, batch=B)
    cell = V1Column(net, mode="event", **ckw)
    z, v, _ = cell.rollout(lgn, bkg)
    oc = OracleCell(tb, **okw)
    oz, ov, oref, _ = oc.forward(lgn, bkg)
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    rng = np.random.default_rng(33)
    gz = rng.normal(0, 1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"))
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz)
    sc = bptt_abs_scale(tb, lgn, bkg, oz, oref, ov, gz_loss=gz, **okw)
    for k in ("rec", "lgn", "bkg"):
        assert_grads_per_element(g[k].cpu().numpy(), og[k], sc[k], what=k)
    # per-tick voltages from identical states
    st = oc.zero_state(B)
    ws = cell.workspace(B, K)
    worst = 0.0
    for t0 in range(T - K):
        dst = _state_dev(cell, st)
        ze, ve, _ = cell.rollout(lgn[t0:t0 + K], bkg[t0:t0 + K], state=dst, ws=ws)
        oz3, ov3, _, _ = oc.forward(lgn[t0:t0 + K], bkg[t0:t0 + K], state=st)
        np.testing.assert_array_equal(ze.cpu().numpy().astype(np.uint8), oz3)
        ve = ve.cpu().numpy().astype(np.float64)
        err = np.abs(ve - ov3)
        assert np.all(err <= 1e-5 * np.abs(ov3) + 1e-6), (t0, float(err.max()))
        worst = max(worst, float(err.max()))
        _, _, _, st = oc.forward(lgn[t0:t0 + 1], bkg[t0:t0 + 1], state=st)
    print("largest per-tick voltage difference", worst)


@pytest.mark.parametrize("mode,B", [("deterministic", 5), ("deterministic", 2), ("event", 5)])
def test_bptt_after_carried_state(mode, B):
    """The reference runs long sequences in chunks with the state carried over
    (osi_dsi_estimator.py:252-305).  The second chunk's BPTT starts from spikes in the
    carried history, which reach the recurrent dW of its first D ticks through the delay
    slots; against the oracle's BPTT with that history (zbuf0), per element."""
    from v1_glif_model_amd.models import V1Column
    ckw, okw = _kw("reference_defaults", True, False)
    cfg = tiny_config(rs=2.0, ins=3.0, delays=5)
    net, tb = network(cfg, seed=41 + B, dense_basis=True)
    T1, T2 = 30, 30
    lgn, bkg = sy.make_inputs(cfg, seed=42, seq_len=T1 + T2, batch=B)
    cell = V1Column(net, mode=mode, **ckw)
    _, _, st = cell.rollout(lgn[:T1], bkg[:T1])
    st0 = _state_np(st)
    assert st0["zbuf"].sum() > 0, "the carried history must hold spikes"
    z, v, _ = cell.rollout(lgn[T1:], bkg[T1:], state=st)
    oc = OracleCell(tb, **okw)
    oz, ov, oref, _ = oc.forward(lgn[T1:], bkg[T1:], state=st0)
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    if mode == "deterministic":
        np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    gz = np.random.default_rng(43).normal(0, 1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"))
    og = oc.backward(lgn[T1:], bkg[T1:], oz, oref, ov, gz_loss=gz, zbuf0=st0["zbuf"])
    sc = bptt_abs_scale(tb, lgn[T1:], bkg[T1:], oz, oref, ov, gz_loss=gz, zbuf0=st0["zbuf"], **okw)
    # the history's share of dW: the same BPTT without the history differs
    og0 = oc.backward(lgn[T1:], bkg[T1:], oz, oref, ov, gz_loss=gz)
    assert np.count_nonzero(og["rec"] != og0["rec"]) > 0
    for k in ("rec", "lgn", "bkg"):
        a = g[k].cpu().numpy()
        assert_grads_per_element(a, og[k], sc[k], what=k)
        print(k, error_summary(a, og[k], sc[k]))
