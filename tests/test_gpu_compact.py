"""GPU parity of the backward with compact G rows.

With synapse types fixed by (presynaptic class, postsynaptic class), the structure of the
reference's 121-type basis table (synaptic_data/basis_function_weights.csv, mapped per edge at
load_sparse.py:113-128), each post neuron receives few of the types, and the cell keeps G rows
for those types only (row post * rows + rank instead of syn_id * N + post).  The forward does
not change; every backward walk reads the compact rows: the grouped row-sliced walk (B = 5 and
B = 12), the type-phased walk (B = 2, 8-float rows; B = 8, one tick per window; B = 20, 32-float
rows), the recurrent dW pass and the LGN / background dW.

Bars: deterministic forward bit-exact with the oracle; weight gradients per element within
1e-5 of the element's sum of absolute terms + 1e-6 (oracle.cpu.bptt_abs_scale).
"""
import dataclasses

import numpy as np
import pytest
import torch

from oracle.cpu import OracleCell, bptt_abs_scale
from tests.helpers import assert_grads_per_element, error_summary, tiny_config
from v1_glif_model_amd import synthetic as sy
from v1_glif_model_amd.tables import build_cell_tables

pytestmark = pytest.mark.gpu

KW = dict(gauss_std=0.3, dampening_factor=0.1, recurrent_dampening_factor=0.1, voltage_gradient_dampening=0.5,
          pseudo_gauss=True)
OKW = dict(gauss_std=0.3, damp=0.1, rd=0.1, vgd=0.5, pseudo_gauss=True)


def _class_net(cfg, seed, n_classes):
    net = sy.class_types(sy.make_network(cfg, seed=seed, dense_basis=True), n_classes=n_classes)
    return net, build_cell_tables(net)


def _bptt_check(cell, tb, lgn, bkg, oz, oref, ov, gz, what):
    oc = OracleCell(tb, **OKW)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"))
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz)
    sc = bptt_abs_scale(tb, lgn, bkg, oz, oref, ov, gz_loss=gz, **OKW)
    for k in ("rec", "lgn", "bkg"):
        a = g[k].cpu().numpy()
        assert np.max(np.abs(og[k])) > 0, (what, k)
        assert_grads_per_element(a, og[k], sc[k], what=f"{what} {k}")
        print(what, k, error_summary(a, og[k], sc[k]))


def test_class_types_give_few_types_per_neuron():
    """The generator's structure: every post receives at most n_classes types (class 0 from the
    inputs, its own post class fixed), and the cell picks compact rows for it."""
    from v1_glif_model_amd.models import V1Column
    cfg = tiny_config(rs=2.0, ins=3.0)
    net, tb = _class_net(cfg, 51, 5)
    cls = net["neuron_class"]
    for pop in (net["network"]["synapses"], net["lgn_input"], net["bkg_input"]):
        post = np.asarray(pop["indices"])[:, 0]
        sid = np.asarray(pop["syn_ids"]).astype(np.int64)
        np.testing.assert_array_equal(sid % 5, cls[post])
    cell = V1Column(net, mode="deterministic", **KW)
    rows, compact = cell.g_layout()
    assert compact and rows <= 5, (rows, compact)
    plain = V1Column(sy.make_network(cfg, seed=51, dense_basis=True), mode="deterministic", **KW)
    assert plain.g_layout() == (5, False)


@pytest.mark.parametrize("B", [2, 5, 8, 12, 20])
def test_compact_rows_bptt(B):
    from v1_glif_model_amd.models import V1Column
    cfg = tiny_config(rs=2.0, ins=3.0)
    net, tb = _class_net(cfg, 52 + B, 5)
    T = 30
    lgn, bkg = sy.make_inputs(cfg, seed=53, seq_len=T, batch=B)
    cell = V1Column(net, mode="deterministic", **KW)
    assert cell.g_layout()[1]
    z, v, _ = cell.rollout(lgn, bkg)
    oz, ov, oref, _ = OracleCell(tb, **OKW).forward(lgn, bkg)
    assert oz.sum() > 0
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    gz = np.random.default_rng(54 + B).normal(0, 1, oz.shape).astype(np.float32)
    _bptt_check(cell, tb, lgn, bkg, oz, oref, ov, gz, f"B={B}")


def test_typed_push_voltages_per_tick():
    """Event forward with per-type slots (a dense basis: each synapse event is one atomic into
    its post's type slot, the step folds the slots through the basis): from the oracle's state
    at every tick, three ticks on, spike trains equal and voltages within 1e-5 relative /
    1e-6 absolute."""
    from tests.test_gpu_params import _state_dev
    from v1_glif_model_amd.models import V1Column
    cfg = tiny_config(rs=2.0, ins=3.0)
    net, tb = _class_net(cfg, 81, 5)
    T, B, K = 40, 3, 3
    lgn, bkg = sy.make_inputs(cfg, seed=82, seq_len=T, batch=B)
    cell = V1Column(net, mode="event", **KW)
    assert cell.g_layout()[1]
    oc = OracleCell(tb, **OKW)
    st = oc.zero_state(B)
    ws = cell.workspace(B, K)
    worst, spikes = 0.0, 0
    for t0 in range(T - K):
        ze, ve, _ = cell.rollout(lgn[t0:t0 + K], bkg[t0:t0 + K], state=_state_dev(cell, st), ws=ws)
        oz3, ov3, _, _ = oc.forward(lgn[t0:t0 + K], bkg[t0:t0 + K], state=st)
        np.testing.assert_array_equal(ze.cpu().numpy().astype(np.uint8), oz3)
        ve = ve.cpu().numpy().astype(np.float64)
        err = np.abs(ve - ov3)
        assert np.all(err <= 1e-5 * np.abs(ov3) + 1e-6), (t0, float(err.max()))
        worst = max(worst, float(err.max()))
        spikes += int(oz3[0].sum())
        _, _, _, st = oc.forward(lgn[t0:t0 + 1], bkg[t0:t0 + 1], state=st)
    assert spikes > 0
    print("largest per-tick voltage difference", worst)


def test_compact_rows_event_mode_and_updated_weights():
    """Event forward, then an ExponentiatedAdam step on all three populations (the compact
    copies of the weights refresh with the others), then a second rollout and BPTT against the
    oracle given the updated weights."""
    from v1_glif_model_amd.models import V1Column
    from v1_glif_model_amd.optim import ExponentiatedAdam
    cfg = tiny_config(rs=2.0, ins=3.0)
    net, tb = _class_net(cfg, 61, 6)
    B, T = 5, 30
    lgn, bkg = sy.make_inputs(cfg, seed=62, seq_len=T, batch=B)
    cell = V1Column(net, mode="event", train_noise=True, **KW)
    assert cell.g_layout()[1]
    z, _, _ = cell.rollout(lgn, bkg)
    oz, ov, oref, _ = OracleCell(tb, **OKW).forward(lgn, bkg)
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    gz = np.random.default_rng(63).normal(0, 1, oz.shape).astype(np.float32)
    _bptt_check(cell, tb, lgn, bkg, oz, oref, ov, gz, "event")
    rng = np.random.default_rng(64)
    grads = [(torch.tensor(rng.normal(0, 1, t.n_syn).astype(np.float32), device="cuda"), var)
             for t, var in ((tb.rec, cell.recurrent_weight_values), (tb.lgn, cell.input_weight_values),
                            (tb.bkg, cell.bkg_input_weights))]
    ExponentiatedAdam(learning_rate=0.2).apply_gradients(grads)
    tb2 = dataclasses.replace(
        tb, rec=dataclasses.replace(tb.rec, weight=cell.recurrent_weight_values.detach().cpu().numpy()),
        lgn=dataclasses.replace(tb.lgn, weight=cell.input_weight_values.detach().cpu().numpy()),
        bkg=dataclasses.replace(tb.bkg, weight=cell.bkg_input_weights.detach().cpu().numpy()))
    assert not np.array_equal(tb2.rec.weight, tb.rec.weight)
    z2, _, _ = cell.rollout(lgn, bkg)
    oz2, ov2, oref2, _ = OracleCell(tb2, **OKW).forward(lgn, bkg)
    np.testing.assert_array_equal(z2.cpu().numpy().astype(np.uint8), oz2)
    _bptt_check(cell, tb2, lgn, bkg, oz2, oref2, ov2, gz, "after update")


@pytest.mark.parametrize("B", [2, 5])
def test_layouts_agree(B):
    """The same cell with type-major and with compact rows (glif_cell_set_g_layout): G holds the
    same values, so the type-phased walk (B = 2, which sums each column type by type in the same
    order under both layouts) gives bit-identical gradients; the grouped walk (B = 5) orders a
    column's sum by G row, so its dz, and through it the gradients, differ by rounding only."""
    from v1_glif_model_amd.models import V1Column
    cfg = tiny_config(rs=2.0, ins=3.0)
    net, tb = _class_net(cfg, 71, 5)
    T = 30
    lgn, bkg = sy.make_inputs(cfg, seed=72, seq_len=T, batch=B)
    cell = V1Column(net, mode="deterministic", **KW)
    gz = None
    out = {}
    for compact in (False, True):
        cell.set_g_layout(compact)
        assert cell.g_layout()[1] == compact
        z, v, _ = cell.rollout(lgn, bkg)
        if gz is None:
            gz = np.random.default_rng(73).normal(0, 1, tuple(z.shape)).astype(np.float32)
        g = cell.backward(gz=torch.tensor(gz, device="cuda"))
        out[compact] = {k: g[k].cpu().numpy() for k in ("rec", "lgn", "bkg")}
    if B == 2:
        for k in out[True]:
            np.testing.assert_array_equal(out[True][k].view(np.uint32), out[False][k].view(np.uint32), err_msg=k)
    else:
        oz, ov, oref, _ = OracleCell(tb, **OKW).forward(lgn, bkg)
        sc = bptt_abs_scale(tb, lgn, bkg, oz, oref, ov, gz_loss=gz, **OKW)
        for k in out[True]:
            assert_grads_per_element(out[True][k], out[False][k], sc[k], what=k)


@pytest.mark.parametrize("B", [2, 5, 12, 20])
def test_op_level_backward_own_compact_rows(B):
    """The op-level custom gradient (glif_syn_bwd, models.py:182-241) on tables whose posts each
    receive few types: the table keeps its own compact rows (G over rows post * rows + rank,
    smaller workspace), walked by the type-phased walk (B = 2, 20) or the grouped walk (B = 5,
    12); dz and dW per element within 1e-5 of the sum of absolute terms + 1e-6 against the
    oracle's op and the float64 brute force.  Recurrent table with spikes, background table
    with Poisson counts."""
    from oracle import cpu as orc
    from oracle import dense
    from v1_glif_model_amd._lib import lib
    from v1_glif_model_amd.ops import SynapseTable
    cfg = tiny_config()
    net, tb = _class_net(cfg, 91, 5)
    rng = np.random.default_rng(92 + B)
    for pop, slots, counts in ((tb.rec, tb.max_delay, False), (tb.bkg, 1, True)):
        t = SynapseTable(pop.indices, pop.syn_id, (tb.n_neurons, pop.n_cols), tb.basis, n_delay_slots=slots)
        t.set_weights(torch.tensor(pop.weight, device="cuda"))
        Bp = 4 if B <= 4 else 8 if B <= 8 else 16 if B <= 16 else 32
        type_major_g = tb.n_neurons * tb.basis.shape[0] * Bp * 4
        assert int(lib().glif_syn_workspace(t.handle, B)) < type_major_g  # compact G rows
        if counts:
            z = ((rng.random((B, pop.n_cols)) < 0.3) * rng.integers(1, 4, (B, pop.n_cols))).astype(np.float32)
        else:
            z = (rng.random((B, pop.n_cols)) < 0.05).astype(np.float32)
        dy = rng.normal(0, 1, (B * tb.n_neurons, tb.n_basis)).astype(np.float32)
        dz, dw = t.backward(torch.tensor(z, device="cuda"), torch.tensor(dy, device="cuda"), counts=counts)
        dz, dw = dz.cpu().numpy(), dw.cpu().numpy()
        rdz, rdw = orc.syn_bwd(pop, z, tb.basis, dy, use_count=counts)
        dz64, dw64, dz_abs, dw_abs = dense.syn_bwd_f64(pop, z, tb.basis, dy, use_count=counts)
        assert np.count_nonzero(dw) > 0
        for got, ref, ex, sc, what in ((dz, rdz, dz64, dz_abs, "dz"), (dw, rdw, dw64, dw_abs, "dW")):
            assert_grads_per_element(got, ref, sc, what=what)
            assert_grads_per_element(got, ex, sc, what=what + " vs float64")
