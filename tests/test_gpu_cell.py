"""GPU parity of the T-step GLIF_3 cell and its BPTT against the CPU oracle.

Bars: deterministic mode reproduces the oracle's spike trains, voltages and final
state bit for bit; event (atomic) mode keeps >= 99.9% per-neuron spike-count
agreement; weight gradients within 1e-5 relative of the oracle, measured against
the gradient's scale (max |dW|) because the BPTT sums cancel.
"""
import numpy as np
import pytest
import torch

from oracle.cpu import OracleCell
from tests.helpers import network, tiny_config
from v1_glif_model_amd import synthetic as sy

pytestmark = pytest.mark.gpu


def _cell(tb_net, mode, **kw):
    from v1_glif_model_amd.models import V1Column
    net, _ = tb_net
    return V1Column(net, mode=mode, **kw)


def _oracle(tb, **kw):
    return OracleCell(tb, **kw)


CELL_KW = dict(gauss_std=0.5, dampening_factor=0.5, recurrent_dampening_factor=0.5,
               voltage_gradient_dampening=0.5, pseudo_gauss=True)
ORC_KW = dict(vgd=0.5, rd=0.5, gauss_std=0.5, damp=0.5, pseudo_gauss=True)


def _inputs(cfg, T, B, seed=1):
    return sy.make_inputs(cfg, seed=seed, seq_len=T, batch=B)


@pytest.mark.parametrize("B", [1, 3])
def test_deterministic_forward_bit_exact_tiny(B):
    cfg = tiny_config(rs=2.0, ins=1.0)
    tn = network(cfg, seed=0, dense_basis=True)
    lgn, bkg = _inputs(cfg, 60, B)
    cell = _cell(tn, "deterministic", **CELL_KW)
    z, v, st = cell.rollout(lgn, bkg)
    oz, ov, oref, ost = _oracle(tn[1], **ORC_KW).forward(lgn, bkg)
    print("rate Hz", oz.mean() * 1000)
    assert oz.sum() > 0
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    np.testing.assert_array_equal(st[0].cpu().numpy(), ost["zbuf"])
    np.testing.assert_array_equal(st[2].cpu().numpy().astype(np.int32), ost["r"])
    for i, k in ((3, "asc"), (4, "psc_rise"), (5, "psc")):
        np.testing.assert_array_equal(st[i].cpu().numpy().view(np.uint32), ost[k].view(np.uint32))


def test_deterministic_forward_bit_exact_config0():
    cfg = sy.config(0)
    tn = network(cfg, seed=0)
    lgn, bkg = _inputs(cfg, 200, cfg.batch)   # 200 ms: past the input ramp, recurrent events on
    cell = _cell(tn, "deterministic", **CELL_KW)
    z, v, _ = cell.rollout(lgn, bkg)
    oz, ov, _, _ = _oracle(tn[1], **ORC_KW).forward(lgn, bkg)
    print("config0 rate Hz", oz.mean() * 1000, "spikes", int(oz.sum()))
    assert oz.sum() > 100
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32))


def test_event_forward_matches_config0():
    cfg = sy.config(0)
    tn = network(cfg, seed=0)
    T = 300
    lgn, bkg = _inputs(cfg, T, 1)
    cell = _cell(tn, "event", **CELL_KW)
    z, v, _ = cell.rollout(lgn, bkg)
    oz, ov, _, _ = _oracle(tn[1], **ORC_KW).forward(lgn, bkg)
    z = z.cpu().numpy().astype(np.uint8)
    first50 = np.array_equal(z[:50], oz[:50])
    counts, ocounts = z.sum(0), oz.sum(0)
    agree = float(np.mean(counts == ocounts))
    print("event: identical first 50 ms", first50, "count agreement", agree, "spikes", int(oz.sum()))
    assert first50
    assert agree >= 0.999


@pytest.mark.parametrize("D,B", [(1, 3), (3, 3), (5, 3), (5, 20)])
def test_event_forward_delays_and_split_rollout(D, B):
    """Event mode over max delays 1, 3 and 5 (with D = 1 the push beside the step has no
    recurrent delay slots; the step's waves push every recurrent event), batch 3 and 20, and
    a rollout split in two, whose second part starts with spikes in the carried history that
    its tick 0 pushes.  Spike trains equal the oracle's; voltages within 1e-4 (the event sums
    differ from the oracle's order by rounding only); the BPTT after the one-piece event
    rollout (the training path) within 1e-5 of the oracle's."""
    cfg = tiny_config(rs=2.0, ins=3.0, delays=D)
    tn = network(cfg, seed=8, dense_basis=True)
    T, T1 = 50, 33
    lgn, bkg = _inputs(cfg, T, B, seed=9)
    oc = _oracle(tn[1], **ORC_KW)
    oz, ov, oref, _ = oc.forward(lgn, bkg)
    assert oz[T1 - D:T1].sum() > 0   # the split point carries spikes in its history
    cell = _cell(tn, "event", **CELL_KW)
    z1, v1, state = cell.rollout(lgn[:T1], bkg[:T1], state=cell.zero_state(B))
    z2, v2, _ = cell.rollout(lgn[T1:], bkg[T1:], state=state)
    z, v, _ = cell.rollout(lgn, bkg)
    for zz, vv in ((z, v), (torch.cat([z1, z2]), torch.cat([v1, v2]))):
        np.testing.assert_array_equal(zz.cpu().numpy().astype(np.uint8), oz)
        assert np.max(np.abs(vv.cpu().numpy() - ov)) <= 1e-4
    gz = np.random.default_rng(D * 10 + B).normal(0, 1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"))
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz)
    for k in ("rec", "lgn", "bkg"):
        a, e = g[k].cpu().numpy(), og[k]
        scale = np.max(np.abs(e))
        assert scale > 0, k
        assert np.max(np.abs(a - e)) <= 1e-5 * scale + 1e-6, k


@pytest.mark.parametrize("D,B", [(1, 2), (4, 3)])
def test_deterministic_split_rollout_bit_exact(D, B):
    """Deterministic mode, one launch per tick with R updated a tick late: a rollout split in
    two (the second part starts from carried R, P and spikes in the history) equals the
    oracle's one-piece rollout bit for bit in spikes, voltages and both final states, so the
    last tick's R update and the first tick's (none: R of tick -1 is the state) are exact."""
    cfg = tiny_config(rs=2.0, ins=3.0, delays=D)
    tn = network(cfg, seed=12, dense_basis=True)
    T, T1 = 40, 30
    lgn, bkg = _inputs(cfg, T, B, seed=13)
    oc = _oracle(tn[1], **ORC_KW)
    oz, ov, _, ost = oc.forward(lgn, bkg)
    _, _, _, ost1 = oc.forward(lgn[:T1], bkg[:T1])
    assert oz[T1 - D:T1].sum() > 0   # the split point carries spikes in its history
    cell = _cell(tn, "deterministic", **CELL_KW)
    z1, v1, state = cell.rollout(lgn[:T1], bkg[:T1], state=cell.zero_state(B))
    mid = [s.clone() for s in state]
    z2, v2, st = cell.rollout(lgn[T1:], bkg[T1:], state=state)
    np.testing.assert_array_equal(torch.cat([z1, z2]).cpu().numpy().astype(np.uint8), oz)
    np.testing.assert_array_equal(torch.cat([v1, v2]).cpu().numpy().view(np.uint32), ov.view(np.uint32))
    for got, exp in ((mid, ost1), (st, ost)):
        np.testing.assert_array_equal(got[0].cpu().numpy(), exp["zbuf"])
        np.testing.assert_array_equal(got[2].cpu().numpy().astype(np.int32), exp["r"])
        for i, k in ((1, "v"), (3, "asc"), (4, "psc_rise"), (5, "psc")):
            np.testing.assert_array_equal(got[i].cpu().numpy().view(np.uint32), exp[k].view(np.uint32), err_msg=k)


@pytest.mark.parametrize("pseudo_gauss,hard_reset", [(True, False), (False, False), (True, True)])
def test_backward_matches_oracle(pseudo_gauss, hard_reset):
    cfg = tiny_config(rs=2.0, ins=1.0)
    tn = network(cfg, seed=1, dense_basis=True)
    T, B = 40, 2
    lgn, bkg = _inputs(cfg, T, B)
    kw = dict(CELL_KW, pseudo_gauss=pseudo_gauss, hard_reset=hard_reset)
    okw = dict(ORC_KW, pseudo_gauss=pseudo_gauss, hard_reset=hard_reset)
    cell = _cell(tn, "deterministic", **kw)
    z, v, _ = cell.rollout(lgn, bkg)
    oc = _oracle(tn[1], **okw)
    oz, ov, oref, _ = oc.forward(lgn, bkg)
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    rng = np.random.default_rng(5)
    gz = rng.normal(0, 1, oz.shape).astype(np.float32)
    gv = rng.normal(0, 0.1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"), gv=torch.tensor(gv, device="cuda"))
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz, gv_loss=gv)
    for k in ("rec", "lgn", "bkg"):
        a, e = g[k].cpu().numpy(), og[k]
        scale = np.max(np.abs(e))
        err = np.max(np.abs(a - e))
        print(k, "max|dW|", scale, "max err", err, "rel", err / scale)
        assert scale > 0
        assert err <= 1e-5 * scale + 1e-6


@pytest.mark.parametrize("B,n,T", [(3, 300, 40), (4, 301, 40), (5, 299, 40), (9, 302, 30), (16, 300, 20)])
def test_backward_grouped_walk_matches_oracle(B, n, T):
    """16-float G rows (B = 3-5 with three-tick windows, B = 9-16 with one-tick windows)
    take the grouped row-sliced recurrent backward: four columns per lane group (n * D
    not a multiple of four leaves a partial last group), a last window of two ticks
    (T = 40: 38 = 12 * 3 + 2); dz and dW of active columns within the bar."""
    cfg = tiny_config(n=n, rs=2.0, ins=3.0)
    tn = network(cfg, seed=n + B, dense_basis=True)
    lgn, bkg = _inputs(cfg, T, B, seed=B)
    cell = _cell(tn, "deterministic", **CELL_KW)
    z, v, _ = cell.rollout(lgn, bkg)
    oc = _oracle(tn[1], **ORC_KW)
    oz, ov, oref, _ = oc.forward(lgn, bkg)
    assert oz.sum() > 0
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    rng = np.random.default_rng(B * 100 + T)
    gz = rng.normal(0, 1, oz.shape).astype(np.float32)
    gv = rng.normal(0, 0.1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"), gv=torch.tensor(gv, device="cuda"))
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz, gv_loss=gv)
    for k in ("rec", "lgn", "bkg"):
        a, e = g[k].cpu().numpy(), og[k]
        scale = np.max(np.abs(e))
        assert scale > 0, k
        assert np.max(np.abs(a - e)) <= 1e-5 * scale + 1e-6, k


@pytest.mark.parametrize("B", [2, 5])
def test_many_synapse_types_forward_and_backward(B):
    """121 synapse types over 4 receptors, the shape of the reference's basis table
    (synaptic_data/basis_function_weights.csv: one row per synaptic model): G has 121 row
    blocks, the grouped walk's rows span all of them (B = 5) and the type-phased walk has
    121 phases (B = 2); deterministic forward bit-exact, BPTT within the bar."""
    import dataclasses
    cfg = dataclasses.replace(tiny_config(rs=3.0, ins=4.0), n_syn_types=121, n_basis=4)
    tn = network(cfg, seed=11, dense_basis=True)
    T = 40
    lgn, bkg = _inputs(cfg, T, B, seed=12)
    cell = _cell(tn, "deterministic", **CELL_KW)
    z, v, _ = cell.rollout(lgn, bkg)
    oc = _oracle(tn[1], **ORC_KW)
    oz, ov, oref, _ = oc.forward(lgn, bkg)
    assert oz.sum() > 0
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    gz = np.random.default_rng(13).normal(0, 1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"))
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz)
    for k in ("rec", "lgn", "bkg"):
        a, e = g[k].cpu().numpy(), og[k]
        scale = np.max(np.abs(e))
        assert scale > 0, k
        assert np.max(np.abs(a - e)) <= 1e-5 * scale + 1e-6, k


def test_backward_rate_loss_per_neuron_grad():
    """gz broadcast per neuron (the rate-loss form) equals the dense form."""
    cfg = tiny_config(rs=2.0, ins=1.0)
    tn = network(cfg, seed=2, dense_basis=True)
    T, B = 30, 2
    lgn, bkg = _inputs(cfg, T, B)
    cell = _cell(tn, "deterministic", **CELL_KW)
    cell.rollout(lgn, bkg)
    rng = np.random.default_rng(8)
    gn = rng.normal(0, 1, tn[1].n_neurons).astype(np.float32)
    g1 = cell.backward(gz_neuron=torch.tensor(gn, device="cuda"))
    dense_gz = np.broadcast_to(gn, (T, B, gn.size)).copy()
    g2 = cell.backward(gz=torch.tensor(dense_gz, device="cuda"))
    # the backward sums in a fixed order (no atomics on dz / dW): bit for bit
    for k in g1:
        np.testing.assert_array_equal(g1[k].cpu().numpy(), g2[k].cpu().numpy())


@pytest.mark.parametrize("B", [8, 20])
def test_wide_batch_forward_and_backward(B):
    """B > 5: one-tick backward windows with 8- and 32-float G rows (2 and 8 lanes per
    synapse); the deterministic forward stays bit-exact and the BPTT within the bar."""
    cfg = tiny_config(rs=2.0, ins=3.0)
    tn = network(cfg, seed=3, dense_basis=True)
    T = 40
    lgn, bkg = _inputs(cfg, T, B, seed=4)
    cell = _cell(tn, "deterministic", **CELL_KW)
    z, v, _ = cell.rollout(lgn, bkg)
    oc = _oracle(tn[1], **ORC_KW)
    oz, ov, oref, _ = oc.forward(lgn, bkg)
    assert oz.sum() > 0
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    rng = np.random.default_rng(6)
    gz = rng.normal(0, 1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"))
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz)
    for k in ("rec", "lgn", "bkg"):
        a, e = g[k].cpu().numpy(), og[k]
        scale = np.max(np.abs(e))
        assert scale > 0
        assert np.max(np.abs(a - e)) <= 1e-5 * scale + 1e-6, k


def test_call_steps_equal_rollout():
    """The per-step Keras-cell API (models.py:1059-1135) over T calls equals one T-step
    rollout (deterministic mode: bit for bit); without counts, call draws the background
    from the device stream and advances the step counter."""
    cfg = tiny_config(rs=2.0, ins=3.0)
    tn = network(cfg, seed=2, dense_basis=True)
    T, B = 20, 2
    lgn, bkg = _inputs(cfg, T, B, seed=3)
    cell = _cell(tn, "deterministic", **CELL_KW)
    zr, vr, _ = cell.rollout(lgn, bkg)
    state = cell.zero_state(B)
    for t in range(T):
        inp = torch.tensor(lgn[t], dtype=torch.float32, device="cuda")
        (z, v), state = cell.call(inp, state, bkg_counts=torch.tensor(bkg[t], device="cuda"))
        np.testing.assert_array_equal(z.detach().cpu().numpy(), zr[t].cpu().numpy())
        np.testing.assert_array_equal(v.detach().cpu().numpy().view(np.uint32), vr[t].cpu().numpy().view(np.uint32))
    assert int(state[6][0].item()) == T
    with torch.no_grad():   # not recorded: plain tensors
        (z, v), st2 = cell.call(torch.tensor(lgn[0], dtype=torch.float32, device="cuda"), state)
    assert z.grad_fn is None and not z.requires_grad
    assert z.shape == (B, tn[1].n_neurons) and int(st2[6][0].item()) == T + 1


@pytest.mark.parametrize("mode,core", [("range", False), ("threshold", False), ("range", True)])
def test_fused_voltage_regularization(mode, core):
    """VoltageRegularization (loss_functions.py:1047-1119) fused into the cell: the loss
    reduced from the kept voltages equals the loss of the output voltages, and the BPTT
    with the fused gradient equals the oracle's BPTT given dL/dv of that loss."""
    from v1_glif_model_amd.losses import VoltageRegularization
    cfg = tiny_config(rs=2.0, ins=3.0)
    tn = network(cfg, seed=5, dense_basis=True)
    T, B = 30, 3
    lgn, bkg = _inputs(cfg, T, B, seed=6)
    cell = _cell(tn, "deterministic", **CELL_KW)
    cost = 0.5
    N = tn[1].n_neurons
    mask = (np.arange(N) % 3 == 0) if core else None
    reg = VoltageRegularization(cell, voltage_cost=cost, penalty_mode=mode, core_mask=mask)
    z, v, _ = cell.rollout(lgn, bkg)
    vn = v.cpu().numpy().astype(np.float64)
    if mode == "range":
        m = np.maximum(np.abs(vn - 0.5) - 0.5, 0.0)
        pen, dpen = m * m, 2.0 * m * np.sign(vn - 0.5)
    else:
        pen, dpen = (vn - 1.0) ** 2, 2.0 * (vn - 1.0)
    sel = np.ones(N, bool) if mask is None else mask
    expect = cost * pen[:, :, sel].mean()
    # the tensor form (autograd's) switches the fused gradient off, the fused form on again
    assert abs(float(reg(v)) - expect) <= 1e-6 * abs(expect) + 1e-12
    loss = float(reg())
    assert abs(loss - expect) <= 1e-6 * abs(expect) + 1e-12
    oc = _oracle(tn[1], **ORC_KW)
    oz, ov, oref, _ = oc.forward(lgn, bkg)
    rng = np.random.default_rng(7)
    gz = rng.normal(0, 1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"))
    gv = (cost * dpen / (vn.shape[0] * vn.shape[1] * sel.sum()) * sel).astype(np.float32)
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz, gv_loss=gv)
    reg.disable()
    for k in ("rec", "lgn", "bkg"):
        a, e = g[k].cpu().numpy(), og[k]
        scale = np.max(np.abs(e))
        assert scale > 0
        assert np.max(np.abs(a - e)) <= 1e-5 * scale + 1e-6, k


@pytest.mark.parametrize("n", [120_000, 270_000])
def test_deterministic_large_bitmaps_bit_exact(n):
    """Large activity bitmaps: at 120k neurons (75 KB) the chunk kernel runs one 1024-lane
    workgroup per CU; at 270k (169 KB, beyond the 160 KB of LDS) the global-memory row pull
    runs instead.  Both bit-exact."""
    cfg = tiny_config(n=n, fanin=6, delays=5, n_lgn=200, lgn_fanin=4, n_bkg=10, bkg_fanin=2,
                      rs=4.0, ins=20.0, lgn_p=0.2)
    tn = network(cfg, seed=4)
    T, B = 20, 2
    lgn, bkg = _inputs(cfg, T, B, seed=5)
    cell = _cell(tn, "deterministic", **CELL_KW)
    z, v, _ = cell.rollout(lgn, bkg)
    oz, ov, _, _ = _oracle(tn[1], **ORC_KW).forward(lgn, bkg)
    assert oz.sum() > 0
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32))


@pytest.mark.parametrize("mode", ["deterministic", "event"])
@pytest.mark.parametrize("B", [2, 5])
@pytest.mark.parametrize("T", [1, 2, 3, 4, 7])
def test_short_sequences_forward_and_backward(T, B, mode):
    """Sequences shorter than / around one backward window (no window for T < 3); B = 5
    takes the grouped row-sliced recurrent backward.  Event mode: T = 1 runs the tick-0 push
    and the last step alone, T = 2 one fused step + push launch between them; voltages within
    1e-4 there, bit-exact in deterministic mode."""
    cfg = tiny_config(rs=2.0, ins=3.0, delays=1)
    tn = network(cfg, seed=6, dense_basis=True)
    lgn, bkg = _inputs(cfg, T, B, seed=7)
    cell = _cell(tn, mode, **CELL_KW)
    z, v, _ = cell.rollout(lgn, bkg)
    oc = _oracle(tn[1], **ORC_KW)
    oz, ov, oref, _ = oc.forward(lgn, bkg)
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    if mode == "deterministic":
        np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    else:
        assert np.max(np.abs(v.cpu().numpy() - ov)) <= 1e-4
    gz = np.random.default_rng(T).normal(0, 1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"))
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz)
    for k in ("rec", "lgn", "bkg"):
        a, e = g[k].cpu().numpy(), og[k]
        assert np.max(np.abs(a - e)) <= 1e-5 * max(np.max(np.abs(e)), 1e-30) + 1e-6, k


def test_voltage_regularization_through_autograd_is_not_doubled():
    """reg(v) on RSNNRollout's voltage output (the reference's usage) differentiated by
    autograd: the gradient reaches the cell as dL/dv once, and the fused form (switched off
    by that call) adds nothing; equals the oracle's BPTT given that dL/dv."""
    from v1_glif_model_amd.losses import VoltageRegularization
    from v1_glif_model_amd.models import RSNNRollout
    cfg = tiny_config(rs=2.0, ins=3.0)
    tn = network(cfg, seed=5, dense_basis=True)
    T, B = 30, 3
    lgn, bkg = _inputs(cfg, T, B, seed=6)
    cell = _cell(tn, "deterministic", train_input=True, train_recurrent_per_type=False, **CELL_KW)
    reg = VoltageRegularization(cell, voltage_cost=0.5, penalty_mode="threshold")
    w = (cell.recurrent_weight_values, cell.input_weight_values, cell.bkg_input_weights)
    z, v = RSNNRollout.apply(cell, torch.tensor(lgn, device="cuda"), torch.tensor(bkg, device="cuda"), *w)
    loss = reg(v)
    loss.backward()
    vn = v.detach().cpu().numpy().astype(np.float64)
    gv = (0.5 * 2.0 * (vn - 1.0) / vn.size).astype(np.float32)
    oc = _oracle(tn[1], **ORC_KW)
    oz, ov, oref, _ = oc.forward(lgn, bkg)
    og = oc.backward(lgn, bkg, oz, oref, ov, gv_loss=gv)
    for k, t in zip(("rec", "lgn", "bkg"), w):
        a, e = t.grad.cpu().numpy(), og[k]
        scale = np.max(np.abs(e))
        assert scale > 0
        assert np.max(np.abs(a - e)) <= 1e-5 * scale + 1e-6, k
    del reg


def test_two_rollouts_before_backward():
    """Each RSNNRollout node keeps its own workspace: two rollouts, then the backward of the
    first, give the first's gradients; a V1Column.backward whose rollout's workspace was
    overwritten raises instead of using the later rollout's activations."""
    from v1_glif_model_amd.models import RSNNRollout
    cfg = tiny_config(rs=2.0, ins=3.0)
    tn = network(cfg, seed=7, dense_basis=True)
    T, B = 25, 2
    lgn, bkg = _inputs(cfg, T, B, seed=8)
    lgn2, bkg2 = _inputs(cfg, T, B, seed=9)
    cell = _cell(tn, "deterministic", train_recurrent_per_type=False, **CELL_KW)
    w = (cell.recurrent_weight_values, cell.input_weight_values, cell.bkg_input_weights)
    gz = torch.tensor(np.random.default_rng(1).normal(0, 1, (T, B, tn[1].n_neurons)).astype(np.float32),
                      device="cuda")
    dev = lambda a: torch.tensor(a, device="cuda")
    z1, _ = RSNNRollout.apply(cell, dev(lgn), dev(bkg), *w)
    z2, _ = RSNNRollout.apply(cell, dev(lgn2), dev(bkg2), *w)
    (z1 * gz).sum().backward()
    g_two = w[0].grad.clone()
    w[0].grad = None
    z1b, _ = RSNNRollout.apply(cell, dev(lgn), dev(bkg), *w)
    (z1b * gz).sum().backward()
    np.testing.assert_array_equal(g_two.cpu().numpy(), w[0].grad.cpu().numpy())
    # the shared workspace: a second rollout invalidates the first one's record
    cell.rollout(lgn, bkg)
    first = cell._last
    cell.rollout(lgn2, bkg2)
    with pytest.raises(RuntimeError, match="overwritten"):
        cell.backward(gz=gz, rollout=first)


@pytest.mark.parametrize("B", [2, 5])
def test_cell_without_recurrent_synapses(B):
    """A network whose recurrent table is empty (fan-in 0; the inputs alone drive it): both
    forwards as the oracle's (deterministic bit-exact, event spike trains equal), the BPTT
    gradients of the input weights within the bar and an empty recurrent gradient."""
    cfg = tiny_config(n=90, fanin=0, ins=2.0)
    tn = network(cfg, seed=3, dense_basis=True)
    assert tn[1].rec.n_syn == 0
    T = 30
    lgn, bkg = _inputs(cfg, T, B)
    oc = _oracle(tn[1], **ORC_KW)
    oz, ov, oref, _ = oc.forward(lgn, bkg)
    assert oz.sum() > 0
    for mode in ("deterministic", "event"):
        cell = _cell(tn, mode, **CELL_KW)
        z, v, _ = cell.rollout(lgn, bkg)
        np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
        if mode == "deterministic":
            np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    rng = np.random.default_rng(B)
    gz = rng.normal(0, 1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"))
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz)
    assert g["rec"].numel() == 0
    for k in ("lgn", "bkg"):
        a, e = g[k].cpu().numpy(), og[k]
        scale = np.max(np.abs(e))
        assert scale > 0
        assert np.max(np.abs(a - e)) <= 1e-5 * scale + 1e-6, k
