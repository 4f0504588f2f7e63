"""The drop-in boundary on the GPU: the reference's state layouts (models.py:1030-1056) with its
int8 refractory counter (:574-583, :1050), refusal of malformed arguments before any kernel
runs, the ownership of the fused voltage loss across regularizer objects, and a backward run
after a switch of the G layout."""
import numpy as np
import pytest
import torch

from oracle.cpu import OracleCell, bptt_abs_scale
from tests.helpers import assert_grads_per_element, network, tiny_config
from v1_glif_model_amd import synthetic as sy

pytestmark = pytest.mark.gpu

KW = dict(gauss_std=0.5, dampening_factor=0.5, recurrent_dampening_factor=0.5, voltage_gradient_dampening=0.5,
          pseudo_gauss=True)
OKW = dict(vgd=0.5, rd=0.5, gauss_std=0.5, damp=0.5, pseudo_gauss=True)


def _cell(mode="deterministic", seed=0, **kw):
    from v1_glif_model_amd.models import V1Column
    cfg = tiny_config(rs=2.0, ins=3.0)
    tn = network(cfg, seed=seed, dense_basis=True)
    return cfg, tn, V1Column(tn[0], mode=mode, **KW, **kw)


@pytest.mark.parametrize("mode", ["deterministic", "event"])
def test_int8_reference_state_matches_int16(mode):
    """A rollout continued from a state in the reference's layout (r int8, as its zero_state
    makes it) equals the same rollout from an int16 state bit for bit, and the caller's int8
    counter holds the final refractory steps."""
    cfg, tn, cell = _cell(mode)
    B, T1, T2 = 3, 40, 30
    lgn, bkg = sy.make_inputs(cfg, seed=3, seq_len=T1 + T2, batch=B)
    st8 = cell.zero_state(B)
    assert st8[2].dtype == torch.int8          # every t_ref of the tiny network is < 128 steps
    _, _, st8 = cell.rollout(lgn[:T1], bkg[:T1], state=st8)
    assert st8[2].dtype == torch.int8 and int(st8[2].max()) > 0   # neurons refractory at the split
    st16 = [s.clone() for s in st8]
    st16[2] = st16[2].to(torch.int16)
    r8 = st8[2]
    z8, v8, out8 = cell.rollout(lgn[T1:], bkg[T1:], state=[s.clone() if i != 2 else s for i, s in enumerate(st8)])
    z16, v16, out16 = cell.rollout(lgn[T1:], bkg[T1:], state=st16)
    assert out8[2] is r8 and out8[2].dtype == torch.int8           # written back in place
    assert out16[2].dtype == torch.int16
    if mode == "deterministic":
        np.testing.assert_array_equal(z8.cpu().numpy(), z16.cpu().numpy())
        np.testing.assert_array_equal(v8.cpu().numpy().view(np.uint32), v16.cpu().numpy().view(np.uint32))
        for a, b in zip(out8[:6], out16[:6]):
            np.testing.assert_array_equal(a.cpu().numpy().astype(np.float64), b.cpu().numpy().astype(np.float64))
    else:
        # atomics: the same refractory counts where the spike trains agree
        assert float((z8 == z16).float().mean()) >= 0.999
    assert int(out8[6][0]) == T1 + T2


def test_malformed_arguments_raise_before_any_kernel():
    """Wrong shapes, dtypes and devices raise ValueError, and nothing is written: the state and
    the cell's rollout count are unchanged afterwards."""
    from v1_glif_model_amd.ops import SynapseTable
    cfg, tn, cell = _cell()
    B, T = 2, 10
    lgn, bkg = sy.make_inputs(cfg, seed=4, seq_len=T, batch=B)
    N, D, nb = tn[1].n_neurons, tn[1].max_delay, tn[1].n_basis
    good = cell.zero_state(B)
    bad_cases = {
        "z_buf short": (0, torch.zeros((B, N * D - 1), device="cuda")),
        "v on the host": (1, torch.zeros((B, N))),
        "r int32": (2, torch.zeros((B, N), dtype=torch.int32, device="cuda")),
        "asc wrong batch": (3, torch.zeros((B + 1, 2 * N), device="cuda")),
        "psc_rise float64": (4, torch.zeros((B, N * nb), dtype=torch.float64, device="cuda")),
        "psc [B, N]": (5, torch.zeros((B, N), device="cuda")),
    }
    gen = cell._gen
    for what, (i, t) in bad_cases.items():
        st = [s.clone() for s in good]
        st[i] = t
        marker = [s.clone() for s in st]
        with pytest.raises(ValueError):
            cell.rollout(lgn, bkg, state=st)
        for a, b in zip(st, marker):
            assert torch.equal(a.cpu(), b.cpu()), what
    assert cell._gen == gen
    with pytest.raises(ValueError):
        cell.rollout(lgn, bkg, state=good, spike_count=torch.zeros((B, N), dtype=torch.int64, device="cuda"))
    with pytest.raises(ValueError):
        cell.rollout(lgn, bkg, state=good, ws=torch.empty(16, dtype=torch.uint8, device="cuda"))
    assert cell._gen == gen
    cell.rollout(lgn, bkg, state=[s.clone() for s in good])
    for gz in (torch.zeros((T, B, N + 1), device="cuda"), torch.zeros((T, B, N)), torch.zeros((T - 1, B, N),
                                                                                             device="cuda")):
        with pytest.raises(ValueError):
            cell.backward(gz=gz)
    with pytest.raises(ValueError):
        cell.backward(gz_neuron=torch.zeros(N + 3, device="cuda"))
    # the op-level table
    tb = tn[1]
    t = SynapseTable(np.stack([tb.rec.post, tb.rec.col], -1), tb.rec.syn_id, (N, tb.rec.n_cols), tb.basis,
                     n_delay_slots=D)
    t.set_weights(torch.tensor(tb.rec.weight, device="cuda"))
    z = torch.zeros((B, tb.rec.n_cols), device="cuda")
    for bad in (torch.zeros((B, tb.rec.n_cols - 1), device="cuda"), torch.zeros((B, tb.rec.n_cols)),
                torch.zeros((33, tb.rec.n_cols), device="cuda"), torch.zeros(tb.rec.n_cols, device="cuda")):
        with pytest.raises(ValueError):
            t.forward(bad)
    for dy in (torch.zeros((B * N, nb + 1), device="cuda"), torch.zeros((B * N, nb)),
               torch.zeros(((B + 1) * N, nb), device="cuda")):
        with pytest.raises(ValueError):
            t.backward(z, dy)
    with pytest.raises(ValueError):
        t.set_weights(torch.tensor(tb.rec.weight))
    dz, dw = t.backward(z, torch.zeros((B * N, nb), device="cuda"))
    assert dz.shape == (B, tb.rec.n_cols) and dw.shape == (tb.rec.n_syn,)


def test_rebound_regularizer_keeps_the_fused_loss():
    """reg = VoltageRegularization(cell, ...) twice in a row (the first object is deleted after
    the second is built): the fused loss and gradient are those of the live object, equal to a
    run with a single regularizer."""
    import gc

    from v1_glif_model_amd.losses import VoltageRegularization
    cfg, tn, cell = _cell(seed=5)
    B, T = 3, 30
    lgn, bkg = sy.make_inputs(cfg, seed=6, seq_len=T, batch=B)
    gz = torch.tensor(np.random.default_rng(7).normal(0, 1, (T, B, tn[1].n_neurons)).astype(np.float32),
                      device="cuda")
    reg = VoltageRegularization(cell, voltage_cost=0.5, penalty_mode="range")
    cell.rollout(lgn, bkg)
    l1 = float(reg())
    g1 = {k: v.clone() for k, v in cell.backward(gz=gz).items()}
    reg.disable()
    reg = VoltageRegularization(cell, voltage_cost=3.0, penalty_mode="threshold")
    reg = VoltageRegularization(cell, voltage_cost=0.5, penalty_mode="range")
    gc.collect()
    cell.rollout(lgn, bkg)
    l2 = float(reg())
    g2 = cell.backward(gz=gz)
    assert l1 == l2
    for k in g1:
        assert torch.equal(g1[k], g2[k]), k
    reg.disable()
    g0 = cell.backward(gz=gz)    # loss off: a different gradient
    assert not torch.equal(g0["rec"], g1["rec"])


def test_backward_after_a_layout_switch():
    """The forward's saved data sits at offsets independent of the G layout: a rollout under
    compact rows, then a switch to type-major rows, then the backward (on a workspace sized for
    the new layout) gives the oracle's gradients within the bar."""
    from v1_glif_model_amd.models import V1Column
    from v1_glif_model_amd.tables import build_cell_tables
    cfg = tiny_config(rs=2.0, ins=3.0)
    net = sy.class_types(sy.make_network(cfg, seed=61, dense_basis=True), n_classes=5)
    tb = build_cell_tables(net)
    B, T = 5, 30
    lgn, bkg = sy.make_inputs(cfg, seed=62, seq_len=T, batch=B)
    cell = V1Column(net, mode="deterministic", **KW)
    assert cell.g_layout()[1]
    from v1_glif_model_amd._lib import lib
    big = max(int(lib().glif_cell_workspace(cell.handle, B, T)), 0)
    cell.set_g_layout(False)
    big = max(big, int(lib().glif_cell_workspace(cell.handle, B, T)))
    cell.set_g_layout(True)
    ws = torch.empty(big, dtype=torch.uint8, device="cuda")
    cell.rollout(lgn, bkg, ws=ws)
    cell.set_g_layout(False)
    gz = np.random.default_rng(63).normal(0, 1, (T, B, tb.n_neurons)).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"))
    oc = OracleCell(tb, **OKW)
    oz, ov, oref, _ = oc.forward(lgn, bkg)
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz)
    sc = bptt_abs_scale(tb, lgn, bkg, oz, oref, ov, gz_loss=gz, **OKW)
    for k in ("rec", "lgn", "bkg"):
        assert np.max(np.abs(og[k])) > 0
        assert_grads_per_element(g[k].cpu().numpy(), og[k], sc[k], what=f"after switch {k}")
