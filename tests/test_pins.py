"""Closed-form pins of the table preprocessing and of the cell's dynamics and BPTT, on hand-built
networks whose expected values are written out here from `v1_model_utils/models.py`, not taken
from `tables.build_cell_tables` or the oracle:

* table preprocessing (models.py:483-593 parameters, :625-773 synapse tables, :528-539 the
  maximum delay), on a four-neuron, three-type network;
* the membrane's impulse response (models.py:979-1028): a spike that reaches the rise current
  R at tick t moves P at t + 1 (P takes the OLD R) and V at t + 2 (V takes the OLD P), by
  cf * (dt * sd) * (w * lr_scale) * p0; then the double-alpha sum V_{t+m} =
  cf * sum_k decay^(m-1-k) * k * dt * sd^k * R_t; a delay-d synapse delivers a spike of
  tick s at tick s + d;
* the BPTT's surrogate and dampening factors (models.py:17-28, 284-296, 1010, 1081): the
  weight gradient of a loss on one spike, through one synapse, in closed form -- which tells
  the Gaussian width from its amplitude, (1 - vgd) from vgd on the voltage self-loop, and
  rd from 1 - rd on the spike buffer.

Each dynamic pin runs on the CPU oracle and (marked gpu) on the library in both modes.
"""
import math

import numpy as np
import pytest

from tests import handnet

E = math.e


# ---------------------------------------------------------------- table pins ----
def test_four_neuron_tables_by_hand():
    from v1_glif_model_amd.tables import build_cell_tables
    tb = build_cell_tables(handnet.four_neuron_network(), dt=1.0, max_delay=4, lr_scale=4.0,
                           recurrent_weight_scale=2.0, input_weight_scale=1.0)
    f32 = np.float32
    # max_delay: the data's maximum is ceil(7.0) = 7 ms, the flag caps it at 4 (models.py:528-539)
    assert tb.max_delay == 4 and tb.n_neurons == 4 and tb.n_basis == 5
    # recurrent columns pre + N * (round(clip(delay, dt, D) / dt) - 1) (models.py:633-635):
    # 0.3 -> 1, 1.5 -> 2, 2.5 -> 2, 7.0 -> 4, 3.5 -> 4, 2.49 -> 2, 1.0 -> 1
    np.testing.assert_array_equal(tb.rec.post, [0, 0, 1, 1, 2, 3, 3])
    np.testing.assert_array_equal(tb.rec.col, [1 + 0, 3 + 4, 0 + 4, 2 + 12, 1 + 12, 0 + 4, 2 + 0])
    assert tb.rec.n_cols == 16
    # weights / (V_th - E_L)[type of post] * recurrent_weight_scale / lr_scale (models.py:631, 664):
    # V_th - E_L = 20, 10, 40, 10 mV for neurons 0..3
    expect = [4.0 / 20, -6.0 / 20, 2.5 / 10, 1.0 / 10, -10.0 / 40, 3.0 / 10, 0.5 / 10]
    np.testing.assert_array_equal(tb.rec.weight, np.array([w * 2.0 / 4.0 for w in expect], dtype=f32))
    np.testing.assert_array_equal(tb.rec.syn_id, [2, 0, 1, 4, 3, 0, 2])
    # inputs: no delays (models.py:715-718, 748-751), weights / vs * input_weight_scale / lr_scale
    np.testing.assert_array_equal(tb.lgn.col, [2, 0, 1])
    np.testing.assert_array_equal(tb.lgn.weight, np.array([2.0 / 20 / 4, 1.0 / 10 / 4, 5.0 / 10 / 4], dtype=f32))
    np.testing.assert_array_equal(tb.bkg.col, [0, 1])
    np.testing.assert_array_equal(tb.bkg.weight, np.array([1.0 / 20 / 4, 4.0 / 40 / 4], dtype=f32))
    # membrane: tau = C_m / g = 10, 10, 20, 10 ms; decay = exp(-dt / tau); cf = (1 - decay) / g
    tau = [10.0, 10.0, 20.0, 10.0]
    g = [10.0, 5.0, 4.0, 5.0]
    decay = [math.exp(-1.0 / x) for x in tau]
    np.testing.assert_allclose(tb.decay, decay, rtol=2e-7)
    np.testing.assert_allclose(tb.current_factor, [(1 - d) / gg for d, gg in zip(decay, g)], rtol=1e-6)
    # t_ref_steps = max(ceil(t_ref / dt), 1): 2.5 -> 3, 0.2 -> 1, 4.0 -> 4 (models.py:574-576)
    np.testing.assert_array_equal(tb.t_ref_steps, [3, 1, 4, 1])
    # asc: exp(-dt * sigmoid(logit(k))) = exp(-k * dt); amps / (V_th - E_L) (models.py:485-490, 588-593)
    k = {0: [0.1, 0.02], 1: [0.3, 0.003], 2: [0.05, 0.2]}
    amps = {0: [10.0 / 20, -4.0 / 20], 1: [-5.0 / 10, 1.0 / 10], 2: [8.0 / 40, 2.0 / 40]}
    types = [0, 1, 2, 1]
    np.testing.assert_allclose(tb.asc_decay, [[math.exp(-x) for x in k[t]] for t in types], rtol=1e-6)
    np.testing.assert_allclose(tb.asc_amps, [amps[t] for t in types], rtol=1e-7)
    # PSC basis: syn_decay = exp(-dt / tau_r), psc_initial = e / tau_r (float64, then float32;
    # models.py:518-526)
    taus = [2.0, 5.0, 10.0, 20.0, 50.0]
    np.testing.assert_array_equal(tb.syn_decay, np.array([math.exp(-1.0 / x) for x in taus], dtype=f32))
    np.testing.assert_array_equal(tb.psc_initial, np.array([E / x for x in taus], dtype=f32))
    np.testing.assert_array_equal(tb.voltage_scale, [20.0, 10.0, 40.0, 10.0])


def test_max_delay_includes_input_delays():
    """models.py:528-539: the maximum runs over the LGN (and background) 'delays' too."""
    from v1_glif_model_amd.tables import build_cell_tables
    assert build_cell_tables(handnet.four_neuron_network()).max_delay == 7
    tb = build_cell_tables(handnet.four_neuron_network(lgn_delays=[9.0, 1.0, 2.0]))
    assert tb.max_delay == 9 and tb.rec.n_cols == 9 * 4
    # the recurrent delays are clipped to the maximum, not the LGN ones (they are not applied)
    np.testing.assert_array_equal(tb.rec.col, [1, 3 + 4, 0 + 4, 2 + 24, 1 + 12, 0 + 4, 2])
    assert build_cell_tables(handnet.four_neuron_network(lgn_delays=[9.0, 1.0, 2.0]), max_delay=5).max_delay == 5


@pytest.mark.parametrize("train_recurrent,per_type,expect", [
    (True, True, False), (True, False, True), (False, True, False), (False, False, False)])
def test_recurrent_trainability(train_recurrent, per_type, expect):
    """models.py:651-669: individual recurrent weights train only with train_recurrent and not
    train_recurrent_per_type (the per-type path is commented out in the reference)."""
    from v1_glif_model_amd.tables import trainable_populations
    t = trainable_populations(train_recurrent=train_recurrent, train_recurrent_per_type=per_type,
                              train_input=True, train_noise=False)
    assert t == {"rec": expect, "lgn": True, "bkg": False}


# ------------------------------------------------------- dynamic pins: runner ----
LR = 2.0   # lr_scale: the tables divide the weights by it, the cell multiplies the currents


def _tables(net):
    from v1_glif_model_amd.tables import build_cell_tables
    return build_cell_tables(net, lr_scale=LR)


def run(backend, net, lgn, bkg, zbuf0=None, gz=None, **kw):
    """Forward (and, with gz, BPTT) on the oracle ("oracle") or the library ("event",
    "deterministic").  Returns z [T,B,N], v [T,B,N], dW dict or None."""
    B, N = lgn.shape[1], net["network"]["n_nodes"]
    okw = dict(vgd=kw.get("vgd", 0.5), rd=kw.get("rd", 0.5), gauss_std=kw.get("gauss_std", 0.5),
               damp=kw.get("damp", 0.5), pseudo_gauss=kw.get("pseudo_gauss", True),
               hard_reset=kw.get("hard_reset", False))
    if backend == "oracle":
        from oracle.cpu import OracleCell
        oc = OracleCell(_tables(net), **okw)
        st = oc.zero_state(B)
        if zbuf0 is not None:
            st["zbuf"][...] = zbuf0
        z, v, ref, _ = oc.forward(lgn, bkg, state=st)
        dW = None if gz is None else oc.backward(lgn, bkg, z, ref, v, gz_loss=gz, zbuf0=zbuf0)
        return z.astype(np.float32), v, dW
    import torch
    from v1_glif_model_amd.models import V1Column
    cell = V1Column(net, mode=backend, lr_scale=LR, gauss_std=okw["gauss_std"],
                    dampening_factor=okw["damp"], recurrent_dampening_factor=okw["rd"],
                    voltage_gradient_dampening=okw["vgd"], pseudo_gauss=okw["pseudo_gauss"],
                    hard_reset=okw["hard_reset"])
    st = list(cell.zero_state(B))
    if zbuf0 is not None:
        st[0] = torch.tensor(zbuf0, device="cuda")
    z, v, _ = cell.rollout(lgn, bkg, state=st)
    dW = None
    if gz is not None:
        dW = {k: t.cpu().numpy() for k, t in cell.backward(gz=torch.tensor(gz, device="cuda")).items()}
    return z.cpu().numpy(), v.cpu().numpy(), dW


BACKENDS = ["oracle", pytest.param("deterministic", marks=pytest.mark.gpu),
            pytest.param("event", marks=pytest.mark.gpu)]


# -------------------------------------------------------- impulse response ----
@pytest.mark.parametrize("backend", BACKENDS)
def test_membrane_impulse_response(backend):
    """Batch 0: LGN input 1 spikes at tick s = 4 into neuron 1 (receptor 2, tau 10 ms).
    Batch 1: neuron 0 spiked at tick -1 (initial history); its delay-3 synapse into neuron 1
    (receptor 1, tau 5 ms) delivers the spike at tick 2.  Neuron 0 of batch 1 is reset by its
    own spike: V = -1 at tick 0, then decays geometrically."""
    net = handnet.chain_network(w_rec=2.0, delay=3.0, sid_rec=1, w_lgn=(1.0, 1.0), sid_lgn=(3, 2))
    tb = _tables(net)
    T, B, N, s = 14, 2, 2, 4
    lgn = np.zeros((T, B, 2), np.uint8)
    lgn[s, 0, 1] = 1
    bkg = np.zeros((T, B, 1), np.uint8)
    zbuf0 = np.zeros((B, tb.max_delay * N), np.float32)
    zbuf0[1, 0] = 1.0       # slot 0 (z_{-1}) of neuron 0, batch 1
    z, v, _ = run(backend, net, lgn, bkg, zbuf0=zbuf0)
    assert z.sum() == 0
    f32 = np.float32
    decay, cf = tb.decay[1], tb.current_factor[1]
    # the hand-built weights: 1 mV / 20 mV / lr and 2 mV / 20 mV / lr
    assert tb.lgn.weight[1] == f32(1.0 / 20 / LR) and tb.rec.weight[0] == f32(2.0 / 20 / LR)
    for b, t_arrive, w, r in ((0, s, tb.lgn.weight[1], 2), (1, 2, tb.rec.weight[0], 1)):
        sd, p0 = tb.syn_decay[r], tb.psc_initial[r]
        R0 = f32(f32(w * f32(LR)) * p0)         # R after the arrival tick
        first = f32(cf * f32(f32(1.0 * sd) * R0))  # V two ticks later: cf * P, P = (dt * sd) * R
        vv = v[:, b, 1].astype(np.float64)
        assert np.all(vv[:t_arrive + 2] == 0.0), (b, vv[:t_arrive + 3])
        assert v[t_arrive + 2, b, 1] == first, (b, v[t_arrive + 2, b, 1], first)
        # double-alpha response: V_{t+m} = cf * sum_{k=1}^{m-1} decay^(m-1-k) * k * dt * sd^k * R_t
        for m in range(2, T - t_arrive):
            expect = float(cf) * sum(float(decay) ** (m - 1 - k) * k * float(sd) ** k
                                     for k in range(1, m)) * float(R0)
            assert abs(vv[t_arrive + m] - expect) <= 1e-6 * abs(expect), (b, m, vv[t_arrive + m], expect)
    # neuron 0, batch 1: reset by the spike of tick -1 (V = -1, models.py:1011), then V_t = -decay^t
    v0 = v[:, 1, 0].astype(np.float64)
    assert v[0, 1, 0] == -1.0
    np.testing.assert_allclose(v0, -float(tb.decay[0]) ** np.arange(T), rtol=1e-6)
    assert np.all(v[:, 0, 0] == 0.0)


# ------------------------------------------------------------ BPTT pins ----
PSETS = {"rd0.2_vgd0.3_d0.3_s0.7": dict(rd=0.2, vgd=0.3, damp=0.3, gauss_std=0.7),
         "reference_defaults": dict(rd=0.1, vgd=0.5, damp=0.1, gauss_std=0.3)}


def _psi(vsc, kw):
    if kw["pseudo_gauss"]:
        return kw["damp"] * math.exp(-vsc * vsc / (kw["gauss_std"] ** 2))     # models.py:17-21
    return kw["damp"] * max(1.0 - abs(vsc), 0.0)                              # models.py:23-28


@pytest.mark.parametrize("backend", BACKENDS)
@pytest.mark.parametrize("pseudo_gauss", [True, False])
@pytest.mark.parametrize("pset", list(PSETS))
def test_bptt_surrogate_and_voltage_dampening(backend, pseudo_gauss, pset):
    """One neuron, one LGN spike at tick s, loss z_{s+3}: dL/dw of that synapse =
    psi(V_{s+3} - 1) * lr * p0 * cf * ((1 - vgd) * decay * dt * sd + 2 * dt * sd * sd)
    (the spike reaches V at s + 2 and s + 3; the self-loop from V_{s+2} to V_{s+3} carries
    decay scaled by 1 - vgd)."""
    kw = dict(PSETS[pset], pseudo_gauss=pseudo_gauss)
    net = handnet.chain_network(w_rec=1.0, w_lgn=(1.0, 2200.0), sid_lgn=(3, 2))
    tb = _tables(net)
    T, B, s = 10, 3, 2
    lgn = np.zeros((T, B, 2), np.uint8)
    lgn[s, :, 1] = 1
    bkg = np.zeros((T, B, 1), np.uint8)
    gz = np.zeros((T, B, 2), np.float32)
    gz[s + 3, 0, 1] = 1.0
    z, v, dW = run(backend, net, lgn, bkg, gz=gz, **kw)
    Vt = float(v[s + 3, 0, 1])
    assert 0.2 < Vt < 1.0 and z[:s + 4, :, 1].sum() == 0, Vt
    r = 2
    sd, p0, decay, cf = (float(tb.syn_decay[r]), float(tb.psc_initial[r]), float(tb.decay[1]),
                         float(tb.current_factor[1]))
    om = 1.0 - kw["vgd"]
    expect = _psi(Vt - 1.0, kw) * LR * p0 * cf * (om * decay * sd + 2.0 * sd * sd)
    got = float(dW["lgn"][1])
    assert abs(got - expect) <= 1e-5 * abs(expect), (got, expect)
    assert np.all(dW["lgn"][[0]] == 0.0) and np.all(dW["rec"] == 0.0) and np.all(dW["bkg"] == 0.0)


@pytest.mark.parametrize("backend", BACKENDS)
@pytest.mark.parametrize("pset", list(PSETS))
def test_bptt_recurrent_dampening(backend, pset):
    """Neuron 0 is driven over threshold once, at tick s0 + 2, by an LGN spike at s0; its
    delay-d synapse moves neuron 1's voltage at t* = s0 + 2 + d + 2; loss z_1 at t*.  With the
    triangular surrogate (zero at V = 0, so no earlier tick of neuron 0 contributes):
      dL/dw_rec  = psi_1 * cf * dt * sd_1 * p0_1 * lr
      dL/dw_lgn0 = psi_1 * cf * dt * sd_1 * p0_1 * lr * w_rec * rd * psi_0 * cf * dt * sd_3 * p0_3 * lr
    with rd the spike buffer's gradient scale (straight_through_dampen(z_buf, 1 - rd))."""
    kw = dict(PSETS[pset], pseudo_gauss=False)
    d = 3
    net = handnet.chain_network(w_rec=2360.0, delay=float(d), sid_rec=1, w_lgn=(24000.0, 1.0), sid_lgn=(3, 2))
    tb = _tables(net)
    T, B, s0 = 16, 3, 2
    ts = s0 + 2 + d + 2
    lgn = np.zeros((T, B, 2), np.uint8)
    lgn[s0, :, 0] = 1
    bkg = np.zeros((T, B, 1), np.uint8)
    gz = np.zeros((T, B, 2), np.float32)
    gz[ts, 0, 1] = 1.0
    z, v, dW = run(backend, net, lgn, bkg, gz=gz, **kw)
    assert z[s0 + 2, 0, 0] == 1 and z[:s0 + 2, :, 0].sum() == 0 and z[:ts + 1, :, 1].sum() == 0
    V0, V1 = float(v[s0 + 2, 0, 0]), float(v[ts, 0, 1])
    assert 1.0 < V0 < 2.0 and 0.0 < V1 < 1.0, (V0, V1)
    cf0, cf1 = float(tb.current_factor[0]), float(tb.current_factor[1])
    a1 = cf1 * float(tb.syn_decay[1]) * float(tb.psc_initial[1]) * LR        # dV_1(t*) / dI (receptor 1)
    a0 = cf0 * float(tb.syn_decay[3]) * float(tb.psc_initial[3]) * LR        # dV_0(s0+2) / dI (receptor 3)
    psi1, psi0 = _psi(V1 - 1.0, kw), _psi(V0 - 1.0, kw)
    rd = kw["rd"]
    exp_rec = psi1 * a1
    exp_lgn0 = psi1 * a1 * float(tb.rec.weight[0]) * rd * psi0 * a0
    assert abs(float(dW["rec"][0]) - exp_rec) <= 1e-5 * abs(exp_rec), (dW["rec"][0], exp_rec)
    assert abs(float(dW["lgn"][0]) - exp_lgn0) <= 1e-5 * abs(exp_lgn0), (dW["lgn"][0], exp_lgn0)
    assert dW["lgn"][1] == 0.0
