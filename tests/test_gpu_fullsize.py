"""Parity at the sizes of the benchmark's configurations, GPU
against the C oracle on identical seeded inputs.

* config 2 (66k neurons, 16.5M recurrent synapses, B = 5, T = 500):
  - deterministic forward: spike trains and voltages bit-exact with the oracle over all
    500 ms;
  - event forward: spike trains identical to the oracle's for the first 50 ms from the
    network's spike onset (it is silent for the first ~70 ms), per-(batch, neuron) spike
    counts agreeing for >= 99.9 % over the run;
  - the benchmarked training step end to end in event mode: rate-MSE loss and its per-neuron
    gradient, BPTT over all 500 ticks (recurrent and LGN weight gradients, per element within
    1e-5 of the element's sum of absolute terms + 1e-6; given the GPU's own event-mode voltages,
    within 1e-5 of the sum of absolute terms with no absolute allowance), one ExponentiatedAdam
    step with the sign constraints (within 1e-6 relative given the gradient);
* config 3 (230k neurons, 69M synapses, B = 1): deterministic forward bit-exact over 500 ms (the
  144 KB-LDS, 1024-lane chunk pull), event counts within the bar;
* config 2's network with the reference's type structure (121 class-pair types, 4 receptors,
  5 Hz): compact G rows, deterministic forward bit-exact over 150 ms and BPTT within the bar;
* config 4 (B = 32, per-batch sinusoidal LGN) with the recurrent weights alone scaled to the
  rate sweep's points (the role of the reference's recurrent_weight_scale, models.py:664; the
  LGN and background weights as generated): 5, 20 and 50 Hz, and for 1 Hz the lowest rate
  recurrent scaling reaches (factor 0: the inputs alone drive the network at ~4.5 Hz).  At
  every point the deterministic forward is bit-exact over 500 ms, the event forward's spike
  trains equal the oracle's for 50 ms from onset and its per-(batch, neuron) counts agree for
  >= 99.9 %; and a B = 32 BPTT at the 50 Hz factor (one-tick windows, 32-float G rows) over
  ticks 300-379 from the carried state, against the oracle.

The oracle runs its OpenMP loops (same bits as one thread).  Each step prints a progress line.
"""
import dataclasses
import os
import time

import numpy as np
import pytest
import torch

from oracle import cpu as orc
from tests.helpers import assert_grads_per_element, error_summary
from v1_glif_model_amd import synthetic as sy

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

CELL_KW = dict(gauss_std=0.5, dampening_factor=0.5, recurrent_dampening_factor=0.5,
               voltage_gradient_dampening=0.5, pseudo_gauss=True)
ORC_KW = dict(vgd=0.5, rd=0.5, gauss_std=0.5, damp=0.5, pseudo_gauss=True)
_T0 = time.time()


def say(*a):
    print(f"[fullsize {time.time() - _T0:7.1f}s]", *a, flush=True)


def onset(z):
    """First tick with a spike anywhere."""
    per = z.reshape(z.shape[0], -1).sum(1)
    return int(np.argmax(per > 0)) if per.any() else z.shape[0]


def count_agreement(a, b):
    return float(np.mean(a.sum(0) == b.sum(0)))


@pytest.fixture(scope="module", autouse=True)
def _threads():
    orc.set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    yield
    orc.set_threads(1)


# ------------------------------------------------------------------ config 2 ----
@pytest.fixture(scope="module")
def config2():
    from v1_glif_model_amd.models import V1Column
    cfg = sy.config(2)
    net = sy.make_network(cfg, seed=0)
    T, B = cfg.seq_len, cfg.batch
    lgn, bkg = sy.make_inputs(cfg, seed=1, seq_len=T, batch=B)
    cell = V1Column(net, mode="deterministic", train_input=True, train_recurrent_per_type=False, **CELL_KW)
    tb = cell.tables
    say("config 2 built:", tb.n_neurons, "neurons,", tb.rec.n_syn, "recurrent synapses")
    oz, ov, oref, _ = orc.OracleCell(tb, **ORC_KW).forward(lgn, bkg)
    say("oracle forward, 500 ms:", int(oz.sum()), "spikes, onset", onset(oz), "ms")
    yield dict(cfg=cfg, net=net, tb=tb, cell=cell, lgn=lgn, bkg=bkg, oz=oz, ov=ov, oref=oref)
    del cell


def test_config2_forward_500ms(config2):
    c = config2
    cell, lgn, bkg, oz, ov = c["cell"], c["lgn"], c["bkg"], c["oz"], c["ov"]
    zd, vd, _ = cell.rollout(lgn, bkg)
    zd, vd = zd.cpu().numpy().astype(np.uint8), vd.cpu().numpy()
    say("deterministic GPU forward:", int(zd.sum()), "spikes")
    assert oz.sum() > 100000
    np.testing.assert_array_equal(zd, oz)
    np.testing.assert_array_equal(vd.view(np.uint32), ov.view(np.uint32))
    ze, ve, _ = cell.rollout(lgn, bkg, mode="event")
    ze = ze.cpu().numpy().astype(np.uint8)
    t0 = onset(oz)
    differ = np.flatnonzero((ze != oz).any(axis=(1, 2)))
    agree = count_agreement(ze, oz)
    say("event vs oracle: onset", t0, "first differing ms", differ[0] if differ.size else None,
        "count agreement", agree)
    assert t0 + 50 <= oz.shape[0]
    np.testing.assert_array_equal(ze[:t0 + 50], oz[:t0 + 50])
    assert agree >= 0.999


def test_config2_training_step_event(config2):
    """The benchmark's step: event forward, rate MSE, BPTT over 500 ticks, ExponentiatedAdam."""
    from oracle import optim_ref
    from oracle.rate_loss_ref import rate_mse
    from v1_glif_model_amd.losses import RateMSE
    from v1_glif_model_amd.models import V1Column
    from v1_glif_model_amd.optim import ExponentiatedAdam, SignedConstraint
    c = config2
    net, tb, lgn, bkg, oz, ov, oref = (c[k] for k in ("net", "tb", "lgn", "bkg", "oz", "ov", "oref"))
    T, B, N = lgn.shape[0], lgn.shape[1], tb.n_neurons
    cell = c["cell"]
    cell.mode = "event"
    targets = sy.make_rate_targets(N, seed=2)
    sc = torch.zeros((B, N), dtype=torch.int32, device="cuda")
    z, v, _ = cell.rollout(lgn, bkg, spike_count=sc)
    ze = z.cpu().numpy().astype(np.uint8)
    same = bool(np.array_equal(ze, oz))
    say("event forward: spike trains equal to the oracle's over 500 ms:", same,
        "count agreement", count_agreement(ze, oz))
    assert count_agreement(ze, oz) >= 0.999
    gzn = torch.zeros(N, dtype=torch.float32, device="cuda")
    loss = float(RateMSE(targets)(sc, T, gz_neuron=gzn))
    g = cell.backward(gz_neuron=gzn, want=("rec", "lgn"))
    g = {k: g[k].cpu().numpy() for k in ("rec", "lgn")}
    w0 = {"rec": cell.recurrent_weight_values.detach().clone(), "lgn": cell.input_weight_values.detach().clone()}
    opt = ExponentiatedAdam(learning_rate=0.005)
    cons = {cell.recurrent_weight_values.data_ptr(): SignedConstraint(cell.recurrent_weight_positive),
            cell.input_weight_values.data_ptr(): SignedConstraint(cell.input_weight_positive)}
    with torch.no_grad():
        opt.apply_gradients([(torch.tensor(g["rec"], device="cuda"), cell.recurrent_weight_values),
                             (torch.tensor(g["lgn"], device="cuda"), cell.input_weight_values)], constraints=cons)
    w1 = {"rec": cell.recurrent_weight_values.detach().cpu().numpy(),
          "lgn": cell.input_weight_values.detach().cpu().numpy()}
    cell.mode = "deterministic"
    say("GPU step done; oracle loss and BPTT over 500 ticks")
    # the oracle's loss on its own spike counts, BPTT through its own trajectory
    ocnt = oz.astype(np.int64).sum((0, 1))
    oloss, ogzn = rate_mse(ocnt, T * B, targets)
    assert abs(loss - float(oloss)) <= 1e-5 * abs(float(oloss))
    og = orc.OracleCell(tb, **ORC_KW).backward(lgn, bkg, oz, oref, ov, gz_neuron=ogzn, want=("rec", "lgn"))
    say("oracle BPTT done; sum-of-absolute-terms scale")
    scale = orc.bptt_abs_scale(tb, lgn, bkg, oz, oref, ov, gz_neuron=ogzn, want=("rec", "lgn"), **ORC_KW)
    for k in ("rec", "lgn"):
        summ = error_summary(g[k], og[k], scale[k])
        say(k, "dW error / sum|terms|:", summ, "nonzero oracle dW", int(np.count_nonzero(og[k])))
        assert np.count_nonzero(og[k]) > 1000
        assert_grads_per_element(g[k], og[k], scale[k], what=k)
    # the same BPTT through the GPU's own event-mode trajectory (its voltages carry the event
    # sums' rounding, which moves the surrogate): isolates the backward's arithmetic
    if same:
        vg = v.cpu().numpy()
        og_tf = orc.OracleCell(tb, **ORC_KW).backward(lgn, bkg, ze, oref, vg, gz_neuron=gzn.cpu().numpy(),
                                                      want=("rec", "lgn"))
        for k in ("rec", "lgn"):
            say(k, "dW error / sum|terms|, oracle on the GPU's voltages:", error_summary(g[k], og_tf[k], scale[k]))
            assert_grads_per_element(g[k], og_tf[k], scale[k], what=k + " (GPU trajectory)", atol=0.0)
    # the update given the gradient (optimizers.py:354-376, models.py:419-427): within 1e-6
    # relative (the device's expf / sqrtf and numpy's differ in the last ulp)
    a = optim_ref.alpha(0.005, 0.9, 0.999, 1)
    for k, pos in (("rec", cell.recurrent_weight_positive), ("lgn", cell.input_weight_positive)):
        w = w0[k].cpu().numpy().copy()
        m, vv = np.zeros_like(w), np.zeros_like(w)
        optim_ref.exp_adam_step(w, m, vv, g[k], a, positive=pos.cpu().numpy())
        np.testing.assert_allclose(w1[k], w, rtol=1e-6, atol=0, err_msg=k)
        say(k, "updated weights equal to the float32 restatement's:", float(np.mean(w1[k] == w)))
    # restore the weights for the other tests of the module
    with torch.no_grad():
        cell.recurrent_weight_values.copy_(w0["rec"])
        cell.input_weight_values.copy_(w0["lgn"])


# ------------------------------------------------------------------ config 3 ----
def test_config3_forward():
    from v1_glif_model_amd.models import V1Column
    cfg = sy.config(3)
    net = sy.make_network(cfg, seed=0)
    T, B = cfg.seq_len, cfg.batch
    lgn, bkg = sy.make_inputs(cfg, seed=1, seq_len=T, batch=B)
    cell = V1Column(net, mode="deterministic", **CELL_KW)
    tb = cell.tables
    say("config 3 built:", tb.n_neurons, "neurons,", tb.rec.n_syn, "recurrent synapses")
    zd, vd, _ = cell.rollout(lgn, bkg)
    ze, _, _ = cell.rollout(lgn, bkg, mode="event")
    zd, vd, ze = zd.cpu().numpy().astype(np.uint8), vd.cpu().numpy(), ze.cpu().numpy().astype(np.uint8)
    del cell
    torch.cuda.empty_cache()
    oz, ov, _, _ = orc.OracleCell(tb, **ORC_KW).forward(lgn, bkg)
    t0 = onset(oz)
    active = int(np.count_nonzero(oz.reshape(T, -1).sum(1)))
    say("config 3 oracle:", int(oz.sum()), "spikes, onset", t0, "ms, active ticks", active)
    assert active >= 100
    np.testing.assert_array_equal(zd, oz)
    np.testing.assert_array_equal(vd.view(np.uint32), ov.view(np.uint32))
    agree = count_agreement(ze, oz)
    say("config 3 event: count agreement", agree)
    np.testing.assert_array_equal(ze[:t0 + 50], oz[:t0 + 50])
    assert agree >= 0.999


# ------------------------------------------------------------------ config 4 ----
# recurrent weight factors of the rate sweep (bench.py --config 4, profiles/rate_sweep_config4.md):
# mean rate 5, 20 and 50 Hz; 1 Hz lies below what recurrent scaling reaches, whose floor (factor 0,
# ~4.5 Hz) stands in for it
REC_FACTORS = {"1Hz_floor": 0.0, "5Hz": 0.70091, "20Hz": 5.28304, "50Hz": 8.45088}


@pytest.fixture(scope="module")
def config4():
    cfg = sy.config(4)
    net = sy.make_network(cfg, seed=0)
    lgn, bkg = sy.make_inputs(cfg, seed=1, seq_len=cfg.seq_len, batch=cfg.batch)
    say("config 4 network built")
    return cfg, net, lgn, bkg


def _scaled_cell(net, f, mode="deterministic"):
    """The network with all three weight populations scaled by f (float32)."""
    from v1_glif_model_amd.models import V1Column
    cell = V1Column(net, mode=mode, **CELL_KW)
    tb = cell.tables
    f32 = np.float32
    scaled = {k: (getattr(tb, k).weight * f32(f)).astype(f32) for k in ("rec", "lgn", "bkg")}
    with torch.no_grad():
        cell.recurrent_weight_values.copy_(torch.tensor(scaled["rec"]))
        cell.input_weight_values.copy_(torch.tensor(scaled["lgn"]))
        cell.bkg_input_weights.copy_(torch.tensor(scaled["bkg"]))
    cell.refresh_weights(force=True)
    tbs = dataclasses.replace(tb, **{k: dataclasses.replace(getattr(tb, k), weight=scaled[k]) for k in scaled})
    return cell, tbs


def _rec_scaled_cell(net, f, mode="deterministic"):
    """The network with its recurrent weights scaled by f through the reference's own knob,
    recurrent_weight_scale (models.py:664): the cell's tables are the oracle's."""
    from v1_glif_model_amd.models import V1Column
    cell = V1Column(net, mode=mode, recurrent_weight_scale=f, **CELL_KW)
    return cell, cell.tables


@pytest.mark.parametrize("rate", list(REC_FACTORS))
def test_config4_forward(config4, rate):
    cfg, net, lgn, bkg = config4
    cell, tbs = _rec_scaled_cell(net, REC_FACTORS[rate])
    T, B, N = lgn.shape[0], lgn.shape[1], tbs.n_neurons
    zd, vd, _ = cell.rollout(lgn, bkg)
    ze, _, _ = cell.rollout(lgn, bkg, mode="event")
    zd, vd, ze = zd.cpu().numpy().astype(np.uint8), vd.cpu().numpy(), ze.cpu().numpy().astype(np.uint8)
    del cell
    say(f"config 4 {rate}: GPU rate", round(float(zd.mean()) * 1000, 2), "Hz")
    oz, ov, _, _ = orc.OracleCell(tbs, **ORC_KW).forward(lgn, bkg)
    say(f"config 4 {rate}: oracle", int(oz.sum()), "spikes, onset", onset(oz))
    np.testing.assert_array_equal(zd, oz)
    np.testing.assert_array_equal(vd.view(np.uint32), ov.view(np.uint32))
    t0 = onset(oz)
    differ = np.flatnonzero((ze != oz).any(axis=(1, 2)))
    agree = count_agreement(ze, oz)
    say(f"config 4 {rate} event: first differing ms", differ[0] if differ.size else None, "count agreement", agree)
    assert t0 + 50 <= T
    np.testing.assert_array_equal(ze[:t0 + 50], oz[:t0 + 50])
    assert agree >= 0.999


def test_config4_bptt_batch32(config4):
    """B = 32: one-tick backward windows, 32-float G rows (8 lanes per column in the
    type-phased walk), at the 50 Hz recurrent factor over 80 ms of the active regime: ticks
    300-379, from the state the deterministic rollout reaches at tick 300 (bit-exact with the
    oracle's), so its spike history feeds the first ticks' recurrent dW."""
    cfg, net, lgn, bkg = config4
    cell, tbs = _rec_scaled_cell(net, REC_FACTORS["50Hz"])
    t_a, T, B = 300, 80, lgn.shape[1]
    _, _, st = cell.rollout(lgn[:t_a], bkg[:t_a], state=cell.zero_state(B), record_z=False, record_v=False)
    st0 = dict(zbuf=st[0].cpu().numpy(), v=st[1].cpu().numpy(), r=st[2].cpu().numpy().astype(np.int32),
               asc=st[3].cpu().numpy(), psc_rise=st[4].cpu().numpy(), psc=st[5].cpu().numpy())
    lgn, bkg = lgn[t_a:t_a + T], bkg[t_a:t_a + T]
    z, v, _ = cell.rollout(lgn, bkg, state=[s.clone() for s in st])
    oc = orc.OracleCell(tbs, **ORC_KW)
    oz, ov, oref, _ = oc.forward(lgn, bkg, state=st0)
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    say("config 4 B=32 BPTT window:", int(oz.sum()), "spikes")
    assert oz.sum() > 1_000_000
    gz = np.random.default_rng(44).normal(0, 1, oz.shape).astype(np.float32)
    g = {k: t.cpu().numpy() for k, t in cell.backward(gz=torch.tensor(gz, device="cuda")).items()}
    del cell
    say("config 4 B=32 GPU BPTT done; oracle")
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz, zbuf0=st0["zbuf"])
    scale = orc.bptt_abs_scale(tbs, lgn, bkg, oz, oref, ov, gz_loss=gz, zbuf0=st0["zbuf"], **ORC_KW)
    for k in ("rec", "lgn", "bkg"):
        say("config 4 B=32", k, error_summary(g[k], og[k], scale[k]))
        assert np.count_nonzero(og[k]) > 0
        assert_grads_per_element(g[k], og[k], scale[k], what=k)


def test_config2_class_types_compact_rows():
    """The config-2 network with the reference's type structure (121 types by (pre class, post
    class) over 11 classes, 4 receptors, dense basis) at the bench's 5 Hz weight factor: the cell
    keeps 11 compact G rows per neuron; deterministic forward bit-exact over 150 ms and the BPTT
    (grouped walk over compact rows, their dW passes) per element within the bar; the event
    forward (per-type slots) with the same spike trains for 50 ms from onset and counts within
    the bar."""
    cfg = dataclasses.replace(sy.config(2), n_basis=4)
    net = sy.class_types(sy.make_network(cfg, seed=0), n_classes=11)
    T, B = 150, cfg.batch
    lgn, bkg = sy.make_inputs(cfg, seed=1, seq_len=T, batch=B)
    cell, tbs = _scaled_cell(net, 0.5179)
    assert cell.g_layout() == (11, True)
    say("config 2, class types: cell built, compact rows", cell.g_layout())
    z, v, _ = cell.rollout(lgn, bkg)
    oc = orc.OracleCell(tbs, **ORC_KW)
    oz, ov, oref, _ = oc.forward(lgn, bkg)
    say("config 2, class types:", int(oz.sum()), "spikes, onset", onset(oz))
    assert oz.sum() > 10000
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    gz = np.random.default_rng(45).normal(0, 1, oz.shape).astype(np.float32)
    g = {k: t.cpu().numpy() for k, t in cell.backward(gz=torch.tensor(gz, device="cuda")).items()}
    # the event forward pushes one atomic per synapse event into the post's type slot and
    # folds the slots through the basis in the step
    ze, _, _ = cell.rollout(lgn, bkg, mode="event")
    ze = ze.cpu().numpy().astype(np.uint8)
    del cell
    t0 = onset(oz)
    differ = np.flatnonzero((ze != oz).any(axis=(1, 2)))
    say("config 2, class types, event: first differing ms", differ[0] if differ.size else None,
        "count agreement", count_agreement(ze, oz))
    np.testing.assert_array_equal(ze[:t0 + 50], oz[:t0 + 50])
    assert count_agreement(ze, oz) >= 0.999
    say("config 2, class types: GPU BPTT done; oracle")
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz)
    scale = orc.bptt_abs_scale(tbs, lgn, bkg, oz, oref, ov, gz_loss=gz, **ORC_KW)
    for k in ("rec", "lgn", "bkg"):
        say("config 2, class types", k, error_summary(g[k], og[k], scale[k]))
        assert_grads_per_element(g[k], og[k], scale[k], what=k)


@pytest.mark.parametrize("name,B", [("lgn", 5), ("lgn", 32), ("bkg", 5), ("bkg", 32)])
def test_config2_op_level_inputs(config2, name, B):
    """calculate_synaptic_currents on config 2's input tables at full size (LGN: 17,400 inputs,
    2.64M synapses; background: 100 inputs of ~6,600 synapses, Poisson counts), one tick of the
    config's inputs at B = 5 and 32 -- the work-unit paths (the LGN's unit push and unit dz at
    B = 5, the background's long-column pull and chunked dz): deterministic forward bit-exact
    with the oracle, event forward, dz and dW within the bar of assert_grads_per_element."""
    from oracle import dense
    from v1_glif_model_amd.ops import SynapseTable
    tb = config2["tb"]
    pop = tb.lgn if name == "lgn" else tb.bkg
    counts = name == "bkg"
    t = SynapseTable(np.stack([pop.post, pop.col], -1), pop.syn_id, (tb.n_neurons, pop.n_cols), tb.basis)
    t.set_weights(torch.tensor(pop.weight, device="cuda"))
    lgn, bkg = sy.make_inputs(config2["cfg"], seed=7, seq_len=1, batch=B)
    z = (lgn if name == "lgn" else bkg)[0].astype(np.float32)
    rng = np.random.default_rng(8)
    dy = rng.normal(0, 1, (B * tb.n_neurons, tb.n_basis)).astype(np.float32)
    zt, dyt = torch.tensor(z, device="cuda"), torch.tensor(dy, device="cuda")
    det = t.forward(zt, counts=counts, mode="deterministic").cpu().numpy()
    ev = t.forward(zt, counts=counts, mode="event").cpu().numpy()
    dz, dw = t.backward(zt, dyt, counts=counts)
    dz, dw = dz.cpu().numpy(), dw.cpu().numpy()
    ref = orc.syn_fwd(pop, z, tb.basis, use_count=counts)
    np.testing.assert_array_equal(det.view(np.uint32), ref.view(np.uint32))
    scale = dense.syn_fwd_abs(pop, z, tb.basis, use_count=counts)
    assert_grads_per_element(ev, ref, scale, what=f"{name} event currents")
    rdz, rdw = orc.syn_bwd(pop, z, tb.basis, dy, use_count=counts)
    _, _, dz_abs, dw_abs = dense.syn_bwd_f64(pop, z, tb.basis, dy, use_count=counts)
    assert np.count_nonzero(rdw) > 0
    say(f"op level {name} B={B}: dz", error_summary(dz, rdz, dz_abs), "dW", error_summary(dw, rdw, dw_abs))
    assert_grads_per_element(dz, rdz, dz_abs, what=f"{name} dz")
    assert_grads_per_element(dw, rdw, dw_abs, what=f"{name} dW")


def test_config2_op_level(config2):
    """calculate_synaptic_currents on the full config-2 recurrent table (models.py:103-263):
    z_buf [5][D*N] at 5 Hz, dy [5*N][nb] normal.  Deterministic forward bit-exact with the
    oracle; event forward, dz and dW within 1e-5 of the float64 brute force's sum of absolute
    terms (+1e-6)."""
    from oracle import dense
    from v1_glif_model_amd.ops import SynapseTable
    tb = config2["tb"]
    N, D, B, nb = tb.n_neurons, tb.max_delay, 5, tb.n_basis
    t = SynapseTable(np.stack([tb.rec.post, tb.rec.col], -1), tb.rec.syn_id, (N, tb.rec.n_cols), tb.basis,
                     n_delay_slots=D)
    t.set_weights(torch.tensor(tb.rec.weight, device="cuda"))
    rng = np.random.default_rng(3)
    z = (rng.uniform(size=(B, D * N)) < 0.005).astype(np.float32)
    dy = rng.normal(0, 1, (B * N, nb)).astype(np.float32)
    zt, dyt = torch.tensor(z, device="cuda"), torch.tensor(dy, device="cuda")
    det = t.forward(zt, mode="deterministic").cpu().numpy()
    ev = t.forward(zt, mode="event").cpu().numpy()
    dz, dw = t.backward(zt, dyt)
    dz, dw = dz.cpu().numpy(), dw.cpu().numpy()
    ref = orc.syn_fwd(tb.rec, z, tb.basis)
    np.testing.assert_array_equal(det.view(np.uint32), ref.view(np.uint32))
    scale = dense.syn_fwd_abs(tb.rec, z, tb.basis)
    say("op level: event currents", error_summary(ev, ref, scale))
    assert_grads_per_element(ev, ref, scale, what="event currents")
    rdz, rdw = orc.syn_bwd(tb.rec, z, tb.basis, dy)
    _, _, dz_abs, dw_abs = dense.syn_bwd_f64(tb.rec, z, tb.basis, dy)
    say("op level: events", int(np.count_nonzero(z)), "max |dz|", float(np.abs(rdz).max()),
        "nonzero dW", int(np.count_nonzero(rdw)))
    assert np.count_nonzero(rdw) > 0
    say("op level: dz", error_summary(dz, rdz, dz_abs), "dW", error_summary(dw, rdw, dw_abs))
    assert_grads_per_element(dz, rdz, dz_abs, what="dz")
    assert_grads_per_element(dw, rdw, dw_abs, what="dW")
