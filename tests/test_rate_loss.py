"""Rate-distribution loss (SpikeRateDistributionTarget, loss_functions.py:782-889).

CPU: the oracle (oracle/rate_loss_ref.py) pinned against the QR-DQN form of the Huber
quantile loss, hand-worked cases, float64 finite differences, order invariance, zero loss at
the targets and a brute-force tie order; the host-side target construction.
GPU: glif_rate_dist_loss against the oracle -- per-neuron dL/dz bit for bit (same fp32
operations per element, same sorted order), the loss within 1e-6 relative (the sum order
differs) -- and fused with the cell: trimmed spike counts from the forward, and the
backward's windowed gz_neuron equal to the dense dL/dz it stands for.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import rate_loss_ref as R
from oracle.sample_ref import words

KAPPA = 0.002


def _pops(n, n_pop, rng, core=None):
    lab = rng.integers(0, n_pop, n)
    sel = np.arange(n) if core is None else np.flatnonzero(core)
    ids = [sel[lab[sel] == k].astype(np.int32) for k in range(n_pop)]
    ptr = np.concatenate([[0], np.cumsum([x.size for x in ids])]).astype(np.int32)
    return np.concatenate(ids), ptr


def _targets(ptr, rng, hi=0.05):
    return np.concatenate([np.sort(rng.uniform(0, hi, ptr[k + 1] - ptr[k])) for k in range(len(ptr) - 1)]
                          ).astype(np.float32)


# ---------------------------------------------------------------- oracle pins ----
def test_huber_quantile_equals_qr_dqn_form():
    """rho_tau^kappa(u) = |tau - [u < 0]| L_kappa(u) / kappa, L_kappa = u^2 / 2 (|u| <= kappa)
    else kappa (|u| - kappa / 2) (Dabney et al. 2018); the reference's [u <= 0] differs only
    at u = 0, where both are 0."""
    rng = np.random.default_rng(0)
    u = np.concatenate([rng.uniform(-0.01, 0.01, 4000), rng.uniform(-1, 1, 1000), [0.0, KAPPA, -KAPPA]])
    tau = rng.uniform(0, 1, u.size)
    # float32 inputs, so that the comparison sees only the arithmetic's rounding
    u, tau = u.astype(np.float32).astype(np.float64), tau.astype(np.float32).astype(np.float64)
    L = np.where(np.abs(u) <= KAPPA, 0.5 * u * u, KAPPA * (np.abs(u) - 0.5 * KAPPA))
    rho = np.abs(tau - (u < 0)) * L / KAPPA
    h = R.huber_quantile(u.astype(np.float32), tau.astype(np.float32), KAPPA).astype(np.float64)
    np.testing.assert_allclose(h, rho, rtol=1e-6, atol=1e-12)
    h64 = R.huber_quantile(u, tau, KAPPA, np.float64)
    np.testing.assert_allclose(h64, rho, rtol=1e-12, atol=1e-18)


def test_hand_worked_cases():
    # one neuron (tau = 1): above the target by more than kappa costs u - kappa / 2, below costs 0
    ids, ptr = np.array([0], np.int32), [0, 1]
    loss, gz = R.rate_dist_loss(np.array([5]), 100, ids, ptr, np.array([0.01], np.float32), rate_cost=2.0)
    assert abs(loss - 2.0 * (0.04 - 0.001)) < 1e-8 and abs(gz[0] - 2.0 / 100) < 1e-9
    loss, gz = R.rate_dist_loss(np.array([0]), 100, ids, ptr, np.array([0.01], np.float32))
    assert loss == 0 and gz[0] == 0
    # two neurons, rates {0.03 (neuron 0), 0.01 (neuron 1)} against targets {0.02, 0.02}:
    # ranks 0 / 1 take tau 0.5 / 1 -> 0.5 (0.01 - 0.001) + (0.01 - 0.001), mean over 2
    loss, gz = R.rate_dist_loss(np.array([3, 1]), 100, np.array([0, 1], np.int32), [0, 2],
                                np.array([0.02, 0.02], np.float32))
    assert abs(loss - 0.0135 / 2) < 1e-9
    np.testing.assert_allclose(gz, [0.5 / 100, -0.25 / 100], rtol=1e-6)
    # inside the quadratic zone: u = 0.001, tau = 1 -> u^2 / (2 kappa) = 2.5e-4
    loss, gz = R.rate_dist_loss(np.array([11]), 1000, np.array([0], np.int32), [0, 1],
                                np.array([0.01], np.float32))
    assert abs(loss - 2.5e-4) < 1e-9 and abs(gz[0] - 0.5 / 1000) < 1e-8


def test_gradient_matches_finite_differences():
    rng = np.random.default_rng(1)
    N = 300
    ids, ptr = _pops(N, 4, rng)
    tg = _targets(ptr, rng).astype(np.float64)
    rates = rng.uniform(0, 0.05, N)
    loss, grad = R.loss_from_rates(rates, ids, ptr, tg, KAPPA, 0.7, dt=np.float64)
    eps = 1e-8
    checked = 0
    srt = np.sort(rates)
    for j in rng.choice(N, 60, replace=False):
        # skip neurons near a tie (the sort order would change) or a kink of h
        if np.min(np.abs(srt - rates[j])[np.abs(srt - rates[j]) > 0], initial=1) < 10 * eps:
            continue
        rp, rm = rates.copy(), rates.copy()
        rp[j] += eps
        rm[j] -= eps
        lp = R.loss_from_rates(rp, ids, ptr, tg, KAPPA, 0.7, dt=np.float64)[0]
        lm = R.loss_from_rates(rm, ids, ptr, tg, KAPPA, 0.7, dt=np.float64)[0]
        fd = (lp - lm) / (2 * eps)
        assert abs(fd - grad[j]) <= 1e-5 * max(abs(grad[j]), 1e-3), (j, fd, grad[j])
        checked += 1
    assert checked >= 40


def test_loss_invariant_to_order_within_population_and_zero_at_targets():
    rng = np.random.default_rng(2)
    N, S = 500, 64
    ids, ptr = _pops(N, 5, rng)
    count = rng.integers(0, 6, N)          # many ties
    tg = _targets(ptr, rng, 0.1)
    l0, g0 = R.rate_dist_loss(count, S, ids, ptr, tg)
    ids2 = ids.copy()
    for k in range(5):
        seg = ids2[ptr[k]:ptr[k + 1]]
        rng.shuffle(seg)
    for shuffle in (False, True):
        l1, g1 = R.rate_dist_loss(count, S, ids2, ptr, tg, shuffle=shuffle, seed=9)
        assert l1 == l0
        # neurons of one (population, count) group share their gradients as a multiset
        for k in range(5):
            seg = ids[ptr[k]:ptr[k + 1]]
            for c in np.unique(count[seg]):
                m = seg[count[seg] == c]
                np.testing.assert_array_equal(np.sort(g1[m]), np.sort(g0[m]))
    # rates equal to the (sorted) targets: zero loss and gradient
    tgt = np.concatenate([np.sort(count[ids[ptr[k]:ptr[k + 1]]]) for k in range(5)]).astype(np.float32) / np.float32(S)
    l2, g2 = R.rate_dist_loss(count, S, ids, ptr, tgt)
    assert l2 == 0 and not np.any(g2)


@pytest.mark.parametrize("shuffle", [False, True])
def test_tie_order_brute_force(shuffle):
    rng = np.random.default_rng(3)
    n = 200
    ids, ptr = _pops(n, 3, rng)
    count = rng.integers(0, 4, n)
    order = R.sorted_order(count[ids], ptr, shuffle, seed=5, offset=77)
    w = words(ids.size, 5, 77) if shuffle else np.zeros(ids.size, np.uint32)
    pop = np.repeat(np.arange(3), np.diff(ptr))
    expect = sorted(range(ids.size), key=lambda i: (pop[i], count[ids[i]], int(w[i])))  # stable
    np.testing.assert_array_equal(order, expect)


def test_rate_mse_oracle_closed_form_and_gradient():
    rng = np.random.default_rng(11)
    N, S = 400, 250
    count = rng.integers(0, 6, N)
    tg = rng.uniform(0, 0.02, N).astype(np.float32)
    loss, gz = R.rate_mse(count, S, tg)
    r = count / S
    assert abs(loss - np.mean((r - tg.astype(np.float64)) ** 2)) <= 1e-6 * loss
    # dL/dz of every tick: dL/drate / S, dL/drate = 2 (r - t) / N (finite differences in float64)
    eps = 1e-7
    for j in rng.choice(N, 10, replace=False):
        rp, rm = r.copy(), r.copy()
        rp[j] += eps
        rm[j] -= eps
        fd = (np.mean((rp - tg) ** 2) - np.mean((rm - tg) ** 2)) / (2 * eps)
        assert abs(gz[j] * S - fd) <= 1e-4 * abs(fd) + 1e-9
    l0, g0 = R.rate_mse(np.zeros(N, int), S, np.zeros(N, np.float32))
    assert l0 == 0 and not np.any(g0)


# ---------------------------------------------------------------- host side ----
def test_sample_firing_rates_properties():
    from v1_glif_model_amd.losses import sample_firing_rates
    rng = np.random.default_rng(4)
    rates = rng.lognormal(0, 1, 300) / 1000
    t = sample_firing_rates(rates, 50000, 42)
    assert t.size == 50000 and np.all(np.diff(t) >= 0)
    assert t.min() >= rates.min() and t.max() <= rates.max()
    # inverse-transform samples: the empirical CDF at a few knots within sampling error
    s = np.sort(rates)
    for q in (0.1, 0.5, 0.9):
        x = np.interp(q, np.linspace(0, 1, s.size), s)
        assert abs(np.mean(t <= x) - q) < 0.01
    np.testing.assert_array_equal(sample_firing_rates(rates, 10, 7), sample_firing_rates(rates, 10, 7))
    np.testing.assert_array_equal(sample_firing_rates(np.array([0.0]), 4, 1), np.zeros(4))


def test_population_ids_and_cell_type_names(tmp_path):
    from v1_glif_model_amd import losses as L
    from v1_glif_model_amd import synthetic as sy
    ct = sy.make_cell_types(400, 320)
    core = np.zeros(400, bool)
    core[::3] = True
    p = L.population_neuron_ids(ct, core)
    assert tuple(p) == L.CELL_TYPE_ORDER
    allids = np.concatenate(list(p.values()))
    np.testing.assert_array_equal(np.sort(allids), np.flatnonzero(core))
    for k, v in p.items():
        assert np.all(ct[v] == k)
    q = L.population_neuron_ids(ct, core, reindex_selected=True)
    assert np.concatenate(list(q.values())).max() == core.sum() - 1
    assert L.neuropixels_cell_type_to_cell_type("EXC_L23") == "L2/3 Exc"
    assert L.neuropixels_cell_type_to_cell_type("PV_L5") == "L5 PV"
    assert L.neuropixels_cell_type_to_cell_type("SST_L1") == "L1 Htr3a"
    assert L.neuropixels_cell_type_to_cell_type("Htr3a_L6") == "L6 VIP"
    assert L.neuropixels_cell_type_to_cell_type("L4 Exc") == "L4 Exc"
    f = tmp_path / "units.csv"
    f.write_text('ecephys_unit_id DSI cell_type firing_rate_sp Ave_Rate(Hz)\n'
                 '1 0.1 "L6 Exc" 0.25 5.4\n2 0.2 PV_L6 18.6 21.3\n3 0.3 EXC_L6 1.0 2.0\n')
    r = L.load_neuropixels_type_rates(str(f), "drifting_gratings")
    np.testing.assert_allclose(r["L6 Exc"], [0.0054, 0.002, 0.0])
    np.testing.assert_allclose(r["L6 PV"], [0.0213, 0.0])
    r = L.load_neuropixels_type_rates(str(f), "spontaneous")
    np.testing.assert_allclose(r["L6 Exc"], [0.00025, 0.001, 0.0])
    g = tmp_path / "units2.csv"
    g.write_text('ecephys_unit_id cell_type Spont_Rate(Hz) Ave_Rate(Hz)\n1 "L4 PV" 3.0 4.0\n')
    np.testing.assert_allclose(L.load_neuropixels_type_rates(str(g), "gray")["L4 PV"], [0.003, 0.0])
    with pytest.raises(ValueError, match="Unknown stimulus_type"):
        L.load_neuropixels_type_rates(str(g), "movies")
    # stimulus types name the rate column (loss_functions.py:796-810)
    with pytest.raises(ValueError, match="Unknown stimulus_type"):
        L._rate_feature("movies")
    assert L._rate_feature("gray") == "firing_rate_sp" and L._rate_feature("natural_images") == "firing_rate_ns"


# ------------------------------------------------------------------------ GPU ----
def _abi_loss(count, rows, N, S, ids, ptr, tg, shuffle, seed, offset, rate_cost=0.5, gz0=None):
    import torch
    from v1_glif_model_amd._lib import lib, check
    dev = "cuda"
    c = torch.tensor(count, dtype=torch.int32, device=dev)
    i = torch.tensor(ids, dtype=torch.int32, device=dev)
    t = torch.tensor(tg, dtype=torch.float32, device=dev)
    gz = torch.zeros(N, dtype=torch.float32, device=dev) if gz0 is None else torch.tensor(gz0, device=dev)
    loss = torch.empty((), dtype=torch.float32, device=dev)
    need = lib().glif_rate_loss_workspace(ids.size)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    pp = (C.c_int32 * len(ptr))(*[int(x) for x in ptr])
    check(lib().glif_rate_dist_loss(C.c_void_p(c.data_ptr()), rows, N, S, C.c_void_p(i.data_ptr()), pp,
                                    len(ptr) - 1, C.c_void_p(t.data_ptr()), KAPPA, rate_cost, shuffle, seed,
                                    offset, C.c_void_p(loss.data_ptr()), C.c_void_p(gz.data_ptr()),
                                    C.c_void_p(ws.data_ptr()), ws.numel(), None))
    torch.cuda.synchronize()
    return float(loss.item()), gz.cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("N,B,S,n_pop,shuffle", [(1, 1, 7, 1, 0), (1000, 3, 300, 17, 0), (1000, 3, 300, 17, 1),
                                                 (70000, 8, 4000, 17, 1), (5000, 2, 2, 5, 1)])
def test_gpu_rate_loss_matches_oracle(N, B, S, n_pop, shuffle):
    rng = np.random.default_rng(N + n_pop + shuffle)
    core = rng.uniform(size=N) < 0.8 if N > 1 else None
    ids, ptr = _pops(N, n_pop, rng, core)
    per_row = max(S // B, 1)
    count = np.minimum(rng.poisson(0.004 * per_row * 3, (B, N)), per_row).astype(np.int32)
    tg = _targets(ptr, rng, 0.02)
    loss, gz = _abi_loss(count, B, N, S, ids, ptr, tg, shuffle, 11, 5)
    el, eg = R.rate_dist_loss(count.sum(0), S, ids, ptr, tg, KAPPA, 0.5, bool(shuffle), 11, 5)
    print("N", N, "loss", loss, el, "nonzero grads", np.count_nonzero(eg))
    np.testing.assert_array_equal(gz.view(np.uint32), eg.view(np.uint32))
    assert abs(loss - el) <= 1e-6 * abs(el) + 1e-12


@pytest.mark.gpu
def test_gpu_rate_loss_accumulates_and_flags_bad_ids():
    rng = np.random.default_rng(7)
    N, S = 300, 50
    ids, ptr = _pops(N, 3, rng)
    count = rng.integers(0, 3, N).astype(np.int32)
    tg = _targets(ptr, rng)
    gz0 = rng.normal(0, 1, N).astype(np.float32)
    _, gz = _abi_loss(count, 1, N, S, ids, ptr, tg, 1, 3, 0, gz0=gz0)
    _, eg = R.rate_dist_loss(count, S, ids, ptr, tg, KAPPA, 0.5, True, 3, 0)
    np.testing.assert_array_equal(gz, gz0 + eg)
    bad = ids.copy()
    bad[5] = N + 10
    loss, gz = _abi_loss(count, 1, N, S, bad, ptr, tg, 1, 3, 0)
    assert np.isnan(loss)
    assert np.all(np.isfinite(gz))


@pytest.mark.gpu
def test_gpu_rate_target_fused_with_cell():
    """Trimmed spike counts from the forward equal the count of the trimmed z; the loss of
    the counts equals the loss of z; the backward's gz_neuron over the trimmed ticks equals
    the dense dL/dz it stands for (bit for bit: the backward sums in a fixed order)."""
    import torch
    from tests.helpers import network, tiny_config
    from v1_glif_model_amd import synthetic as sy
    from v1_glif_model_amd.losses import SpikeRateDistributionTarget
    from v1_glif_model_amd.models import V1Column
    cfg = tiny_config(rs=2.0, ins=3.0)
    net, tb = network(cfg, seed=4, dense_basis=True)
    N = tb.n_neurons
    T, B, pre, post = 40, 3, 6, 4
    lgn, bkg = sy.make_inputs(cfg, seed=5, seq_len=T, batch=B)
    cell = V1Column(net, mode="deterministic", gauss_std=0.5, dampening_factor=0.5,
                    recurrent_dampening_factor=0.5, voltage_gradient_dampening=0.5, pseudo_gauss=True)
    pops = {k: v for k, v in zip(("L2/3 Exc", "L4 PV", "L5 SST"), np.array_split(np.arange(N, dtype=np.int32), 3))}
    loss_fn = SpikeRateDistributionTarget(populations=pops, type_rates=sy.make_type_rates(), rate_cost=0.5,
                                          pre_delay=pre, post_delay=post, cell=cell, shuffle_seed=3)
    cnt = torch.zeros((B, N), dtype=torch.int32, device="cuda")
    z, v, _ = cell.rollout(lgn, bkg, spike_count=cnt)
    zn = z.cpu().numpy()
    assert zn[pre:T - post].sum() > 0
    np.testing.assert_array_equal(cnt.cpu().numpy(), zn[pre:T - post].sum(0).astype(np.int32))
    l1 = loss_fn(spike_count=cnt, T=T)
    g1 = loss_fn.gz_neuron.clone()
    loss_fn._offset = 0
    l2 = loss_fn(z)
    assert float(l1) == float(l2)
    np.testing.assert_array_equal(g1.cpu().numpy(), loss_fn.gz_neuron.cpu().numpy())
    assert torch.count_nonzero(g1) > 0
    gw = cell.backward(gz_neuron=g1)
    dense = torch.zeros((T, B, N), dtype=torch.float32, device="cuda")
    dense[pre:T - post] = g1
    gd = cell.backward(gz=dense)
    for k in gw:
        np.testing.assert_array_equal(gw[k].cpu().numpy(), gd[k].cpu().numpy())


@pytest.mark.gpu
def test_gpu_rate_mse_matches_oracle():
    import torch
    from v1_glif_model_amd.losses import RateMSE
    rng = np.random.default_rng(12)
    B, N, T = 5, 70000, 500
    count = rng.poisson(2.5, (B, N)).astype(np.int32)
    tg = rng.lognormal(np.log(0.004), 1.0, N).astype(np.float32)
    f = RateMSE(tg)
    gz0 = rng.normal(0, 1e-6, N).astype(np.float32)
    g = torch.tensor(gz0, device="cuda")
    loss = float(f(torch.tensor(count, device="cuda"), T, gz_neuron=g))
    el, eg = R.rate_mse(count.sum(0), T * B, tg)
    np.testing.assert_array_equal(g.cpu().numpy(), gz0 + eg)
    assert abs(loss - el) <= 1e-6 * el
