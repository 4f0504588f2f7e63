"""Test infrastructure only (never imported by the product): a float32 numpy restatement of
the rate-distribution loss, SpikeRateDistributionTarget.__call__ (v1_model_utils/
loss_functions.py:873-889) -> compute_spike_rate_target_loss (:634-664) ->
compute_spike_rate_distribution_loss (:666-681) -> huber_quantile_loss (:626-632), with the
gradient TF's autograd takes through it, in TF's operation order.

The reference shuffles each population with tf.random.shuffle before tf.sort; the shuffle
only decides which of several neurons with equal rates takes which sorted position.  Here
the order among equal rates is a Philox4x32-10 word per selection position (or the input
order), so the GPU kernel's assignment can be checked exactly.

Pinned in tests/test_rate_loss.py by: the QR-DQN form of the Huber quantile loss (Dabney et
al., AAAI 2018, rho = |tau - [u < 0]| L_kappa(u) / kappa), hand-worked one- and two-neuron
cases, finite differences of the loss in float64, invariance of the loss to the order of
ids within a population, zero loss and gradient when rates equal the targets, and numpy's
own stable sort for the tie order.
"""
import numpy as np

from oracle.sample_ref import words

f32 = np.float32


def huber_quantile(u, tau, kappa, dt=f32):
    """loss_functions.py:626-632 (float32 by default)."""
    u, tau, kappa = dt(u), dt(tau), dt(kappa)
    au = np.abs(u)
    num = np.abs(tau - (u <= 0).astype(dt))
    b1 = num / (dt(2) * kappa) * np.square(u)
    b2 = num * (au - dt(0.5) * kappa)
    return np.where(au <= kappa, b1, b2).astype(dt)


def huber_quantile_grad(u, tau, kappa, g, dt=f32):
    """d/du of huber_quantile times upstream g, as TF's gradients of Select / Mul / Square /
    Abs chain it: branch 1 (g * (num / 2 kappa)) * (2 u), branch 2 (g * num) * sign(u)."""
    u, tau, kappa, g = dt(u), dt(tau), dt(kappa), dt(g)
    au = np.abs(u)
    num = np.abs(tau - (u <= 0).astype(dt))
    d1 = (g * (num / (dt(2) * kappa))) * (u * dt(2))
    d2 = (g * num) * np.sign(u).astype(dt)
    return np.where(au <= kappa, d1, d2).astype(dt)


def sorted_order(keys, pop_ptr, shuffle=False, seed=0, offset=0):
    """Selection positions in sorted order: by (population, key, tie word, position);
    keys [n_sel] are the selected neurons' counts (or rates)."""
    n_sel = int(pop_ptr[-1])
    pop = np.repeat(np.arange(len(pop_ptr) - 1), np.diff(pop_ptr))
    tie = words(n_sel, seed, offset).astype(np.int64) if shuffle else np.zeros(n_sel, np.int64)
    return np.lexsort((np.arange(n_sel), tie, keys, pop))


def loss_from_rates(rates, ids, pop_ptr, targets, kappa=0.002, rate_cost=1.0, order=None, dt=f32):
    """compute_spike_rate_target_loss (:634-664) on rates [N] -> (loss, dL/drate [N]).

    order: selection positions in sorted order (sorted_order); by default a stable sort of
    the selected rates within each population."""
    rates = np.asarray(rates, dt)
    pop_ptr = np.asarray(pop_ptr, np.int64)
    n_sel = int(pop_ptr[-1])
    if order is None:
        order = sorted_order(rates[ids], pop_ptr)
    pop = np.repeat(np.arange(len(pop_ptr) - 1), np.diff(pop_ptr))
    rank = np.arange(n_sel) - pop_ptr[pop]
    nk = (pop_ptr[1:] - pop_ptr[:-1])[pop]
    tau = (rank.astype(dt) + dt(1)) / nk.astype(dt)
    u = rates[ids[order]] - np.asarray(targets, dt)
    h = huber_quantile(u, tau, kappa, dt)
    loss = dt(dt(np.sum(h, dtype=np.float64)) / dt(n_sel)) * dt(rate_cost)
    g = dt(rate_cost) / dt(n_sel)
    grad = np.zeros(rates.shape, dt)
    grad[ids[order]] = huber_quantile_grad(u, tau, kappa, g, dt)
    return loss, grad


def rate_dist_loss(count, n_samples, ids, pop_ptr, targets, kappa=0.002, rate_cost=1.0, shuffle=False,
                   seed=0, offset=0):
    """SpikeRateDistributionTarget.__call__ (:873-889) on spike counts [N] (summed over the
    batch and the trimmed ticks, n_samples of them per neuron) -> (loss f32, gz_neuron [N]
    f32), gz_neuron = 0 + dL/drate / n_samples, the dL/dz of every (tick, batch)
    (reduce_mean, :885)."""
    count = np.asarray(count)
    S = f32(n_samples)
    order = sorted_order(count[ids].astype(np.int64), pop_ptr, shuffle, seed, offset)
    loss, grad = loss_from_rates(count.astype(f32) / S, ids, pop_ptr, targets, kappa, rate_cost, order)
    # added into a zero buffer, as the library adds into the caller's (-0 becomes +0)
    return loss, (np.zeros(count.shape, f32) + grad / S).astype(f32)


def rate_mse(count, n_samples, targets):
    """Mean-squared firing-rate error (the benchmark configuration's loss): count [N]
    (summed over batch rows), rbar = count / S in float32; loss = mean (rbar - target)^2,
    gz_neuron = 0 + (rbar - target) * float32(2 / (N * S)) per tick."""
    count = np.asarray(count)
    N = count.shape[-1]
    diff = count.astype(f32) / f32(n_samples) - np.asarray(targets, f32)
    loss = f32(np.sum(diff.astype(np.float64) ** 2) / N)
    scale = f32(2.0 / (float(N) * float(n_samples)))
    return loss, (np.zeros(N, f32) + diff * scale).astype(f32)
