"""ExponentiatedAdam + SignedConstraint (optimizers.py:268-376, models.py:419-427).

CPU: the float32 oracle (oracle/optim_ref.py) is pinned by Adam's first-step closed
form (the update's magnitude is the learning rate: w1 = w0 * exp(-lr * sign(g * w0))
when |g| >> epsilon), exact invariants (zero gradient leaves everything unchanged; the
update never flips a sign; the constraint clips wrong-signed weights to zero; the
AMSGrad slot is the running maximum of v) and a float64 restatement over many steps.
GPU: libglif's fused kernel against the oracle over several steps (1e-6 relative,
the gap of the exp / sqrt roundings).
"""
import numpy as np
import pytest

from oracle import optim_ref as orf

f32 = np.float32


def _data(n=2000, seed=0):
    rng = np.random.default_rng(seed)
    w = rng.lognormal(-1, 1, n).astype(f32) * rng.choice([-1, 1], n).astype(f32)
    w[:10] = 0.0
    return w, rng


def test_first_step_closed_form():
    w0, rng = _data()
    g = rng.normal(0, 1, w0.size).astype(f32)
    g[np.abs(g) < 0.1] = 0.1   # the closed form neglects epsilon / sqrt(v) ~ lr * 3e-6 / |g|
    lr = 0.005
    w, m, v = w0.copy(), np.zeros_like(w0), np.zeros_like(w0)
    orf.exp_adam_step(w, m, v, g, orf.alpha(lr, 0.9, 0.999, 1))
    s = np.where(w0 == 0, 1.0, np.sign(w0))
    expect = w0.astype(np.float64) * np.exp(-lr * np.sign(g) * s)
    np.testing.assert_allclose(w, expect, rtol=2e-6, atol=0)


def test_zero_gradient_is_identity():
    w0, _ = _data(seed=1)
    w, m, v = w0.copy(), np.zeros_like(w0), np.zeros_like(w0)
    for t in range(1, 6):
        orf.exp_adam_step(w, m, v, np.zeros_like(w0), orf.alpha(0.01, 0.9, 0.999, t))
    np.testing.assert_array_equal(w, w0)
    assert not m.any() and not v.any()


def test_sign_preserved_and_constraint_clips():
    w0, rng = _data(seed=2)
    positive = rng.random(w0.size) < 0.5
    w, m, v = w0.copy(), np.zeros_like(w0), np.zeros_like(w0)
    for t in range(1, 4):
        g = rng.normal(0, 1, w0.size).astype(f32)
        orf.exp_adam_step(w, m, v, g, orf.alpha(0.05, 0.9, 0.999, t), positive=positive)
    wrong = np.sign(w0) != np.where(positive, 1, -1)
    assert np.all(w[wrong & (w0 != 0)] == 0)          # wrong sign -> clipped to zero
    ok = ~wrong & (w0 != 0)
    assert np.all(np.sign(w[ok]) == np.sign(w0[ok]))  # right sign: kept, magnitude moved
    assert np.all(w[w0 == 0] == 0)                    # zero stays zero (multiplicative)


def test_amsgrad_slot_is_running_max():
    w0, rng = _data(seed=3)
    w, m, v, vh = w0.copy(), np.zeros_like(w0), np.zeros_like(w0), np.zeros_like(w0)
    vmax = np.zeros_like(w0)
    for t in range(1, 6):
        g = (rng.normal(0, 1, w0.size) * (3.0 if t == 2 else 1.0)).astype(f32)
        orf.exp_adam_step(w, m, v, g, orf.alpha(0.01, 0.9, 0.999, t), vhat=vh)
        vmax = np.maximum(vmax, v)
        np.testing.assert_array_equal(vh, vmax)


def test_oracle_matches_float64_over_steps():
    w0, rng = _data(seed=4)
    w, m, v = w0.copy(), np.zeros_like(w0), np.zeros_like(w0)
    W, M, V = w0.astype(np.float64), np.zeros(w0.size), np.zeros(w0.size)
    lr, b1, b2, eps = 0.01, 0.9, 0.999, 1e-7
    for t in range(1, 21):
        g = rng.normal(0, 1, w0.size).astype(f32)
        orf.exp_adam_step(w, m, v, g, orf.alpha(lr, b1, b2, t))
        M += (g - M) * (1 - b1)
        V += (g.astype(np.float64) ** 2 - V) * (1 - b2)
        a = lr * np.sqrt(1 - b2 ** t) / (1 - b1 ** t)
        s = np.where(W == 0, 1.0, np.sign(W))
        W *= np.exp(-a * M / (np.sqrt(V) + eps) * s)
    np.testing.assert_allclose(w, W, rtol=2e-5, atol=1e-12)


# ------------------------------------------------------------------------ GPU ----
@pytest.mark.gpu
@pytest.mark.parametrize("amsgrad,constrained", [(False, False), (True, False), (False, True), (True, True)])
def test_gpu_exp_adam_matches_oracle(amsgrad, constrained):
    import torch
    from v1_glif_model_amd.optim import ExponentiatedAdam, SignedConstraint
    w0, rng = _data(n=100_003, seed=5)
    positive = rng.random(w0.size) < 0.6
    wt = torch.tensor(w0, device="cuda")
    opt = ExponentiatedAdam(learning_rate=0.01, amsgrad=amsgrad)
    cons = {wt.data_ptr(): SignedConstraint(torch.tensor(positive))} if constrained else None
    w, m, v = w0.copy(), np.zeros_like(w0), np.zeros_like(w0)
    vh = np.zeros_like(w0) if amsgrad else None
    for t in range(1, 8):
        g = rng.normal(0, 1, w0.size).astype(f32)
        g[::97] = 0.0
        opt.apply_gradients([(torch.tensor(g, device="cuda"), wt)], constraints=cons)
        orf.exp_adam_step(w, m, v, g, orf.alpha(0.01, 0.9, 0.999, t), vhat=vh,
                          positive=positive if constrained else None)
    got = wt.cpu().numpy()
    np.testing.assert_allclose(got, w, rtol=1e-6, atol=1e-12)
    s = opt.slots(wt)
    np.testing.assert_allclose(s["m"].cpu().numpy(), m, rtol=1e-6, atol=1e-12)
    np.testing.assert_allclose(s["v"].cpu().numpy(), v, rtol=1e-6, atol=1e-12)
    assert opt.iterations == 7


@pytest.mark.gpu
def test_gpu_update_reaches_the_next_rollout():
    """The optimizer writes the weights through a raw pointer; the next rollout must use the
    updated weights (the synapse tables refresh their copies when the tensor's version moves):
    a rollout after the step equals one of a fresh cell given the updated weights."""
    import torch
    from tests.helpers import network, tiny_config
    from v1_glif_model_amd import synthetic as sy
    from v1_glif_model_amd.models import V1Column
    from v1_glif_model_amd.optim import ExponentiatedAdam
    cfg = tiny_config(rs=2.0, ins=3.0)
    net, tb = network(cfg, seed=12, dense_basis=True)
    lgn, bkg = sy.make_inputs(cfg, seed=13, seq_len=30, batch=2)
    kw = dict(gauss_std=0.5, dampening_factor=0.5, pseudo_gauss=True, train_recurrent_per_type=False)
    a = V1Column(net, mode="deterministic", **kw)
    a.rollout(lgn, bkg)
    g = {k: torch.tensor(np.random.default_rng(1).normal(0, 1, n).astype(f32), device="cuda")
         for k, n in (("rec", tb.rec.n_syn), ("lgn", tb.lgn.n_syn))}
    ExponentiatedAdam(learning_rate=0.3).apply_gradients(
        [(g["rec"], a.recurrent_weight_values), (g["lgn"], a.input_weight_values)])
    za, va, _ = a.rollout(lgn, bkg)
    b = V1Column(net, mode="deterministic", **kw)
    with torch.no_grad():
        b.recurrent_weight_values.copy_(a.recurrent_weight_values)
        b.input_weight_values.copy_(a.input_weight_values)
    zb, vb, _ = b.rollout(lgn, bkg)
    assert not torch.equal(a.recurrent_weight_values, torch.tensor(tb.rec.weight, device="cuda"))
    np.testing.assert_array_equal(za.cpu().numpy(), zb.cpu().numpy())
    np.testing.assert_array_equal(va.cpu().numpy().view(np.uint32), vb.cpu().numpy().view(np.uint32))
