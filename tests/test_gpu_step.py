"""The per-step backward (glif_step_backward) behind ``V1Column.call``: the gradient of a loop of
``call``s, as the reference's GradientTape takes it through the Keras RNN step by step
(models.py:1059-1135 under :1317-1322; multi_training.py:368-372, 485-493).

Bars: the forward of the loop equals the oracle's bit for bit (deterministic mode); the weight
gradients and the gradients of the loop's initial state (spike buffer, v, asc, psc_rise, psc)
equal the float64 autograd restatement (oracle/torch_ref.py, teacher-forced on the oracle's
spikes) per element within 1e-5 of the element's sum of absolute terms + 1e-6, and the literal
1e-5 relative / 1e-6 absolute on every element that is not a cancellation case; the loop's
weight gradients equal those of the fused rollout's BPTT within the same bar.
"""
import numpy as np
import pytest
import torch

from oracle import torch_ref
from oracle.cpu import OracleCell, bptt_abs_scale
from tests.helpers import assert_grads_per_element, error_summary, network, tiny_config
from v1_glif_model_amd import synthetic as sy

pytestmark = pytest.mark.gpu

PARAMS = {
    "gauss_sym": dict(pseudo_gauss=True, hard_reset=False, rd=0.5, vgd=0.5, gauss_std=0.5, damp=0.5),
    "reference_defaults_hard_reset": dict(pseudo_gauss=True, hard_reset=True, rd=0.1, vgd=0.5, gauss_std=0.3,
                                          damp=0.1),
    "triangular_asym": dict(pseudo_gauss=False, hard_reset=False, rd=0.2, vgd=0.3, gauss_std=0.7, damp=0.3),
}


def _cell_kw(p):
    return dict(pseudo_gauss=p["pseudo_gauss"], hard_reset=p["hard_reset"], recurrent_dampening_factor=p["rd"],
                voltage_gradient_dampening=p["vgd"], gauss_std=p["gauss_std"], dampening_factor=p["damp"])


@pytest.mark.parametrize("name", list(PARAMS))
def test_call_loop_gradients(name):
    from v1_glif_model_amd.models import V1Column
    p = PARAMS[name]
    cfg = tiny_config(n=200, fanin=20, rs=2.0, ins=3.0)
    net, tb = network(cfg, seed=21, dense_basis=True)
    T1, T2, B = 40, 25, 3
    lgn, bkg = sy.make_inputs(cfg, seed=22, seq_len=T1 + T2, batch=B)
    oc = OracleCell(tb, **p)
    # a carried state with spikes in its history and refractory neurons
    _, _, _, st1 = oc.forward(lgn[:T1], bkg[:T1])
    assert st1["zbuf"].sum() > 0 and st1["r"].max() > 0
    lgn2, bkg2 = lgn[T1:], bkg[T1:]
    oz, ov, oref, _ = oc.forward(lgn2, bkg2, state=st1)
    assert oz.sum() > 0
    rng = np.random.default_rng(23)
    gz = rng.normal(0, 1, oz.shape).astype(np.float32)
    gv = rng.normal(0, 0.1, oz.shape).astype(np.float32)

    cell = V1Column(net, mode="deterministic", train_recurrent_per_type=False, train_input=True, **_cell_kw(p))
    dev = "cuda"
    leaves = {k: torch.tensor(st1[k], device=dev).requires_grad_(True)
              for k in ("zbuf", "v", "asc", "psc_rise", "psc")}
    state = (leaves["zbuf"], leaves["v"], torch.tensor(st1["r"].astype(np.int8), device=dev), leaves["asc"],
             leaves["psc_rise"], leaves["psc"], torch.zeros(B, dtype=torch.int32, device=dev))
    loss = torch.zeros((), device=dev)
    zs, vs = [], []
    for t in range(T2):
        (z, v), state = cell.call(torch.tensor(lgn2[t], dtype=torch.float32, device=dev), state,
                                  bkg_counts=torch.tensor(bkg2[t], device=dev))
        loss = loss + (z * torch.tensor(gz[t], device=dev)).sum() + (v * torch.tensor(gv[t], device=dev)).sum()
        zs.append(z.detach())
        vs.append(v.detach())
    assert state[2].dtype == torch.int8
    loss.backward()
    np.testing.assert_array_equal(torch.stack(zs).cpu().numpy().astype(np.uint8), oz)
    np.testing.assert_array_equal(torch.stack(vs).cpu().numpy().view(np.uint32), ov.view(np.uint32))
    got_w = {"rec": cell.recurrent_weight_values.grad, "lgn": cell.input_weight_values.grad,
             "bkg": cell.bkg_input_weights.grad}
    got_w = {k: g.cpu().numpy() for k, g in got_w.items()}
    got_s = {k: leaves[k].grad.cpu().numpy() for k in leaves}

    s0 = {k: st1[k].astype(np.float64) for k in st1}
    tg, tv, tg0 = torch_ref.bptt(tb, lgn2, bkg2, oz, gz, gv, state0=s0, state_grad=True, **p)
    assert np.max(np.abs(tv - ov)) < 1e-5
    sw, _, ss0 = torch_ref.bptt(tb, lgn2, bkg2, oz, gz, gv, state0=s0, state_grad=True, psi_v=ov, absolute=True,
                                **p)
    for k in ("rec", "lgn", "bkg"):
        assert np.max(np.abs(tg[k])) > 0, k
        print(name, k, error_summary(got_w[k], tg[k], sw[k]))
        assert_grads_per_element(got_w[k], tg[k], sw[k], what=f"{name} dW {k}")
    for k in ("zbuf", "v", "asc", "psc_rise", "psc"):
        assert np.max(np.abs(tg0[k])) > 0, k
        print(name, "initial", k, error_summary(got_s[k], tg0[k], ss0[k]))
        assert_grads_per_element(got_s[k], tg0[k], ss0[k], what=f"{name} d(initial {k})")

    # the fused rollout's BPTT of the same loop (from the same carried state) gives the same dW
    st_dev = [torch.tensor(st1[k], device=dev) for k in ("zbuf", "v")] + \
        [torch.tensor(st1["r"].astype(np.int16), device=dev)] + \
        [torch.tensor(st1[k], device=dev) for k in ("asc", "psc_rise", "psc")]
    cell.rollout(lgn2, bkg2, state=st_dev)
    g = cell.backward(gz=torch.tensor(gz, device=dev), gv=torch.tensor(gv, device=dev))
    og_scale = bptt_abs_scale(tb, lgn2, bkg2, oz, oref, ov, gz_loss=gz, gv_loss=gv, zbuf0=st1["zbuf"], **{
        k: p[k] for k in ("vgd", "rd", "gauss_std", "damp", "pseudo_gauss", "hard_reset")})
    for k in ("rec", "lgn", "bkg"):
        assert_grads_per_element(got_w[k], g[k].cpu().numpy(), og_scale[k], what=f"{name} loop vs rollout {k}")


def test_step_backward_of_one_call_alone():
    """One call's gradients given dL/d(new state) only (no output loss): the adjoint of the
    step on its own, against the float64 restatement of that one step."""
    from v1_glif_model_amd.models import V1Column
    p = PARAMS["gauss_sym"]
    cfg = tiny_config(n=150, fanin=15, rs=2.0, ins=3.0)
    net, tb = network(cfg, seed=31, dense_basis=True)
    B = 2
    lgn, bkg = sy.make_inputs(cfg, seed=32, seq_len=31, batch=B)
    oc = OracleCell(tb, **p)
    _, _, _, st = oc.forward(lgn[:30], bkg[:30])
    oz, ov, _, st_new = oc.forward(lgn[30:], bkg[30:], state=st)
    cell = V1Column(net, mode="deterministic", train_recurrent_per_type=False, train_input=True, **_cell_kw(p))
    dev = "cuda"
    leaves = {k: torch.tensor(st[k], device=dev).requires_grad_(True) for k in ("zbuf", "v", "asc", "psc_rise", "psc")}
    state = (leaves["zbuf"], leaves["v"], torch.tensor(st["r"].astype(np.int8), device=dev), leaves["asc"],
             leaves["psc_rise"], leaves["psc"], torch.zeros(B, dtype=torch.int32, device=dev))
    (z, v), new = cell.call(torch.tensor(lgn[30], dtype=torch.float32, device=dev), state,
                            bkg_counts=torch.tensor(bkg[30], device=dev))
    rng = np.random.default_rng(33)
    g_new = {k: rng.normal(0, 1, st[k].shape).astype(np.float32) for k in ("zbuf", "v", "asc", "psc_rise", "psc")}
    idx = {"zbuf": 0, "v": 1, "asc": 3, "psc_rise": 4, "psc": 5}
    loss = sum((new[idx[k]] * torch.tensor(g_new[k], device=dev)).sum() for k in idx)
    loss.backward()
    # float64 closed forms of the step's adjoint (the kernel comment's equations, from models.py)
    N, D, nb = tb.n_neurons, tb.max_delay, tb.n_basis
    decay = tb.decay.astype(np.float64)
    cf = tb.current_factor.astype(np.float64)
    ad = tb.asc_decay.reshape(-1).astype(np.float64)
    sd = tb.syn_decay.astype(np.float64)
    dtsd = (np.float64(tb.dt) * sd)
    vnew = ov[0].astype(np.float64)
    refr = st_new["r"] > 0
    vsc = vnew - 1.0
    psi = np.exp(-vsc * vsc / p["gauss_std"] ** 2) * p["damp"]
    gV = np.where(refr, 0.0, g_new["zbuf"][:, :N] * psi) + g_new["v"]
    gc = (gV * cf)
    exp_v = gV * decay * (1 - p["vgd"])
    exp_asc = g_new["asc"] * ad[None] + np.repeat(gc, 2, axis=1)
    gPn = g_new["psc"].reshape(B, N, nb)
    gRn = g_new["psc_rise"].reshape(B, N, nb)
    exp_P = (gPn * sd + gc[:, :, None]).reshape(B, -1)
    exp_R = (gRn * sd + gPn * dtsd).reshape(B, -1)
    for k, e in (("v", exp_v), ("asc", exp_asc), ("psc", exp_P), ("psc_rise", exp_R)):
        a = leaves[k].grad.cpu().numpy()
        np.testing.assert_allclose(a, e, rtol=1e-5, atol=1e-6, err_msg=k)
    # the spike buffer: the shifted slots plus rd times the op's dz of dy = (gR' p0) lr
    from oracle import cpu as orc
    dy = (gRn * tb.psc_initial.astype(np.float64) * tb.lr_scale).reshape(B * N, nb).astype(np.float32)
    dz, _ = orc.syn_bwd(tb.rec, st["zbuf"], tb.basis, dy)
    exp_zb = p["rd"] * dz.astype(np.float64)
    exp_zb[:, :-N] += g_new["zbuf"][:, N:]
    np.testing.assert_allclose(leaves["zbuf"].grad.cpu().numpy(), exp_zb, rtol=1e-5,
                               atol=1e-5 * np.abs(exp_zb).max())


@pytest.mark.parametrize("i", [0, 1, 3, 4, 7, 9])
def test_call_loop_gradients_irregular_shapes(i):
    """The per-step backward over the shape sweep's irregular networks (1-200 neurons, 1-9 delay
    slots, 1-8 receptors, 1-20 types, batch 1-17, both surrogates; case 9 has one delay slot, so
    the spike buffer has no shifted slots): a loop of calls from rest, its weight gradients and
    the gradients of its initial state against the float64 restatement, within both bars."""
    from tests.test_gpu_shapes import _case
    from v1_glif_model_amd.models import V1Column
    net, tb, lgn, bkg, kw, ckw = _case(i)
    T, B = lgn.shape[:2]
    T = min(T, 12)
    lgn, bkg = lgn[:T], bkg[:T]
    oc = OracleCell(tb, **kw)
    oz, ov, _, _ = oc.forward(lgn, bkg)
    rng = np.random.default_rng(300 + i)
    gz = rng.normal(0, 1, oz.shape).astype(np.float32)
    gv = rng.normal(0, 0.1, oz.shape).astype(np.float32)
    cell = V1Column(net, mode="deterministic", train_recurrent_per_type=False, train_input=True, **ckw)
    dev = "cuda"
    st0 = oc.zero_state(B)
    leaves = {k: torch.tensor(st0[k], device=dev).requires_grad_(True) for k in ("zbuf", "v", "asc", "psc_rise", "psc")}
    state = (leaves["zbuf"], leaves["v"], torch.tensor(st0["r"].astype(np.int8), device=dev), leaves["asc"],
             leaves["psc_rise"], leaves["psc"], None)
    loss = torch.zeros((), device=dev)
    zs = []
    for t in range(T):
        (z, v), state = cell.call(torch.tensor(lgn[t], dtype=torch.float32, device=dev), state,
                                  bkg_counts=torch.tensor(bkg[t], device=dev))
        loss = loss + (z * torch.tensor(gz[t], device=dev)).sum() + (v * torch.tensor(gv[t], device=dev)).sum()
        zs.append(z.detach())
    loss.backward()
    np.testing.assert_array_equal(torch.stack(zs).cpu().numpy().astype(np.uint8), oz)
    s0 = {k: st0[k].astype(np.float64) for k in st0}
    tg, _, tg0 = torch_ref.bptt(tb, lgn, bkg, oz, gz, gv, state0=s0, state_grad=True, **kw)
    sw, _, ss0 = torch_ref.bptt(tb, lgn, bkg, oz, gz, gv, state0=s0, state_grad=True, psi_v=ov, absolute=True,
                                **kw)
    got_w = {"rec": cell.recurrent_weight_values.grad, "lgn": cell.input_weight_values.grad,
             "bkg": cell.bkg_input_weights.grad}
    for k in ("rec", "lgn", "bkg"):
        assert_grads_per_element(got_w[k].cpu().numpy(), tg[k], sw[k], what=f"case {i} dW {k}")
    for k in ("zbuf", "v", "asc", "psc_rise", "psc"):
        assert_grads_per_element(leaves[k].grad.cpu().numpy(), tg0[k], ss0[k], what=f"case {i} d(initial {k})")
