"""float64 PyTorch autograd restatement of V1Column.call (TEST INFRASTRUCTURE ONLY).

Pins the hand-derived BPTT of ``glif_oracle.c`` (orc_backward) and, through it, the
HIP adjoint.  Every line restates `v1_model_utils/models.py` with torch ops and lets
autograd build the reverse pass, exactly as TF's GradientTape does for the
reference:

* straight_through_dampen (models.py:284-296): ``x * (1 - d) + (x * d).detach()``;
* the spike buffer is dampened with ``1 - recurrent_dampening`` before the
  synaptic op (models.py:1081);
* calculate_synaptic_currents (models.py:103-263): for binary spikes its custom
  gradient equals autograd of the bilinear form sum_syn z[b, col] W basis[syn_id, r]
  (dense dz over all synapses, dW over active events only), which is used here;
  the background source multiplies by the Poisson count (models.py:917-931);
* _dense_update_impl (models.py:985-1028) with stop_gradient on prev_z and r;
* spike_function / spike_gauss (models.py:17-66) with the refractory ``tf.where``
  (models.py:1113-1114).

Spikes are teacher-forced to a given train (the CPU oracle's) so the float64 graph
follows the same trajectory as the float32 run it checks; the surrogate is still
evaluated on this run's own voltage (or on given voltages, ``psi_v``).

The rollout may start from a given state and also return the gradients of that initial
state (what the reference's tape gives for the RNN's initial state), and with
``absolute=True`` every signed factor (weights, basis entries, loss gradients) is replaced by
its absolute value, so each returned gradient is the sum of the absolute values of its terms:
the scale fp32 rounding in any summation order is proportional to.
"""
from __future__ import annotations

import numpy as np
import torch


class _SpikeForced(torch.autograd.Function):
    @staticmethod
    def forward(ctx, v_sc, z, pseudo_gauss, sigma, amp, v_sc_psi=None):
        ctx.save_for_backward(v_sc if v_sc_psi is None else v_sc_psi)
        ctx.p = (pseudo_gauss, sigma, amp)
        return z.clone()

    @staticmethod
    def backward(ctx, dy):
        (v_sc,) = ctx.saved_tensors
        pseudo_gauss, sigma, amp = ctx.p
        if pseudo_gauss:
            psi = torch.exp(-torch.square(v_sc) / (sigma * sigma)) * amp      # models.py:17-21
        else:
            psi = amp * torch.clamp(1.0 - torch.abs(v_sc), min=0.0)           # models.py:23-28
        return dy * psi, None, None, None, None, None


def _st_dampen(x, d):
    d = min(max(float(d), 0.0), 1.0)
    return x * (1.0 - d) + (x * d).detach()


def _syn(z_src, table, w, basis, B, N, nb):
    """sum over synapses of z_src[b, col] * w * basis[syn_id, :], scattered to post."""
    col = torch.as_tensor(table.col)
    post = torch.as_tensor(table.post)
    bs = basis[torch.as_tensor(table.syn_id.astype(np.int64))]           # [S, nb]
    contrib = (z_src[:, col] * w[None, :])[:, :, None] * bs[None]       # [B, S, nb]
    out = torch.zeros((B, N, nb), dtype=torch.float64)
    return out.index_add(1, post, contrib)


def bptt(tb, lgn, bkg, z_forced, gz, gv, vgd=0.5, rd=0.5, gauss_std=0.5, damp=0.5,
         pseudo_gauss=True, hard_reset=False, zbuf0=None, state0=None, state_grad=False, psi_v=None,
         absolute=False):
    """Returns ({'rec','lgn','bkg'}: dL/dW float64 arrays, v [T,B,N]) for
    L = sum(z * gz) + sum(v * gv), from a zero state with the spike history zbuf0 [B, D*N]
    (None: no spikes), or from state0 (dict of the state tuple's arrays in the reference
    layouts: zbuf, v, r, asc, psc_rise, psc).  The history's spikes are inputs; with
    state_grad a third dict holds dL/d(initial state) for zbuf, v, asc, psc_rise, psc, in the
    same layouts (the gradient that flows into the initial spike buffer included).  psi_v
    [T,B,N]: voltages the surrogate is evaluated at (default: this run's); absolute: every
    signed factor by its absolute value (the sum-of-absolute-terms scale)."""
    T, B = lgn.shape[:2]
    N, D, nb = tb.n_neurons, tb.max_delay, tb.n_basis
    f = lambda a: torch.tensor(np.asarray(a, dtype=np.float64))
    fa = (lambda a: torch.tensor(np.abs(np.asarray(a, dtype=np.float64)))) if absolute else f
    W = {k: fa(getattr(tb, k).weight).requires_grad_(True) for k in ("rec", "lgn", "bkg")}
    basis = fa(tb.basis)
    decay, cf = f(tb.decay), f(tb.current_factor)
    ad, amp = f(tb.asc_decay), f(tb.asc_amps)
    tref = torch.tensor(tb.t_ref_steps.astype(np.int64))
    sd, p0 = f(tb.syn_decay), f(tb.psc_initial)
    dt, lr = tb.dt, tb.lr_scale
    zf = torch.tensor(np.asarray(z_forced, dtype=np.float64))
    x_lgn = torch.tensor((np.asarray(lgn) > 0).astype(np.float64))
    x_bkg = torch.tensor(np.asarray(bkg).astype(np.float64))
    vpsi = None if psi_v is None else torch.tensor(np.asarray(psi_v, dtype=np.float64)) - 1.0

    z_buf = torch.zeros((B, D * N), dtype=torch.float64)
    if zbuf0 is not None:
        z_buf = torch.tensor(np.asarray(zbuf0, dtype=np.float64))
    v = torch.zeros((B, N), dtype=torch.float64)
    r = torch.zeros((B, N), dtype=torch.int64)
    asc = torch.zeros((B, N, 2), dtype=torch.float64)
    R = torch.zeros((B, N, nb), dtype=torch.float64)
    P = torch.zeros((B, N, nb), dtype=torch.float64)
    if state0 is not None:
        z_buf, v = f(state0["zbuf"]).reshape(B, D * N), f(state0["v"]).reshape(B, N)
        r = torch.tensor(np.asarray(state0["r"]).astype(np.int64)).reshape(B, N)
        asc = f(state0["asc"]).reshape(B, N, 2)
        R, P = f(state0["psc_rise"]).reshape(B, N, nb), f(state0["psc"]).reshape(B, N, nb)
    leaves = {}
    if state_grad:
        leaves = {"zbuf": z_buf.clone().requires_grad_(True), "v": v.clone().requires_grad_(True),
                  "asc": asc.clone().requires_grad_(True), "psc_rise": R.clone().requires_grad_(True),
                  "psc": P.clone().requires_grad_(True)}
        z_buf, v, asc, R, P = (leaves[k] for k in ("zbuf", "v", "asc", "psc_rise", "psc"))
    loss = torch.zeros((), dtype=torch.float64)
    vs = []
    gz_t, gv_t = fa(gz), fa(gv)
    for t in range(T):
        prev_z = z_buf[:, :N]
        rec_z_buf = _st_dampen(z_buf, 1.0 - rd)
        i_rec = _syn(rec_z_buf, tb.rec, W["rec"], basis, B, N, nb)
        i_lgn = _syn(x_lgn[t], tb.lgn, W["lgn"], basis, B, N, nb)
        i_bkg = _syn(x_bkg[t], tb.bkg, W["bkg"], basis, B, N, nb)
        rec_inputs = (i_rec + i_lgn + i_bkg) * lr
        new_R = R * sd + rec_inputs * p0
        new_P = P * sd + dt * sd * R
        new_asc = ad[None] * asc + prev_z.detach()[:, :, None] * amp[None]
        c1 = P.sum(-1) + asc.sum(-1)
        new_v = decay * _st_dampen(v, vgd) + cf * c1 - prev_z.detach()
        new_r = torch.clamp(r + prev_z.detach().long() * tref - 1, min=0)
        if hard_reset:
            new_v = torch.where(new_r > 0, torch.zeros_like(new_v), new_v)
        z = _SpikeForced.apply(new_v - 1.0, zf[t], pseudo_gauss, gauss_std, damp,
                               None if vpsi is None else vpsi[t])
        z = torch.where(new_r > 0, torch.zeros_like(z), z)
        z_buf = torch.cat([z, z_buf[:, :-N]], dim=1)
        loss = loss + (z * gz_t[t]).sum() + (new_v * gv_t[t]).sum()
        vs.append(new_v.detach())
        v, r, asc, R, P = new_v, new_r, new_asc, new_R, new_P
    loss.backward()
    dw = {k: W[k].grad.numpy() for k in W}
    if not state_grad:
        return dw, torch.stack(vs).numpy()
    g0 = {k: (t.grad if t.grad is not None else torch.zeros_like(t)).reshape(B, -1).numpy()
          for k, t in leaves.items()}
    return dw, torch.stack(vs).numpy(), g0
