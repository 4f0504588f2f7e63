"""V1Column: the GLIF_3 recurrent cell of `v1_model_utils/models.py:450-1135` on libglif.

Same constructor arguments, state tuple, per-step ``call`` and Keras-RNN-style
rollout as the reference; the T-step loop and its BPTT run as HIP kernels on one
stream (libglif ``glif_cell_forward`` / ``glif_cell_backward``).

Differences from the reference, by necessity:
* ``tau_basis`` and ``synaptic_basis_weights`` come from the network dictionary
  (keys ``tau_basis`` / ``basis``) instead of ``synaptic_data/tau_basis.npy`` and the
  network's pickle (models.py:518, 614-622).
* The background Poisson counts are an input (``bkg`` tensors): TF's stateless
  Poisson stream (models.py:865-887) cannot be reproduced.  ``call`` draws them from
  the device Philox sampler (``inputs.poisson``) when they are not given.
* The kernels keep the refractory counter as int16.  ``zero_state`` returns the
  reference's dtype (int8, or int16 when some t_ref exceeds 127 steps, models.py:574-583,
  1050), and a rollout from an int8 state widens it on entry and writes the counter back
  into the caller's int8 tensor.
"""
from __future__ import annotations

import ctypes as C
import weakref
from typing import Optional

import numpy as np
import torch

from . import _lib
from ._lib import check, lib, ptr, stream_ptr
from .ops import MODES, SynapseTable
from .tables import build_cell_tables, trainable_populations

__all__ = ["V1Column", "RSNNRollout", "Rollout"]


class V1Column:
    """models.py:450 V1Column with the same keyword arguments (plus ``mode``)."""

    def __init__(self, network, lgn_input=None, bkg_input=None, dt=1.0, gauss_std=0.5,
                 dampening_factor=0.3, recurrent_dampening_factor=0.5,
                 voltage_gradient_dampening=0.5, input_weight_scale=1.0, recurrent_weight_scale=1.0,
                 lr_scale=1.0, spike_gradient=False, max_delay=0, batch_size=1, bkg_firing_rate=250,
                 pseudo_gauss=False, train_recurrent=True, train_recurrent_per_type=True,
                 train_input=False, train_noise=True, noise_seed=0, hard_reset=False,
                 current_input=False, mode: str = "event", device="cuda"):
        _lib.require_gpu()
        if current_input:
            raise NotImplementedError("current_input (firing-probability LGN input) is not on the hot path")
        if mode not in MODES:
            raise ValueError(f"mode must be one of {sorted(MODES)}")
        net = network if "network" in network else dict(network=network, lgn_input=lgn_input,
                                                          bkg_input=bkg_input)
        self.tables = tb = build_cell_tables(net, dt=dt, max_delay=max_delay, lr_scale=lr_scale,
                                             recurrent_weight_scale=recurrent_weight_scale,
                                             input_weight_scale=input_weight_scale)
        self.device = _concrete_device(device)
        self.mode = mode
        self._n_neurons, self.max_delay, self._n_syn_basis = tb.n_neurons, tb.max_delay, tb.n_basis
        self.input_dim = tb.lgn.n_cols
        self.n_bkg = tb.bkg.n_cols
        self._dt, self._lr_scale = float(dt), float(lr_scale)
        self._gauss_std, self._dampening_factor = float(gauss_std), float(dampening_factor)
        self._recurrent_dampening = float(recurrent_dampening_factor)
        self._voltage_gradient_dampening = float(voltage_gradient_dampening)
        self._pseudo_gauss, self._hard_reset = bool(pseudo_gauss), bool(hard_reset)
        self.bkg_spike_prob = bkg_firing_rate * 0.001
        self.noise_seed = int(noise_seed)
        # models.py:577-583: int8 unless some neuron's refractory period exceeds 127 steps
        self._refractory_state_dtype = torch.int16 if int(tb.t_ref_steps.max()) > 127 else torch.int8

        self.recurrent_dense_shape = (tb.n_neurons, tb.max_delay * tb.n_neurons)
        self.rec_table = SynapseTable(tb.rec.indices, tb.rec.syn_id, self.recurrent_dense_shape,
                                      tb.basis, n_delay_slots=tb.max_delay)
        self.lgn_table = SynapseTable(tb.lgn.indices, tb.lgn.syn_id, (tb.n_neurons, tb.lgn.n_cols),
                                      tb.basis)
        self.bkg_table = SynapseTable(tb.bkg.indices, tb.bkg.syn_id, (tb.n_neurons, tb.bkg.n_cols),
                                      tb.basis)
        dev = self.device
        tr = trainable_populations(train_recurrent, train_recurrent_per_type, train_input, train_noise)
        # trainable weight vectors in reference order (models.py:663-669, 725-731, 758-764)
        self.recurrent_weight_values = torch.tensor(tb.rec.weight, device=dev).requires_grad_(tr["rec"])
        self.input_weight_values = torch.tensor(tb.lgn.weight, device=dev).requires_grad_(tr["lgn"])
        self.bkg_input_weights = torch.tensor(tb.bkg.weight, device=dev).requires_grad_(tr["bkg"])
        self._individual_training = tr["rec"]
        # sign masks for SignedConstraint (models.py:419-427)
        self.recurrent_weight_positive = torch.tensor(tb.rec.weight >= 0, device=dev)
        self.input_weight_positive = torch.tensor(tb.lgn.weight >= 0, device=dev)
        self.bkg_weight_positive = torch.tensor(tb.bkg.weight >= 0, device=dev)

        cfg = _lib.CellConfig(tb.n_neurons, tb.max_delay, tb.n_basis, float(dt), float(lr_scale),
                              float(voltage_gradient_dampening), float(recurrent_dampening_factor),
                              float(gauss_std), float(dampening_factor), int(pseudo_gauss),
                              int(hard_reset))
        self._keep = [np.ascontiguousarray(a) for a in (
            tb.decay, tb.current_factor, tb.asc_decay.reshape(-1), tb.asc_amps.reshape(-1),
            tb.t_ref_steps.astype(np.int32), tb.syn_decay, tb.psc_initial)]
        h = C.c_void_p()
        check(lib().glif_cell_create(C.byref(cfg), *[a.ctypes.data_as(C.c_void_p) for a in self._keep],
                                     self.rec_table.handle, self.lgn_table.handle,
                                     self.bkg_table.handle, C.byref(h)))
        self.handle = h
        self._ws = {}
        self._gen = 0                  # rollouts run so far
        self._ledger = WorkspaceLedger()   # which rollout last wrote each workspace
        self._last = None

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            try:
                lib().glif_cell_destroy(h)
            except Exception:
                pass
            self.handle = None

    # ---- state ---------------------------------------------------------------
    @property
    def state_size(self):
        N, D, nb = self._n_neurons, self.max_delay, self._n_syn_basis
        return (N * D, N, N, N * 2, N * nb, N * nb, ())

    def zero_state(self, batch_size, dtype=torch.float32):
        """models.py:1043-1056, r in the reference's dtype (int8; int16 above 127 steps)."""
        B, N, D, nb, dev = batch_size, self._n_neurons, self.max_delay, self._n_syn_basis, self.device
        return (torch.zeros((B, N * D), dtype=torch.float32, device=dev),
                torch.zeros((B, N), dtype=torch.float32, device=dev),
                torch.zeros((B, N), dtype=self._refractory_state_dtype, device=dev),
                torch.zeros((B, N * 2), dtype=torch.float32, device=dev),
                torch.zeros((B, N * nb), dtype=torch.float32, device=dev),
                torch.zeros((B, N * nb), dtype=torch.float32, device=dev),
                torch.zeros((B,), dtype=torch.int32, device=dev))

    def refresh_weights(self, force: bool = False):
        """refresh_recurrent_weight_shadow (models.py:966-976) for all three populations."""
        self.rec_table.set_weights(self.recurrent_weight_values, force)
        self.lgn_table.set_weights(self.input_weight_values, force)
        self.bkg_table.set_weights(self.bkg_input_weights, force)

    def g_layout(self):
        """(rows per neuron, compact) of the backward's per-synapse-type projection: compact
        when no neuron receives more than three quarters of the synapse types (the
        reference's class-pair types: 11 of 121 per neuron), each neuron then keeping rows for
        its own types only."""
        rows, compact = C.c_int32(), C.c_int32()
        check(lib().glif_cell_g_layout(self.handle, C.byref(rows), C.byref(compact)))
        return int(rows.value), bool(compact.value)

    def set_g_layout(self, compact: bool):
        """Select compact (True, when available) or type-major G rows for the next rollout and
        backward."""
        check(lib().glif_cell_set_g_layout(self.handle, int(bool(compact))))

    def workspace(self, B: int, T: int) -> torch.Tensor:
        n = int(lib().glif_cell_workspace(self.handle, int(B), int(T)))
        ws = self._ws.get("ws")
        if ws is None or ws.numel() < n:
            self._ws.clear()
            ws = torch.empty(n, dtype=torch.uint8, device=self.device)
            self._ws["ws"] = ws
        return ws

    # ---- forward ---------------------------------------------------------------
    def _prep_inputs(self, lgn, bkg):
        lgn = torch.as_tensor(lgn, device=self.device)
        bkg = torch.as_tensor(bkg, device=self.device)
        if lgn.dtype != torch.uint8:
            lgn = (lgn > 0).to(torch.uint8)
        if bkg.dtype != torch.uint8:
            if torch.any(bkg > 255):
                raise ValueError("background counts above 255")
            bkg = bkg.to(torch.uint8)
        return lgn.contiguous(), bkg.contiguous()

    def rollout(self, lgn, bkg, state=None, record_z=True, record_v=True, spike_count=None,
                mode: Optional[str] = None, ws: Optional[torch.Tensor] = None):
        """Run T steps (the Keras RNN over `call`, models.py:1317-1322).

        lgn [T, B, n_lgn] (spike where > 0), bkg [T, B, n_bkg] Poisson counts.
        Returns (z [T, B, N] or None, v [T, B, N] or None, new_state).  The state is
        updated in place (pass a copy to keep it)."""
        lgn, bkg = self._prep_inputs(lgn, bkg)
        if lgn.dim() != 3 or bkg.dim() != 3:
            raise ValueError("lgn and bkg must be [T, B, n_inputs]")
        T, B = int(lgn.shape[0]), int(lgn.shape[1])
        if lgn.shape[2] != self.input_dim or bkg.shape[:2] != lgn.shape[:2] or bkg.shape[2] != self.n_bkg:
            raise ValueError("input shapes do not match the network")
        if not 1 <= B <= 32 or T < 1:
            raise ValueError(f"batch size must be in [1, 32] and T >= 1, got B={B}, T={T}")
        if mode is not None and mode not in MODES:
            raise ValueError(f"mode must be one of {sorted(MODES)}")
        if state is None:
            state = self.zero_state(B)
        self.check_state(state, B)
        st = list(state)
        for i in range(6):
            st[i] = st[i].contiguous()
        r_caller = None
        if st[2].dtype == torch.int8:   # the reference's refractory dtype: widen for the kernels
            r_caller, st[2] = st[2], st[2].to(torch.int16)
        N = self._n_neurons
        if spike_count is not None:
            _check_tensor(spike_count, "spike_count", (B, N), (torch.int32,), self.device, contiguous=True)
        if ws is not None:
            _check_tensor(ws, "ws", None, (torch.uint8,), self.device, contiguous=True)
            if ws.numel() < int(lib().glif_cell_workspace(self.handle, B, T)):
                raise ValueError("workspace too small for this batch size and T")
        z = torch.empty((T, B, N), dtype=torch.float32, device=self.device) if record_z else None
        v = torch.empty((T, B, N), dtype=torch.float32, device=self.device) if record_v else None
        self.refresh_weights()
        if ws is None:
            ws = self.workspace(B, T)
        cstate = _lib.State(*[C.c_void_p(t.data_ptr()) for t in st[:6]])
        check(lib().glif_cell_forward(self.handle, B, T, MODES[mode or self.mode], ptr(lgn), ptr(bkg),
                                      C.byref(cstate), ptr(z), ptr(v), ptr(spike_count), ptr(ws),
                                      ws.numel(), stream_ptr(self.device)))
        if r_caller is not None:
            r_caller.copy_(st[2])
            st[2] = r_caller
        if len(st) > 6 and st[6] is not None:
            st[6] = st[6] + T
        self._gen += 1
        self._ledger.record(ws, self._gen)
        self._last = Rollout(B, T, ws, self._gen)
        return z, v, tuple(st)

    def check_state(self, state, B: int):
        """Refuse a state tuple whose tensors do not have the reference's layouts
        (models.py:1030-1056) on this cell's device: z_buf [B, N*D], v [B, N], r [B, N] int8 or
        int16, asc [B, 2N], psc_rise and psc [B, N*nb] float32, and noise_step [B] int32 when
        present.  Raises ValueError."""
        if not isinstance(state, (tuple, list)) or len(state) not in (6, 7):
            raise ValueError("state must be the 7-tuple (z_buf, v, r, asc, psc_rise, psc, noise_step)")
        N, D, nb = self._n_neurons, self.max_delay, self._n_syn_basis
        f32 = (torch.float32,)
        spec = (("z_buf", (B, N * D), f32), ("v", (B, N), f32), ("r", (B, N), (torch.int8, torch.int16)),
                ("asc", (B, 2 * N), f32), ("psc_rise", (B, N * nb), f32), ("psc", (B, N * nb), f32))
        for t, (name, shape, dtypes) in zip(state[:6], spec):
            _check_tensor(t, name, shape, dtypes, self.device)
        if len(state) == 7 and state[6] is not None:
            _check_tensor(state[6], "noise_step", (B,), (torch.int32, torch.int64), self.device)
        if state[2].dtype == torch.int8 and self._refractory_state_dtype != torch.int8:
            raise ValueError("r must be int16: some refractory period exceeds 127 steps (models.py:577-583)")

    def call(self, inputs, state, bkg_counts=None, constants=None):
        """One step (models.py:1059-1135): returns ((z, v), new_state).

        Differentiable, as the reference's step is under a GradientTape: with grad mode on and
        a weight vector or state tensor that requires grad, the step is an autograd node
        (``StepFunction``) whose backward is libglif's ``glif_step_backward``, so a loop of
        ``call``s (the Keras RNN) can be differentiated step by step.  ``rollout`` +
        ``backward`` (or ``RSNNRollout``) is the fused, faster form of the same loop."""
        B = int(inputs.shape[0])
        self.check_state(state, B)
        if bkg_counts is None:
            # the reference seeds its stateless Poisson per step with (noise_seed, step)
            # (models.py:867-887); here the step picks the offset in the noise_seed stream
            from .inputs import poisson
            step = int(state[6][0].item())
            bkg_counts = poisson(self.bkg_spike_prob, (B, self.n_bkg), self.noise_seed,
                                 offset=step * B * self.n_bkg, device=self.device)
        lgn, bkg = self._prep_inputs(inputs[:, :self.input_dim][None], torch.as_tensor(bkg_counts)[None])
        z, v, z_buf, r, asc, psc_rise, psc = StepFunction.apply(
            self, lgn[0], bkg[0], *state[:6], self.recurrent_weight_values, self.input_weight_values,
            self.bkg_input_weights)
        noise_step = state[6] + 1 if len(state) > 6 and state[6] is not None else None
        return (z, v), (z_buf, v, r, asc, psc_rise, psc, noise_step)

    __call__ = call

    # ---- backward ------------------------------------------------------------
    def check_rollout(self, rollout: Optional["Rollout"] = None) -> "Rollout":
        """The rollout record a backward or fused loss reads (default: the last rollout); raises
        if a later rollout has overwritten its workspace (saved voltages, spike bits)."""
        rec = self._last if rollout is None else rollout
        if rec is None:
            raise RuntimeError("no rollout to take the saved activations from")
        if not self._ledger.holds(rec.ws, rec.gen):
            raise RuntimeError("the workspace of this rollout was overwritten by a later rollout on the same "
                               "workspace; give each rollout that is to be differentiated its own workspace "
                               "(rollout(..., ws=...)) or run its backward first")
        return rec

    def backward(self, gz=None, gz_neuron=None, gv=None, want=("rec", "lgn", "bkg"),
                 rollout: Optional["Rollout"] = None):
        """BPTT through a rollout (default: the last one; zero initial adjoint).

        gz / gv: dL/dz, dL/dv [T, B, N] (or None); gz_neuron: dL/dz [N] broadcast over
        (t, b).  Returns dict of weight gradients in reference order."""
        rec = self.check_rollout(rollout)
        B, T, ws = rec.B, rec.T, rec.ws
        dev = self.device
        N = self._n_neurons
        for name, t, shape in (("gz", gz, (T, B, N)), ("gv", gv, (T, B, N)), ("gz_neuron", gz_neuron, (N,))):
            if t is not None:
                _check_tensor(t, name, shape, (torch.float32, torch.float64, torch.float16, torch.bfloat16), dev)
        out = {}
        for name, table in (("rec", self.rec_table), ("lgn", self.lgn_table), ("bkg", self.bkg_table)):
            out[name] = torch.empty(table.n_syn, dtype=torch.float32, device=dev) if name in want else None
        prep = lambda t: None if t is None else t.detach().contiguous().float()
        gz, gz_neuron, gv = prep(gz), prep(gz_neuron), prep(gv)
        check(lib().glif_cell_backward(self.handle, B, T, ptr(gz), ptr(gz_neuron), ptr(gv),
                                       ptr(out["rec"]), ptr(out["lgn"]), ptr(out["bkg"]), ptr(ws),
                                       ws.numel(), stream_ptr(dev)))
        return out


def _concrete_device(device) -> torch.device:
    """torch.device with an index ("cuda" -> "cuda:<current>"), so tensors compare equal."""
    dev = torch.device(device)
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


def _check_tensor(t, name, shape, dtypes, device, contiguous=False):
    """ValueError unless `t` is a tensor of one of `dtypes`, of exactly `shape` (None: any), on
    `device`, and contiguous where asked (a buffer the library writes in place); the kernels
    take its data pointer, so nothing else may reach them."""
    if not torch.is_tensor(t):
        raise ValueError(f"{name} must be a tensor, got {type(t).__name__}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, the cell's tensors on {device}")
    if t.dtype not in dtypes:
        raise ValueError(f"{name} must be {' or '.join(str(d) for d in dtypes)}, got {t.dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous (the library writes it in place)")


class WorkspaceLedger:
    """Which rollout last wrote each workspace, keyed by its device address.

    An entry lives while the tensor that wrote it does: when that tensor is freed (its
    rollouts are gone, so nothing can ask about it) the entry goes, and a later tensor at the
    same address starts a new one.  Any number of workspaces can be pending."""

    def __init__(self):
        self._last = {}    # data_ptr -> (rollout number, weakref to the workspace tensor)

    def record(self, ws: torch.Tensor, gen: int):
        key = ws.data_ptr()
        old = self._last.get(key)
        if old is None or old[1]() is not ws:
            weakref.finalize(ws, WorkspaceLedger._forget, weakref.ref(self), key)
        self._last[key] = (gen, weakref.ref(ws))

    def holds(self, ws: torch.Tensor, gen: int) -> bool:
        """True while rollout `gen` is still the last writer of `ws`."""
        entry = self._last.get(ws.data_ptr())
        return entry is not None and entry[0] == gen

    def __len__(self):
        return len(self._last)

    @staticmethod
    def _forget(ledger_ref, key):
        ledger = ledger_ref()
        if ledger is None:
            return
        entry = ledger._last.get(key)
        if entry is not None and entry[1]() is None:   # its writer is gone (not a later tensor)
            del ledger._last[key]


class Rollout:
    """What a backward needs of one rollout: its batch, length and workspace (which holds the
    saved voltages and spike bits), and the rollout's number on its cell."""
    __slots__ = ("B", "T", "ws", "gen")

    def __init__(self, B, T, ws, gen):
        self.B, self.T, self.ws, self.gen = B, T, ws, gen


class StepFunction(torch.autograd.Function):
    """Autograd node over one V1Column.call (models.py:1059-1135): (old state, weights) ->
    (z, v, new z_buf, new r, new asc, new psc_rise, new psc).  The forward is a one-tick
    rollout; the backward is ``glif_step_backward``, from the saved old spike buffer, the
    step's voltage and refractory counter and its inputs: dL/d(old state) for every state
    tensor that requires grad, and the step's weight gradients (the reference's tape through
    the step, with its straight-through dampening and stop_gradients)."""

    @staticmethod
    def forward(ctx, cell, lgn, bkg, z_buf, v, r, asc, psc_rise, psc, w_rec, w_lgn, w_bkg):
        st = [z_buf.clone(), v.clone(), r.clone(), asc.clone(), psc_rise.clone(), psc.clone()]
        z, vout, st = cell.rollout(lgn[None], bkg[None], state=st)
        z, vout = z[0], vout[0]
        ctx.cell = cell
        ctx.mark_non_differentiable(st[2])
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(z_buf, vout, st[2], lgn, bkg, w_rec, w_lgn, w_bkg)
        return z, vout, st[0], st[2], st[3], st[4], st[5]

    @staticmethod
    def backward(ctx, gz, gv, gzb, _gr, gasc, gR, gP):
        cell = ctx.cell
        z_buf, v_new, r_new, lgn, bkg, w_rec, w_lgn, w_bkg = ctx.saved_tensors
        need = ctx.needs_input_grad
        B, dev = int(v_new.shape[0]), v_new.device
        N, D, nb = cell._n_neurons, cell.max_delay, cell._n_syn_basis
        prep = lambda t: None if t is None else t.detach().contiguous().float()
        gz, gv, gzb, gasc, gR, gP = (prep(t) for t in (gz, gv, gzb, gasc, gR, gP))
        shapes = {"z_buf": (3, (B, D * N)), "v": (4, (B, N)), "asc": (6, (B, 2 * N)),
                  "psc_rise": (7, (B, N * nb)), "psc": (8, (B, N * nb))}
        g_old = {k: torch.empty(shp, dtype=torch.float32, device=dev) if need[i] else None
                 for k, (i, shp) in shapes.items()}
        dw = [torch.empty(t.n_syn, dtype=torch.float32, device=dev) if need[9 + i] else None
              for i, t in enumerate((cell.rec_table, cell.lgn_table, cell.bkg_table))]
        cell.refresh_weights()   # the saved weights' values (autograd refuses them if changed since)
        sg = lambda d: _lib.StateGrad(*[ptr(d[k]) for k in ("z_buf", "v", "asc", "psc_rise", "psc")])
        g_new = sg({"z_buf": gzb, "v": None, "asc": gasc, "psc_rise": gR, "psc": gP})
        c_old = sg(g_old)
        r16 = r_new.to(torch.int16).contiguous()
        zb = z_buf.detach().contiguous()
        n = int(lib().glif_step_workspace(cell.handle, B))
        ws = torch.empty(max(n, 1), dtype=torch.uint8, device=dev)
        # the state's v and the output v are one tensor: its gradient arrives once, as gv
        check(lib().glif_step_backward(cell.handle, B, ptr(lgn), ptr(bkg), ptr(zb),
                                       ptr(v_new), ptr(r16), ptr(gz), ptr(gv), C.byref(g_new), C.byref(c_old),
                                       ptr(dw[0]), ptr(dw[1]), ptr(dw[2]), ptr(ws), ws.numel(),
                                       stream_ptr(dev)))
        return (None, None, None, g_old["z_buf"], g_old["v"], None, g_old["asc"], g_old["psc_rise"],
                g_old["psc"], dw[0], dw[1], dw[2])


class RSNNRollout(torch.autograd.Function):
    """Autograd node over a whole rollout: weights -> (z [T,B,N], v [T,B,N]).

    Each node runs on a workspace of its own (from torch's caching allocator), so several
    rollouts, or per-step ``call``s, may run before the backward of any of them."""

    @staticmethod
    def forward(ctx, cell: V1Column, lgn, bkg, w_rec, w_lgn, w_bkg):
        T, B = int(lgn.shape[0]), int(lgn.shape[1])
        n = int(lib().glif_cell_workspace(cell.handle, B, T))
        ws = torch.empty(n, dtype=torch.uint8, device=cell.device)
        z, v, _ = cell.rollout(lgn, bkg, ws=ws)
        ctx.cell = cell
        ctx.rollout = cell._last
        ctx.want = tuple(n for n, w in (("rec", w_rec), ("lgn", w_lgn), ("bkg", w_bkg)) if w.requires_grad)
        return z, v

    @staticmethod
    def backward(ctx, gz, gv):
        g = ctx.cell.backward(gz=gz, gv=gv, want=ctx.want, rollout=ctx.rollout)
        return None, None, None, g["rec"], g["lgn"], g["bkg"]

