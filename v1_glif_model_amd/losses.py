"""Losses on the cell's outputs, fused with the GLIF_3 path (loss_functions.py).

``SpikeRateDistributionTarget`` (loss_functions.py:782-889): per cell-type population,
the Huber quantile loss between the sorted model rates and sorted target rates sampled
from recorded per-type rates.  One libglif call turns the forward's spike counts into the
loss and a per-neuron dL/dz, which ``V1Column.backward(gz_neuron=...)`` broadcasts over
the (trimmed) ticks, so no [T, B, N] spike gradient has to exist.

``VoltageRegularization`` (loss_functions.py:1047-1119): the penalty of the cell's output
voltages, "range" relu(|v - 0.5| - 0.5)^2 or "threshold" (v - 1)^2, cost * mean over
(B, T, N) -- over the core-mask neurons only when a ``core_mask`` is given.  Two forms:

* ``reg()`` (fused): the loss of the cell's last rollout is reduced from the voltages the
  cell keeps for BPTT, and the next ``V1Column.backward`` adds the gradient inside the
  adjoint, so no [T, B, N] voltage tensor has to exist;
* ``reg(voltages)``: the reference's form on a voltage tensor (e.g. the ``v`` output of
  ``RSNNRollout``), differentiated by autograd, which hands dL/dv to the backward as ``gv``.
  This call switches the fused gradient off, so the gradient is never applied twice.

Constructing the object selects the fused form; it is switched off again when the object
is deleted or ``disable()`` is called.
"""
from __future__ import annotations

import ctypes as C
from typing import Dict, Optional

import numpy as np
import torch

from ._lib import check, lib, ptr, stream_ptr

__all__ = ["VoltageRegularization", "SpikeRateDistributionTarget", "RateMSE", "CELL_TYPE_ORDER",
           "population_neuron_ids", "sample_firing_rates", "load_neuropixels_type_rates",
           "neuropixels_cell_type_to_cell_type"]

# loss_functions.py:724-743 (the values of CELL_TYPE_QUERY_MAPPING, in its order)
CELL_TYPE_ORDER = ("L1 Htr3a", "L2/3 Exc", "L2/3 PV", "L2/3 SST", "L2/3 VIP", "L4 Exc", "L4 PV",
                   "L4 SST", "L4 VIP", "L5 Exc", "L5 PV", "L5 SST", "L5 VIP", "L6 Exc", "L6 PV",
                   "L6 SST", "L6 VIP")

_MODES = {"range": 1, "threshold": 2}


class VoltageRegularization:
    """The cell holds one fused voltage loss: the regularizer that claimed it last (by being
    constructed, or by a fused ``reg()`` call) owns it, and only the owner switches it off
    (``disable()``, or when it is deleted).  A fused ``reg()`` re-claims it, with this object's
    penalty, cost and core mask, if another regularizer took it meanwhile."""

    def __init__(self, cell, voltage_cost=1e-5, dtype=torch.float32, core_mask=None, penalty_mode="range"):
        self._cell = None
        self._tok = object()   # the marker the cell keeps of its owner (it does not keep this object alive)
        if penalty_mode not in _MODES:
            raise ValueError("penalty_mode must be 'range' or 'threshold'")
        self._cell = cell
        self._voltage_cost = float(voltage_cost)
        self._penalty_mode = penalty_mode
        self._core_mask = None
        self._mask_u8 = None
        self._fused = False
        if core_mask is not None:
            m = torch.as_tensor(core_mask, device=cell.device).to(torch.bool).reshape(-1)
            if m.numel() != cell._n_neurons or not bool(m.any()):
                raise ValueError("core_mask must select at least one of the cell's neurons")
            self._core_mask = m
            self._mask_u8 = m.to(torch.uint8).contiguous()   # kept alive while this object owns the loss
        self._claim()

    def _owns(self) -> bool:
        cell = self._cell
        return cell is not None and getattr(cell, "_vloss_owner", None) is self._tok

    def _claim(self):
        """Enable the fused loss on the cell with this object's penalty, cost and mask."""
        cell = self._cell
        n_sel = int(self._core_mask.sum().item()) if self._core_mask is not None else 0
        check(lib().glif_cell_set_voltage_mask(cell.handle, ptr(self._mask_u8), n_sel))
        check(lib().glif_cell_set_voltage_loss(cell.handle, _MODES[self._penalty_mode], self._voltage_cost))
        cell._vloss_owner = self._tok
        cell._vloss_mask_ref = self._mask_u8
        self._fused = True

    def _release(self):
        """Switch the fused loss off, if this object still owns it."""
        cell = self._cell
        if self._owns() and getattr(cell, "handle", None) is not None:
            check(lib().glif_cell_set_voltage_loss(cell.handle, 0, 0.0))
            check(lib().glif_cell_set_voltage_mask(cell.handle, None, 0))
            cell._vloss_owner = None
            cell._vloss_mask_ref = None
        self._fused = False

    def disable(self):
        """Switch the fused gradient off (if this object still owns it) and detach from the cell."""
        if getattr(self, "_cell", None) is None:
            return
        self._release()
        self._cell = None

    def __del__(self):
        try:
            self.disable()
        except Exception:
            pass

    @staticmethod
    def penalty(v, mode="range"):
        """Elementwise penalty (the reference's _compute_range_loss / _compute_threshold_loss)."""
        if mode == "range":
            return torch.square(torch.relu(torch.abs(v - 0.5) - 0.5))
        return torch.square(v - 1.0)

    def __call__(self, voltages=None):
        """Loss of ``voltages`` [T, B, N] if given, else (fused) of the cell's last rollout."""
        cell = self._cell
        if cell is None:
            raise RuntimeError("this VoltageRegularization was disabled")
        if voltages is not None:
            # autograd carries this gradient (as gv): the fused one must not be added too
            if self._fused:
                self._release()
            if self._core_mask is not None:
                voltages = voltages[:, :, self._core_mask]   # tf.boolean_mask(..., axis=2)
            return self.penalty(voltages, self._penalty_mode).mean() * self._voltage_cost
        if not self._fused or not self._owns():
            self._claim()
        rec = cell.check_rollout()
        out = torch.empty((), dtype=torch.float32, device=cell.device)
        check(lib().glif_cell_voltage_loss(cell.handle, rec.B, rec.T, ptr(out), ptr(rec.ws), rec.ws.numel(),
                                           stream_ptr(cell.device)))
        return out


# ------------------------------------------------------------ rate distribution ----
def neuropixels_cell_type_to_cell_type(name):
    """loss_functions.py:702-721: 'EXC_L23' -> 'L2/3 Exc', 'PV_L5' -> 'L5 PV', 'x_L1' ->
    'L1 Htr3a', 'Htr3a_L4' -> 'L4 VIP'; names that contain a space pass through."""
    if not isinstance(name, str) or " " in name:
        return name
    cls, layer = name.split("_")[0], name.split("_")[1]
    if "2" in layer:
        layer = "L2/3"
    elif layer == "L1":
        return "L1 Htr3a"
    cls = {"EXC": "Exc", "Htr3a": "VIP"}.get(cls, cls)
    return f"{layer} {cls}"


def sample_firing_rates(firing_rates, n_neurons, rnd_seed):
    """loss_functions.py:613-624: n_neurons inverse-transform samples of the empirical CDF
    of `firing_rates` (RandomState(rnd_seed) uniforms through np.interp), sorted."""
    s = np.sort(np.asarray(firing_rates))
    percentiles = np.linspace(0, 1, s.size)
    x = np.random.RandomState(seed=rnd_seed).uniform(low=0, high=1, size=n_neurons)
    return np.sort(np.interp(x, percentiles, s))


def load_neuropixels_type_rates(path, stimulus_type="drifting_gratings"):
    """Per cell type recorded rates in spikes/ms with a 0 appended
    (SpikeRateDistributionTarget.get_neuropixels_firing_rates, loss_functions.py:808-858):
    a space-separated table with columns ecephys_unit_id, cell_type, firing_rate_sp (or
    Spont_Rate(Hz)) and Ave_Rate(Hz)."""
    import pandas as pd
    feature = _rate_feature(stimulus_type)
    cols = ["ecephys_unit_id", "cell_type", "firing_rate_sp", "Ave_Rate(Hz)"]
    try:
        df = pd.read_csv(path, index_col=0, sep=" ", usecols=cols).dropna(how="all")
    except ValueError:
        cols = ["ecephys_unit_id", "cell_type", "Spont_Rate(Hz)", "Ave_Rate(Hz)"]
        df = pd.read_csv(path, index_col=0, sep=" ", usecols=cols).dropna(how="all")
        df = df.rename(columns={"Spont_Rate(Hz)": "firing_rate_sp"})
    df["cell_type"] = df["cell_type"].apply(neuropixels_cell_type_to_cell_type)
    return {ct: np.append(sub[feature].dropna().values / 1000, 0) for ct, sub in df.groupby("cell_type")}


def _rate_feature(stimulus_type):
    """loss_functions.py:796-810."""
    if stimulus_type in ("spontaneous", "gray"):
        return "firing_rate_sp"
    if stimulus_type in ("natural_stimuli", "natural_images"):
        return "firing_rate_ns"
    if stimulus_type == "drifting_gratings":
        return "Ave_Rate(Hz)"
    raise ValueError(f"Unknown stimulus_type: {stimulus_type}. Choose among 'spontaneous/gray', "
                     "'drifting_gratings', or 'natural_stimuli'.")


def population_neuron_ids(cell_types, core_mask=None, reindex_selected=False):
    """get_population_neuron_ids (loss_functions.py:759-779) from per-neuron cell-type
    labels: {cell type: int32 ids of the selected neurons of that type}, CELL_TYPE_ORDER."""
    cell_types = np.asarray(cell_types)
    mask = np.ones(cell_types.size, bool) if core_mask is None else np.asarray(core_mask, bool)
    if mask.shape != cell_types.shape:
        raise ValueError("core_mask must have one entry per neuron")
    sel = (np.arange(np.count_nonzero(mask), dtype=np.int32) if reindex_selected
           else np.flatnonzero(mask).astype(np.int32))
    sel_types = cell_types[mask]
    return {ct: sel[sel_types == ct] for ct in CELL_TYPE_ORDER}


class SpikeRateDistributionTarget:
    """loss_functions.py:782-889.

    network: the network dictionary; its ``cell_type`` labels (one per neuron) give the
    populations, or pass ``populations`` {cell type: ids} directly.  The recorded per-type
    rates come from ``neuropixels_df`` (a path, see ``load_neuropixels_type_rates``) or
    from ``type_rates`` {cell type: rates in spikes/ms}.  Targets per population:
    ``rates_dampening * sample_firing_rates(rates, n_k, seed)``.

    ``cell`` (a V1Column) makes the forward count spikes over the trimmed ticks
    [pre_delay, T - post_delay) and its backward broadcast gz_neuron over those ticks.
    Each call draws a fresh tie order among equal rates (tf.random.shuffle in the
    reference) from a Philox stream keyed by ``shuffle_seed``.
    """

    def __init__(self, network=None, stimulus_type="drifting_gratings", rate_cost=0.5, pre_delay=None,
                 post_delay=None, data_dir=None, core_mask=None, rates_dampening=1.0, seed=42,
                 dtype=torch.float32, neuropixels_df=None, populations: Optional[Dict] = None,
                 type_rates: Optional[Dict] = None, cell=None, kappa=0.002, shuffle_seed=0,
                 device="cuda", **kwargs):
        # deprecated flags of the reference map to a stimulus type (loss_functions.py:796-801)
        if kwargs.get("spontaneous_fr"):
            stimulus_type = "spontaneous"
        elif kwargs.get("natural_images"):
            stimulus_type = "natural_stimuli"
        _rate_feature(stimulus_type)  # validates it
        if dtype != torch.float32:
            raise NotImplementedError("the rate loss computes in float32")
        self._rate_cost = float(rate_cost)
        self._pre_delay, self._post_delay = pre_delay, post_delay
        self._kappa = float(kappa)
        self._seed = seed
        self.device = torch.device(device)
        if populations is None:
            if network is None:
                raise ValueError("pass a network with cell_type labels or populations")
            net = network.get("network", network)
            if "cell_type" not in net:
                raise ValueError("the network has no per-neuron cell_type labels; pass populations")
            populations = population_neuron_ids(net["cell_type"], core_mask)
            self._n_neurons = int(net["n_nodes"])
        else:
            self._n_neurons = None
        if type_rates is None:
            if neuropixels_df is None:
                raise ValueError("pass neuropixels_df (a path) or type_rates")
            type_rates = load_neuropixels_type_rates(neuropixels_df, stimulus_type)
        self.populations = {}
        self.target_rates = {}
        ids, ptrs, tgts = [], [0], []
        for ct in CELL_TYPE_ORDER:
            nid = np.asarray(populations.get(ct, np.zeros(0, np.int32)), np.int32)
            rates = type_rates.get(ct, np.array([0.0], dtype=np.float32))
            tgt = (rates_dampening * sample_firing_rates(rates, nid.size, seed)).astype(np.float32)
            self.populations[ct] = nid
            self.target_rates[ct] = dict(rates=rates, neuron_ids=nid, sorted_target_rates=tgt)
            ids.append(nid)
            tgts.append(tgt)
            ptrs.append(ptrs[-1] + nid.size)
        ids = np.concatenate(ids)
        if ids.size == 0:
            raise ValueError("no neuron selected")
        if np.unique(ids).size != ids.size:
            raise ValueError("a neuron belongs to more than one population")
        if self._n_neurons is None:
            self._n_neurons = int(ids.max()) + 1
        self._pop_ptr = (C.c_int32 * len(ptrs))(*ptrs)
        self._n_pop = len(ptrs) - 1
        self._ids = torch.tensor(ids, dtype=torch.int32, device=self.device)
        self._targets = torch.tensor(np.concatenate(tgts), dtype=torch.float32, device=self.device)
        self._n_sel = int(ids.size)
        self._shuffle_seed = int(shuffle_seed)
        self._offset = 0
        self._ws = None
        self._cell = cell
        if cell is not None:
            check(lib().glif_cell_set_trim(cell.handle, int(pre_delay or 0), int(post_delay or 0)))
        self.gz_neuron = None

    def _window(self, T):
        pre = int(self._pre_delay or 0)
        post = int(self._post_delay or 0)
        return pre, T - post

    def __call__(self, spikes=None, trim=True, spike_count=None, T=None, gz_neuron=None, shuffle=True):
        """Loss of ``spikes`` [T, B, N] (trimmed here as spike_trimming, loss_functions.py:
        604-611), or of ``spike_count`` [B, N] int32 that a forward of ``T`` ticks counted over
        the trimmed ticks (the fused form).  dL/dz per tick is added into ``gz_neuron`` [N]
        (a new zero tensor when None) and kept as ``self.gz_neuron``."""
        if spike_count is None:
            if spikes is None:
                raise ValueError("pass spikes or spike_count")
            T, B = int(spikes.shape[0]), int(spikes.shape[1])
            t0, t1 = self._window(T) if trim else (int(self._pre_delay or 0), T)
            spike_count = (spikes[t0:t1] > 0).sum(0, dtype=torch.int32)
        else:
            if T is None:
                raise ValueError("spike_count needs the forward's T")
            B = int(spike_count.shape[0])
            t0, t1 = self._window(int(T))
        n_samples = (t1 - t0) * B
        if n_samples <= 0:
            raise ValueError("the trimmed window is empty")
        spike_count = spike_count.contiguous()
        if spike_count.dtype != torch.int32:
            raise TypeError("spike_count must be int32")
        N = int(spike_count.shape[-1])
        rows = spike_count.numel() // N
        need = int(lib().glif_rate_loss_workspace(self._n_sel))
        if need == 0:
            raise RuntimeError("glif_rate_loss_workspace failed")
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        if gz_neuron is None:
            gz_neuron = torch.zeros(N, dtype=torch.float32, device=self.device)
        loss = torch.empty((), dtype=torch.float32, device=self.device)
        check(lib().glif_rate_dist_loss(ptr(spike_count), rows, N, n_samples, ptr(self._ids), self._pop_ptr,
                                        self._n_pop, ptr(self._targets), self._kappa, self._rate_cost,
                                        1 if shuffle else 0, self._shuffle_seed, self._offset, ptr(loss),
                                        ptr(gz_neuron), ptr(self._ws), self._ws.numel(),
                                        stream_ptr(self.device)))
        self._offset += self._n_sel
        self.gz_neuron = gz_neuron
        return loss


class RateMSE:
    """Mean-squared firing-rate error against per-neuron targets (spikes per tick): the loss
    the benchmark's training configuration names.  ``__call__(spike_count, T)`` takes the
    forward's spike counts [B, N] over T ticks; dL/dz per tick is added into ``gz_neuron``."""

    def __init__(self, targets, device="cuda"):
        self.device = torch.device(device)
        self.targets = torch.as_tensor(targets, dtype=torch.float32, device=self.device).contiguous()
        self._ws = torch.empty(int(lib().glif_rate_mse_workspace()), dtype=torch.uint8, device=self.device)
        self.gz_neuron = None

    def __call__(self, spike_count, T, gz_neuron=None):
        spike_count = spike_count.contiguous()
        if spike_count.dtype != torch.int32:
            raise TypeError("spike_count must be int32")
        N = int(spike_count.shape[-1])
        if N != self.targets.numel():
            raise ValueError("one target per neuron")
        rows = spike_count.numel() // N
        if gz_neuron is None:
            gz_neuron = torch.zeros(N, dtype=torch.float32, device=self.device)
        loss = torch.empty((), dtype=torch.float32, device=self.device)
        check(lib().glif_rate_mse_loss(ptr(spike_count), rows, N, int(T) * rows, ptr(self.targets), ptr(loss),
                                       ptr(gz_neuron), ptr(self._ws), self._ws.numel(), stream_ptr(self.device)))
        self.gz_neuron = gz_neuron
        return loss
