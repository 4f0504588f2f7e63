"""One-time host preprocessing of a V1 network into the GLIF_3 cell's tables.

This mirrors `V1Column.__init__` (`v1_model_utils/models.py:451-773`) step for step,
in the same floating-point types, so the HIP path and the CPU restatement start
from identical numbers:

* ``voltage_scale = V_th - E_L``; ``asc_amps /= voltage_scale`` (`models.py:483-490`);
* ``tau = C_m / g``, ``decay = exp(-dt / tau)``, ``current_factor = (1 - decay) / g``
  in float32 (`models.py:512-515`);
* ``syn_decay = exp(-dt / tau_basis)``, ``psc_initial = e / tau_basis`` computed in
  float64 then cast to float32 (`models.py:518-526`);
* ``t_ref_steps = max(ceil(t_ref / dt), 1)`` (`models.py:574-583`);
* ``asc_decay = exp(-dt * sigmoid(logit(k)))`` in float32 (`models.py:556-593`);
* ``max_delay = min(ceil(max delay / dt), flag)`` over the recurrent delays and the LGN /
  background ``delays`` when present (`models.py:528-539`);
* recurrent weights ``w / voltage_scale[post] * recurrent_weight_scale / lr_scale``,
  delays ``round(clip(d, dt, max_delay) / dt)``, column ``pre + N * (delay - 1)``,
  dense shape ``(N, max_delay * N)`` (`models.py:625-669`);
* LGN and background weights ``w / voltage_scale[post] * input_weight_scale / lr_scale``
  with no delays (`models.py:707-773`).
"""
from __future__ import annotations

import dataclasses
import numpy as np

__all__ = ["SynapseTable", "CellTables", "build_cell_tables", "trainable_populations"]


def trainable_populations(train_recurrent=True, train_recurrent_per_type=True, train_input=False,
                          train_noise=True) -> dict:
    """Which weight vectors V1Column trains (models.py:651-669, 728-731, 761-764): the
    individual recurrent weights only with train_recurrent and not train_recurrent_per_type
    (the per-type factors of that mode are commented out in the reference, so the recurrent
    weights are then frozen), the LGN weights with train_input, the background weights with
    train_noise."""
    return {"rec": bool(train_recurrent) and not bool(train_recurrent_per_type),
            "lgn": bool(train_input), "bkg": bool(train_noise)}


@dataclasses.dataclass
class SynapseTable:
    """One synapse population in reference order (sorted by (post, pre)).

    ``post``/``col`` are the two columns of the reference's ``indices`` after the
    delay fold (`models.py:635`); ``n_cols`` is ``dense_shape[1]``.
    """
    post: np.ndarray      # int64 [S]
    col: np.ndarray       # int64 [S]  (pre + N*(delay-1) for the recurrent table)
    weight: np.ndarray    # float32 [S]  trainable variable value
    syn_id: np.ndarray    # uint8 [S]
    n_post: int
    n_cols: int

    @property
    def n_syn(self) -> int:
        return int(self.post.size)

    @property
    def indices(self) -> np.ndarray:
        """[S, 2] int64 (post, col): the reference's ``synapse_indices``."""
        return np.stack([self.post, self.col], -1)


@dataclasses.dataclass
class CellTables:
    n_neurons: int
    max_delay: int
    n_basis: int
    dt: float
    decay: np.ndarray           # float32 [N]
    current_factor: np.ndarray  # float32 [N]
    asc_decay: np.ndarray       # float32 [N, 2]
    asc_amps: np.ndarray        # float32 [N, 2]
    t_ref_steps: np.ndarray     # int32 [N]
    syn_decay: np.ndarray       # float32 [n_basis]
    psc_initial: np.ndarray     # float32 [n_basis]
    basis: np.ndarray           # float32 [n_syn_types, n_basis]
    voltage_scale: np.ndarray   # float32 [N]
    rec: SynapseTable
    lgn: SynapseTable
    bkg: SynapseTable
    lr_scale: float = 1.0


def _sigmoid_f32(x: np.ndarray) -> np.ndarray:
    one = np.float32(1.0)
    return (one / (one + np.exp(-x))).astype(np.float32)


def build_cell_tables(net: dict, dt: float = 1.0, max_delay: int = 0, lr_scale: float = 1.0,
                      recurrent_weight_scale: float = 1.0,
                      input_weight_scale: float = 1.0) -> CellTables:
    """Derive the cell's tables from the dictionaries `synthetic.make_network` returns
    (keys ``network``, ``lgn_input``, ``bkg_input``, ``tau_basis``, ``basis``)."""
    network, lgn_input, bkg_input = net["network"], net["lgn_input"], net["bkg_input"]
    p = {k: np.asarray(v) for k, v in network["node_params"].items()}
    type_ids = np.asarray(network["node_type_ids"])
    N = int(network["n_nodes"])

    vs = (p["V_th"] - p["E_L"]).astype(np.float32)
    asc_amps = (p["asc_amps"] / vs[..., None]).astype(np.float32)
    tau = (p["C_m"] / p["g"]).astype(np.float32)
    decay = np.exp(np.float32(-dt) / tau).astype(np.float32)
    current_factor = ((np.float32(1.0) - decay) / p["g"]).astype(np.float32)

    tau_syns = np.asarray(net["tau_basis"], dtype=np.float64)
    syn_decay = np.exp(-dt / tau_syns).astype(np.float32)
    psc_initial = (np.e / tau_syns).astype(np.float32)

    t_ref_steps = np.maximum(np.ceil(p["t_ref"][type_ids] / dt).astype(np.int32), 1)
    if int(t_ref_steps.max()) > 32767:
        raise ValueError("refractory period exceeds the int16 range")

    k = p["k"].astype(np.float32)
    logit = np.log(k / (np.float32(1.0) - k)).astype(np.float32)
    asc_decay = np.exp(np.float32(-dt) * _sigmoid_f32(logit)).astype(np.float32)

    syn = network["synapses"]
    indices = np.array(syn["indices"], dtype=np.int64)
    delays = np.asarray(syn["delays"], dtype=np.float64)
    # models.py:528-539: the largest delay of the recurrent synapses and of the LGN and
    # background populations when they carry one (their delays are not applied, :715-718)
    all_delays = [delays] + [np.asarray(pop["delays"], dtype=np.float64).reshape(-1)
                             for pop in (lgn_input, bkg_input) if "delays" in pop]
    all_delays = np.concatenate(all_delays)
    data_max_delay = int(np.ceil(np.max(all_delays) / dt)) if all_delays.size else 1
    D = min(data_max_delay, max_delay) if max_delay > 0 else data_max_delay
    w = (np.asarray(syn["weights"], dtype=np.float32) / vs[type_ids[indices[:, 0]]]).astype(np.float32)
    d_steps = np.round(np.clip(delays, dt, D) / dt).astype(np.int64)
    col = indices[:, 1] + N * (d_steps - 1)
    w_var = (w * np.float32(recurrent_weight_scale) / np.float32(lr_scale)).astype(np.float32)
    rec = SynapseTable(post=indices[:, 0].copy(), col=col, weight=w_var,
                       syn_id=np.asarray(syn["syn_ids"], dtype=np.uint8), n_post=N, n_cols=D * N)

    def _input(pop):
        ind = np.asarray(pop["indices"], dtype=np.int64)
        pw = (np.asarray(pop["weights"], dtype=np.float32) / vs[type_ids[ind[:, 0]]]).astype(np.float32)
        pw = (pw * np.float32(input_weight_scale) / np.float32(lr_scale)).astype(np.float32)
        return SynapseTable(post=ind[:, 0].copy(), col=ind[:, 1].copy(), weight=pw,
                            syn_id=np.asarray(pop["syn_ids"], dtype=np.uint8), n_post=N,
                            n_cols=int(pop["n_inputs"]))

    return CellTables(
        n_neurons=N, max_delay=D, n_basis=int(tau_syns.size), dt=float(dt),
        decay=decay[type_ids], current_factor=current_factor[type_ids],
        asc_decay=asc_decay[type_ids], asc_amps=asc_amps[type_ids],
        t_ref_steps=t_ref_steps.astype(np.int32), syn_decay=syn_decay, psc_initial=psc_initial,
        basis=np.asarray(net["basis"], dtype=np.float32), voltage_scale=vs[type_ids],
        rec=rec, lgn=_input(lgn_input), bkg=_input(bkg_input), lr_scale=float(lr_scale))
