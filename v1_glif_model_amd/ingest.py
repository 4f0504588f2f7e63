"""Network ingestion: the dictionaries ``load_sparse.load_v1`` returns, plus the data the
reference's ``V1Column`` and rate losses read from disk beside them.

* ``network`` / ``lgn_input`` / ``bkg_input``: as ``load_sparse.py:364-377`` and
  ``:464-470`` build them (synapses sorted by (post, pre), ``load_sparse.py:15-22``);
  ``build_cell_tables`` consumes them unchanged.
* ``tau_basis``: ``synaptic_data/tau_basis.npy`` (``models.py:518-519``), read with
  ``numpy.load`` (no pickle).
* The basis table, one row of receptor weights per synapse type: the reference pickles
  ``{syn_id: weights}`` (``load_sparse.py:75-97``), built from
  ``synaptic_data/basis_function_weights.csv`` and the listing of
  ``<data_dir>/components/synaptic_models``: syn_id = position in the listing, a row for
  every ``.json`` file in listing order, and ``models.py:614-622`` stacks the dictionary's
  values.  ``load_basis_table`` rebuilds exactly that from the two sources (no pickle).
* Per-neuron cell types for the rate losses: ``pop_names`` (``other_v1_utils.py:63-84``) maps
  each neuron's SONATA ``node_type_id`` to its ``pop_name`` through
  ``network/v1_node_types.csv``; ``pop_name_to_cell_type`` (``other_v1_utils.py:23-52``)
  turns that into the cell type.  The reference re-reads the node ids from the SONATA h5
  file; ``network["node_type_id"]`` holds the same ids in the network's neuron order
  (``load_sparse.py:225, 274, 367``), so no h5 reader is needed.
"""
from __future__ import annotations

import os
from typing import Dict, Optional, Tuple

import numpy as np

__all__ = ["load_tau_basis", "load_basis_table", "pop_name_to_cell_type", "cell_types_from_node_types",
           "prepare_network"]


def load_tau_basis(path: str) -> np.ndarray:
    """Receptor time constants (ms), ``models.py:518-519``."""
    tau = np.load(path, allow_pickle=False)
    tau = np.asarray(tau, dtype=np.float64).reshape(-1)
    if tau.size == 0 or not np.all(tau > 0):
        raise ValueError("tau_basis must be a non-empty array of positive time constants")
    return tau


def load_basis_table(basis_csv: str, synaptic_models_dir: str) -> Tuple[np.ndarray, Dict[str, int]]:
    """(basis [n_types, n_basis] float32, {synaptic model: syn_id}) as ``load_sparse.py:75-97``
    and ``models.py:614-622`` produce them: syn_id is the position in
    ``os.listdir(synaptic_models_dir)``; every ``.json`` entry, in listing order, adds the row
    of its model from the weights table."""
    import pandas as pd
    weights = pd.read_csv(basis_csv, index_col=0)
    model_to_id: Dict[str, int] = {}
    rows = []
    for syn_id, name in enumerate(os.listdir(synaptic_models_dir)):
        if name.endswith(".json"):
            model = name.split(".")[0]
            model_to_id[model] = syn_id
            rows.append(weights.loc[model].values)
    if not rows:
        raise ValueError(f"no synaptic model (.json) in {synaptic_models_dir}")
    return np.asarray(rows, dtype=np.float32), model_to_id


# Inhibitory classes of a population name and the subclass each maps to; every other class
# is excitatory (other_v1_utils.py:23-52).
_INHIBITORY_SUBCLASS = {"Pvalb": "PV", "Sst": "SST", "Vip": "VIP", "Htr3a": "VIP"}


def pop_name_to_cell_type(pop_name: str, ignore_l5e_subtypes: bool = False) -> str:
    """``other_v1_utils.py:23-52``: 'e4Rorb' -> 'L4 Exc', 'i4Pvalb' -> 'L4 PV',
    'i23Sst' -> 'L2/3 SST', 'e5ET' -> 'L5 ET' (or 'L5 Exc' with ignore_l5e_subtypes),
    layer 1 -> 'L1 Htr3a'.  A name is <e|i><layer><class>; layer 2/3 is written with two
    digits, every other layer with one."""
    layer_char = pop_name[1]
    if layer_char == "1":
        return "L1 Htr3a"
    layer, cls = ("2/3", pop_name[3:]) if layer_char == "2" else (layer_char, pop_name[2:])
    sub = _INHIBITORY_SUBCLASS.get(cls)
    if sub is None:   # excitatory: layer 5 keeps its subtype unless asked not to
        sub = cls if layer == "5" and not ignore_l5e_subtypes else "Exc"
    return f"L{layer} {sub}"


def cell_types_from_node_types(node_types_csv: str, node_type_id: np.ndarray,
                               ignore_l5e_subtypes: bool = True) -> np.ndarray:
    """Per-neuron cell types from the space-separated SONATA node-types table (columns
    ``node_type_id`` and ``pop_name``) and the neurons' ``node_type_id`` (the rate losses use
    ``ignore_l5e_subtypes=True``, ``loss_functions.py:769-774``)."""
    import pandas as pd
    nt = pd.read_csv(node_types_csv, sep=" ")
    to_pop = dict(zip(nt["node_type_id"].to_numpy(), nt["pop_name"].to_numpy()))
    ids = np.asarray(node_type_id)
    missing = set(np.unique(ids).tolist()) - set(to_pop)
    if missing:
        raise ValueError(f"node_type_id(s) {sorted(missing)[:5]} not in {node_types_csv}")
    return np.array([pop_name_to_cell_type(str(to_pop[i]), ignore_l5e_subtypes) for i in ids])


def prepare_network(network: dict, lgn_input: dict, bkg_input: dict, tau_basis: np.ndarray,
                    basis: np.ndarray, cell_types: Optional[np.ndarray] = None) -> dict:
    """The dictionary ``V1Column`` and ``build_cell_tables`` take: the three reference
    dictionaries plus the receptor time constants and the basis table, checked against the
    synapse types the tables use."""
    tau_basis = np.asarray(tau_basis, dtype=np.float64).reshape(-1)
    basis = np.asarray(basis, dtype=np.float32)
    if basis.ndim != 2 or basis.shape[1] != tau_basis.size:
        raise ValueError(f"basis must be [n_types, {tau_basis.size}] (one weight per receptor)")
    for name, pop in (("network", network.get("synapses", {})), ("lgn_input", lgn_input), ("bkg_input", bkg_input)):
        sid = np.asarray(pop.get("syn_ids", []))
        if sid.size and (sid.min() < 0 or sid.max() >= basis.shape[0]):
            raise ValueError(f"{name} uses syn_id {int(sid.max())} but the basis table has {basis.shape[0]} rows")
    net = dict(network)
    if cell_types is not None:
        cell_types = np.asarray(cell_types)
        if cell_types.shape != (int(network["n_nodes"]),):
            raise ValueError("cell_types must have one entry per neuron")
        net["cell_type"] = cell_types
    return dict(network=net, lgn_input=lgn_input, bkg_input=bkg_input, tau_basis=tau_basis, basis=basis)
