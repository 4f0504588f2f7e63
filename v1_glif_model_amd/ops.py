"""The synaptic-current operator with the reference's Python signature.

Mirrors `v1_model_utils/models.py`:

* ``make_pre_ind_table``          models.py:343-373 (with _validate_inputs :299-315)
* ``calculate_synaptic_currents`` models.py:103-263 (forward + custom gradient)

Both run in libglif (HIP, gfx950); there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional

import numpy as np
import torch

from . import _lib
from ._lib import check, lib, ptr, stream_ptr

__all__ = ["PreIndTable", "make_pre_ind_table", "SynapseTable", "calculate_synaptic_currents",
           "where_gt0"]

MODES = {"event": _lib.MODE_EVENT, "deterministic": _lib.MODE_DETERMINISTIC}


class PreIndTable:
    """Ragged table of synapse ids grouped by presynaptic column.

    The reference keeps it as ``tf.RaggedTensor.from_row_splits(order, row_splits)``
    (models.py:367-373); ``values`` is ``order`` (int32) and ``row_splits`` int32.
    """

    def __init__(self, order: np.ndarray, row_splits: np.ndarray):
        self.values = order
        self.row_splits = row_splits
        self._tables = {}

    @property
    def flat_values(self):
        return self.values

    def row_lengths(self):
        return np.diff(self.row_splits)

    def __getitem__(self, col):
        return self.values[self.row_splits[col]:self.row_splits[col + 1]]

    def nrows(self):
        return self.row_splits.size - 1


def make_pre_ind_table(indices, n_source_neurons=197613) -> PreIndTable:
    """Stable counting sort of synapse ids by ``indices[:, 1]`` (models.py:343-373).

    Raises ValueError exactly where `_validate_inputs` (models.py:299-315) does.
    Runs on the host inside libglif (the reference builds it on the host with numba).
    """
    n_source_neurons = int(n_source_neurons)
    if n_source_neurons <= 0:
        raise ValueError(f'`n_source_neurons` must be > 0, got {n_source_neurons}.')
    ind = np.asarray(indices)
    if ind.ndim != 2 or ind.shape[1] < 2:
        raise ValueError(f'`indices` must have shape [n_synapses, >=2], got {ind.shape}.')
    cols = np.ascontiguousarray(ind[:, 1], dtype=np.int64)
    S = cols.size
    if S > np.iinfo(np.int32).max:
        raise ValueError("more than 2^31-1 synapses: int32 order is not enough")
    order = np.empty(S, dtype=np.int32)
    splits = np.empty(n_source_neurons + 1, dtype=np.int32)
    bad = C.c_int64(-1)
    rc = lib().glif_make_pre_ind_table(cols.ctypes.data_as(C.c_void_p), S, n_source_neurons,
                                       order.ctypes.data_as(C.c_void_p),
                                       splits.ctypes.data_as(C.c_void_p), C.byref(bad))
    if rc != 0:
        if rc == _lib.GLIF_ERANGE:
            raise ValueError(f'Presynaptic index {int(cols[bad.value])} is out of bounds for '
                             f'`n_source_neurons={n_source_neurons}`.')
        check(rc)
    return PreIndTable(order, splits)


class SynapseTable:
    """Device-resident synapse population (libglif ``glif_table``).

    Built once from the reference-order arrays V1Column keeps (models.py:625-773):
    ``indices`` [S, 2] (post, col), ``syn_ids`` [S], ``dense_shape`` (n_post, n_cols),
    ``basis`` [n_types, n_basis].  ``n_delay_slots`` is D for the recurrent table
    (col = pre + n_post * (delay - 1)), 1 for the input populations.
    """

    def __init__(self, indices, syn_ids, dense_shape, basis, n_delay_slots: int = 1):
        _lib.require_gpu()
        ind = np.asarray(indices)
        post = np.ascontiguousarray(ind[:, 0], dtype=np.int64)
        col = np.ascontiguousarray(ind[:, 1], dtype=np.int64)
        sid = np.ascontiguousarray(np.asarray(syn_ids), dtype=np.int64)
        if sid.size and (sid.min() < 0 or sid.max() > 255):
            raise ValueError("syn_ids must be in [0, 255]")
        sid = sid.astype(np.uint8)
        basis = np.ascontiguousarray(np.asarray(basis, dtype=np.float32))
        self.n_post, self.n_cols = int(dense_shape[0]), int(dense_shape[1])
        self.n_syn = post.size
        self.n_types, self.n_basis = basis.shape
        self.n_delay_slots = int(n_delay_slots)
        # the device the table is uploaded to (the current one); its entry points take tensors there
        self.device = torch.device("cuda", torch.cuda.current_device())
        h = C.c_void_p()
        check(lib().glif_table_create(post.ctypes.data_as(C.c_void_p), col.ctypes.data_as(C.c_void_p),
                                      sid.ctypes.data_as(C.c_void_p), self.n_syn, self.n_post,
                                      self.n_cols, self.n_delay_slots,
                                      basis.ctypes.data_as(C.c_void_p), self.n_types, self.n_basis,
                                      C.byref(h)))
        self.handle = h
        self._w_key = None
        self._ws = {}

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            try:
                lib().glif_table_destroy(h)
            except Exception:
                pass
            self.handle = None

    def pre_ind_device(self):
        """(order, row_splits) device pointers of the bit-exact pre_ind_table."""
        o, r = C.c_void_p(), C.c_void_p()
        check(lib().glif_table_pre_ind(self.handle, C.byref(o), C.byref(r)))
        return o.value, r.value

    def set_weights(self, w: torch.Tensor, force: bool = False):
        """refresh_recurrent_weight_shadow (models.py:966-976): copy w into the table.

        Skipped when the same tensor at the same version was copied last time."""
        if not torch.is_tensor(w) or w.dtype != torch.float32 or w.device != self.device or w.numel() != self.n_syn:
            raise ValueError(f"weights must be a float32 tensor on {self.device} with one entry per synapse")
        w = w.detach().contiguous()
        key = (w.data_ptr(), w._version)
        if force or key != self._w_key:
            check(lib().glif_table_set_weights(self.handle, ptr(w), stream_ptr(w.device)))
            self._w_key = key
            self._w_ref = w

    def workspace(self, B: int, device) -> torch.Tensor:
        n = int(lib().glif_syn_workspace(self.handle, int(B)))
        ws = self._ws.get((B, str(device)))
        if ws is None or ws.numel() < n:
            ws = torch.empty(max(n, 1), dtype=torch.uint8, device=device)
            self._ws[(B, str(device))] = ws
        return ws

    def _check_z(self, z):
        """ValueError unless z is a [B, n_cols] tensor on the table's device with 1 <= B <= 32."""
        if not torch.is_tensor(z) or z.dim() != 2:
            raise ValueError("z must be a 2-D tensor [B, n_cols]")
        if z.device != self.device:
            raise ValueError(f"z is on {z.device}, the table on {self.device}")
        if z.shape[1] != self.n_cols:
            raise ValueError(f"z must have {self.n_cols} columns (dense_shape[1]), got {z.shape[1]}")
        if not 1 <= z.shape[0] <= 32:
            raise ValueError(f"batch size must be in [1, 32], got {z.shape[0]}")
        if z.dtype.is_complex:
            raise ValueError(f"z must be a real tensor, got {z.dtype}")

    def forward(self, z: torch.Tensor, counts: bool = False, mode: str = "event") -> torch.Tensor:
        self._check_z(z)
        if mode not in MODES:
            raise ValueError(f"mode must be one of {sorted(MODES)}")
        B = z.shape[0]
        z = z.contiguous()
        if z.dtype != torch.float32:
            z = z.float()
        I = torch.empty((B * self.n_post, self.n_basis), dtype=torch.float32, device=z.device)
        ws = self.workspace(B, z.device)
        check(lib().glif_syn_fwd(self.handle, ptr(z), B, int(counts), MODES[mode], ptr(I), ptr(ws),
                                 ws.numel(), stream_ptr(z.device)))
        return I

    def backward(self, z: torch.Tensor, dy: torch.Tensor, counts: bool = False, want_dz: bool = True,
                 want_dw: bool = True):
        self._check_z(z)
        B = z.shape[0]
        if not torch.is_tensor(dy) or tuple(dy.shape) != (B * self.n_post, self.n_basis):
            raise ValueError(f"dy must have shape {(B * self.n_post, self.n_basis)} ([B * n_post, n_basis]), "
                             f"got {tuple(dy.shape) if torch.is_tensor(dy) else type(dy).__name__}")
        if dy.device != self.device:
            raise ValueError(f"dy is on {dy.device}, the table on {self.device}")
        z = z.contiguous().float()
        dy = dy.contiguous().float()
        dz = torch.empty((B, self.n_cols), dtype=torch.float32, device=z.device) if want_dz else None
        dw = torch.empty(self.n_syn, dtype=torch.float32, device=z.device) if want_dw else None
        ws = self.workspace(B, z.device)
        check(lib().glif_syn_bwd(self.handle, ptr(z), ptr(dy), B, int(counts), ptr(dz), ptr(dw),
                                 ptr(ws), ws.numel(), stream_ptr(z.device)))
        return dz, dw


def where_gt0(z: torch.Tensor) -> torch.Tensor:
    """tf.where(z > 0) for a 2-D float32 CUDA tensor (models.py:128): [n, 2] int64, row-major."""
    if not torch.is_tensor(z) or z.dim() != 2:
        raise ValueError("where_gt0 takes a 2-D tensor")
    if not z.is_cuda:
        raise ValueError("where_gt0 takes a device tensor")
    z = z.contiguous().float()
    rows, cols = z.shape
    pairs = torch.empty((max(rows * cols, 1), 2), dtype=torch.int64, device=z.device)
    count = torch.zeros(1, dtype=torch.int64, device=z.device)
    n = int(lib().glif_where_workspace(rows, cols))
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=z.device)
    check(lib().glif_where_gt0(ptr(z), rows, cols, ptr(pairs), ptr(count), ptr(ws), ws.numel(),
                               stream_ptr(z.device)))
    return pairs[: int(count.item())]


def _array_key(a):
    """Identity of a table input: the object (held by the cache entry, so its id is not
    reused), its shape and, for a tensor, its in-place version counter."""
    if torch.is_tensor(a):
        return (id(a), tuple(a.shape), a._version)
    return (id(a), tuple(np.shape(a)))


def _table_for(pre_ind_table: PreIndTable, synapse_indices, syn_ids, dense_shape, basis):
    """The device table of these arrays, built on first use and cached on ``pre_ind_table``.
    The cache is keyed on the dense shape and on the identity of ``synapse_indices``,
    ``syn_ids`` and ``basis`` (new objects, or a tensor modified in place, build a new table;
    the reference builds its tables once, models.py:636-705)."""
    key = ((int(dense_shape[0]), int(dense_shape[1])), _array_key(synapse_indices), _array_key(syn_ids),
           _array_key(basis))
    hit = pre_ind_table._tables.get(key)
    if hit is None:
        n_post, n_cols = key[0]
        slots = n_cols // n_post if n_cols % n_post == 0 and n_cols > n_post else 1
        ind = synapse_indices.cpu().numpy() if torch.is_tensor(synapse_indices) else synapse_indices
        sid = syn_ids.cpu().numpy() if torch.is_tensor(syn_ids) else syn_ids
        bs = basis.detach().cpu().numpy() if torch.is_tensor(basis) else basis
        if np.asarray(ind).shape[0] != pre_ind_table.values.size:
            raise ValueError("synapse_indices and pre_ind_table hold different numbers of synapses")
        t = SynapseTable(ind, sid, key[0], bs, n_delay_slots=slots)
        # one table per pre_ind_table: a new key replaces the old entry (and frees its device table)
        pre_ind_table._tables.clear()
        hit = (t, (synapse_indices, syn_ids, basis))
        pre_ind_table._tables[key] = hit
    return hit[0]


class _SynCurrents(torch.autograd.Function):
    @staticmethod
    def forward(ctx, rec_z_buf, weight_values, weight_values_compute, table, mode):
        table.set_weights(weight_values_compute)
        ctx.table = table
        ctx.save_for_backward(rec_z_buf)
        ctx.w_needs = weight_values.requires_grad
        return table.forward(rec_z_buf, mode=mode)

    @staticmethod
    def backward(ctx, dy):
        (z,) = ctx.saved_tensors
        want_dz = ctx.needs_input_grad[0]
        dz, dw = ctx.table.backward(z, dy, want_dz=want_dz, want_dw=ctx.w_needs)
        return dz, dw, None, None, None


def calculate_synaptic_currents(rec_z_buf, synapse_indices, weight_values, weight_values_compute,
                                dense_shape, synaptic_basis_weights, syn_ids, pre_ind_table,
                                mode: str = "event"):
    """I[b*N + post, r] = sum over active (b, col) of W * basis[syn_id, r]  (models.py:103-169).

    Gradients (models.py:174-261): w.r.t. ``rec_z_buf`` the dense
    ``sum_r dy_r @ W_r`` over all synapses; w.r.t. ``weight_values`` the per-synapse
    sum over active events of ``dy[b*N + post] . basis[syn_id]``; None elsewhere
    (``weight_values_compute`` is the forward's copy and gets no gradient).

    ``pre_ind_table`` is the `PreIndTable` of `make_pre_ind_table`; the device table
    is built on first use and cached on it.  ``mode``: "event" (atomic push, fast)
    or "deterministic" (reference accumulation order, bit-reproducible).
    """
    if mode not in MODES:
        raise ValueError(f"mode must be one of {sorted(MODES)}")
    table = _table_for(pre_ind_table, synapse_indices, syn_ids, dense_shape, synaptic_basis_weights)
    if weight_values_compute is None:
        weight_values_compute = weight_values
    return _SynCurrents.apply(rec_z_buf, weight_values, weight_values_compute, table, mode)
