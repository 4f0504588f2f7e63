"""numpy float64 brute force of the synaptic operator (TEST INFRASTRUCTURE ONLY).

An independent restatement (vectorised scatter-adds in float64, no ordering) used
to pin both the C oracle and the HIP kernels:

* ``csr_build_numpy``  the reference's own numpy fallback of make_pre_ind_table,
                       models.py:360-365 (argsort kind='stable' + bincount + cumsum).
* ``syn_fwd_f64``      forward of calculate_synaptic_currents, models.py:126-169:
                       I[b, post, r] = sum over synapses with z[b, col] > 0 of
                       (w * mult) * basis[syn_id, r].
* ``syn_bwd_f64``      its custom gradient, models.py:182-241:
                       dz[b, col] = sum_syn sum_r dy[b, post, r] w basis[syn_id, r]
                       dW[syn]    = sum_{b: z[b, col] > 0} mult * sum_r dy[b, post, r] basis[syn_id, r]
The ``*_abs`` companions return the same sums over |terms|, the scale a float32
sum's rounding error is proportional to.
"""
from __future__ import annotations

import numpy as np


def csr_build_numpy(cols, n_source):
    """models.py:360-365, verbatim in behaviour: (order int32, row_splits int32)."""
    pre_ids = np.asarray(cols, dtype=np.int64)
    order_np = np.argsort(pre_ids, kind="stable")
    counts_np = np.bincount(pre_ids[order_np], minlength=n_source)
    row_splits_np = np.empty((n_source + 1,), dtype=np.int64)
    row_splits_np[0] = 0
    np.cumsum(counts_np, dtype=np.int64, out=row_splits_np[1:])
    return order_np.astype(np.int32), row_splits_np.astype(np.int32)


def _act(table, z, use_count):
    z = np.asarray(z, dtype=np.float64)
    a = z[:, table.col]                       # [B, S]
    on = a > 0
    mult = np.where(on, a if use_count else 1.0, 0.0)
    return mult


def syn_fwd_f64(table, z, basis, use_count=False, absolute=False):
    basis = np.asarray(basis, dtype=np.float64)
    mult = _act(table, z, use_count)
    B = mult.shape[0]
    N, nb = table.n_post, basis.shape[1]
    w = table.weight.astype(np.float64)
    I = np.zeros((B, N, nb))
    for b in range(B):
        # bincount adds each bin's terms in input order, as a scatter-add would; zero terms
        # (inactive columns) are left out, which does not change a float64 sum
        on = mult[b] != 0
        terms = (mult[b][on] * w[on])[:, None] * basis[table.syn_id[on]]   # [active, nb]
        if absolute:
            terms = np.abs(terms)
        for r in range(nb):
            I[b, :, r] = np.bincount(table.post[on], weights=terms[:, r], minlength=N)
    return I.reshape(B * N, nb)


def syn_fwd_abs(table, z, basis, use_count=False):
    return syn_fwd_f64(table, z, basis, use_count, absolute=True)


def syn_bwd_f64(table, z, basis, dy, use_count=False):
    """Returns (dz [B, n_cols], dW [S], |dz| scale, |dW| scale), all float64."""
    basis = np.asarray(basis, dtype=np.float64)
    mult = _act(table, z, use_count)
    B = mult.shape[0]
    N, nb = table.n_post, basis.shape[1]
    dy = np.asarray(dy, dtype=np.float64).reshape(B, N, nb)
    bs = basis[table.syn_id]                          # [S, nb]
    w = table.weight.astype(np.float64)
    dz = np.zeros((B, table.n_cols))
    dz_abs = np.zeros((B, table.n_cols))
    dW = np.zeros(table.n_syn)
    dW_abs = np.zeros(table.n_syn)
    for b in range(B):
        prod = dy[b][table.post] * bs                 # [S, nb]
        g = prod.sum(1)
        pa = np.abs(prod).sum(1)
        dz[b] = np.bincount(table.col, weights=w * g, minlength=table.n_cols)
        dz_abs[b] = np.bincount(table.col, weights=np.abs(w) * pa, minlength=table.n_cols)
        dW += mult[b] * g
        dW_abs += np.abs(mult[b]) * pa
    return dz, dW, dz_abs, dW_abs
