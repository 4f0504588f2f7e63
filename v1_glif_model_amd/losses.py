"""Losses on the cell's outputs, fused with the GLIF_3 path (loss_functions.py).

``VoltageRegularization`` (loss_functions.py:1047-1119): the penalty of the cell's output
voltages, "range" relu(|v - 0.5| - 0.5)^2 or "threshold" (v - 1)^2, cost * mean over
(B, T, N).  Constructing it enables the fused form on the cell: the loss of the last
rollout is reduced from the voltages the cell keeps for BPTT, and ``V1Column.backward``
adds the gradient inside the adjoint, so no [T, B, N] voltage tensor has to exist.
"""
from __future__ import annotations

import torch

from ._lib import check, lib, ptr, stream_ptr

__all__ = ["VoltageRegularization"]

_MODES = {"range": 1, "threshold": 2}


class VoltageRegularization:
    def __init__(self, cell, voltage_cost=1e-5, dtype=torch.float32, core_mask=None, penalty_mode="range"):
        if penalty_mode not in _MODES:
            raise ValueError("penalty_mode must be 'range' or 'threshold'")
        if core_mask is not None:
            raise NotImplementedError("core_mask is not supported by the fused form")
        self._cell = cell
        self._voltage_cost = float(voltage_cost)
        self._penalty_mode = penalty_mode
        check(lib().glif_cell_set_voltage_loss(cell.handle, _MODES[penalty_mode], self._voltage_cost))

    def disable(self):
        check(lib().glif_cell_set_voltage_loss(self._cell.handle, 0, 0.0))

    @staticmethod
    def penalty(v, mode="range"):
        """Elementwise penalty (the reference's _compute_range_loss / _compute_threshold_loss)."""
        if mode == "range":
            return torch.square(torch.relu(torch.abs(v - 0.5) - 0.5))
        return torch.square(v - 1.0)

    def __call__(self, voltages=None):
        """Loss of ``voltages`` [T, B, N] if given, else (fused) of the cell's last rollout."""
        if voltages is not None:
            return self.penalty(voltages, self._penalty_mode).mean() * self._voltage_cost
        cell = self._cell
        if getattr(cell, "_last", None) is None:
            raise RuntimeError("no rollout to take the voltages from")
        B, T, ws = cell._last
        out = torch.empty((), dtype=torch.float32, device=cell.device)
        check(lib().glif_cell_voltage_loss(cell.handle, B, T, ptr(out), ptr(ws), ws.numel(),
                                           stream_ptr(cell.device)))
        return out
