"""ExponentiatedAdam and SignedConstraint on the GPU (v1_model_utils/optimizers.py:154-390,
models.py:419-427).

Same names and arguments as the reference.  ``apply_gradients`` runs the dense
``update_step`` and then the variable's sign constraint in one libglif kernel
(``glif_exp_adam``) per variable; the moment slots live on the device beside the
weights.  Weight vectors are fp32 device tensors updated in place.
"""
from __future__ import annotations

import numpy as np
import torch

from ._lib import check, lib, ptr, require_gpu, stream_ptr

__all__ = ["ExponentiatedAdam", "SignedConstraint"]


class SignedConstraint:
    """``w -> where(positive, relu(w), -relu(-w))`` (models.py:419-427).

    ``positive``: bool / uint8 tensor, True where the weight must stay >= 0."""

    def __init__(self, positive):
        self.condition = torch.as_tensor(positive).to(torch.uint8).contiguous()

    def __call__(self, w):
        return torch.where(self.condition.bool().to(w.device), torch.relu(w), -torch.relu(-w))


class ExponentiatedAdam:
    """Adam moments with the exponentiated update ``w <- w * exp(-alpha * m / (sqrt(v) + eps)
    * sign(w))`` (sign(0) = +1), optionally AMSGrad; the dense branch of
    ``ExponentiatedAdam.update_step`` (optimizers.py:268-376, dense branch :354-376)."""

    def __init__(self, learning_rate=0.001, beta_1=0.9, beta_2=0.999, epsilon=1e-7, amsgrad=False,
                 name="ExponentiatedAdam"):
        self.learning_rate = learning_rate
        self.beta_1, self.beta_2, self.epsilon = beta_1, beta_2, epsilon
        self.amsgrad = bool(amsgrad)
        self.name = name
        self.iterations = 0
        self._slots = {}

    def _lr(self):
        lr = self.learning_rate
        return float(lr(self.iterations) if callable(lr) else lr)

    def alpha(self):
        """alpha of the next step in fp32, as update_step forms it (optimizers.py:273-283)."""
        f = np.float32
        t = f(self.iterations + 1)
        b1p = np.power(f(self.beta_1), t)
        b2p = np.power(f(self.beta_2), t)
        return f(f(self._lr()) * np.sqrt(f(1) - b2p)) / (f(1) - b1p)

    def slots(self, var):
        key = var.data_ptr()
        s = self._slots.get(key)
        if s is None:
            z = lambda: torch.zeros_like(var)   # noqa: E731
            s = {"m": z(), "v": z(), "vhat": z() if self.amsgrad else None}
            self._slots[key] = s
        return s

    def apply_gradients(self, grads_and_vars, constraints=None):
        """One step over every (gradient, variable) pair, then iterations += 1.

        ``constraints``: optional {id(var) or var.data_ptr(): SignedConstraint or a
        positive-mask tensor}; a constrained variable is projected in the same kernel."""
        require_gpu()
        alpha = self.alpha()
        for g, var in grads_and_vars:
            if g is None:
                continue
            if var.dtype != torch.float32 or not var.is_cuda or not var.is_contiguous():
                raise ValueError("variables must be contiguous fp32 device tensors")
            g = g.to(device=var.device, dtype=torch.float32).contiguous()
            if g.shape != var.shape:
                raise ValueError("gradient and variable shapes differ")
            pos = None
            if constraints:
                c = constraints.get(var.data_ptr(), constraints.get(id(var)))
                if c is not None:
                    pos = (c.condition if isinstance(c, SignedConstraint) else torch.as_tensor(c))
                    pos = pos.to(device=var.device, dtype=torch.uint8).contiguous()
            s = self.slots(var)
            with torch.no_grad():
                check(lib().glif_exp_adam(ptr(var), ptr(s["m"]), ptr(s["v"]), ptr(s["vhat"]), ptr(g),
                                          ptr(pos), var.numel(), float(alpha), float(self.beta_1),
                                          float(self.beta_2), float(self.epsilon), stream_ptr(var.device)))
            # the kernel wrote through a raw pointer: mark the tensor modified, so the weight
            # copies the synapse tables keep (keyed on the tensor's version) are refreshed
            torch.autograd.graph.increment_version(var)
        self.iterations += 1
