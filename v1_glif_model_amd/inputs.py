"""Input spikes sampled on the device (libglif's Philox4x32-10 streams).

``sample_lgn``: LGN spikes, Bernoulli with p = 1 - exp(-rate * dt / 1000)
(stim_dataset.py:182-197).  ``sample_bkg``: background Poisson counts with
lambda = rate * dt / 1000 (models.py:865-887).  TF's stateless streams cannot be
reproduced; a (seed, offset) pair names a stream here, element i of a [T, B, n] draw
being stream element offset + i, so consecutive calls can continue one stream.
"""
from __future__ import annotations

import numpy as np
import torch

from ._lib import check, lib, ptr, require_gpu, stream_ptr

__all__ = ["sample_lgn", "sample_bkg", "bernoulli", "poisson"]


def bernoulli(p: torch.Tensor, seed: int, offset: int = 0) -> torch.Tensor:
    """uint8 tensor of p's shape: 1 where u < p (p fp32 on the device)."""
    require_gpu()
    p = p.to(torch.float32).contiguous()
    out = torch.empty(p.shape, dtype=torch.uint8, device=p.device)
    check(lib().glif_sample_bernoulli(ptr(p), p.numel(), int(seed) & (2 ** 64 - 1), int(offset), ptr(out),
                                      stream_ptr(p.device)))
    return out


def poisson(lam: float, shape, seed: int, offset: int = 0, device="cuda") -> torch.Tensor:
    """uint8 Poisson(lam) counts (capped at 255)."""
    require_gpu()
    device = torch.device(device)
    out = torch.empty(tuple(shape), dtype=torch.uint8, device=device)
    lam32 = np.float32(lam)
    check(lib().glif_sample_poisson(float(lam32), float(np.exp(-lam32)), out.numel(), int(seed) & (2 ** 64 - 1),
                                    int(offset), ptr(out), stream_ptr(device)))
    return out


def sample_lgn(rates_hz, seed: int, dt: float = 1.0, offset: int = 0) -> torch.Tensor:
    """rates_hz [T, B, n_lgn] (tensor or array) -> spikes [T, B, n_lgn] uint8 on the device."""
    r = torch.as_tensor(rates_hz, dtype=torch.float32, device="cuda")
    p = 1.0 - torch.exp(-r * (dt / 1000.0))
    return bernoulli(p, seed, offset)


def sample_bkg(T: int, B: int, n_bkg: int, seed: int, rate_hz: float = 250.0, dt: float = 1.0,
               offset: int = 0, device="cuda") -> torch.Tensor:
    """Background counts [T, B, n_bkg] uint8 with lambda = rate_hz * dt / 1000."""
    return poisson(rate_hz * dt / 1000.0, (T, B, n_bkg), seed, offset, device)
