"""Shared builders for the tests: seeded synthetic networks and tolerance checks."""
import dataclasses

import numpy as np

from v1_glif_model_amd import synthetic as sy
from v1_glif_model_amd.tables import build_cell_tables

# fp32 parity bar of the benchmark definition: 1e-5 relative / 1e-6 absolute
RTOL, ATOL = 1e-5, 1e-6


def tiny_config(n=300, fanin=30, delays=3, n_lgn=80, lgn_fanin=8, n_bkg=10, bkg_fanin=3,
                rs=0.5, ins=0.5, lgn_p=0.05, seq_len=40, batch=2):
    return dataclasses.replace(
        sy.CONFIGS[0], n_neurons=n, fanin_mean=fanin, max_delay=delays, n_lgn=n_lgn,
        lgn_fanin=lgn_fanin, n_bkg=n_bkg, bkg_fanin=bkg_fanin, recurrent_weight_scale=rs,
        input_weight_scale=ins, lgn_p=lgn_p, seq_len=seq_len, batch=batch)


def network(cfg, seed=0, dense_basis=False):
    net = sy.make_network(cfg, seed=seed, dense_basis=dense_basis)
    return net, build_cell_tables(net)


def assert_close(actual, expected, rtol=RTOL, atol=ATOL, what=""):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (what, a.shape, e.shape)
    err = np.abs(a - e)
    bad = err > atol + rtol * np.abs(e)
    if np.any(bad):
        i = np.flatnonzero(bad)[0]
        raise AssertionError(
            f"{what}: {bad.sum()} of {bad.size} outside rtol={rtol} atol={atol}; first at {i}: "
            f"{a.flat[i]!r} vs {e.flat[i]!r}; max abs err {err.max():.3e}")


def rel_to_scale(actual, expected, scale):
    """Max |a - e| / scale (scale: the sum of |terms| a value is accumulated from)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return float(np.max(np.abs(a - e) / np.maximum(scale, 1e-30)))


def device_to_numpy(dev_ptr, n, dtype):
    """Copy n elements from a raw device pointer (libglif-owned) to a numpy array."""
    import ctypes

    import torch
    out = np.empty(n, dtype=dtype)
    if n == 0:
        return out
    hip = ctypes.CDLL("libamdhip64.so.7")   # the runtime torch already loaded
    torch.cuda.synchronize()
    rc = hip.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(dev_ptr),
                       ctypes.c_size_t(out.nbytes), ctypes.c_int(2))  # hipMemcpyDeviceToHost
    assert rc == 0, rc
    return out


def assert_grads_per_element(got, exp, scale, what="", rtol=RTOL, atol=ATOL):
    """North star's bar per gradient element: |got - exp| <= rtol * scale + atol, with scale
    the element's sum of absolute terms (oracle.cpu.bptt_abs_scale).  Returns the largest
    |got - exp| / scale over the elements with a nonzero scale (the error distribution's
    tail, printed by the callers)."""
    a = np.asarray(got, dtype=np.float64)
    e = np.asarray(exp, dtype=np.float64)
    s = np.asarray(scale, dtype=np.float64)
    assert a.shape == e.shape == s.shape, (what, a.shape, e.shape, s.shape)
    err = np.abs(a - e)
    bad = err > rtol * s + atol
    if np.any(bad):
        i = np.flatnonzero(bad)[0]
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} elements outside {rtol:g}*sum|terms| + "
                             f"{atol:g}; first at {i}: {a.flat[i]!r} vs {e.flat[i]!r} (scale {s.flat[i]!r})")
    nz = s > 0
    return float(np.max(err[nz] / s[nz])) if np.any(nz) else 0.0


def error_summary(got, exp, scale):
    """Quantiles of |got - exp| / scale over the nonzero-scale elements."""
    a, e, s = (np.asarray(x, dtype=np.float64) for x in (got, exp, scale))
    nz = s > 0
    if not np.any(nz):
        return {}
    r = np.abs(a - e)[nz] / s[nz]
    return {"n": int(nz.sum()), "p50": float(np.quantile(r, 0.5)), "p99": float(np.quantile(r, 0.99)),
            "max": float(r.max()), "exact_frac": float(np.mean(r == 0))}
