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


# An element whose value is at most this fraction of its sum of absolute terms is a
# cancellation case: its excitatory and inhibitory terms nearly cancel, so fp32 rounding in any
# summation order is large against the value itself.
CANCEL = 1e-2


def literal_bar(got, exp, scale, rtol=RTOL, atol=ATOL, cancel=CANCEL):
    """The north star's literal bar |got - exp| <= rtol * |exp| + atol, element by element:
    how many elements meet it, and of those that do not, how many are cancellation cases
    (|exp| <= cancel * sum|terms|) and how many are not (the latter must be none)."""
    a, e, s = (np.asarray(x, dtype=np.float64) for x in (got, exp, scale))
    err = np.abs(a - e)
    miss = err > rtol * np.abs(e) + atol
    canc = np.abs(e) <= cancel * s
    out = {"n": int(a.size), "literal_frac": float(1.0 - miss.mean()) if a.size else 1.0,
           "miss": int(miss.sum()), "miss_cancelling": int((miss & canc).sum()),
           "miss_not_cancelling": int((miss & ~canc).sum())}
    if out["miss"]:
        out["miss_max_value_over_terms"] = float(np.max(np.abs(e[miss]) / np.maximum(s[miss], 1e-30)))
    return out


def assert_literal_bar(got, exp, scale, what="", rtol=RTOL, atol=ATOL, cancel=CANCEL):
    """Every element meets |got - exp| <= rtol * |exp| + atol unless it is a cancellation case
    (|exp| <= cancel * sum|terms|).  Returns the literal_bar report (printed by the callers)."""
    rep = literal_bar(got, exp, scale, rtol, atol, cancel)
    if rep["miss_not_cancelling"]:
        a, e, s = (np.asarray(x, dtype=np.float64) for x in (got, exp, scale))
        bad = (np.abs(a - e) > rtol * np.abs(e) + atol) & (np.abs(e) > cancel * s)
        i = np.flatnonzero(bad)[0]
        raise AssertionError(f"{what}: {rep['miss_not_cancelling']} non-cancelling elements outside "
                             f"{rtol:g}*|e| + {atol:g}; first at {i}: {a.flat[i]!r} vs {e.flat[i]!r} "
                             f"(sum|terms| {s.flat[i]!r}); {rep}")
    return rep


def assert_grads_per_element(got, exp, scale, what="", rtol=RTOL, atol=ATOL):
    """North star's bar per gradient element, in two forms.  (1) |got - exp| <= rtol * scale +
    atol, with scale the element's sum of absolute terms (oracle.cpu.bptt_abs_scale), the bound
    fp32 rounding in any summation order obeys.  (2) The literal |got - exp| <= rtol * |exp| +
    atol on every element that is not a cancellation case (assert_literal_bar); the report of
    (2) is printed.  Returns the largest |got - exp| / scale over the elements with a nonzero
    scale (the error distribution's tail, printed by the callers)."""
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
    rep = assert_literal_bar(a, e, s, what, rtol, atol)
    print(f"{what}: literal bar {rep}")
    nz = s > 0
    return float(np.max(err[nz] / s[nz])) if np.any(nz) else 0.0


def error_summary(got, exp, scale):
    """Quantiles of |got - exp| / scale over the nonzero-scale elements, and the share of all
    elements within the literal 1e-5 * |exp| + 1e-6."""
    a, e, s = (np.asarray(x, dtype=np.float64) for x in (got, exp, scale))
    nz = s > 0
    if not np.any(nz):
        return {}
    r = np.abs(a - e)[nz] / s[nz]
    return {"n": int(nz.sum()), "p50": float(np.quantile(r, 0.5)), "p99": float(np.quantile(r, 0.99)),
            "max": float(r.max()), "exact_frac": float(np.mean(r == 0)),
            "literal_frac": literal_bar(a, e, s)["literal_frac"]}
