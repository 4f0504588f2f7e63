"""ctypes binding of libglif.so (the C ABI declared in include/glif.h).

The library is loaded from this package directory.  There is no fallback: a
missing library, or a call on a machine without a GPU, raises.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

import torch  # noqa: F401  (loads torch's HIP runtime first, so libglif binds to the same one)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libglif.so")

GLIF_OK, GLIF_EINVAL, GLIF_ERANGE, GLIF_ENOMEM, GLIF_EHIP = 0, -22, -34, -12, -1000
MODE_EVENT, MODE_DETERMINISTIC = 0, 1

# Every symbol include/glif.h declares, with (restype, argtypes).
vp, i32, i64, f32p, sz = C.c_void_p, C.c_int32, C.c_int64, C.c_void_p, C.c_size_t


class CellConfig(C.Structure):
    """glif_cell_config."""
    _fields_ = [("n_neurons", C.c_int32), ("n_delay", C.c_int32), ("n_basis", C.c_int32),
                ("dt", C.c_float), ("lr_scale", C.c_float),
                ("voltage_gradient_dampening", C.c_float), ("recurrent_dampening", C.c_float),
                ("gauss_std", C.c_float), ("dampening_factor", C.c_float),
                ("pseudo_gauss", C.c_int32), ("hard_reset", C.c_int32)]


class State(C.Structure):
    """glif_state: device pointers of the reference state tuple."""
    _fields_ = [("z_buf", vp), ("v", vp), ("r", vp), ("asc", vp), ("psc_rise", vp), ("psc", vp)]


class StateGrad(C.Structure):
    """glif_state_grad: device pointers of the gradients of the state tuple (NULL: none)."""
    _fields_ = [("z_buf", vp), ("v", vp), ("asc", vp), ("psc_rise", vp), ("psc", vp)]


SIGNATURES = {
    "glif_last_error": (C.c_char_p, []),
    "glif_version": (C.c_int, []),
    "glif_make_pre_ind_table": (C.c_int, [vp, i64, i64, vp, vp, vp]),
    "glif_where_workspace": (sz, [i64, i64]),
    "glif_where_gt0": (C.c_int, [vp, i64, i64, vp, vp, vp, sz, vp]),
    "glif_table_create": (C.c_int, [vp, vp, vp, i64, i32, i64, i32, vp, i32, i32, C.POINTER(vp)]),
    "glif_table_destroy": (None, [vp]),
    "glif_table_n_syn": (i64, [vp]),
    "glif_table_pre_ind": (C.c_int, [vp, C.POINTER(vp), C.POINTER(vp)]),
    "glif_table_set_weights": (C.c_int, [vp, vp, vp]),
    "glif_syn_workspace": (sz, [vp, i32]),
    "glif_syn_fwd": (C.c_int, [vp, vp, i32, i32, i32, vp, vp, sz, vp]),
    "glif_syn_bwd": (C.c_int, [vp, vp, vp, i32, i32, vp, vp, vp, sz, vp]),
    "glif_syn_fwd_noalloc": (C.c_int, [vp, vp, i32, i32, i32, vp, vp]),
    "glif_cell_create": (C.c_int, [C.POINTER(CellConfig), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                   C.POINTER(vp)]),
    "glif_cell_destroy": (None, [vp]),
    "glif_cell_workspace": (sz, [vp, i32, i32]),
    "glif_cell_forward": (C.c_int, [vp, i32, i32, i32, vp, vp, C.POINTER(State), vp, vp, vp, vp,
                                    sz, vp]),
    "glif_cell_backward": (C.c_int, [vp, i32, i32, vp, vp, vp, vp, vp, vp, vp, sz, vp]),
    "glif_step_workspace": (sz, [vp, i32]),
    "glif_step_backward": (C.c_int, [vp, i32, vp, vp, vp, vp, vp, vp, vp, C.POINTER(StateGrad),
                                     C.POINTER(StateGrad), vp, vp, vp, vp, sz, vp]),
    "glif_cell_set_voltage_loss": (C.c_int, [vp, i32, C.c_float]),
    "glif_cell_voltage_loss": (C.c_int, [vp, i32, i32, vp, vp, sz, vp]),
    "glif_cell_set_trim": (C.c_int, [vp, i32, i32]),
    "glif_cell_g_layout": (C.c_int, [vp, vp, vp]),
    "glif_cell_set_g_layout": (C.c_int, [vp, i32]),
    "glif_cell_set_voltage_mask": (C.c_int, [vp, vp, i32]),
    "glif_rate_loss_workspace": (sz, [i64]),
    "glif_rate_mse_workspace": (sz, []),
    "glif_rate_mse_loss": (C.c_int, [vp, i32, i32, i32, vp, vp, vp, vp, sz, vp]),
    "glif_rate_dist_loss": (C.c_int, [vp, i32, i32, i32, vp, vp, i32, vp, C.c_float, C.c_float, i32,
                                      C.c_uint64, C.c_uint64, vp, vp, vp, sz, vp]),
    "glif_exp_adam": (C.c_int, [vp, vp, vp, vp, vp, vp, i64, C.c_float, C.c_float, C.c_float, C.c_float,
                                vp]),
    "glif_sample_bernoulli": (C.c_int, [vp, i64, C.c_uint64, C.c_uint64, vp, vp]),
    "glif_sample_poisson": (C.c_int, [C.c_float, C.c_float, i64, C.c_uint64, C.c_uint64, vp, vp]),
    "glif_prof_enable": (C.c_int, [C.c_uint32]),
    "glif_prof_stride": (C.c_int, [i32]),
    "glif_prof_collect": (C.c_int, [vp, vp, i32]),
    "glif_prof_name": (C.c_char_p, [i32]),
}

PROF_KINDS = ("push", "step", "adj", "bwd_rec", "bwd_lgn", "bwd_bkg", "syn_fwd", "syn_bwd", "lgn")


class GlifError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"libglif error {code}: {msg}")
        self.code = code


class GlifValueError(GlifError, ValueError):
    """Argument errors: the reference raises ValueError for these (models.py:299-315)."""


_lock = threading.Lock()
_lib = None


def lib():
    """Load libglif.so (raises if it was not built)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m v1_glif_model_amd.build` "
                    "(there is no CPU fallback)")
            L = C.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def check(rc: int):
    if rc != GLIF_OK:
        msg = lib().glif_last_error().decode(errors="replace")
        if rc in (GLIF_EINVAL, GLIF_ERANGE):
            raise GlifValueError(rc, msg)
        raise GlifError(rc, msg)


def stream_ptr(device=None):
    """The current torch stream of `device` as a hipStream_t (void*)."""
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(t):
    """Data pointer of a tensor (None for None)."""
    if t is None:
        return None
    return C.c_void_p(t.data_ptr())


def prof_enable(kinds):
    """Enable HIP-event timing of the named kernel classes (empty: off)."""
    mask = 0
    for k in kinds:
        mask |= 1 << PROF_KINDS.index(k)
    check(lib().glif_prof_enable(mask))


def prof_stride(every: int):
    """Bracket only every `every`-th launch of an enabled class (1: all)."""
    check(lib().glif_prof_stride(int(every)))


def prof_collect():
    """{kind: (total_ms, launches)} since the last collect (waits for the events)."""
    import numpy as np
    n = len(PROF_KINDS)
    tot = np.zeros(n, dtype=np.float64)
    cnt = np.zeros(n, dtype=np.int64)
    check(lib().glif_prof_collect(tot.ctypes.data_as(C.c_void_p), cnt.ctypes.data_as(C.c_void_p), n))
    return {k: (float(tot[i]), int(cnt[i])) for i, k in enumerate(PROF_KINDS) if cnt[i]}


def require_gpu():
    if not torch.cuda.is_available():
        raise RuntimeError("libglif needs a HIP GPU; none is visible (there is no CPU fallback)")
