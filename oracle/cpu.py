"""ctypes front end of ``glif_oracle.c`` (TEST INFRASTRUCTURE ONLY).

Builds ``oracle/_build/libglif_oracle.so`` with ``make`` on first use when it is
missing (gcc only, no GPU).  Every function mirrors one C entry point; see the C
file's header for the reference file:line each restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
import threading

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libglif_oracle.so")
_lock = threading.Lock()
_lib = None

i64p = C.POINTER(C.c_int64)
f32p = C.POINTER(C.c_float)
u8p = C.POINTER(C.c_uint8)
i32p = C.POINTER(C.c_int32)


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                build()
            L = C.CDLL(_LIB_PATH)
            L.orc_csr_build.restype = C.c_int
            L.orc_csr_build.argtypes = [i64p, C.c_int64, C.c_int64, i64p, i64p, i64p]
            L.orc_where_gt0.restype = C.c_int64
            L.orc_where_gt0.argtypes = [f32p, C.c_int64, C.c_int64, i64p]
            L.orc_syn_fwd.restype = None
            L.orc_syn_fwd.argtypes = [C.c_int, C.c_int64, C.c_int64, C.c_int, f32p, C.c_int,
                                      i64p, f32p, u8p, f32p, i64p, i64p, f32p]
            L.orc_syn_bwd.restype = None
            L.orc_syn_bwd.argtypes = [C.c_int, C.c_int64, C.c_int64, C.c_int, C.c_int64, f32p,
                                      C.c_int, i64p, i64p, f32p, u8p, f32p, i64p, i64p, f32p,
                                      f32p, f32p, f32p]
            L.orc_forward.restype = C.c_int
            L.orc_forward.argtypes = [C.POINTER(OrcCell), C.c_int, C.c_int, u8p, u8p, f32p, f32p,
                                      i32p, f32p, f32p, f32p, u8p, f32p, u8p]
            L.orc_set_threads.restype = C.c_int
            L.orc_set_threads.argtypes = [C.c_int]
            L.orc_backward.restype = C.c_int
            L.orc_backward.argtypes = [C.POINTER(OrcCell), C.c_int, C.c_int, u8p, u8p, f32p, u8p, u8p,
                                       f32p, f32p, f32p, f32p, f32p, f32p, f32p, f32p]
            _lib = L
    return _lib


def set_threads(n):
    """Threads of the oracle's OpenMP loops (results are the same for any count); returns
    the number in use."""
    return int(lib().orc_set_threads(int(n)))


def _p(a, t):
    if a is None:
        return None
    return a.ctypes.data_as(t)


class OrcTable(C.Structure):
    _fields_ = [("S", C.c_int64), ("n_cols", C.c_int64), ("post", i64p), ("col", i64p),
                ("order", i64p), ("row_splits", i64p), ("w", f32p), ("sid", u8p)]


class OrcCell(C.Structure):
    _fields_ = [("N", C.c_int64), ("D", C.c_int64), ("nb", C.c_int32), ("n_types", C.c_int32),
                ("decay", f32p), ("cf", f32p), ("asc_decay", f32p), ("asc_amps", f32p),
                ("tref", i32p), ("syn_decay", f32p), ("psc_initial", f32p), ("basis", f32p),
                ("dt", C.c_float), ("lr_scale", C.c_float), ("vgd", C.c_float), ("rd", C.c_float),
                ("gauss_std", C.c_float), ("damp", C.c_float), ("pseudo_gauss", C.c_int32),
                ("hard_reset", C.c_int32), ("rec", OrcTable), ("lgn", OrcTable), ("bkg", OrcTable)]


class OracleError(ValueError):
    pass


def csr_build(cols, n_cols):
    """models.py:317-341 restated in C: returns (order int64 [S], row_splits int64 [n_cols+1])."""
    cols = np.ascontiguousarray(cols, dtype=np.int64)
    S = cols.size
    order = np.empty(S, dtype=np.int64)
    splits = np.empty(int(n_cols) + 1 if n_cols > 0 else 1, dtype=np.int64)
    bad = np.zeros(1, dtype=np.int64)
    rc = lib().orc_csr_build(_p(cols, i64p), S, int(n_cols), _p(order, i64p), _p(splits, i64p),
                             _p(bad, i64p))
    if rc == -22:
        raise OracleError(f"`n_source_neurons` must be > 0, got {n_cols}.")
    if rc == -34:
        raise OracleError(f"Presynaptic index {int(cols[bad[0]])} is out of bounds for "
                          f"`n_source_neurons={n_cols}`.")
    if rc != 0:
        raise OracleError(f"orc_csr_build failed: {rc}")
    return order, splits


def where_gt0(z):
    """models.py:128: row-major [n, 2] int64 list of entries > 0."""
    z = np.ascontiguousarray(z, dtype=np.float32)
    rows, cols = z.shape
    n = lib().orc_where_gt0(_p(z, f32p), rows, cols, None)
    out = np.empty((n, 2), dtype=np.int64)
    lib().orc_where_gt0(_p(z, f32p), rows, cols, _p(out, i64p))
    return out


class _Tab:
    """Table arrays kept alive for the C structs that point into them."""

    def __init__(self, tab):
        self.post = np.ascontiguousarray(tab.post, dtype=np.int64)
        self.col = np.ascontiguousarray(tab.col, dtype=np.int64)
        self.w = np.ascontiguousarray(tab.weight, dtype=np.float32)
        self.sid = np.ascontiguousarray(tab.syn_id, dtype=np.uint8)
        self.order, self.splits = csr_build(self.col, tab.n_cols)
        self.n_post, self.n_cols = tab.n_post, tab.n_cols

    def set_weight(self, w):
        self.w[...] = np.asarray(w, dtype=np.float32)

    def struct(self):
        return OrcTable(self.post.size, self.n_cols, _p(self.post, i64p), _p(self.col, i64p),
                        _p(self.order, i64p), _p(self.splits, i64p), _p(self.w, f32p),
                        _p(self.sid, u8p))


def syn_fwd(table, act, basis, use_count=False):
    """Forward of calculate_synaptic_currents (models.py:126-169) in fp32 reference order.

    act: [B, n_cols] float (event where > 0).  Returns I [B*n_post, nb] float32.
    """
    t = table if isinstance(table, _Tab) else _Tab(table)
    act = np.ascontiguousarray(act, dtype=np.float32)
    basis = np.ascontiguousarray(basis, dtype=np.float32)
    B = act.shape[0]
    nb = basis.shape[1]
    I = np.zeros((B * t.n_post, nb), dtype=np.float32)
    lib().orc_syn_fwd(B, t.n_post, t.n_cols, nb, _p(act, f32p), int(use_count), _p(t.post, i64p),
                      _p(t.w, f32p), _p(t.sid, u8p), _p(basis, f32p), _p(t.order, i64p),
                      _p(t.splits, i64p), _p(I, f32p))
    return I


def syn_bwd(table, act, basis, dy, want_dz=True, want_dw=True, use_count=False):
    """Custom gradient of calculate_synaptic_currents (models.py:174-261), fp32.

    Returns (dz [B, n_cols] or None, dW [S] or None).
    """
    t = table if isinstance(table, _Tab) else _Tab(table)
    act = np.ascontiguousarray(act, dtype=np.float32)
    basis = np.ascontiguousarray(basis, dtype=np.float32)
    dy = np.ascontiguousarray(dy, dtype=np.float32)
    B = act.shape[0]
    nb = basis.shape[1]
    dz = np.empty((B, t.n_cols), dtype=np.float32) if want_dz else None
    scr = np.empty((B, t.n_cols), dtype=np.float32) if want_dz else None
    dW = np.zeros(t.post.size, dtype=np.float32) if want_dw else None
    lib().orc_syn_bwd(B, t.n_post, t.n_cols, nb, t.post.size, _p(act, f32p), int(use_count),
                      _p(t.post, i64p), _p(t.col, i64p), _p(t.w, f32p), _p(t.sid, u8p),
                      _p(basis, f32p), _p(t.order, i64p), _p(t.splits, i64p), _p(dy, f32p),
                      _p(dz, f32p), _p(dW, f32p), _p(scr, f32p))
    return dz, dW


class OracleCell:
    """The T-step GLIF_3 cell (models.py:1059-1135) and its BPTT on the CPU."""

    def __init__(self, tables, vgd=0.5, rd=0.5, gauss_std=0.5, damp=0.5, pseudo_gauss=True,
                 hard_reset=False):
        tb = tables
        self.tb = tb
        self.N, self.D, self.nb = tb.n_neurons, tb.max_delay, tb.n_basis
        self._keep = dict(
            decay=np.ascontiguousarray(tb.decay, np.float32),
            cf=np.ascontiguousarray(tb.current_factor, np.float32),
            ad=np.ascontiguousarray(tb.asc_decay, np.float32),
            amp=np.ascontiguousarray(tb.asc_amps, np.float32),
            tref=np.ascontiguousarray(tb.t_ref_steps, np.int32),
            sd=np.ascontiguousarray(tb.syn_decay, np.float32),
            p0=np.ascontiguousarray(tb.psc_initial, np.float32),
            basis=np.ascontiguousarray(tb.basis, np.float32))
        self.rec, self.lgn, self.bkg = _Tab(tb.rec), _Tab(tb.lgn), _Tab(tb.bkg)
        k = self._keep
        self.c = OrcCell(self.N, self.D, self.nb, tb.basis.shape[0], _p(k["decay"], f32p),
                         _p(k["cf"], f32p), _p(k["ad"], f32p), _p(k["amp"], f32p),
                         _p(k["tref"], i32p), _p(k["sd"], f32p), _p(k["p0"], f32p),
                         _p(k["basis"], f32p), tb.dt, tb.lr_scale, vgd, rd, gauss_std, damp,
                         int(pseudo_gauss), int(hard_reset), self.rec.struct(), self.lgn.struct(),
                         self.bkg.struct())

    def zero_state(self, B):
        N, D, nb = self.N, self.D, self.nb
        return dict(zbuf=np.zeros((B, D * N), np.float32), v=np.zeros((B, N), np.float32),
                    r=np.zeros((B, N), np.int32), asc=np.zeros((B, N * 2), np.float32),
                    psc_rise=np.zeros((B, N * nb), np.float32),
                    psc=np.zeros((B, N * nb), np.float32))

    def forward(self, lgn, bkg, state=None, record=True):
        """Run T steps.  lgn [T,B,n_lgn] uint8, bkg [T,B,n_bkg] uint8.

        Returns (z [T,B,N] uint8, v [T,B,N] float32, ref [T,B,N] uint8, state)."""
        lgn = np.ascontiguousarray(lgn, np.uint8)
        bkg = np.ascontiguousarray(bkg, np.uint8)
        T, B = lgn.shape[:2]
        st = self.zero_state(B) if state is None else {k: np.ascontiguousarray(v).copy()
                                                        for k, v in state.items()}
        z = np.zeros((T, B, self.N), np.uint8) if record else None
        v = np.zeros((T, B, self.N), np.float32) if record else None
        ref = np.zeros((T, B, self.N), np.uint8) if record else None
        rc = lib().orc_forward(C.byref(self.c), T, B, _p(lgn, u8p), _p(bkg, u8p),
                               _p(st["zbuf"], f32p), _p(st["v"], f32p), _p(st["r"], i32p),
                               _p(st["asc"], f32p), _p(st["psc_rise"], f32p), _p(st["psc"], f32p),
                               _p(z, u8p), _p(v, f32p), _p(ref, u8p))
        if rc != 0:
            raise OracleError(f"orc_forward failed: {rc}")
        return z, v, ref, st

    def backward(self, lgn, bkg, z, ref, v, gz_loss=None, gz_neuron=None, gv_loss=None,
                 want=("rec", "lgn", "bkg"), want_gz=False, zbuf0=None):
        """BPTT of a forward with outputs z, ref, v (and initial spike history zbuf0
        [B, D*N], None for zero); returns the weight gradients {rec, lgn, bkg}."""
        zb0 = None if zbuf0 is None else np.ascontiguousarray(zbuf0, np.float32)
        lgn = np.ascontiguousarray(lgn, np.uint8)
        bkg = np.ascontiguousarray(bkg, np.uint8)
        T, B = lgn.shape[:2]
        z = np.ascontiguousarray(z, np.uint8)
        ref = np.ascontiguousarray(ref, np.uint8)
        v = np.ascontiguousarray(v, np.float32)
        gzl = None if gz_loss is None else np.ascontiguousarray(gz_loss, np.float32)
        gzn = None if gz_neuron is None else np.ascontiguousarray(gz_neuron, np.float32)
        gvl = None if gv_loss is None else np.ascontiguousarray(gv_loss, np.float32)
        dW = {k: (np.zeros(getattr(self, k).post.size, np.float32) if k in want else None)
              for k in ("rec", "lgn", "bkg")}
        gz_out = np.zeros((T, B, self.N), np.float32) if want_gz else None
        if zb0 is not None and zb0.shape != (B, self.D * self.N):
            raise OracleError("zbuf0 must be [B, D*N]")
        rc = lib().orc_backward(C.byref(self.c), T, B, _p(lgn, u8p), _p(bkg, u8p), _p(zb0, f32p), _p(z, u8p),
                                _p(ref, u8p), _p(v, f32p), _p(gzl, f32p), _p(gzn, f32p),
                                _p(gvl, f32p), _p(dW["rec"], f32p), _p(dW["lgn"], f32p),
                                _p(dW["bkg"], f32p), _p(gz_out, f32p))
        if rc != 0:
            raise OracleError(f"orc_backward failed: {rc}")
        if want_gz:
            return dW, gz_out
        return dW


def abs_tables(tables):
    """The cell tables with every weight and basis entry replaced by its absolute value."""
    import dataclasses
    tb = tables
    return dataclasses.replace(
        tb, basis=np.abs(np.asarray(tb.basis, np.float32)),
        rec=dataclasses.replace(tb.rec, weight=np.abs(tb.rec.weight)),
        lgn=dataclasses.replace(tb.lgn, weight=np.abs(tb.lgn.weight)),
        bkg=dataclasses.replace(tb.bkg, weight=np.abs(tb.bkg.weight)))


def bptt_abs_scale(tables, lgn, bkg, z, ref, v, gz_loss=None, gz_neuron=None, gv_loss=None,
                   want=("rec", "lgn", "bkg"), zbuf0=None, **cell_kw):
    """Per-element scale of the BPTT weight gradients: the same reverse pass with every
    signed factor (weights, basis entries, loss gradients) replaced by its absolute value.
    Every other factor of the adjoint (surrogate, decays, current factors, PSC constants,
    dampening scales) is non-negative, so each output is the sum of the absolute values of
    all the terms that make up that gradient element -- the quantity fp32 rounding errors of
    any summation order are proportional to."""
    ab = lambda a: None if a is None else np.abs(np.asarray(a, np.float32))
    oc = OracleCell(abs_tables(tables), **cell_kw)
    return oc.backward(lgn, bkg, z, ref, v, gz_loss=ab(gz_loss), gz_neuron=ab(gz_neuron),
                       gv_loss=ab(gv_loss), want=want, zbuf0=zbuf0)
