"""Writes ``cell_small.npz``: a small GLIF_3 network, its inputs, and the C oracle's
outputs for them (forward spikes, voltages and final state; BPTT weight gradients of a
fixed loss gradient; op-level currents and gradients).

The reference's own tests hold no golden vectors for this path, so the fixture is the
oracle's (``oracle/glif_oracle.c``, itself pinned by ``tests/test_oracle.py`` against
closed forms and a float64 autograd restatement).  It stores the network dictionaries
that ``V1Column.__init__`` takes (``models.py:450-773``; layout of
``load_sparse.load_v1``, ``load_sparse.py:364-377``) as flat arrays, not a seed, so it
stays valid if the synthetic generator changes.

Run from the repository root:  ``python tests/golden/make_golden.py``
"""
from __future__ import annotations

import dataclasses
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
PATH = os.path.join(HERE, "cell_small.npz")

# network and run of the fixture: 300 neurons, 3 delay slots, a dense basis table
NET = dict(n=300, fanin=30, delays=3, n_lgn=80, lgn_fanin=8, n_bkg=10, bkg_fanin=3,
           rs=2.0, ins=3.0, lgn_p=0.05)
T, B = 40, 2
ORC_KW = dict(vgd=0.5, rd=0.5, gauss_std=0.5, damp=0.5, pseudo_gauss=True)


def flatten(d, prefix=""):
    """Nested dict of arrays / scalars -> flat {"a/b/c": array}."""
    out = {}
    for k, v in d.items():
        key = f"{prefix}{k}"
        if isinstance(v, dict):
            out.update(flatten(v, key + "/"))
        else:
            out[key] = np.asarray(v)
    return out


def unflatten(flat, prefix):
    """Inverse of flatten for the keys under ``prefix`` (0-d arrays become scalars)."""
    out = {}
    for key, v in flat.items():
        if not key.startswith(prefix):
            continue
        parts = key[len(prefix):].split("/")
        node = out
        for p in parts[:-1]:
            node = node.setdefault(p, {})
        node[parts[-1]] = v.item() if v.ndim == 0 else v
    return out


def load():
    """(net dict, lgn [T,B,n_lgn] u8, bkg [T,B,n_bkg] u8, expected outputs dict)."""
    with np.load(PATH, allow_pickle=False) as f:
        flat = {k: f[k] for k in f.files}
    net = unflatten(flat, "net/")
    net["network"]["synapses"]["dense_shape"] = tuple(int(x) for x in net["network"]["synapses"]["dense_shape"])
    exp = unflatten(flat, "out/")
    for k in ("z", "ref"):
        exp[k] = np.unpackbits(exp[k + "_bits"])[: T * B * int(net["network"]["n_nodes"])].reshape(
            T, B, -1)
    return net, flat["in/lgn"], flat["in/bkg"], exp


def main():
    sys.path.insert(0, ROOT)
    from oracle.cpu import OracleCell, build, syn_bwd, syn_fwd
    from v1_glif_model_amd import synthetic as sy
    from v1_glif_model_amd.tables import build_cell_tables

    build()
    cfg = dataclasses.replace(
        sy.CONFIGS[0], n_neurons=NET["n"], fanin_mean=NET["fanin"], max_delay=NET["delays"],
        n_lgn=NET["n_lgn"], lgn_fanin=NET["lgn_fanin"], n_bkg=NET["n_bkg"], bkg_fanin=NET["bkg_fanin"],
        recurrent_weight_scale=NET["rs"], input_weight_scale=NET["ins"], lgn_p=NET["lgn_p"],
        seq_len=T, batch=B)
    net = sy.make_network(cfg, seed=11, dense_basis=True)
    lgn, bkg = sy.make_inputs(cfg, seed=12, seq_len=T, batch=B)
    tb = build_cell_tables(net)
    oc = OracleCell(tb, **ORC_KW)
    z, v, ref, st = oc.forward(lgn, bkg)
    rng = np.random.default_rng(13)
    gz = rng.normal(0, 1, z.shape).astype(np.float32)
    gv = rng.normal(0, 0.1, z.shape).astype(np.float32)
    dW = oc.backward(lgn, bkg, z, ref, v, gz_loss=gz, gv_loss=gv)
    # op level (currents, dz, dW) on the recurrent table: a random binary z and dy
    zop = (rng.random((B, tb.rec.n_cols)) < 0.05).astype(np.float32)
    dy = rng.normal(0, 1, (B * tb.n_neurons, tb.n_basis)).astype(np.float32)
    I_op = syn_fwd(tb.rec, zop, tb.basis)
    dz_op, dw_op = syn_bwd(tb.rec, zop, tb.basis, dy)
    # the generator's own config record is not part of the network dictionaries
    flat = flatten({k: v for k, v in net.items() if k != "cfg"}, "net/")
    flat.update({"in/lgn": lgn, "in/bkg": bkg, "in/gz": gz, "in/gv": gv, "in/z_op": zop, "in/dy_op": dy})
    out = {"z_bits": np.packbits(z.ravel()), "ref_bits": np.packbits(ref.ravel()), "v": v,
           "state": {k: st[k] for k in ("zbuf", "v", "r", "asc", "psc_rise", "psc")},
           "dW": {k: dW[k] for k in ("rec", "lgn", "bkg")},
           "op": {"I": I_op, "dz": dz_op, "dw": dw_op}}
    flat.update(flatten(out, "out/"))
    np.savez_compressed(PATH, **flat)
    print(f"wrote {PATH}: {os.path.getsize(PATH)} bytes; spikes {int(z.sum())}, "
          f"rate {z.mean() * 1000:.1f} Hz")


if __name__ == "__main__":
    main()
