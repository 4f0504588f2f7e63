"""synthetic.expand_receptors: the receptor-space form of a many-type network (each synapse split
into one synapse per receptor, weight w * basis[syn_id][r], identity basis) carries the same
synaptic currents and, through the chain rule dW = sum_r basis[syn_id][r] * dW_r, the same weight
gradient (checked on the CPU oracle's op, models.py:103-263)."""
import dataclasses

import numpy as np

from oracle import cpu as orc
from tests.helpers import tiny_config
from v1_glif_model_amd import synthetic as sy
from v1_glif_model_amd.tables import build_cell_tables


def test_expanded_network_has_the_same_currents_and_gradients():
    cfg = dataclasses.replace(tiny_config(n=200, fanin=20, delays=3), n_syn_types=121, n_basis=4)
    net = sy.make_network(cfg, seed=3, dense_basis=True)
    ex = sy.expand_receptors(net)
    tb, te = build_cell_tables(net), build_cell_tables(ex)
    nb = tb.n_basis
    assert te.rec.n_syn == nb * tb.rec.n_syn and te.basis.shape == (nb, nb)
    np.testing.assert_array_equal(te.rec.col, np.repeat(tb.rec.col, nb))
    rng = np.random.default_rng(4)
    B = 3
    z = (rng.uniform(size=(B, tb.rec.n_cols)) < 0.1).astype(np.float32)
    I0 = orc.syn_fwd(tb.rec, z, tb.basis)
    I1 = orc.syn_fwd(te.rec, z, te.basis)
    # (w / vs) * b against (w * b) / vs: a few ulp apart
    np.testing.assert_allclose(I1, I0, rtol=1e-5, atol=1e-7)
    dy = rng.normal(0, 1, (B * tb.n_neurons, nb)).astype(np.float32)
    dz0, dw0 = orc.syn_bwd(tb.rec, z, tb.basis, dy)
    dz1, dw1 = orc.syn_bwd(te.rec, z, te.basis, dy)
    scale = np.abs(dz0).max()
    assert np.max(np.abs(dz1 - dz0)) <= 1e-5 * scale
    b = tb.basis[tb.rec.syn_id.astype(np.int64)]                 # [S, nb]
    dw_chain = (dw1.reshape(-1, nb).astype(np.float64) * b).sum(1)
    assert np.max(np.abs(dw_chain - dw0)) <= 1e-5 * np.abs(dw0).max()


def test_class_types_structure():
    """synthetic.class_types: syn_id = pre_class * K + post_class (class 0 for the inputs), so a
    neuron receives at most K distinct types out of K * K, and the tables keep every synapse."""
    K = 11
    cfg = tiny_config(n=400, fanin=40, delays=3)
    net = sy.make_network(cfg, seed=5)
    ct = sy.class_types(net, n_classes=K)
    cls = ct["neuron_class"]
    n_exc = net["network"]["n_exc"]
    assert set(np.unique(cls[:n_exc])) <= set(range(1, K // 2 + 1))
    assert set(np.unique(cls[n_exc:])) <= set(range(K // 2 + 1, K))
    assert ct["basis"].shape == (K * K, net["basis"].shape[1])
    seen = [set() for _ in range(cfg.n_neurons)]
    for pop, src in ((ct["network"]["synapses"], cls), (ct["lgn_input"], None), (ct["bkg_input"], None)):
        post, pre = np.asarray(pop["indices"]).T
        sid = np.asarray(pop["syn_ids"]).astype(np.int64)
        np.testing.assert_array_equal(sid % K, cls[post])
        np.testing.assert_array_equal(sid // K, src[pre] if src is not None else 0)
        for p, s in zip(post, sid):
            seen[p].add(int(s))
    assert max(len(s) for s in seen) <= K
    tb = build_cell_tables(ct)
    assert tb.rec.n_syn == len(net["network"]["synapses"]["weights"])
