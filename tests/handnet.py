"""Hand-built networks for the closed-form tests: a few neurons, every parameter and synapse
written out, in the dictionary layout `load_sparse.load_v1` hands to `V1Column`
(`load_sparse.py:364-377, 464-470`)."""
import numpy as np

# tau of the five PSC basis functions (ms)
TAU_BASIS = np.array([2.0, 5.0, 10.0, 20.0, 50.0])


def node_params(types):
    """types: list of dicts with V_th, E_L, C_m, g, t_ref, k (2), asc_amps (2)."""
    f = lambda key: np.array([t[key] for t in types], dtype=np.float32)
    E_L = f("E_L")
    return dict(V_th=f("V_th"), E_L=E_L, V_reset=E_L.copy(), C_m=f("C_m"), g=f("g"), t_ref=f("t_ref"),
                k=f("k"), asc_amps=f("asc_amps"))


def population(n_inputs, rows, delays=None):
    """rows: (post, pre, weight, syn_id) sorted by (post, pre)."""
    d = dict(n_inputs=n_inputs,
             indices=np.array([[r[0], r[1]] for r in rows], dtype=np.int64).reshape(-1, 2),
             weights=np.array([r[2] for r in rows], dtype=np.float32),
             syn_ids=np.array([r[3] for r in rows], dtype=np.uint8))
    if delays is not None:
        d["delays"] = np.asarray(delays, dtype=np.float32)
    return d


def network(types, type_ids, rec_rows, lgn_rows, n_lgn, bkg_rows, n_bkg, lgn_delays=None, n_types=5):
    """rec_rows: (post, pre, weight, delay_ms, syn_id) sorted by (post, pre)."""
    N = len(type_ids)
    rec = dict(indices=np.array([[r[0], r[1]] for r in rec_rows], dtype=np.int64).reshape(-1, 2),
               weights=np.array([r[2] for r in rec_rows], dtype=np.float32),
               delays=np.array([r[3] for r in rec_rows], dtype=np.float32),
               syn_ids=np.array([r[4] for r in rec_rows], dtype=np.uint8),
               dense_shape=(N, N))
    net = dict(n_nodes=N, node_params=node_params(types), node_type_ids=np.asarray(type_ids, dtype=np.int64),
               synapses=rec, n_exc=N)
    return dict(network=net, lgn_input=population(n_lgn, lgn_rows, lgn_delays),
                bkg_input=population(n_bkg, bkg_rows), tau_basis=TAU_BASIS.copy(),
                basis=np.eye(n_types, TAU_BASIS.size, dtype=np.float32))


# three node types (V_th - E_L = 20, 10, 40 mV; tau_m = 10, 10, 20 ms)
TYPES = [
    dict(V_th=-50.0, E_L=-70.0, C_m=100.0, g=10.0, t_ref=2.5, k=[0.1, 0.02], asc_amps=[10.0, -4.0]),
    dict(V_th=-55.0, E_L=-65.0, C_m=50.0, g=5.0, t_ref=0.2, k=[0.3, 0.003], asc_amps=[-5.0, 1.0]),
    dict(V_th=-40.0, E_L=-80.0, C_m=80.0, g=4.0, t_ref=4.0, k=[0.05, 0.2], asc_amps=[8.0, 2.0]),
]


def four_neuron_network(lgn_delays=None):
    """Neurons 0..3 of types 0, 1, 2, 1.  Recurrent delays (ms) below dt, on x.5 (numpy
    rounds half to even), just below x.5 and above any max_delay flag used in the tests."""
    rec = [(0, 1, 4.0, 0.3, 2),     # delay below dt: clipped up to 1 step
           (0, 3, -6.0, 1.5, 0),    # 1.5 -> 2 (half to even)
           (1, 0, 2.5, 2.5, 1),     # 2.5 -> 2 (half to even)
           (1, 2, 1.0, 7.0, 4),     # beyond the max_delay flag 4: clipped to 4
           (2, 1, -10.0, 3.5, 3),   # 3.5 -> 4 (half to even)
           (3, 0, 3.0, 2.49, 0),    # 2.49 -> 2
           (3, 2, 0.5, 1.0, 2)]
    lgn = [(0, 2, 2.0, 0), (1, 0, 1.0, 1), (3, 1, 5.0, 2)]
    bkg = [(0, 0, 1.0, 3), (2, 1, 4.0, 4)]
    return network(TYPES, [0, 1, 2, 1], rec, lgn, 3, bkg, 2, lgn_delays=lgn_delays)


# one node type for the response tests: V_th - E_L = 20 mV, tau_m = 10 ms, g = 10 nS, no ASC
PLAIN = dict(V_th=-50.0, E_L=-70.0, C_m=100.0, g=10.0, t_ref=3.0, k=[0.1, 0.1], asc_amps=[0.0, 0.0])


def chain_network(w_rec=2.0, delay=3.0, sid_rec=1, w_lgn=(1.0, 1.0), sid_lgn=(3, 2)):
    """Neuron 0 -> neuron 1 through one recurrent synapse (weight w_rec mV, delay, syn_id
    sid_rec); LGN input 0 -> neuron 0 and input 1 -> neuron 1 (weights w_lgn, syn_ids
    sid_lgn); one background input wired to neuron 0 and never active."""
    rec = [(1, 0, w_rec, delay, sid_rec)]
    lgn = [(0, 0, w_lgn[0], sid_lgn[0]), (1, 1, w_lgn[1], sid_lgn[1])]
    bkg = [(0, 0, 1.0, 0)]
    return network([PLAIN, PLAIN], [0, 1], rec, lgn, 2, bkg, 1)
