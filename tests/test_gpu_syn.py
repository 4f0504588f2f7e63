"""GPU parity of the synaptic-current operator (CSR build, spike compaction, currents, dz, dW) against the CPU oracle.

Bars: compaction and CSR/CSC bit-exact; deterministic forward bit-exact with the
oracle's reference-order fp32 sum; event (atomic) forward and the backward within
1e-5 relative / 1e-6 absolute (scaled, where a value is a sum with cancellation,
by the sum of absolute terms -- see each test).
"""
import numpy as np
import pytest
import torch

from oracle import cpu as orc
from oracle import dense
from tests.helpers import device_to_numpy, network, tiny_config

pytestmark = pytest.mark.gpu


def _setup(seed=0, dense_basis=True, **kw):
    from v1_glif_model_amd.ops import SynapseTable
    cfg = tiny_config(**kw)
    net, tb = network(cfg, seed=seed, dense_basis=dense_basis)
    t = SynapseTable(tb.rec.indices, tb.rec.syn_id, (tb.n_neurons, tb.rec.n_cols), tb.basis,
                     n_delay_slots=tb.max_delay)
    w = torch.tensor(tb.rec.weight, device="cuda")
    t.set_weights(w)
    return tb, t, w


def _spikes(rng, B, cols, p):
    return (rng.random((B, cols)) < p).astype(np.float32)


def test_pre_ind_table_on_device_matches_reference_build():
    """The table's device order/row_splits equal the reference's numpy fallback."""
    tb, t, _ = _setup()
    o_ptr, r_ptr = t.pre_ind_device()
    S, C = tb.rec.n_syn, tb.rec.n_cols
    ref_o, ref_r = dense.csr_build_numpy(tb.rec.col, C)
    np.testing.assert_array_equal(device_to_numpy(o_ptr, S, np.int32), ref_o)
    np.testing.assert_array_equal(device_to_numpy(r_ptr, C + 1, np.int32), ref_r)


@pytest.mark.parametrize("rows,cols,p", [(1, 1, 1.0), (3, 1000, 0.01), (5, 5000, 0.3), (2, 70001, 0.001),
                                         (4, 0, 0.5), (0, 10, 0.5)])
def test_where_matches_argwhere(rows, cols, p):
    from v1_glif_model_amd.ops import where_gt0
    rng = np.random.default_rng(rows * 7919 + cols)
    z = (rng.random((rows, cols)) < p).astype(np.float32) * rng.choice([1.0, 0.5, 2.0], (rows, cols)).astype(np.float32)
    if rows and cols:
        z[0, -1] = -1.0  # negative values are not events
    got = where_gt0(torch.tensor(z, device="cuda")).cpu().numpy()
    np.testing.assert_array_equal(got, np.argwhere(z > 0))


@pytest.mark.parametrize("seed", [0, 1])
@pytest.mark.parametrize("B", [1, 3, 8, 20, 32])
def test_syn_fwd_deterministic_is_bit_exact(seed, B):
    tb, t, _ = _setup(seed=seed)
    rng = np.random.default_rng(100 + seed)
    z = _spikes(rng, B, tb.rec.n_cols, 0.05)
    got = t.forward(torch.tensor(z, device="cuda"), mode="deterministic").cpu().numpy()
    ref = orc.syn_fwd(tb.rec, z, tb.basis)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_syn_fwd_deterministic_widest_accumulators():
    """B = 32 and 8 receptors: 256 (batch, receptor) sums per row, all 8 accumulator slots of
    every lane of the half-wave row pull; bit-exact with the oracle, spikes and counts."""
    import dataclasses
    from v1_glif_model_amd.ops import SynapseTable
    cfg = dataclasses.replace(tiny_config(n=257), n_basis=8)
    _, tb = network(cfg, seed=13, dense_basis=True)
    t = SynapseTable(tb.rec.indices, tb.rec.syn_id, (tb.n_neurons, tb.rec.n_cols), tb.basis,
                     n_delay_slots=tb.max_delay)
    t.set_weights(torch.tensor(tb.rec.weight, device="cuda"))
    rng = np.random.default_rng(14)
    for counts in (False, True):
        z = _spikes(rng, 32, tb.rec.n_cols, 0.05)
        if counts:
            z *= rng.integers(1, 4, z.shape)
        got = t.forward(torch.tensor(z, device="cuda"), counts=counts, mode="deterministic").cpu().numpy()
        ref = orc.syn_fwd(tb.rec, z, tb.basis, use_count=counts)
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("B,nb", [(13, 5), (20, 5), (32, 5), (32, 8)])
def test_syn_fwd_deterministic_long_rows(B, nb):
    """The op's row pull with a whole wave per post row, taken by tables whose rows average at
    least 64 synapses when B * nb exceeds the chunk form's 64 lanes (2 and 4 slots per lane):
    bit-exact with the oracle."""
    import dataclasses
    from v1_glif_model_amd.ops import SynapseTable
    cfg = dataclasses.replace(tiny_config(n=300, fanin=100), n_basis=nb)
    _, tb = network(cfg, seed=17, dense_basis=True)
    assert tb.rec.n_syn >= 64 * tb.n_neurons
    t = SynapseTable(tb.rec.indices, tb.rec.syn_id, (tb.n_neurons, tb.rec.n_cols), tb.basis,
                     n_delay_slots=tb.max_delay)
    t.set_weights(torch.tensor(tb.rec.weight, device="cuda"))
    rng = np.random.default_rng(B * 10 + nb)
    for p in (0.01, 0.2):
        z = _spikes(rng, B, tb.rec.n_cols, p)
        got = t.forward(torch.tensor(z, device="cuda"), mode="deterministic").cpu().numpy()
        ref = orc.syn_fwd(tb.rec, z, tb.basis)
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("B", [4, 8, 20])
def test_syn_fwd_deterministic_bitmaps_beyond_lds(B):
    """An input table whose activity bitmap exceeds LDS (1.5M inputs: 183 KB of bits), so the
    row pulls read it from global memory: two rows per wave at B * nb = 20, a wave per row (rows
    of ~100 synapses) at 40 and 100; bit-exact with the oracle."""
    from v1_glif_model_amd.tables import SynapseTable as Tab
    from v1_glif_model_amd.ops import SynapseTable
    rng = np.random.default_rng(19)
    n_post, n_cols, fan = 600, 1500000, 100
    post = np.repeat(np.arange(n_post), fan)
    col = rng.integers(0, n_cols, post.size)
    _, first = np.unique(post * n_cols + col, return_index=True)
    post, col = post[first], col[first]
    o = np.lexsort((col, post))
    tab = Tab(post=post[o].astype(np.int64), col=col[o].astype(np.int64),
              weight=rng.normal(0, 1, o.size).astype(np.float32),
              syn_id=rng.integers(0, 5, o.size).astype(np.uint8), n_post=n_post, n_cols=n_cols)
    basis = rng.random((5, 5)).astype(np.float32)
    t = SynapseTable(tab.indices, tab.syn_id, (n_post, n_cols), basis)
    t.set_weights(torch.tensor(tab.weight, device="cuda"))
    z = _spikes(rng, B, tab.n_cols, 0.01)
    got = t.forward(torch.tensor(z, device="cuda"), mode="deterministic").cpu().numpy()
    ref = orc.syn_fwd(tab, z, basis)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_syn_fwd_deterministic_input_table_bit_exact():
    """The op on an input population's table (one delay slot, n_pre != n_post)."""
    from v1_glif_model_amd.ops import SynapseTable
    cfg = tiny_config(n_lgn=333, lgn_fanin=12)
    net, tb = network(cfg, seed=5, dense_basis=True)
    t = SynapseTable(tb.lgn.indices, tb.lgn.syn_id, (tb.n_neurons, tb.lgn.n_cols), tb.basis)
    t.set_weights(torch.tensor(tb.lgn.weight, device="cuda"))
    rng = np.random.default_rng(12)
    for B in (2, 9, 32):   # 32 x 5 receptors: the half-wave row pull, not the chunk form
        z = _spikes(rng, B, tb.lgn.n_cols, 0.1)
        got = t.forward(torch.tensor(z, device="cuda"), mode="deterministic").cpu().numpy()
        ref = orc.syn_fwd(tb.lgn, z, tb.basis)
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("B", [1, 5, 17])
def test_syn_fwd_event_within_tolerance(B):
    tb, t, _ = _setup(seed=2)
    rng = np.random.default_rng(7)
    z = _spikes(rng, B, tb.rec.n_cols, 0.05)
    got = t.forward(torch.tensor(z, device="cuda"), mode="event").cpu().numpy()
    ref = orc.syn_fwd(tb.rec, z, tb.basis)
    scale = dense.syn_fwd_abs(tb.rec, z, tb.basis)
    assert np.max(np.abs(got - ref) - 1e-5 * scale) <= 1e-6
    exact = dense.syn_fwd_f64(tb.rec, z, tb.basis)
    assert np.max(np.abs(got - exact) - 1e-5 * scale) <= 1e-6


def test_syn_fwd_counts_scale_weights():
    """Background form: events carry a count and the weight is scaled by it."""
    tb, t, _ = _setup(seed=3)
    rng = np.random.default_rng(9)
    z = rng.poisson(0.3, (2, tb.rec.n_cols)).astype(np.float32)
    for mode in ("deterministic", "event"):
        got = t.forward(torch.tensor(z, device="cuda"), counts=True, mode=mode).cpu().numpy()
        ref = orc.syn_fwd(tb.rec, z, tb.basis, use_count=True)
        if mode == "deterministic":
            np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
        else:
            scale = dense.syn_fwd_abs(tb.rec, z, tb.basis, use_count=True)
            assert np.max(np.abs(got - ref) - 1e-5 * scale) <= 1e-6


@pytest.mark.parametrize("B", [1, 5, 9])
def test_syn_bwd_matches_oracle(B):
    tb, t, _ = _setup(seed=4)
    rng = np.random.default_rng(11)
    z = _spikes(rng, B, tb.rec.n_cols, 0.05)
    dy = rng.normal(0, 1, (B * tb.n_neurons, tb.n_basis)).astype(np.float32)
    dz, dw = t.backward(torch.tensor(z, device="cuda"), torch.tensor(dy, device="cuda"))
    dz, dw = dz.cpu().numpy(), dw.cpu().numpy()
    rdz, rdw = orc.syn_bwd(tb.rec, z, tb.basis, dy)
    dz64, dw64, dz_abs, dw_abs = dense.syn_bwd_f64(tb.rec, z, tb.basis, dy)
    for got, ref, ex, sc, what in ((dz, rdz, dz64, dz_abs, "dz"), (dw, rdw, dw64, dw_abs, "dW")):
        assert np.max(np.abs(got - ref) - 1e-5 * sc) <= 1e-6, what
        assert np.max(np.abs(got - ex) - 1e-5 * sc) <= 1e-6, what


@pytest.mark.parametrize("B", [1, 5])
def test_op_on_a_table_without_synapses(B):
    """S = 0 (every column empty): both forwards give zero currents, the gradient zero dz and an
    empty dW, without a launch of zero workgroups."""
    from v1_glif_model_amd.ops import SynapseTable
    n_post, D, nb = 70, 3, 5
    t = SynapseTable(np.zeros((0, 2), np.int64), np.zeros(0, np.uint8), (n_post, D * n_post),
                     np.eye(5, nb, dtype=np.float32), n_delay_slots=D)
    t.set_weights(torch.zeros(0, dtype=torch.float32, device="cuda"))
    z = torch.tensor(_spikes(np.random.default_rng(B), B, D * n_post, 0.3), device="cuda")
    for mode in ("deterministic", "event"):
        I = t.forward(z, mode=mode).cpu().numpy()
        assert I.shape == (B * n_post, nb) and not np.any(I)
    dz, dw = t.backward(z, torch.ones((B * n_post, nb), dtype=torch.float32, device="cuda"))
    assert dz.shape == (B, D * n_post) and not torch.any(dz).item()
    assert dw.numel() == 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("B,nb", [(17, 8), (32, 8), (32, 1), (3, 2)])
def test_syn_bwd_wide_and_narrow_rows(B, nb):
    """G rows of 32 floats (B = 17-32, the type-phased column walk) and of 4 floats (B <= 4),
    8 receptors and 1: the G build's dy tile at its smallest (8 posts of 32 batch entries x 8
    receptors) and its largest, padding entries written as zero."""
    import dataclasses
    from v1_glif_model_amd.ops import SynapseTable
    cfg = dataclasses.replace(tiny_config(n=257), n_basis=nb)
    _, tb = network(cfg, seed=9, dense_basis=True)
    t = SynapseTable(tb.rec.indices, tb.rec.syn_id, (tb.n_neurons, tb.rec.n_cols), tb.basis,
                     n_delay_slots=tb.max_delay)
    t.set_weights(torch.tensor(tb.rec.weight, device="cuda"))
    rng = np.random.default_rng(B * 10 + nb)
    z = _spikes(rng, B, tb.rec.n_cols, 0.05)
    dy = rng.normal(0, 1, (B * tb.n_neurons, tb.n_basis)).astype(np.float32)
    dz, dw = t.backward(torch.tensor(z, device="cuda"), torch.tensor(dy, device="cuda"))
    dz, dw = dz.cpu().numpy(), dw.cpu().numpy()
    rdz, rdw = orc.syn_bwd(tb.rec, z, tb.basis, dy)
    _, _, dz_abs, dw_abs = dense.syn_bwd_f64(tb.rec, z, tb.basis, dy)
    assert np.max(np.abs(dz - rdz) - 1e-5 * dz_abs) <= 1e-6
    assert np.max(np.abs(dw - rdw) - 1e-5 * dw_abs) <= 1e-6
    assert np.count_nonzero(dw) > 0


@pytest.mark.parametrize("B", [5, 12])
def test_syn_bwd_counts_and_partial_requests(B):
    """Poisson-count inputs (dW scaled by the count, models.py:917-931) through the grouped
    row-sliced dz walk (8- and 16-float G rows) and the active-column dW pass; dz-only and
    dW-only calls give the same values as the full call."""
    tb, t, _ = _setup(seed=7, n=301)
    rng = np.random.default_rng(B)
    z = (rng.random((B, tb.rec.n_cols)) < 0.08).astype(np.float32) * rng.integers(1, 4, (B, tb.rec.n_cols))
    z = z.astype(np.float32)
    dy = rng.normal(0, 1, (B * tb.n_neurons, tb.n_basis)).astype(np.float32)
    zt, dyt = torch.tensor(z, device="cuda"), torch.tensor(dy, device="cuda")
    dz, dw = t.backward(zt, dyt, counts=True)
    dz, dw = dz.cpu().numpy(), dw.cpu().numpy()
    rdz, rdw = orc.syn_bwd(tb.rec, z, tb.basis, dy, use_count=True)
    _, _, dz_abs, dw_abs = dense.syn_bwd_f64(tb.rec, z, tb.basis, dy, use_count=True)
    assert np.max(np.abs(dz - rdz) - 1e-5 * dz_abs) <= 1e-6
    assert np.max(np.abs(dw - rdw) - 1e-5 * dw_abs) <= 1e-6
    assert np.count_nonzero(dw) > 0
    dz_only, none_w = t.backward(zt, dyt, counts=True, want_dw=False)
    none_z, dw_only = t.backward(zt, dyt, counts=True, want_dz=False)
    assert none_w is None and none_z is None
    np.testing.assert_array_equal(dz_only.cpu().numpy(), dz)
    np.testing.assert_array_equal(dw_only.cpu().numpy(), dw)


def _long_column_table(seed=3, n_post=6000, lens=None):
    """A table with columns longer than the dz walk handles well (the background table's
    shape) beside the other work-unit kinds: long columns split into 1024-synapse chunks
    (4097 entries: a 1-synapse last chunk), columns of 1025-2049, single columns too long to
    share a run (700), runs of up to 64 short columns, and empty columns among them."""
    from v1_glif_model_amd.tables import SynapseTable as Tab
    rng = np.random.default_rng(seed)
    if lens is None:
        lens = [5000, 0, 700, 700, 4097, 1025, 3, 0] + list(rng.integers(0, 40, 70)) + [2049, 1024, 0, 6000]
    post, col = [], []
    for c, n in enumerate(lens):
        p = rng.choice(n_post, size=int(n), replace=False)
        post.append(p)
        col.append(np.full(int(n), c))
    post, col = np.concatenate(post).astype(np.int64), np.concatenate(col).astype(np.int64)
    o = np.lexsort((col, post))            # the reference's (post, pre) order
    post, col = post[o], col[o]
    S = post.size
    return Tab(post=post, col=col, weight=rng.normal(0, 1, S).astype(np.float32),
               syn_id=rng.integers(0, 5, S).astype(np.uint8), n_post=n_post, n_cols=len(lens))


@pytest.mark.parametrize("B", [1, 5, 12, 32])
def test_syn_bwd_long_columns(B):
    """dz of a table with columns of thousands of synapses over the weight-gradient work
    units (a wave per unit; a chunked column's units summed in order), with the dW pass
    beside it; Poisson-count inputs, and dz-only / dW-only calls equal to the full call."""
    from v1_glif_model_amd.ops import SynapseTable
    tab = _long_column_table()
    rng = np.random.default_rng(B + 70)
    basis = rng.random((5, 3)).astype(np.float32)
    t = SynapseTable(tab.indices, tab.syn_id, (tab.n_post, tab.n_cols), basis)
    t.set_weights(torch.tensor(tab.weight, device="cuda"))
    z = ((rng.random((B, tab.n_cols)) < 0.5) * rng.integers(1, 3, (B, tab.n_cols))).astype(np.float32)
    dy = rng.normal(0, 1, (B * tab.n_post, 3)).astype(np.float32)
    zt, dyt = torch.tensor(z, device="cuda"), torch.tensor(dy, device="cuda")
    dz, dw = t.backward(zt, dyt, counts=True)
    dz, dw = dz.cpu().numpy(), dw.cpu().numpy()
    rdz, rdw = orc.syn_bwd(tab, z, basis, dy, use_count=True)
    _, _, dz_abs, dw_abs = dense.syn_bwd_f64(tab, z, basis, dy, use_count=True)
    assert np.max(np.abs(dz - rdz) - 1e-5 * dz_abs) <= 1e-6
    assert np.max(np.abs(dw - rdw) - 1e-5 * dw_abs) <= 1e-6
    assert np.all(dz[:, [1, 7]] == 0) and np.count_nonzero(dz[:, 0]) == B
    dz_only, _ = t.backward(zt, dyt, counts=True, want_dw=False)
    _, dw_only = t.backward(zt, dyt, counts=True, want_dz=False)
    np.testing.assert_array_equal(dz_only.cpu().numpy(), dz)
    np.testing.assert_array_equal(dw_only.cpu().numpy(), dw)


@pytest.mark.parametrize("B", [1, 5, 17])
def test_syn_fwd_long_columns(B):
    """Both forwards on the long-column table (event mode pulls there as well: each active
    input would cost an atomic per synapse of its column), spikes and Poisson counts; the
    deterministic pull bit-exact."""
    from v1_glif_model_amd.ops import SynapseTable
    tab = _long_column_table(seed=4)
    rng = np.random.default_rng(B + 90)
    basis = rng.random((5, 3)).astype(np.float32)
    t = SynapseTable(tab.indices, tab.syn_id, (tab.n_post, tab.n_cols), basis)
    t.set_weights(torch.tensor(tab.weight, device="cuda"))
    for counts in (False, True):
        z = (rng.random((B, tab.n_cols)) < 0.5).astype(np.float32)
        if counts:
            z *= rng.integers(1, 4, z.shape)
        zt = torch.tensor(z, device="cuda")
        got = t.forward(zt, counts=counts, mode="event").cpu().numpy()
        ref = orc.syn_fwd(tab, z, basis, use_count=counts)
        scale = dense.syn_fwd_abs(tab, z, basis, use_count=counts)
        assert np.max(np.abs(got - ref) - 1e-5 * scale) <= 1e-6
        assert np.max(np.abs(got - dense.syn_fwd_f64(tab, z, basis, use_count=counts)) - 1e-5 * scale) <= 1e-6
        det = t.forward(zt, counts=counts, mode="deterministic").cpu().numpy()
        np.testing.assert_array_equal(det.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("B", [1, 5, 32])
def test_syn_fwd_event_medium_columns(B):
    """The event push over work units on a table whose longest column (2048 synapses) still
    pushes: columns of 1025-2048 split into 1024-synapse chunks on waves of their own, runs of
    short columns, empty columns; spikes and Poisson counts."""
    from v1_glif_model_amd.ops import SynapseTable
    rng0 = np.random.default_rng(21)
    lens = [2048, 0, 1025, 700, 700, 1500, 3, 0] + list(rng0.integers(0, 40, 70)) + [1024, 2000, 0]
    tab = _long_column_table(seed=6, lens=lens)
    rng = np.random.default_rng(B + 120)
    basis = rng.random((5, 3)).astype(np.float32)
    t = SynapseTable(tab.indices, tab.syn_id, (tab.n_post, tab.n_cols), basis)
    t.set_weights(torch.tensor(tab.weight, device="cuda"))
    for counts in (False, True):
        z = (rng.random((B, tab.n_cols)) < 0.5).astype(np.float32)
        if counts:
            z *= rng.integers(1, 4, z.shape)
        got = t.forward(torch.tensor(z, device="cuda"), counts=counts, mode="event").cpu().numpy()
        ref = orc.syn_fwd(tab, z, basis, use_count=counts)
        scale = dense.syn_fwd_abs(tab, z, basis, use_count=counts)
        assert np.max(np.abs(got - ref) - 1e-5 * scale) <= 1e-6


def test_syn_fwd_workspace_rules():
    """glif_syn_fwd refuses a NULL or short workspace wherever its pull builds batch masks
    there (spikes in deterministic mode; spikes on a table with columns over 2048 synapses in
    event mode too) before any launch, and runs without one where nothing uses it (the event
    push, the pull of counts), with the results of a call that has one."""
    from v1_glif_model_amd import _lib
    from v1_glif_model_amd.ops import MODES, SynapseTable
    rng = np.random.default_rng(33)
    long_tab = _long_column_table(seed=8)
    long_basis = rng.random((5, 3)).astype(np.float32)
    t_long = SynapseTable(long_tab.indices, long_tab.syn_id, (long_tab.n_post, long_tab.n_cols), long_basis)
    t_long.set_weights(torch.tensor(long_tab.weight, device="cuda"))
    tb, t_short, _ = _setup(seed=4)
    B = 3
    for tab, t, basis, long_cols in ((long_tab, t_long, long_basis, True), (tb.rec, t_short, tb.basis, False)):
        for mode in ("event", "deterministic"):
            for counts in (False, True):
                z = (rng.random((B, tab.n_cols)) < 0.2).astype(np.float32)
                zt = torch.tensor(z, device="cuda")
                I = torch.empty((B * t.n_post, t.n_basis), dtype=torch.float32, device="cuda")
                ws = t.workspace(B, zt.device)
                needs = not counts and (mode == "deterministic" or long_cols)
                for w_ptr, w_bytes in ((None, 0), (_lib.ptr(ws), 1)):   # none, and one byte short of all
                    rc = _lib.lib().glif_syn_fwd(t.handle, _lib.ptr(zt), B, int(counts), MODES[mode],
                                                 _lib.ptr(I), w_ptr, w_bytes, _lib.stream_ptr())
                    what = (long_cols, mode, counts, w_bytes)
                    if needs:
                        assert rc == -12, what   # GLIF_ENOMEM, nothing launched
                        continue
                    assert rc == 0, (what, _lib.lib().glif_last_error())
                    got = I.cpu().numpy()
                    ref = orc.syn_fwd(tab, z, basis, use_count=counts)
                    if mode == "deterministic" or long_cols:   # pulled: the reference's sums
                        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
                    else:
                        scale = dense.syn_fwd_abs(tab, z, basis, use_count=counts)
                        assert np.max(np.abs(got - ref) - 1e-5 * scale) <= 1e-6


def test_syn_fwd_event_column_scan():
    """The event push's column scan (a wave per 64 columns), taken by tables of at least
    131,072 columns with no long column: 150,001 columns of 0-3 synapses."""
    from v1_glif_model_amd.ops import SynapseTable
    tab = _wide_table()
    rng = np.random.default_rng(12)
    basis = rng.random((3, 2)).astype(np.float32)
    t = SynapseTable(tab.indices, tab.syn_id, (tab.n_post, tab.n_cols), basis)
    t.set_weights(torch.tensor(tab.weight, device="cuda"))
    z = (rng.random((3, tab.n_cols)) < 0.05).astype(np.float32)
    got = t.forward(torch.tensor(z, device="cuda"), mode="event").cpu().numpy()
    ref = orc.syn_fwd(tab, z, basis)
    scale = dense.syn_fwd_abs(tab, z, basis)
    assert np.max(np.abs(got - ref) - 1e-5 * scale) <= 1e-6


def _wide_table(seed=11, n_post=2000, n_cols=150001, n_types=3):
    """A table of many short columns (0-3 synapses each): its dz walk has enough lanes at every
    batch width, so the op walks it (grouped or type-phased) instead of using the work units."""
    from v1_glif_model_amd.tables import SynapseTable as Tab
    rng = np.random.default_rng(seed)
    col = np.repeat(np.arange(n_cols), rng.integers(0, 4, n_cols))
    post = rng.integers(0, n_post, col.size)
    _, first = np.unique(post * n_cols + col, return_index=True)   # distinct (post, column) pairs
    post, col = post[first], col[first]
    o = np.lexsort((col, post))
    return Tab(post=post[o].astype(np.int64), col=col[o].astype(np.int64),
               weight=rng.normal(0, 1, o.size).astype(np.float32),
               syn_id=rng.integers(0, n_types, o.size).astype(np.uint8), n_post=n_post, n_cols=n_cols)


@pytest.mark.parametrize("B", [2, 12, 32])
def test_syn_bwd_wide_table_walks(B):
    """The op's dz walks on a 150,001-column table: the type-phased column walk at 4- and
    32-float G rows (B = 2, 32; dW in the same walk) and the grouped row-sliced walk at 16-float
    rows (B = 12, dW over the work units beside it); spike and count inputs."""
    from v1_glif_model_amd.ops import SynapseTable
    tab = _wide_table()
    rng = np.random.default_rng(B + 140)
    basis = rng.random((3, 2)).astype(np.float32)
    t = SynapseTable(tab.indices, tab.syn_id, (tab.n_post, tab.n_cols), basis)
    t.set_weights(torch.tensor(tab.weight, device="cuda"))
    for counts in (False, True):
        z = (rng.random((B, tab.n_cols)) < 0.05).astype(np.float32)
        if counts:
            z *= rng.integers(1, 4, z.shape)
        dy = rng.normal(0, 1, (B * tab.n_post, 2)).astype(np.float32)
        dz, dw = t.backward(torch.tensor(z, device="cuda"), torch.tensor(dy, device="cuda"), counts=counts)
        dz, dw = dz.cpu().numpy(), dw.cpu().numpy()
        rdz, rdw = orc.syn_bwd(tab, z, basis, dy, use_count=counts)
        _, _, dz_abs, dw_abs = dense.syn_bwd_f64(tab, z, basis, dy, use_count=counts)
        assert np.max(np.abs(dz - rdz) - 1e-5 * dz_abs) <= 1e-6
        assert np.max(np.abs(dw - rdw) - 1e-5 * dw_abs) <= 1e-6
        assert np.count_nonzero(dw) > 0


@pytest.mark.parametrize("B", [5, 9])
def test_syn_bwd_input_table(B):
    """The backward on an input population's table (one delay slot, n_pre != n_post)."""
    from v1_glif_model_amd.ops import SynapseTable
    cfg = tiny_config(n_lgn=333, lgn_fanin=12)
    net, tb = network(cfg, seed=5, dense_basis=True)
    t = SynapseTable(tb.lgn.indices, tb.lgn.syn_id, (tb.n_neurons, tb.lgn.n_cols), tb.basis)
    t.set_weights(torch.tensor(tb.lgn.weight, device="cuda"))
    rng = np.random.default_rng(B + 40)
    z = _spikes(rng, B, tb.lgn.n_cols, 0.1)
    dy = rng.normal(0, 1, (B * tb.n_neurons, tb.n_basis)).astype(np.float32)
    dz, dw = t.backward(torch.tensor(z, device="cuda"), torch.tensor(dy, device="cuda"))
    rdz, rdw = orc.syn_bwd(tb.lgn, z, tb.basis, dy)
    _, _, dz_abs, dw_abs = dense.syn_bwd_f64(tb.lgn, z, tb.basis, dy)
    assert np.max(np.abs(dz.cpu().numpy() - rdz) - 1e-5 * dz_abs) <= 1e-6
    assert np.max(np.abs(dw.cpu().numpy() - rdw) - 1e-5 * dw_abs) <= 1e-6


def test_calculate_synaptic_currents_autograd():
    from v1_glif_model_amd.ops import calculate_synaptic_currents, make_pre_ind_table
    cfg = tiny_config()
    net, tb = network(cfg, seed=5, dense_basis=True)
    pre = make_pre_ind_table(tb.rec.indices, n_source_neurons=tb.rec.n_cols)
    rng = np.random.default_rng(3)
    B = 4
    z = torch.tensor(_spikes(rng, B, tb.rec.n_cols, 0.05), device="cuda", requires_grad=True)
    w = torch.tensor(tb.rec.weight, device="cuda", requires_grad=True)
    basis = torch.tensor(tb.basis)
    I = calculate_synaptic_currents(z, tb.rec.indices, w, w, (tb.n_neurons, tb.rec.n_cols), basis,
                                    tb.rec.syn_id, pre)
    dy = torch.tensor(rng.normal(0, 1, tuple(I.shape)).astype(np.float32), device="cuda")
    (I * dy).sum().backward()
    ref_I = orc.syn_fwd(tb.rec, z.detach().cpu().numpy(), tb.basis)
    scale = dense.syn_fwd_abs(tb.rec, z.detach().cpu().numpy(), tb.basis)
    assert np.max(np.abs(I.detach().cpu().numpy() - ref_I) - 1e-5 * scale) <= 1e-6
    rdz, rdw = orc.syn_bwd(tb.rec, z.detach().cpu().numpy(), tb.basis, dy.cpu().numpy())
    _, _, dz_abs, dw_abs = dense.syn_bwd_f64(tb.rec, z.detach().cpu().numpy(), tb.basis, dy.cpu().numpy())
    assert np.max(np.abs(z.grad.cpu().numpy() - rdz) - 1e-5 * dz_abs) <= 1e-6
    assert np.max(np.abs(w.grad.cpu().numpy() - rdw) - 1e-5 * dw_abs) <= 1e-6
