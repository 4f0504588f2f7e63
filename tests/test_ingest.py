"""Network ingestion (load_sparse.py:75-97, 364-377; models.py:518-519, 614-622;
other_v1_utils.py:23-84): the loaders on small files of the reference's formats, and a
4-receptor network (the real model's receptor count) through the cell on the GPU,
bit-exact with the oracle in deterministic mode."""
import json
import os

import numpy as np
import pytest

from v1_glif_model_amd import ingest

REF_SYN = "/root/reference/synaptic_data"


def _basis_files(tmp_path, models, listing_extra=()):
    d = tmp_path / "synaptic_models"
    d.mkdir()
    for m in models:
        (d / f"{m}.json").write_text(json.dumps({"model": m}))
    for x in listing_extra:
        (d / x).write_text("not a model")
    csv = tmp_path / "basis_function_weights.csv"
    rng = np.random.default_rng(0)
    rows = {m: rng.uniform(-0.1, 1.3, 4) for m in list(models) + ["unused_model"]}
    csv.write_text("connection_name,w0,w1,w2,w3\n" +
                   "".join(f"{m},{','.join(repr(float(v)) for v in w)}\n" for m, w in rows.items()))
    return str(csv), str(d), rows


def test_tau_basis(tmp_path):
    p = tmp_path / "tau.npy"
    np.save(p, np.array([1.0, 2.0, 3.5, 5.5]))
    np.testing.assert_array_equal(ingest.load_tau_basis(str(p)), [1.0, 2.0, 3.5, 5.5])
    np.save(p, np.array([1.0, -2.0]))
    with pytest.raises(ValueError):
        ingest.load_tau_basis(str(p))


def test_basis_table_follows_the_listing(tmp_path):
    models = ["exc_to_exc", "exc_to_pv", "pv_to_exc", "sst_to_vip"]
    csv, d, rows = _basis_files(tmp_path, models, listing_extra=("README.txt",))
    basis, m2id = ingest.load_basis_table(csv, d)
    listing = os.listdir(d)
    json_in_order = [x.split(".")[0] for x in listing if x.endswith(".json")]
    # one row per .json entry in listing order; syn_id = position in the listing
    assert basis.shape == (4, 4) and basis.dtype == np.float32
    for i, m in enumerate(json_in_order):
        np.testing.assert_array_equal(basis[i], np.float32(rows[m]))
        assert m2id[m] == listing.index(f"{m}.json")


def test_pop_names_to_cell_types(tmp_path):
    f = ingest.pop_name_to_cell_type
    assert f("e4Rorb") == "L4 Exc" and f("i4Pvalb") == "L4 PV" and f("i23Sst") == "L2/3 SST"
    assert f("e5ET") == "L5 ET" and f("e5ET", ignore_l5e_subtypes=True) == "L5 Exc"
    assert f("i1Htr3a") == "L1 Htr3a" and f("i6Vip") == "L6 VIP" and f("i5Htr3a") == "L5 VIP"
    assert f("e23Cux2") == "L2/3 Exc" and f("i23Vip") == "L2/3 VIP" and f("e5IT") == "L5 IT"
    assert f("e6Ntsr1") == "L6 Exc" and f("i6Sst") == "L6 SST" and f("i1Vip") == "L1 Htr3a"
    nt = tmp_path / "v1_node_types.csv"
    nt.write_text("node_type_id pop_name model_type\n100 e23Cux2 point\n101 i4Pvalb point\n102 e5IT point\n")
    ct = ingest.cell_types_from_node_types(str(nt), np.array([102, 100, 101, 100]))
    assert ct.tolist() == ["L5 Exc", "L2/3 Exc", "L4 PV", "L2/3 Exc"]
    with pytest.raises(ValueError, match="not in"):
        ingest.cell_types_from_node_types(str(nt), np.array([7]))


def test_prepare_network_checks_shapes():
    from v1_glif_model_amd import synthetic as sy
    from tests.helpers import tiny_config
    net = sy.make_network(tiny_config(), seed=0)
    tau = np.array([1.0, 2.0, 3.5, 5.5])
    with pytest.raises(ValueError, match="one weight per receptor"):
        ingest.prepare_network(net["network"], net["lgn_input"], net["bkg_input"], tau, np.ones((5, 5)))
    with pytest.raises(ValueError, match="syn_id"):
        ingest.prepare_network(net["network"], net["lgn_input"], net["bkg_input"], tau, np.ones((2, 4)))
    p = ingest.prepare_network(net["network"], net["lgn_input"], net["bkg_input"], tau, np.ones((5, 4)),
                               cell_types=np.array(["L4 Exc"] * net["network"]["n_nodes"]))
    assert p["basis"].shape == (5, 4) and p["network"]["cell_type"].size == net["network"]["n_nodes"]


@pytest.mark.skipif(not os.path.isdir(REF_SYN), reason="reference synaptic data not mounted")
def test_reference_synaptic_data_formats(tmp_path):
    """The reference's own tau_basis.npy and basis_function_weights.csv load with the safe
    readers: 4 receptors, one weight row per synaptic model."""
    tau = ingest.load_tau_basis(os.path.join(REF_SYN, "tau_basis.npy"))
    assert tau.shape == (4,)
    import pandas as pd
    names = pd.read_csv(os.path.join(REF_SYN, "basis_function_weights.csv"), index_col=0).index[:3]
    d = tmp_path / "models"
    d.mkdir()
    for n in names:
        (d / f"{n}.json").write_text("{}")
    basis, m2id = ingest.load_basis_table(os.path.join(REF_SYN, "basis_function_weights.csv"), str(d))
    assert basis.shape == (3, tau.size) and set(m2id) == set(names)


@pytest.mark.gpu
def test_gpu_four_receptor_network_bit_exact(tmp_path):
    """A network with the real model's 4 receptors, prepared through the ingestion path,
    runs through the cell bit-exactly with the oracle (deterministic mode), and its BPTT
    is within the 1e-5 bar."""
    import torch
    from oracle.cpu import OracleCell
    from tests.helpers import tiny_config
    from v1_glif_model_amd import synthetic as sy
    from v1_glif_model_amd.models import V1Column
    from v1_glif_model_amd.tables import build_cell_tables
    cfg = tiny_config(rs=2.0, ins=3.0)
    raw = sy.make_network(cfg, seed=7)
    csv, d, _ = _basis_files(tmp_path, [f"m{i}" for i in range(cfg.n_syn_types)])
    basis, _ = ingest.load_basis_table(csv, d)
    tau = np.array([0.98958772, 1.88019093, 3.62895928, 5.65340431])
    net = ingest.prepare_network(raw["network"], raw["lgn_input"], raw["bkg_input"], tau, basis)
    T, B = 40, 3
    lgn, bkg = sy.make_inputs(cfg, seed=8, seq_len=T, batch=B)
    cell = V1Column(net, mode="deterministic", gauss_std=0.5, dampening_factor=0.5,
                    recurrent_dampening_factor=0.5, voltage_gradient_dampening=0.5, pseudo_gauss=True)
    z, v, _ = cell.rollout(lgn, bkg)
    oc = OracleCell(build_cell_tables(net), vgd=0.5, rd=0.5, gauss_std=0.5, damp=0.5, pseudo_gauss=True)
    oz, ov, oref, _ = oc.forward(lgn, bkg)
    assert oz.sum() > 0
    np.testing.assert_array_equal(z.cpu().numpy().astype(np.uint8), oz)
    np.testing.assert_array_equal(v.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    gz = np.random.default_rng(9).normal(0, 1, oz.shape).astype(np.float32)
    g = cell.backward(gz=torch.tensor(gz, device="cuda"))
    og = oc.backward(lgn, bkg, oz, oref, ov, gz_loss=gz)
    for k in ("rec", "lgn", "bkg"):
        a, e = g[k].cpu().numpy(), og[k]
        assert np.max(np.abs(a - e)) <= 1e-5 * np.max(np.abs(e)) + 1e-6, k
