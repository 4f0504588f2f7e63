"""Device input sampling (Philox4x32-10 streams): LGN Bernoulli spikes
(stim_dataset.py:182-197) and background Poisson counts (models.py:865-887).

CPU: the numpy restatement (oracle/sample_ref.py) reproduces the published Philox4x32-10
known-answer vectors (Salmon et al. 2011, Random123), and its samples have the right
moments.  GPU: libglif's draws equal the restatement's bit for bit (integer work), for any
offset, length and probability, including 0 and 1.
"""
import numpy as np
import pytest

from oracle import sample_ref as sr

KAT = [((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
       ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
       ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
        (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1))]


@pytest.mark.parametrize("ctr,key,expect", KAT)
def test_philox_known_answers(ctr, key, expect):
    out = sr.philox4x32_10(np.array([ctr], np.uint32), np.array([key], np.uint32))[0]
    assert tuple(int(x) for x in out) == expect


def test_stream_offsets_continue_and_seeds_differ():
    a = sr.words(1000, seed=7)
    np.testing.assert_array_equal(sr.words(600, seed=7, offset=400), a[400:])
    assert np.mean(sr.words(1000, seed=8) == a) < 0.01


def test_moments():
    u = sr.uniform(200_000, seed=3)
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 5e-3
    p = np.full(200_000, 0.01, np.float32)
    assert abs(sr.bernoulli(p, seed=4).mean() - 0.01) < 1.5e-3
    for lam in (0.25, 3.0):
        k = sr.poisson(lam, 200_000, seed=5).astype(np.float64)
        assert abs(k.mean() - lam) < 0.02 * max(lam, 1.0)
        assert abs(k.var() - lam) < 0.05 * max(lam, 1.0)


@pytest.mark.gpu
@pytest.mark.parametrize("n,offset", [(1, 0), (1003, 0), (100_001, 5), (4096, 123_456_789_013)])
def test_gpu_bernoulli_bit_exact(n, offset):
    import torch
    from v1_glif_model_amd.inputs import bernoulli
    rng = np.random.default_rng(n)
    p = rng.random(n).astype(np.float32)
    p[::7] = 0.0
    p[::11] = 1.0
    got = bernoulli(torch.tensor(p, device="cuda"), seed=0xDEADBEEFCAFE, offset=offset).cpu().numpy()
    np.testing.assert_array_equal(got, sr.bernoulli(p, seed=0xDEADBEEFCAFE, offset=offset))


@pytest.mark.gpu
@pytest.mark.parametrize("lam,n,offset", [(0.25, 100_003, 0), (2.5, 50_000, 17), (30.0, 5000, 3)])
def test_gpu_poisson_bit_exact(lam, n, offset):
    from v1_glif_model_amd.inputs import poisson
    got = poisson(lam, (n,), seed=12345, offset=offset).cpu().numpy()
    np.testing.assert_array_equal(got, sr.poisson(lam, n, seed=12345, offset=offset))


@pytest.mark.gpu
def test_gpu_sample_helpers_shapes():
    from v1_glif_model_amd.inputs import sample_bkg, sample_lgn
    x = sample_lgn(np.full((20, 3, 50), 10.0, np.float32), seed=1)
    assert x.shape == (20, 3, 50) and x.dtype.is_floating_point is False
    k = sample_bkg(20, 3, 100, seed=2)
    assert k.shape == (20, 3, 100)
    assert abs(float(k.float().mean()) - 0.25) < 0.05
