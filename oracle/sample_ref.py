"""Test infrastructure only (never imported by the product): numpy restatement of the
counter-based input sampler (Philox4x32-10, Salmon et al., "Parallel random numbers: as
easy as 1, 2, 3", SC 2011) used for the LGN Bernoulli spikes (stim_dataset.py:182-197) and
the background Poisson counts (models.py:865-887; TF's stateless stream itself cannot be
reproduced, so these replace it)."""
import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
MASK = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr, key):
    """ctr [..., 4] uint32, key [..., 2] uint32 -> [..., 4] uint32."""
    c = [ctr[..., i].astype(np.uint64) for i in range(4)]
    k0, k1 = key[..., 0].astype(np.uint32), key[..., 1].astype(np.uint32)
    for r in range(10):
        p0, p1 = M0 * c[0], M1 * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & MASK
        hi1, lo1 = p1 >> np.uint64(32), p1 & MASK
        c = [hi1 ^ c[1] ^ k0.astype(np.uint64), lo1, hi0 ^ c[3] ^ k1.astype(np.uint64), lo0]
        k0, k1 = k0 + W0, k1 + W1
    return np.stack([x.astype(np.uint32) for x in c], -1)


def words(n, seed, offset=0):
    """Random 32-bit words of elements offset..offset+n-1: element i uses word i % 4 of the
    block for counter (i // 4, 0, 0, 0) and key (seed_lo, seed_hi)."""
    i = np.arange(offset, offset + n, dtype=np.uint64)
    blk = i // np.uint64(4)
    ctr = np.zeros((n, 4), np.uint32)
    ctr[:, 0] = (blk & MASK).astype(np.uint32)
    ctr[:, 1] = (blk >> np.uint64(32)).astype(np.uint32)
    key = np.zeros((n, 2), np.uint32)
    key[:, 0] = np.uint32(seed & 0xFFFFFFFF)
    key[:, 1] = np.uint32((seed >> 32) & 0xFFFFFFFF)
    out = philox4x32_10(ctr, key)
    return out[np.arange(n), (i % np.uint64(4)).astype(np.int64)]


def uniform(n, seed, offset=0):
    """fp32 in [0, 1): the top 24 bits of the word times 2^-24."""
    return (words(n, seed, offset) >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)


def bernoulli(p, seed, offset=0):
    """uint8 spikes: u < p (p float32, any shape)."""
    p = np.asarray(p, np.float32)
    return (uniform(p.size, seed, offset).reshape(p.shape) < p).astype(np.uint8)


def poisson(lam, n, seed, offset=0, kmax=255):
    """uint8 counts by sequential inverse CDF in fp32: k = 0, pk = exp(-lam), cdf = pk;
    while u > cdf and k < kmax: k += 1; pk = pk * (lam / k); cdf = cdf + pk."""
    f = np.float32
    u = uniform(n, seed, offset)
    lam = f(lam)
    pk = np.full(n, np.exp(-lam), f)
    cdf = pk.copy()
    k = np.zeros(n, np.int32)
    for j in range(1, kmax + 1):
        more = (u > cdf) & (k < kmax)
        if not more.any():
            break
        pk = np.where(more, pk * (lam / f(j)), pk).astype(f)
        cdf = np.where(more, cdf + pk, cdf).astype(f)
        k = np.where(more, j, k)
    return k.astype(np.uint8)
