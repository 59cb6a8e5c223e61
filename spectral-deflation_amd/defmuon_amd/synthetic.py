"""Seeded synthetic momenta with a designed singular spectrum.

A = U diag(s) V^T with Haar-distributed U (rows x m) and V (cols x m), m = min(rows,
cols).  The bulk of s is the top of the singular spectrum of an independent
rows x cols Gaussian matrix with N(0, 1/max(rows, cols)) entries (Marchenko-Pastur),
and the head is `n_spikes` values beta * logspace(log10 hi, log10 lo), beta being the
bulk's largest value.  With n_spikes = 0 the whole spectrum is bulk, which the
deflation gate declines.

Everything is generated in fp64 on `device` from torch Generators seeded with
`seed`, then rounded to fp32.
"""

import math

import torch


def _gen(seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def haar(rows, cols, gen, device, dtype=torch.float64):
    """rows x cols (rows >= cols) matrix with Haar-distributed orthonormal columns:
    QR of a Gaussian with the signs of diag(R) folded into Q."""
    Z = torch.randn(rows, cols, generator=gen, device=device, dtype=dtype)
    Q, R = torch.linalg.qr(Z)
    d = torch.sign(torch.diagonal(R))
    d[d == 0] = 1
    return Q * d[None, :]


def bulk_values(rows, cols, gen, device, count=None):
    """Descending singular values of a rows x cols N(0, 1/max(rows,cols)) matrix
    (from the eigenvalues of its small-side Gram), the top `count` of them."""
    n, m = max(rows, cols), min(rows, cols)
    Gm = torch.randn(n, m, generator=gen, device=device, dtype=torch.float64) / math.sqrt(n)
    ev = torch.linalg.eigvalsh(Gm.mT @ Gm).clamp_min(0).sqrt()
    s = torch.flip(ev, dims=[0])
    return s if count is None else s[:count]


def spiked_spectrum(m, n_spikes, hi, lo, bulk):
    """Concatenate spikes beta*logspace(log10 hi, log10 lo, n_spikes) over the bulk."""
    beta = float(bulk[0])
    if n_spikes == 0:
        return bulk.clone()
    spikes = beta * torch.logspace(math.log10(hi), math.log10(lo), n_spikes,
                                   dtype=torch.float64, device=bulk.device)
    return torch.cat([spikes, bulk[: m - n_spikes]])


def spiked_matrix(rows, cols, seed, n_spikes=8, hi=50.0, lo=10.0, device="cpu",
                  dtype=torch.float32, return_spectrum=False):
    """One synthetic rows x cols momentum with a designed spectrum."""
    gen = _gen(seed, device)
    m = min(rows, cols)
    U = haar(rows, m, gen, device)
    V = haar(cols, m, gen, device)
    bulk = bulk_values(rows, cols, gen, device, count=m)
    s = spiked_spectrum(m, n_spikes, hi, lo, bulk)
    A = (U * s[None, :]) @ V.mT
    A = A.to(dtype)
    if return_spectrum:
        return A, s
    return A


def expected_k(n_spikes, hi, lo, thresh=0.10):
    """Deflation width the gate picks on the exact spectrum: the number of spikes
    above thresh * the top one (bulk values are <= beta <= thresh * beta*hi when
    hi >= 1/thresh)."""
    if n_spikes == 0:
        return 0
    vals = [hi * (lo / hi) ** (i / max(n_spikes - 1, 1)) for i in range(n_spikes)]
    return sum(1 for v in vals if v > thresh * vals[0])


def mp_quantile_values(rows, cols, count=None):
    """Descending singular values at the quantiles (i + 1/2)/m of the
    Marchenko-Pastur law of a rows x cols N(0, 1/max(rows, cols)) matrix: the
    deterministic 'typical' bulk, eigenvalues of the Gram in
    [(1 - sqrt c)^2, (1 + sqrt c)^2] with c = m / n."""
    import numpy as np
    n, m = max(rows, cols), min(rows, cols)
    c = m / n
    a, b = (1 - math.sqrt(c)) ** 2, (1 + math.sqrt(c)) ** 2
    # substitution lambda = a + (b - a) sin^2(t) removes the edge singularities
    t = np.linspace(0.0, math.pi / 2, 200001)
    lam = a + (b - a) * np.sin(t) ** 2
    dlam = 2 * (b - a) * np.sin(t) * np.cos(t)
    with np.errstate(divide="ignore", invalid="ignore"):
        dens = np.sqrt(np.maximum((b - lam) * (lam - a), 0.0)) / (2 * math.pi * c * lam)
    w = np.nan_to_num(dens * dlam)
    cdf = np.concatenate([[0.0], np.cumsum(0.5 * (w[1:] + w[:-1]) * np.diff(t))])
    cdf /= cdf[-1]
    q = (np.arange(m) + 0.5) / m
    ev = np.interp(q, cdf, lam)[::-1]
    s = np.sqrt(np.maximum(ev, 0.0))
    return s if count is None else s[:count]


def spiked_batch(batch, rows, cols, seed, n_spikes=8, hi=50.0, lo=10.0, device="cpu",
                 dtype=torch.float32, unspiked=()):
    """A (batch, rows, cols) stack of synthetic momenta generated on `device`:
    Haar singular vectors (QR of Gaussians, fp32), the Marchenko-Pastur quantile
    bulk, and n_spikes values beta*logspace(hi..lo) on top (beta = the bulk's top
    value).  Matrices whose index is in `unspiked` keep the pure bulk."""
    import numpy as np
    gen = _gen(seed, device)
    m = min(rows, cols)
    U, _ = torch.linalg.qr(torch.randn(batch, rows, m, generator=gen, device=device))
    V, _ = torch.linalg.qr(torch.randn(batch, cols, m, generator=gen, device=device))
    bulk = mp_quantile_values(rows, cols)
    beta = float(bulk[0])
    s = np.tile(bulk, (batch, 1))
    if n_spikes:
        spikes = beta * np.logspace(math.log10(hi), math.log10(lo), n_spikes)
        for i in range(batch):
            if i not in unspiked:
                s[i, :n_spikes] = spikes
                s[i, n_spikes:] = bulk[: m - n_spikes]
    sv = torch.from_numpy(s).to(device=device, dtype=torch.float32)
    return ((U * sv[:, None, :]) @ V.mT).to(dtype)
