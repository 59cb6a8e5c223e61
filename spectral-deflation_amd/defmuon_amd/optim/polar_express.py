"""Polar Express polar factor on the HIP bf16 MFMA chain.

Drop-in for defmuon/optim/polar_express.py: the same `coeffs_list` schedule
(Amsel et al., 2025, arXiv:2505.16932, l = 1e-3, safety factor 1.01 on all but
the last triple; polar_express.py:7-19) and the same `PolarExpress(G, steps)`
contract (polar_express.py:21-34): bf16 output of G's shape, entry divisor
1.01 ||X||_F + 1e-7, the first `steps` triples with the last one repeated, and
the chain run on the wide side (transposed when size(-2) > size(-1)).
"""

from itertools import repeat

from defmuon_amd import _native

_PE_TRIPLES = [
    (8.28721201814563, -23.595886519098837, 17.300387312530933),
    (4.107059111542203, -2.9478499167379106, 0.5448431082926601),
    (3.9486908534822946, -2.908902115962949, 0.5518191394370137),
    (3.3184196573706015, -2.488488024314874, 0.51004894012372),
    (2.300652019954817, -1.6689039845747493, 0.4188073119525673),
    (1.891301407787398, -1.2679958271945868, 0.37680408948524835),
    (1.8750014808534479, -1.2500016453999487, 0.3750001645474248),
    (1.875, -1.25, 0.375),  # subsequent coefficients equal this numerically
]
coeffs_list = [(a / 1.01, b / 1.01 ** 3, c / 1.01 ** 5) for (a, b, c) in _PE_TRIPLES[:-1]] \
    + [_PE_TRIPLES[-1]]


def pe_schedule(steps):
    return list(coeffs_list[:steps]) + list(repeat(coeffs_list[-1], steps - len(coeffs_list)))


def as_batch(G):
    """View G (..., R, C) as (batch, R, C)."""
    if G.ndim == 2:
        return G[None]
    return G.reshape(-1, G.shape[-2], G.shape[-1])


def PolarExpress(G, steps):
    assert G.ndim >= 2
    tall = G.size(-2) > G.size(-1)
    out = _native.ns_chain(as_batch(G), tall, 2, pe_schedule(steps))
    return out.reshape(G.shape)
