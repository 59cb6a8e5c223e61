"""Pin the CPU oracle with closed forms and invariants (independent of the
reference's vectors): every polynomial iterate of G = U diag(sigma) V^T is
U diag(p(sigma)) V^T, CholeskyQR is a QR, the rSVD is exact on low-rank input, and
the gate / deflation entry have closed forms on designed spectra."""

import math

import numpy as np
import pytest
import torch

from defmuon_amd import synthetic as S
from oracle import polar_oracle as O

F64 = torch.float64


def _svd_input(rows, cols, sigma, seed):
    g = torch.Generator().manual_seed(seed)
    m = min(rows, cols)
    U = S.haar(rows, m, g, "cpu")
    V = S.haar(cols, m, g, "cpu")
    return (U * sigma[None, :]) @ V.mT, U, V


def _scalar_map(x, hs):
    """Composition of p(x) = a x + b x^3 + c x^5 (numpy, fp64); the reference's
    own scalar restatement is spectra/plot_spectra.py:79-84."""
    x = np.asarray(x, dtype=np.float64)
    for a, b, c in hs:
        x = a * x + b * x ** 3 + c * x ** 5
    return x


@pytest.mark.parametrize("rows,cols", [(40, 96), (96, 40), (64, 64)])
def test_ns5_fp64_equals_scalar_map(rows, cols):
    m = min(rows, cols)
    sigma = torch.logspace(0, -3, m, dtype=F64) * 7.0
    G, U, V = _svd_input(rows, cols, sigma, 1)
    delta = float(G.norm()) + 1e-7
    want = (U * torch.from_numpy(_scalar_map(sigma.numpy() / delta, O.ns_schedule(5)))) @ V.mT
    got = O.ns5(G, 5, dtype=F64)
    assert got.shape == G.shape
    assert float((got - want).norm() / want.norm()) < 1e-10


@pytest.mark.parametrize("rows,cols", [(40, 96), (96, 40)])
def test_polar_express_fp64_equals_scalar_map(rows, cols):
    m = min(rows, cols)
    sigma = torch.linspace(3.0, 0.01, m, dtype=F64)
    G, U, V = _svd_input(rows, cols, sigma, 2)
    delta = 1.01 * float(G.norm()) + 1e-7
    want = (U * torch.from_numpy(_scalar_map(sigma.numpy() / delta, O.pe_schedule(5)))) @ V.mT
    got = O.polar_express(G, 5, dtype=F64)
    assert float((got - want).norm() / want.norm()) < 1e-10


def test_pe_schedule_repeats_last_triple():
    hs = O.pe_schedule(10)
    assert len(hs) == 10 and hs[8] == hs[7] == hs[9] == (1.875, -1.25, 0.375)
    # safety factor on all but the last triple (polar_express.py:18-19)
    a0, b0, c0 = O.PE_COEFFS[0]
    assert math.isclose(a0 * 1.01, 8.28721201814563, rel_tol=1e-15)
    assert math.isclose(b0 * 1.01 ** 3, -23.595886519098837, rel_tol=1e-15)
    assert math.isclose(c0 * 1.01 ** 5, 17.300387312530933, rel_tol=1e-15)


def test_horner_fp64_equals_scalar_map_tall():
    sigma = torch.linspace(0.99, 0.001, 32, dtype=F64)
    X, U, V = _svd_input(80, 32, sigma, 3)
    want = (U * torch.from_numpy(_scalar_map(sigma.numpy(), O.ns_schedule(5)))) @ V.mT
    got = O.horner_iterate(X[None], O.ns_schedule(5))[0]
    assert float((got - want).norm() / want.norm()) < 1e-10


def test_zeros_are_a_fixed_point():
    Z = torch.zeros(3, 64, 32, dtype=torch.bfloat16)
    assert torch.count_nonzero(O.horner_iterate(Z, O.ns_schedule(5)).float()) == 0
    assert torch.count_nonzero(O.ns5(torch.zeros(48, 96)).float()) == 0


def test_transpose_equivariance_and_forms_agree_fp64():
    g = torch.Generator().manual_seed(4)
    M = torch.randn(48, 120, generator=g, dtype=F64)
    a = O.ns5(M, 5, dtype=F64)
    b = O.ns5(M.mT.contiguous(), 5, dtype=F64)
    assert float((a - b.mT).norm()) < 1e-10
    # tall form X(aI+bG+cG^2) equals the wide form on the transposed side
    X0 = M.mT / (M.norm() + 1e-7)
    t = O.horner_iterate(X0[None].contiguous(), O.ns_schedule(5))[0]
    assert float((t.mT - a).norm()) < 1e-10


def test_orth_b_is_a_qr():
    g = torch.Generator().manual_seed(5)
    X = torch.randn(3, 300, 12, generator=g)
    Q = O.orth_b(X)
    I = torch.eye(12)
    assert float((Q.mT @ Q - I).abs().max()) < 1e-5
    # span(Q) = span(X): the projector of X onto Q's complement vanishes
    assert float((X - Q @ (Q.mT @ X)).norm() / X.norm()) < 1e-5
    Qr, _ = torch.linalg.qr(X.double())
    assert float((Q.double() @ Q.double().mT - Qr @ Qr.mT).norm()) < 1e-4


def test_rsvd_exact_on_low_rank():
    """rank(A) = r: the subspace iteration captures A exactly, so s equals the
    exact singular values and U diag(s) V^T reproduces A.  (rank < r makes the
    sketch Gram singular, where the reference's CholeskyQR is undefined.)"""
    sigma = torch.tensor([9.0, 5.0, 2.0, 1.0, 0.5, 0.25], dtype=F64)
    A64, _, _ = _svd_input(200, 90, torch.cat([sigma, torch.zeros(84, dtype=F64)]), 6)
    A = A64.float()[None]
    r, kw = O.sketch_dims(90)
    assert (r, kw) == (6, 3)
    Om = O.draw_omega(1, 90, r, 11)
    U, s, V = O.rsvd_b(A, Om)
    np.testing.assert_allclose(s[0].double().numpy(), sigma.numpy(), rtol=1e-4)
    rec = (U * s[:, None, :]) @ V.mT
    assert float((rec - A).norm() / A.norm()) < 1e-5


@pytest.mark.parametrize("m,expect", [(768, (40, 20)), (1024, (52, 26)), (1280, (64, 32)),
                                      (96, (6, 3)), (80, (4, 2)), (1, (1, 1))])
def test_sketch_dims(m, expect):
    assert O.sketch_dims(m) == expect


def test_gate_closed_form_on_designed_spectrum():
    """Config-2 design (8 spikes 50x..10x): k = 8.  Config-4 design (16 spikes
    100x..5x): k = 12.  Pure bulk: the gate declines (k = 0)."""
    assert S.expected_k(8, 50.0, 10.0) == 8
    assert S.expected_k(16, 100.0, 5.0) == 12
    for (n, m, ns, hi, lo, kexp) in [(1536, 384, 8, 50.0, 10.0, 8),     # kw = 10
                                     (1536, 768, 16, 100.0, 5.0, 12),    # kw = 20
                                     (1536, 384, 0, 1.0, 1.0, 0)]:
        A = S.spiked_matrix(n, m, seed=31, n_spikes=ns, hi=hi, lo=lo)[None]
        r, _ = O.sketch_dims(m)
        _, k, _ = O.rmfro_clip(A, O.draw_omega(1, m, r, 3))
        assert int(k[0]) == kexp


def test_gate_rule_on_explicit_values():
    s = torch.tensor([[10.0, 5.0, 0.5, 0.4, 0.3, 0.2],     # k=2, fires
                      [10.0, 9.0, 8.0, 0.4, 0.3, 0.2],     # window value 8 >= 1: declines
                      [10.0, 0.5, 0.4, 0.4, 0.3, 0.2],     # k=1, fires
                      [10.0, 9.0, 9.0, 9.0, 9.0, 9.0]])    # kr = r: declines
    kk, fired, head = O.gate(s, kw=3)
    assert fired.tolist() == [True, False, True, False]
    assert (kk * fired).tolist() == [2, 0, 1, 0]
    assert head.sum(1).tolist() == [2, 0, 1, 0]


def test_clip_entry_closed_form():
    """With a gap the estimated head is accurate: X0's spectrum is 1/pad (k times)
    over sigma_bulk / ||W||_F, with ||W||_F^2 = sum of the bulk's squares."""
    A, s = S.spiked_matrix(1200, 300, seed=41, n_spikes=4, hi=60.0, lo=20.0,
                           return_spectrum=True)
    r, _ = O.sketch_dims(300)
    X0, k, d = O.rmfro_clip(A[None], O.draw_omega(1, 300, r, 5), pad=1.01)
    assert int(k[0]) == 4
    bulk = s[4:]
    wn = float(bulk.norm())
    assert abs(float(d[0]) - wn) / wn < 1e-4
    sv = torch.linalg.svdvals(X0[0].double())
    np.testing.assert_allclose(sv[:4].numpy(), 1 / 1.01, rtol=1e-4)
    np.testing.assert_allclose(sv[4:].numpy(), (bulk / wn).numpy(), rtol=2e-3, atol=1e-6)


def test_clip_declined_is_plain_entry():
    A = S.spiked_matrix(400, 200, seed=42, n_spikes=0)[None]
    r, _ = O.sketch_dims(200)
    X0, k, d = O.rmfro_clip(A, O.draw_omega(1, 200, r, 6))
    assert int(k[0]) == 0
    want = A / (A.norm(dim=(-2, -1), keepdim=True) + 1e-7)
    assert torch.equal(X0, want)


def test_group_seed_formula():
    assert O.group_seed(1, 0) == 1009
    assert O.group_seed(3, 2) == 3 * 1009 + 2 * 9176867
    assert O.group_seed(2 ** 61, 1) == (2 ** 61 * 1009 + 9176867) % 2 ** 62
