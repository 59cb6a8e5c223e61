"""GPU parity of the rSVD deflation front-end (dmh_orth / dmh_project / dmh_rsvd /
dmh_rmfro_clip) against the CPU oracle and the reference's own vectors."""

import numpy as np
import pytest
import torch

from conftest import bf16_from_bits
from oracle import polar_oracle as O
from parity import SUBSPACE_TOL, log_parity, rel

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def N():
    from defmuon_amd import _native
    _native.load()
    assert torch.cuda.is_available()
    return _native


def _spiked_batch(shapes_seeds):
    from defmuon_amd import synthetic as S
    return torch.stack([S.spiked_matrix(*a, **kw) for a, kw in shapes_seeds])


def _head_proj(U, s, V, k):
    """Sign-invariant head: U_k diag(s_k) V_k^T (fp64)."""
    U, s, V = U.double().cpu(), s.double().cpu(), V.double().cpu()
    return (U[..., :k] * s[..., None, :k]) @ V[..., :k].mT


def test_orth_matches_oracle(N):
    X = torch.randn(3, 500, 40, generator=torch.Generator().manual_seed(1))
    Q = N.orth(X.to(DEV), 1).cpu()
    Qo = O.orth_b(X)
    assert float((Q - Qo).abs().max()) < 1e-4
    I = torch.eye(40)
    assert float((Q.mT @ Q - I).abs().max()) < 1e-4


def test_orth_two_passes(N):
    X = torch.randn(2, 300, 24, generator=torch.Generator().manual_seed(2))
    Q = N.orth(X.to(DEV), 2).cpu()
    Qo = O.orth_b(X, passes=2)
    assert float((Q - Qo).abs().max()) < 1e-4


def test_project_matches_oracle(N):
    A = _spiked_batch([((600, 200), dict(seed=3, n_spikes=3, hi=40.0, lo=10.0))])
    Q = O.orth_b(A @ torch.randn(1, 200, 10, generator=torch.Generator().manual_seed(4)))
    U, s, V = N.project(Q.to(DEV), A.to(DEV))
    Uo, so, Vo = O.project_b(Q, A)
    np.testing.assert_allclose(s.cpu().numpy(), so.numpy(), rtol=SUBSPACE_TOL)
    assert rel(_head_proj(U, s, V, 10), _head_proj(Uo, so, Vo, 10)) < SUBSPACE_TOL


@pytest.mark.parametrize("key", ["clip", "clip2"])
def test_rsvd_matches_reference_vectors(N, golden, key):
    A = torch.from_numpy(golden["inputs"][f"{key}_A"])
    Om = torch.from_numpy(golden["inputs"][f"{key}_Omega"])
    ref = golden["eager"]
    U, s, V = N.rsvd(A.to(DEV), Om.to(DEV), 1, 1)
    np.testing.assert_allclose(s.cpu().numpy(), ref[f"{key}_s"], rtol=SUBSPACE_TOL, atol=1e-6)
    # head subspace where the gate fires (a declined, pure-bulk matrix has no
    # separated head, so its leading vectors are not determined to 1e-4)
    Uo, so, Vo = O.rsvd_b(A, Om)
    for b, k in enumerate(ref[f"{key}_k"].tolist()):
        if k == 0:
            continue
        got = (U[b, :, :k] @ V[b, :, :k].mT).double().cpu()
        if k == 2:
            assert rel(got, torch.from_numpy(ref[f"{key}_head_proj"][b]).double()) < SUBSPACE_TOL
        assert rel(got, (Uo[b, :, :k] @ Vo[b, :, :k].mT).double()) < SUBSPACE_TOL


@pytest.mark.parametrize("key", ["clip", "clip2"])
def test_clip_matches_reference_vectors(N, golden, key):
    A = torch.from_numpy(golden["inputs"][f"{key}_A"])
    Om = torch.from_numpy(golden["inputs"][f"{key}_Omega"])
    ref = golden["eager"]
    r, kw = O.sketch_dims(A.shape[-1])
    X0, k, d = N.rmfro_clip(A.to(DEV), Om.to(DEV), kw, O.GATE_RATIO, O.DEFLATE_THRESH,
                            O.DIVISOR_PAD, 1, 1, None)
    assert k.cpu().tolist() == ref[f"{key}_k"].tolist()
    # d = ||A - U_k S_k V_k^T||_F + 1e-7 depends at first order on the rounding of the
    # sketch products (single-pass fp32 CholeskyQR leaves Q^T Q - I ~ kappa*eps, and
    # the head-to-remainder energy ratio, ~33 on clip2's first matrix, amplifies it):
    # two correct fp32 implementations agree to the front-end tolerance, 1e-4.  The
    # accuracy against the same algorithm in fp64 is held in test_config2_clip.
    np.testing.assert_allclose(d.cpu().numpy(), ref[f"{key}_d"], rtol=SUBSPACE_TOL)
    assert rel(X0, torch.from_numpy(ref[f"{key}_X0f32"])) < SUBSPACE_TOL
    X0b, kb, _ = N.rmfro_clip(A.to(DEV), Om.to(DEV), kw, O.GATE_RATIO, O.DEFLATE_THRESH,
                              O.PE_PAD, 1, 1, torch.bfloat16)
    assert kb.cpu().tolist() == ref[f"{key}_kpe"].tolist()
    want = bf16_from_bits(ref[f"{key}_X0pe"])
    assert rel(X0b, want) < 4e-3           # bf16 rounding of an fp32 result within 1e-4
    eq = (X0b.cpu().view(torch.int16) == want.view(torch.int16)).float().mean().item()
    assert eq > 0.97


def test_config2_clip(N):
    """one spiked 3072x768 tall momentum, r=40, kw=20, k=8."""
    from defmuon_amd import synthetic as S
    A = S.spiked_matrix(3072, 768, seed=0)[None]
    r, kw = O.sketch_dims(768)
    assert (r, kw) == (40, 20)
    Om = O.draw_omega(1, 768, r, 123)
    X0, k, d = N.rmfro_clip(A.to(DEV), Om.to(DEV), kw, O.GATE_RATIO, O.DEFLATE_THRESH,
                            O.DIVISOR_PAD, 1, 1, torch.bfloat16)
    Xo, ko, do = O.rmfro_clip(A, Om, out_dtype=torch.bfloat16)
    assert int(k[0]) == int(ko[0]) == 8
    U, s, V = N.rsvd(A.to(DEV), Om.to(DEV), 1, 1)
    Uo, so, Vo = O.rsvd_b(A, Om)
    log_parity("frontend", "config 2 clip 1x(3072,768)",
               s=float(((s.cpu()[0, :8] - so[0, :8]).abs() / so[0, :8]).max()),
               head=rel(_head_proj(U, s, V, 8), _head_proj(Uo, so, Vo, 8)),
               d=abs(float(d[0]) - float(do[0])) / float(do[0]), x0=rel(X0, Xo))
    assert abs(float(d[0]) - float(do[0])) / float(do[0]) < SUBSPACE_TOL
    assert rel(X0, Xo) < 4e-3
    np.testing.assert_allclose(s.cpu().numpy()[0, :8], so.numpy()[0, :8], rtol=SUBSPACE_TOL)
    assert rel(_head_proj(U, s, V, 8), _head_proj(Uo, so, Vo, 8)) < SUBSPACE_TOL
    # The same algorithm in fp64 is the yardstick: single-pass CholeskyQR in fp32
    # loses ~kappa * eps of orthogonality on the power-iterated sketch, in the
    # reference arithmetic as here.  The library must be no less accurate.
    U8, s8, V8 = O.rsvd_b(A.double(), Om.double())
    _, _, d8 = O.rmfro_clip(A.double(), Om.double())
    e_lib = rel(_head_proj(U, s, V, 8), _head_proj(U8, s8, V8, 8))
    e_ref = rel(_head_proj(Uo, so, Vo, 8), _head_proj(U8, s8, V8, 8))
    assert e_lib <= 2 * e_ref + 1e-6, (e_lib, e_ref)
    dd_lib = abs(float(d[0]) - float(d8[0])) / float(d8[0])
    dd_ref = abs(float(do[0]) - float(d8[0])) / float(d8[0])
    assert dd_lib <= 2 * dd_ref + 1e-6, (dd_lib, dd_ref)


def test_gate_identity_mixed_batch(N):
    """Config-4 style design at reduced size: 16 spikes 100x..5x (k = 12) and
    every 4th matrix with no spike (k = 0); gate decisions identical to the
    oracle's."""
    spec = []
    for i in range(8):
        ns = 0 if i % 4 == 3 else 16
        spec.append(((1536, 768), dict(seed=100 + i, n_spikes=ns, hi=100.0, lo=5.0)))
    A = _spiked_batch(spec)
    r, kw = O.sketch_dims(768)
    Om = O.draw_omega(8, 768, r, 77)
    _, k, d = N.rmfro_clip(A.to(DEV), Om.to(DEV), kw, O.GATE_RATIO, O.DEFLATE_THRESH,
                           O.PE_PAD, 1, 1, torch.bfloat16)
    _, ko, do = O.rmfro_clip(A, Om, pad=O.PE_PAD)
    assert k.cpu().tolist() == ko.tolist() == [12, 12, 12, 0, 12, 12, 12, 0]
    np.testing.assert_allclose(d.cpu().numpy(), do.numpy(), rtol=SUBSPACE_TOL)


def test_zero_matrix_is_declined_and_finite(N):
    """A rank-deficient sketch Gram: the reference is undefined (NaN); the
    library declines the matrix and returns the plain entry (zeros here)."""
    from defmuon_amd import synthetic as S
    A = torch.stack([torch.zeros(400, 200), S.spiked_matrix(400, 200, seed=5, n_spikes=2,
                                                            hi=40.0, lo=20.0)])
    r, kw = O.sketch_dims(200)
    Om = O.draw_omega(2, 200, r, 9)
    X0, k, d = N.rmfro_clip(A.to(DEV), Om.to(DEV), kw, O.GATE_RATIO, O.DEFLATE_THRESH,
                            O.DIVISOR_PAD, 1, 1, torch.bfloat16)
    assert torch.isfinite(X0.float()).all()
    assert int(k[0]) == 0 and float(X0[0].float().abs().max()) == 0.0
    assert int(k[1]) == 2
    _, ko, _ = O.rmfro_clip(A[1:], Om[1:])
    assert int(ko[0]) == 2


def test_empty_group(N):
    """An empty shape group (batch 0): every entry returns empty outputs of the right
    shapes without launching anything."""
    from defmuon_amd.optim import deflation_batched as DB
    A = torch.empty(0, 512, 256, device=DEV)
    r, kw = O.sketch_dims(256)
    Om = torch.empty(0, 256, r, device=DEV)
    X0, k, d = N.rmfro_clip(A, Om, kw, O.GATE_RATIO, O.DEFLATE_THRESH, O.DIVISOR_PAD, 1, 1,
                            torch.bfloat16)
    assert X0.shape == (0, 512, 256) and k.shape == (0,) and d.shape == (0,)
    U, s, V = N.rsvd(A, Om, 1, 1)
    assert U.shape[0] == s.shape[0] == V.shape[0] == 0
    P, k2, d2 = DB.DeflatedNSPolar().polar_group(A, Omega=Om, steps=5)
    assert P.shape == (0, 512, 256) and P.dtype == torch.bfloat16 and k2.numel() == 0
    Y = N.ns_chain(torch.empty(0, 300, 200, device=DEV), True, 1, [O.NS_ABC] * 5)
    assert Y.shape == (0, 300, 200)
    torch.cuda.synchronize()


def test_non_finite_matrix_is_isolated(N):
    """A momentum holding a NaN (undefined in the reference: its NaN sketch reaches
    cholesky_ex) is declined (k = 0), and every other matrix of the batch comes out
    bit-identical to a batch without it: no kernel mixes matrices."""
    from defmuon_amd.optim import deflation_batched as DB
    fac = DB.DeflatedNSPolar()
    spec = [((640, 256), dict(seed=70 + i, n_spikes=3, hi=50.0, lo=20.0)) for i in range(3)]
    A = _spiked_batch(spec)
    r, kw = O.sketch_dims(256)
    Om = O.draw_omega(3, 256, r, 21)
    Ap = A.clone()
    Ap[1, 17, 5] = float("nan")
    U0, k0, d0 = fac.polar_group(A.to(DEV), Omega=Om.to(DEV), steps=5)
    U1, k1, d1 = fac.polar_group(Ap.to(DEV), Omega=Om.to(DEV), steps=5)
    assert int(k1[1]) == 0 and int(k0[1]) == 3
    for b in (0, 2):
        assert int(k1[b]) == int(k0[b]) == 3
        assert float(d1[b]) == float(d0[b])
        assert torch.equal(U1[b].view(torch.int16), U0[b].view(torch.int16)), b


@pytest.mark.parametrize("arm", ["ns", "pe"])
def test_fused_deflated_polar_matches_two_calls(N, arm):
    """dmh_deflated_polar (clip written straight into the chain's operands) gives
    bit-identical results to BATCHED_CLIP followed by _iterate, and both agree
    with the oracle."""
    from defmuon_amd.optim import deflation_batched as DB
    fac = DB.DeflatedNSPolar() if arm == "ns" else DB.DeflatedPEPolar()
    spec = [((900, 300), dict(seed=60 + i, n_spikes=4, hi=60.0, lo=20.0)) for i in range(3)]
    spec.append(((900, 300), dict(seed=63, n_spikes=0)))
    A = _spiked_batch(spec)
    r, kw = O.sketch_dims(300)
    Om = O.draw_omega(4, 300, r, 5)
    Ad, Omd = A.to(DEV), Om.to(DEV)
    U1, k1, d1 = fac.polar_group(Ad, Omega=Omd, steps=5)
    X0, k2, d2 = fac.BATCHED_CLIP(Ad, Omega=Omd, pad=fac.PAD, out_dtype=torch.bfloat16)
    U2 = fac._iterate(X0, 5)
    assert torch.equal(k1, k2) and torch.equal(d1, d2)
    assert torch.equal(U1.view(torch.int16), U2.view(torch.int16))
    assert k1.cpu().tolist() == [4, 4, 4, 0]
    Xo, ko, do = O.rmfro_clip(A, Om, pad=fac.PAD, out_dtype=torch.bfloat16)
    hs = O.ns_schedule(5) if arm == "ns" else O.pe_schedule(5)
    Uo = O.horner_iterate(Xo, hs)
    from parity import assert_polar_parity
    for b in range(4):
        assert_polar_parity(U1[b], Uo[b], A[b], f"fused {arm}[{b}]")


@pytest.mark.parametrize("B,n,m,ns", [(3, 1000, 264, 3), (2, 536, 520, 4), (1, 2056, 136, 2),
                                      (2, 1001, 259, 3)])
def test_rsvd_ragged_shapes_match_oracle(N, B, n, m, ns):
    """The split-bf16 skinny products on shapes whose rows and columns end mid-chunk
    (m % 64 = 8, 8 or 8; n % 16 = 8 or 0; a last row block of a few rows): the
    out-of-range loads read zeros and the results match the oracle on the same sketch.
    (2, 1001, 259): n and m not multiples of 8, which the split-bf16 kernels do not
    take: the fp32-MFMA skinny products (skinny_gemm) and their |A|^2 partials run."""
    A = _spiked_batch([((n, m), dict(seed=40 + b, n_spikes=ns, hi=60.0, lo=15.0))
                       for b in range(B)])
    r, kw = O.sketch_dims(m)
    Om = O.draw_omega(B, m, r, 77)
    U, s, V = N.rsvd(A.to(DEV), Om.to(DEV), 1, 1)
    Uo, so, Vo = O.rsvd_b(A, Om)
    np.testing.assert_allclose(s.cpu().numpy()[:, :ns], so.numpy()[:, :ns], rtol=SUBSPACE_TOL)
    for b in range(B):
        assert rel(_head_proj(U[b:b + 1], s[b:b + 1], V[b:b + 1], ns),
                   _head_proj(Uo[b:b + 1], so[b:b + 1], Vo[b:b + 1], ns)) < SUBSPACE_TOL, b
    X0, k, d = N.rmfro_clip(A.to(DEV), Om.to(DEV), kw, O.GATE_RATIO, O.DEFLATE_THRESH,
                            O.DIVISOR_PAD, 1, 1, torch.bfloat16)
    Xo, ko, do = O.rmfro_clip(A, Om, out_dtype=torch.bfloat16)
    assert torch.equal(k.cpu(), ko)
    s_err = float(((s.cpu()[:, :ns] - so[:, :ns]).abs() / so[:, :ns]).max())
    d_err = float(((d.cpu() - do).abs() / do).max())
    head = max(rel(_head_proj(U[b:b + 1], s[b:b + 1], V[b:b + 1], ns),
                   _head_proj(Uo[b:b + 1], so[b:b + 1], Vo[b:b + 1], ns)) for b in range(B))
    log_parity("frontend", f"rsvd/clip {B}x({n},{m})", s=s_err, head=head, d=d_err,
               x0=rel(X0.float().cpu(), Xo.float()))
    np.testing.assert_allclose(d.cpu().numpy(), do.numpy(), rtol=1e-4)
    assert rel(X0.float().cpu(), Xo.float()) < 4e-3


@pytest.mark.parametrize("bulk", [1e-3, 1e-4])
def test_head_dominated_divisor(N, bulk):
    """Rank-1 matrices with a bulk at `bulk` of sigma_1 (the head holds all but
    ~m bulk^2 of the energy): d = ||A - U_k S_k V_k^T||_F + 1e-7 must match the
    reference's explicit norm (the oracle) to 1e-4 and the entry must stay finite.
    The algebraic ||A||^2 - sum lambda (2 - G) loses its digits here (its error grows
    as ||A||^2 / ||W||^2), so the library recomputes d from W for such matrices."""
    B, n, m = 4, 512, 512
    g = torch.Generator().manual_seed(int(1 / bulk))
    A = torch.empty(B, n, m)
    for b in range(B):
        u = torch.randn(n, 1, generator=g, dtype=torch.float64)
        v = torch.randn(m, 1, generator=g, dtype=torch.float64)
        noise = torch.randn(n, m, generator=g, dtype=torch.float64) / (n ** 0.5 + m ** 0.5)
        A[b] = ((u / u.norm()) @ (v / v.norm()).mT + bulk * noise).float()
    r, kw = O.sketch_dims(m)
    Om = O.draw_omega(B, m, r, seed=5)
    X0, k, d = N.rmfro_clip(A.to(DEV), Om.to(DEV), kw, O.GATE_RATIO, O.DEFLATE_THRESH,
                            O.DIVISOR_PAD, out_dtype=torch.float32)
    X0o, ko, do = O.rmfro_clip(A, Om)
    assert k.cpu().tolist() == ko.tolist() == [1] * B
    log_parity("frontend", f"head-dominated bulk {bulk:g} {B}x({n},{m})",
               d=float(((d.cpu() - do).abs() / do).max()), x0=rel(X0, X0o))
    np.testing.assert_allclose(d.cpu().numpy(), do.numpy(), rtol=1e-4)
    assert bool(torch.isfinite(X0).all())
    # the deflated entry: 1/pad on the head, the bulk at unit Frobenius norm
    assert rel(X0, X0o) < 1e-3


def _clip_vs_fp64(N, A, kw, ratio, thresh, name):
    """rmfro_clip on the GPU, the oracle in fp32 (the reference arithmetic) and the same
    algorithm in fp64; returns (k, k_oracle, k_fp64) and checks that the library's d and
    X0 are at least as close to the fp64 result as the oracle's fp32 ones."""
    B, n, m = A.shape
    r, _ = O.sketch_dims(m)
    Om = O.draw_omega(B, m, r, seed=m + B)
    X0, k, d = N.rmfro_clip(A.to(DEV), Om.to(DEV), kw, ratio, thresh, O.DIVISOR_PAD,
                            out_dtype=torch.float32)
    X0o, ko, do = O.rmfro_clip(A, Om, ratio=ratio, thresh=thresh)
    X08, k8, d8 = O.rmfro_clip(A.double(), Om.double(), ratio=ratio, thresh=thresh)
    e_lib, e_ref = rel(X0.cpu().double(), X08), rel(X0o.double(), X08)
    dd_lib = float(((d.cpu().double() - d8).abs() / d8).max())
    dd_ref = float(((do.double() - d8).abs() / d8).max())
    log_parity("frontend", name, x0_vs_fp64=e_lib, oracle_x0_vs_fp64=e_ref, d_vs_fp64=dd_lib,
               oracle_d_vs_fp64=dd_ref)
    assert e_lib <= 2 * e_ref + 1e-6, (e_lib, e_ref)
    assert dd_lib <= 2 * dd_ref + 1e-6, (dd_lib, dd_ref)
    return k.cpu().tolist(), ko.tolist(), k8.tolist()


@pytest.mark.parametrize("case", ["repeated_head", "wide_head", "two_column_sketch"])
def test_clip_head_eigenpairs(N, case):
    """The clip's gate eigen-solve (tridiagonal reduction, multisection for the top kw
    eigenvalues, inverse iteration on the deflated head): four equal head singular
    values (an eigenvalue cluster, re-orthogonalised), a 30-direction head in the
    widest gate window (kw = 32), and a 2-column sketch (r = 2, kw = 1: the gate cannot
    fire).  Gate decisions identical to the oracle's in fp32 and fp64."""
    from defmuon_amd import synthetic as S
    if case == "repeated_head":
        A = S.spiked_batch(3, 2048, 512, seed=21, n_spikes=4, hi=30.0, lo=30.0)
        want = [4, 4, 4]
    elif case == "wide_head":
        A = S.spiked_batch(2, 2560, 1280, seed=22, n_spikes=30, hi=60.0, lo=12.0)
        want = [30, 30]
    else:
        A = S.spiked_batch(3, 300, 40, seed=23, n_spikes=1, hi=20.0, lo=20.0)
        want = [0, 0, 0]
    _, kw = O.sketch_dims(A.shape[-1])
    k, ko, k8 = _clip_vs_fp64(N, A, kw, O.GATE_RATIO, O.DEFLATE_THRESH, f"clip head {case}")
    assert k == ko == k8 == want


def test_clip_threshold_below_ratio(N):
    """A clip threshold below the gate ratio (DEFMUON_DEFL_THRESH < DEFMUON_DEFL_RATIO)
    deflates past the gate window (16 directions, kw = 13): the library takes its
    full Jacobi eigen-solve there; k, d and X0 as the oracle's at those thresholds."""
    from defmuon_amd import synthetic as S
    A = S.spiked_batch(3, 2048, 512, seed=24, n_spikes=16, hi=100.0, lo=5.0)
    _, kw = O.sketch_dims(512)
    assert kw == 13
    k, ko, k8 = _clip_vs_fp64(N, A, kw, 0.10, 0.04, "clip thresh 0.04 < ratio 0.10")
    assert k == ko == k8 == [16, 16, 16]


@pytest.mark.parametrize("B,n,m", [(3, 1000, 768), (2, 3072, 768), (2, 1280, 1280), (1, 264, 128)])
def test_skinny_rows_direct_to_lds_matches_register_kernel(N, B, n, m, monkeypatch):
    """The direct-to-LDS A x X kernel (rows of A streamed through an LDS ring, the
    default where m % 64 == 0) and the register-load kernel (DMH_SKR_DTL=0) make the
    same products in the same order: the rSVD outputs are bit-identical (partial last
    row blocks included).  Their per-workgroup sums of squares of A, behind the
    divisor, add the same values in another order, so k is equal and d and X0 agree
    to fp32 rounding."""
    from defmuon_amd import synthetic as S
    A = torch.stack([S.spiked_matrix(n, m, seed=7 * b + n, n_spikes=4, hi=40.0, lo=12.0)
                     for b in range(B)]).to(DEV)
    r, kw = O.sketch_dims(m)
    Om = O.draw_omega(B, m, r, 99).to(DEV)
    outs = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("DMH_SKR_DTL", mode)
        X0, k, d = N.rmfro_clip(A, Om, kw, O.GATE_RATIO, O.DEFLATE_THRESH, O.DIVISOR_PAD, 1, 1)
        U, s, V = N.rsvd(A, Om, 1, 1)
        outs[mode] = [t.cpu() for t in (X0, k, d, U, s, V)]
    (X0r, kr, dr, Ur, sr, Vr), (X0, k, d, U, s, V) = outs["0"], outs["1"]
    for a, b in ((U, Ur), (s, sr), (V, Vr), (k, kr)):
        assert torch.equal(a, b)
    assert float(((d - dr).abs() / dr).max()) < 1e-6
    assert rel(X0, X0r) < 1e-6
