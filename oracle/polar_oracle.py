"""CPU restatement of the deflated-Muon polar-factor path (TEST INFRASTRUCTURE).

This module is the parity oracle.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or
as the timed CPU baseline -- never as the product path.  The product path is the
HIP library behind ``defmuon_amd``; it raises if that library is missing.

Every function restates the reference's arithmetic with plain torch ops on the
CPU, citing the reference file:line it follows (paths are relative to the
ComputationalRobotics/Spectral-Deflation tree):

    ns5                 defmuon/optim/muon.py:16-44
    polar_express       defmuon/optim/polar_express.py:7-34
    horner_iterate      defmuon/optim/deflation_batched.py:196-204
    orth_b              defmuon/optim/deflation_batched.py:117-128
    project_b           defmuon/optim/deflation_batched.py:131-139
    rsvd_b              defmuon/optim/deflation_batched.py:142-148
    sketch_dims         defmuon/optim/deflation_batched.py:170-171
    gate                defmuon/optim/deflation_batched.py:177-183
    rmfro_clip          defmuon/optim/deflation_batched.py:155-189
    group_seed          defmuon/optim/muon.py:290-291
    exact_polar/rel_err spectra/polar_convergence.py:138-141, 173-174

Rounding.  The reference runs the bf16 chains under ``torch.compile`` (inductor,
default config).  ``rounding="compiled"`` (the default) reproduces the graph
inductor emits for them:

  * entry: the cast to bf16 is folded away, so X = bf16(G / (||G||_F + 1e-7)) with
    the norm taken over the un-rounded input (muon.py:29-33);
  * 2-D operands: `b*A + (c*A) @ A` becomes addmm(bf16(b*A), bf16(c*A), A), i.e.
    one rounding of bias + fp32 accumulator; `a*X + B @ X` likewise;
  * 3-D operands: the products are bmm's with bf16 outputs, and the axpy is a
    separate fused pointwise kernel in fp32 with one final rounding.

``rounding="eager"`` rounds after every op as torch eager mode does (TorchDynamo
disabled).  ``dtype=torch.float64`` runs the same chain in fp64, which is what the
closed-form pins use.

Parity status of each function is recorded beside the test that pins it; every
function here is pinned by a closed form, an invariant or a reference golden
vector (tests/test_oracle_*.py).
"""

import math
from itertools import repeat

import torch

# ---------------------------------------------------------------------------
# constants (defmuon/optim/muon.py:28, deflation_batched.py:42-59,229,
# polar_express.py:8-19)
# ---------------------------------------------------------------------------
NS_ABC = (3.4445, -4.7750, 2.0315)

_PE_RAW = [
    (8.28721201814563, -23.595886519098837, 17.300387312530933),
    (4.107059111542203, -2.9478499167379106, 0.5448431082926601),
    (3.9486908534822946, -2.908902115962949, 0.5518191394370137),
    (3.3184196573706015, -2.488488024314874, 0.51004894012372),
    (2.300652019954817, -1.6689039845747493, 0.4188073119525673),
    (1.891301407787398, -1.2679958271945868, 0.37680408948524835),
    (1.8750014808534479, -1.2500016453999487, 0.3750001645474248),
    (1.875, -1.25, 0.375),
]
# safety factor 1.01 on all but the last triple (polar_express.py:18-19)
PE_COEFFS = [(a / 1.01, b / 1.01 ** 3, c / 1.01 ** 5) for (a, b, c) in _PE_RAW[:-1]] \
    + [_PE_RAW[-1]]

DIVISOR_PAD = 1.01
PE_PAD = 1.1
RSVD_NITER = 1
CHOLQR_PASSES = 1
GATE_WINDOW = 0.025
SKETCH_FRAC = GATE_WINDOW
OVERSAMPLE_FRAC = 0.025
GATE_RATIO = 0.10
DEFLATE_THRESH = GATE_RATIO


def pe_schedule(steps):
    """First `steps` PE triples, the last one repeated (polar_express.py:27-28)."""
    return list(PE_COEFFS[:steps]) + list(repeat(PE_COEFFS[-1], steps - len(PE_COEFFS)))


def ns_schedule(steps):
    return [NS_ABC] * steps


# ---------------------------------------------------------------------------
# polynomial chains
# ---------------------------------------------------------------------------

def _rnd(t, dtype):
    return t.to(dtype)


# depth at which inductor stops inlining the running axpy chain (measured against
# torch.compile output on the CPU; tests/golden holds the reference's vectors)
_INLINE_DEPTH = 4


def _compiled_chain(Xs, Xe, hs, tall, dtype):
    """The bf16 chain as inductor lowers it (default config, which does not
    emulate intermediate bf16 casts).

    Every tensor has a stored value (bf16, what matmuls read) and an fp32
    expression value (what fused pointwise kernels read; they recompute their
    pointwise producers instead of loading the stored copy):

      2-D operands -- B = addmm(bf16(b*A), bf16(c*A), A) and
                      X' = addmm(bf16(a*Xe), B, X): one rounding of bias + fp32
                      accumulator; X' is an extern output, so Xe' = float(X').
      3-D operands -- products are bmm's with bf16 outputs, and
                      B = bf16(b*A + (cA)@A), Xe' = a*Xe + float(bf16(product)),
                      X' = bf16(Xe'): the fp32 running value Xe is inlined into
                      the next axpy until the inlined chain holds
                      _INLINE_DEPTH products, where inductor realizes it (stores
                      bf16) and the running value restarts from the stored copy.

    `tall` selects the deflated arm's form G = X^T X, X' = aX + X B
    (deflation_batched.py:200-203) instead of A = X X^T, X' = aX + B X
    (muon.py:36-40, polar_express.py:30-32)."""
    three_d = Xs.ndim == 3
    depth = 0
    for a, b, c in hs:
        A = Xs.mT @ Xs if tall else Xs @ Xs.mT
        Ae = A.float()
        cA = _rnd(c * Ae, dtype)
        if three_d:
            B = _rnd(b * Ae + (cA @ A).float(), dtype)
            P = Xs @ B if tall else B @ Xs
            Xe = a * Xe + P.float()
            Xs = _rnd(Xe, dtype)
            depth += 1
            if depth == _INLINE_DEPTH:
                Xe, depth = Xs.float(), 0
        else:
            B = torch.addmm(_rnd(b * Ae, dtype), cA, A)
            bias = _rnd(a * Xe, dtype)
            Xs = torch.addmm(bias, Xs, B) if tall else torch.addmm(bias, B, Xs)
            Xe = Xs.float()
    return Xs


def _wide_step(X, a, b, c, dtype):
    """One step A=XX^T; B=bA+(cA)@A; X=aX+B@X (muon.py:36-40) with torch's own
    per-op rounding (eager) or in fp32/fp64.  Python precedence makes
    `c * A @ A` mean (c*A) @ A."""
    A = X @ X.mT
    B = b * A + (c * A) @ A
    return a * X + B @ X


def _tall_step(X, a, b, c, dtype):
    """One step G=X^TX; B=bG+(cG)@G; X=aX+X@B (deflation_batched.py:200-203)."""
    G = X.mT @ X
    B = b * G + (c * G) @ G
    return a * X + X @ B


def _wide_chain(G, scale, hs, dtype, rounding, tr):
    X = G.to(dtype)
    if tr:
        X = X.mT
    if dtype == torch.bfloat16 and rounding == "compiled":
        gf = (G.mT if tr else G).float()
        nrm = gf.norm(dim=(-2, -1), keepdim=True)
        den = nrm * scale + 1e-7 if scale != 1.0 else nrm + 1e-7
        Xe = gf / den
        X = _compiled_chain(_rnd(Xe, dtype), Xe, hs, False, dtype)
    else:
        nrm = X.norm(dim=(-2, -1), keepdim=True)
        if scale != 1.0:
            nrm = nrm * scale
        X = X / (nrm + 1e-7)
        for a, b, c in hs:
            X = _wide_step(X, a, b, c, dtype)
    return X.mT if tr else X


def ns5(G, steps=5, dtype=torch.bfloat16, rounding="compiled"):
    """zeropower_via_newtonschulz5 (muon.py:16-44): entry X/(||X||_F+1e-7), NS_ABC
    for `steps` steps.  The transpose test compares size(0) with size(1), as the
    reference does (muon.py:30,42)."""
    assert G.ndim >= 2
    return _wide_chain(G, 1.0, ns_schedule(steps), dtype, rounding, G.size(0) > G.size(1))


def polar_express(G, steps=5, dtype=torch.bfloat16, rounding="compiled"):
    """PolarExpress (polar_express.py:21-34): divisor 1.01*||X||_F+1e-7, the PE
    schedule, transpose test on the last two dims."""
    assert G.ndim >= 2
    return _wide_chain(G, 1.01, pe_schedule(steps), dtype, rounding,
                       G.size(-2) > G.size(-1))


def horner_iterate(X, hs, rounding="compiled"):
    """_horner_iterate (deflation_batched.py:196-204), tall convention, in X.dtype."""
    dtype = X.dtype
    if dtype == torch.bfloat16 and rounding == "compiled":
        return _compiled_chain(X, X.float(), hs, True, dtype)
    for a, b, c in hs:
        X = _tall_step(X, a, b, c, dtype)
    return X


# ---------------------------------------------------------------------------
# randomized SVD front-end (fp32, fp64 Gram)
# ---------------------------------------------------------------------------

def sketch_dims(m, sketch=SKETCH_FRAC, oversample=OVERSAMPLE_FRAC, window=GATE_WINDOW):
    """(r, kw) from deflation_batched.py:170-171."""
    r = min(int(math.ceil(sketch * m)) + int(math.ceil(oversample * m)), m)
    kw = min(max(1, int(math.ceil(window * m))), r)
    return r, kw


def orth_b(X, passes=CHOLQR_PASSES):
    """Batched CholeskyQR (deflation_batched.py:117-128): fp64 Gram and Cholesky,
    fp32 triangular solve Q = X L^-T.  cholesky_ex's info is ignored, as in the
    reference."""
    Q = X
    for _ in range(passes):
        Xd = Q.to(torch.float64)
        G = Xd.mT @ Xd
        L, _ = torch.linalg.cholesky_ex(G)
        Q = torch.linalg.solve_triangular(L.to(Q.dtype).mT, Q, upper=True, left=False)
    return Q


def project_b(Q, A):
    """Rayleigh-Ritz (deflation_batched.py:131-139): Bp = Q^T A, thin SVD (LAPACK
    on the CPU), U = Q Ub, V = Vh^T."""
    Bp = Q.mT @ A
    Ub, s, Vh = torch.linalg.svd(Bp, full_matrices=False)
    return Q @ Ub, s, Vh.mT


def rsvd_b(A, Omega, n_iter=RSVD_NITER, passes=CHOLQR_PASSES):
    """Batched subspace iteration (deflation_batched.py:142-148)."""
    Q = orth_b(A @ Omega, passes)
    for _ in range(n_iter):
        Z = orth_b(A.mT @ Q, passes)
        Q = orth_b(A @ Z, passes)
    return project_b(Q, A)


def gate(s, kw, ratio=GATE_RATIO, thresh=DEFLATE_THRESH):
    """Gate on descending s (B, r) (deflation_batched.py:177-183).
    Returns (kk, fired, head) with head the (B, r) top-block mask."""
    r = s.shape[1]
    kr = (s > thresh * s[:, :1]).sum(dim=1)
    fired = (s[:, kw - 1] < ratio * s[:, 0]) & (kr >= 1) & (kr < r)
    kk = kr.clamp(1, r - 1)
    idx = torch.arange(r)[None, :]
    head = (idx < kk[:, None]) * fired[:, None]
    return kk, fired, head


def rmfro_clip(A, Omega, pad=DIVISOR_PAD, out_dtype=None, n_iter=RSVD_NITER,
               passes=CHOLQR_PASSES, window=GATE_WINDOW, ratio=GATE_RATIO,
               thresh=DEFLATE_THRESH):
    """batched_rmfro_clip (deflation_batched.py:155-189) with an injected sketch.
    A (B, n, m) fp32 with n >= m; Omega (B, m, r).  Returns (X0, k, d)."""
    Bn, n, m = A.shape
    r = Omega.shape[-1]
    kw = min(max(1, int(math.ceil(window * m))), r)
    U, s, V = rsvd_b(A, Omega, n_iter, passes)
    kk, fired, head = gate(s, kw, ratio, thresh)
    W = A - (U * (s * head)[:, None, :]) @ V.mT
    d = W.norm(dim=(-2, -1), keepdim=True) + 1e-7
    X0 = W / d + (U * ((1.0 / pad) * head)[:, None, :]) @ V.mT
    if out_dtype is not None:
        X0 = X0.to(out_dtype)
    return X0, kk * fired, d.reshape(Bn)


def draw_omega(B, m, r, seed, device="cpu"):
    """The sketch as the reference draws it: randn(B, m, r) fp32 from a Generator
    seeded with `seed` on `device` (deflation_batched.py:172-174)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.randn(B, m, r, device=device, dtype=torch.float32, generator=g)


def group_seed(bd_step, gi):
    """Sketch seed of shape group gi at batched step bd_step (muon.py:290-291)."""
    return (bd_step * 1009 + gi * 9176867) % (2 ** 62)


def deflated_polar(A, Omega, arm="ns", steps=5, rounding="compiled"):
    """One deflated arm end to end on a tall batch: clip to bf16, then the arm's
    Horner schedule (deflation_batched.py:221-256)."""
    pad = DIVISOR_PAD if arm == "ns" else PE_PAD
    X0, k, d = rmfro_clip(A, Omega, pad=pad, out_dtype=torch.bfloat16)
    hs = ns_schedule(steps) if arm == "ns" else pe_schedule(steps)
    return horner_iterate(X0, hs, rounding), k, d


# ---------------------------------------------------------------------------
# accuracy measures (spectra/polar_convergence.py:138-141, 173-174)
# ---------------------------------------------------------------------------

def exact_polar(A):
    U, _, Vh = torch.linalg.svd(A.double(), full_matrices=False)
    return U @ Vh


def rel_err(X, P):
    return float((X.double() - P).norm() / P.norm())


def orth_residual(O):
    """||O^T O - I||_F (tall) / ||O O^T - I||_F (wide), in fp64."""
    O = O.double()
    if O.shape[-2] < O.shape[-1]:
        O = O.mT
    I = torch.eye(O.shape[-1], dtype=torch.float64)
    return float((O.mT @ O - I).norm())
