"""Accuracy studies of the deflated polar path on dumped momenta, on the GPU.

rSVD head accuracy (spectra/rsvd_accuracy.py): for every matrix and sketch seed, the
production front-end's randomized SVD (this library's `_rsvd_b`, Gaussian sketch of
ceil(2.5% m) + ceil(2.5% m) columns drawn on the CPU generator exactly as
rsvd_accuracy.py:40-48 does) and the production gate; where the gate fires, the k
deflated singular values against the leading k of an fp64 SVD:
    sv_err = max_{i<k} |s_i - sigma_i| / sigma_i
Rows: step, label, seed, fired, k, sv_err (rsvd_accuracy.py:86-92).

Polar-factor convergence (spectra/polar_convergence.py): for every matrix, the four
methods with their production entries (polar_convergence.py:151-170) and the relative
Frobenius error ||X_k - UV^T||_F / ||UV^T||_F against the fp64 polar factor after each
of the 5 iterations (polar_convergence.py:173-188).  Entries and the deflation front-end
run through this library, and so does the iteration: `_horner_iterate` one step at a
time in the study's dtype, as the reference's `run` does (polar_convergence.py:177-185),
i.e. the library's bf16 MFMA chain (the training precision) or, with iter_dtype fp32
(the reference's default, which isolates estimation and mapping effects from bf16
rounding), its fp32 chain.  Rows: tag, step, matrix, method, rel_err_k0..k5,
k_deflated, iter_dtype (polar_convergence.py:309-320).
"""

import csv
import math
import zlib

import torch

from defmuon_amd.optim import deflation_batched as DB
from defmuon_amd.optim.polar_express import coeffs_list as PE_COEFFS
from defmuon_amd.spectra.dumps import PANEL_COLS, ROW_NAME

NS_ABC = (3.4445, -4.7750, 2.0315)
NS_STEPS = 5
SEED = 20260915                 # sketch seed base (polar_convergence.py:84)
METHODS = ["ns5", "polarexpress", "deflated_ns", "deflated_pe"]
ITER_DTYPES = {"bf16": torch.bfloat16, "fp32": torch.float32}


def sketch_seed(step, lbl):
    """Per-matrix sketch seed (polar_convergence.py:144-145)."""
    return SEED + 7919 * int(step) + zlib.crc32(lbl.encode()) % 1000


def exact_polar(A):
    """UV^T from an fp64 SVD (polar_convergence.py:138-141)."""
    U, _, Vh = torch.linalg.svd(A.double(), full_matrices=False)
    return U @ Vh


# ---------------------------------------------------------------------------
# rSVD head accuracy
# ---------------------------------------------------------------------------

def rsvd_one(A, se, seed):
    """(fired, k, sv_err) for one sketch of the tall fp32 matrix A (on the GPU) with
    exact singular values se (fp64, descending) (rsvd_accuracy.py:40-54)."""
    n, m = A.shape
    r = min(math.ceil(DB.SKETCH_FRAC * m) + math.ceil(DB.OVERSAMPLE_FRAC * m), m)
    kw = min(max(1, math.ceil(DB.GATE_WINDOW * m)), r)
    gen = torch.Generator().manual_seed(seed)
    Omega = torch.randn(1, m, r, dtype=A.dtype, generator=gen).to(A.device)
    _, s, _ = DB._rsvd_b(A[None], Omega, DB.RSVD_NITER)
    s = s[0].double().cpu()
    k = int((s > DB.DEFLATE_THRESH * s[0]).sum())
    fired = bool(s[kw - 1] < DB.GATE_RATIO * s[0]) and 1 <= k < r
    if not fired:
        return False, 0, float("nan")
    se = se.cpu()
    return True, k, float(((s[:k] - se[:k]).abs() / se[:k]).max())


def rsvd_accuracy(data, seeds, device="cuda", log=None):
    """Rows (step, label, seed, fired, k, sv_err) over {step: {label: A}}
    (rsvd_accuracy.py:78-92)."""
    rows = []
    for step in sorted(data):
        for lbl in [c for c in PANEL_COLS if c in data[step]]:
            A = data[step][lbl].to(device)
            se = torch.linalg.svdvals(A.double().cpu())
            for sidx in range(seeds):
                fired, k, err = rsvd_one(A, se, sketch_seed(step, lbl) + 100003 * sidx)
                rows.append(dict(step=step, label=lbl, seed=sidx, fired=int(fired), k=k, sv_err=err))
            if log:
                fr = sorted(r["sv_err"] for r in rows
                            if r["step"] == step and r["label"] == lbl and r["fired"])
                log(f"step {step:>4} {lbl:9s} {tuple(A.shape)}  fired {len(fr)}/{seeds}"
                    + (f"  median sv_err {fr[len(fr) // 2]:.2e}" if fr else ""))
    return rows


def write_rsvd_csv(rows, path):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["step", "label", "seed", "fired", "k", "sv_err"])
        w.writeheader()
        w.writerows(rows)


# ---------------------------------------------------------------------------
# polar-factor convergence
# ---------------------------------------------------------------------------

def entry(method, A, seed):
    """(X0 fp32, k) for the tall matrix A (on the GPU): the method's production entry
    and the deflation width its front-end chose (polar_convergence.py:151-165)."""
    fro = A.norm()
    if method == "ns5":
        return A / (fro + 1e-7), 0
    if method == "polarexpress":
        return A / (1.01 * fro + 1e-7), 0
    pad = DB.DIVISOR_PAD if method == "deflated_ns" else DB.DeflatedPEPolar.PAD
    gen = torch.Generator(device=A.device).manual_seed(seed)
    X0, k, _ = DB.batched_rmfro_clip(A[None], generator=gen, pad=pad)
    return X0[0], int(k[0])


def schedule(method):
    """polar_convergence.py:168-171"""
    if method in ("polarexpress", "deflated_pe"):
        return PE_COEFFS[:NS_STEPS]
    return [NS_ABC] * NS_STEPS


def rel_err(X, P):
    return float((X.double() - P).norm() / P.norm())


def run(method, A, P, seed, iter_dtype="bf16"):
    """(rel_err after k = 0..NS_STEPS iterations, deflation width) for one method on
    the tall matrix A with exact polar factor P (polar_convergence.py:178-188)."""
    X0, k = entry(method, A, seed)
    X = X0.to(ITER_DTYPES[iter_dtype])
    rel = [rel_err(X, P)]
    for coef in schedule(method):
        X = DB._horner_iterate(X, [coef])
        rel.append(rel_err(X, P))
    return rel, k


def polar_convergence(data, iter_dtype="bf16", tag="", device="cuda", log=None):
    """Rows as polar_convergence.py:309-320 writes them, over {step: {label: A}}."""
    rows = []
    for step in sorted(data):
        for lbl in [c for c in PANEL_COLS if c in data[step]]:
            A = data[step][lbl].to(device)
            P = exact_polar(A)
            seed = sketch_seed(step, lbl)
            res = {m: run(m, A, P, seed, iter_dtype) for m in METHODS}
            for meth in METHODS:
                rel, k = res[meth]
                row = dict(tag=tag, step=step, matrix=ROW_NAME[lbl].replace("$", ""), method=meth)
                row.update({f"rel_err_k{i}": f"{v:.6g}" for i, v in enumerate(rel)})
                row["k_deflated"] = k if meth.startswith("deflated") else ""
                row["iter_dtype"] = iter_dtype
                rows.append(row)
            if log:
                log(f"step {step:>4} {lbl:9s} {tuple(A.shape)}  "
                    + "  ".join(f"{m}: k5={res[m][0][-1]:.4f}"
                                + (f" (k={res[m][1]})" if m.startswith("deflated") else "")
                                for m in METHODS))
    return rows


def write_convergence_csv(rows, path):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0].keys()))
        w.writeheader()
        w.writerows(rows)
