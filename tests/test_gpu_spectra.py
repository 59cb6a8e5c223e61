"""GPU checks of the spectra harness (defmuon_amd.spectra): the rSVD accuracy and
polar-convergence studies of spectra/rsvd_accuracy.py and spectra/polar_convergence.py
run through the library, checked against the CPU oracle on the same sketches, and the
collector's dumps against the optimizer's own momentum."""

import json
import os

import pytest
import torch

from oracle import polar_oracle as O
from parity import POLAR_TOL, log_parity

pytestmark = pytest.mark.gpu
DEV = "cuda"
E = 256          # m = 256: r = 14, kw = 7
K_DESIGN = 3     # three spikes, 50..20 times the bulk edge: k = 3 where the gate looks


@pytest.fixture(scope="module")
def dump_dir(tmp_path_factory):
    from defmuon_amd import synthetic as S
    from defmuon_amd.spectra import dumps as SD
    d = str(tmp_path_factory.mktemp("dumps"))
    for step in (1, 500):
        sp = lambda r, c, s: S.spiked_matrix(r, c, seed=10 * step + s, n_spikes=K_DESIGN,
                                             hi=50.0, lo=20.0)
        SD.save_dump(d, step, "attn_qkv", torch.cat([sp(E, E, j) for j in range(3)]), 0.95, True)
        SD.save_dump(d, step, "attn_o", sp(E, E, 5), 0.95, True)
        SD.save_dump(d, step, "mlp_fc", sp(4 * E, E, 6), 0.95, True)
        SD.save_dump(d, step, "mlp_proj", sp(E, 4 * E, 7), 0.95, True)
    return d


def test_rsvd_accuracy_matches_oracle(dump_dir):
    """Every sketch fires with the designed k, and sv_err agrees with the oracle's
    rSVD (CPU, fp32, the reference's arithmetic) on the same sketch."""
    from defmuon_amd.spectra import accuracy as SA
    from defmuon_amd.spectra.dumps import load_matrices
    data = load_matrices(dump_dir)
    rows = SA.rsvd_accuracy(data, seeds=2)
    assert len(rows) == 2 * 6 * 2
    for row in rows:
        assert row["fired"] == 1 and row["k"] == K_DESIGN, row
        A = data[row["step"]][row["label"]]
        m = A.shape[1]
        r, kw = O.sketch_dims(m)
        g = torch.Generator().manual_seed(SA.sketch_seed(row["step"], row["label"])
                                          + 100003 * row["seed"])
        Om = torch.randn(1, m, r, generator=g)
        _, s, _ = O.rsvd_b(A[None], Om)
        se = torch.linalg.svdvals(A.double())
        err_o = float(((s[0, :K_DESIGN].double() - se[:K_DESIGN]).abs() / se[:K_DESIGN]).max())
        assert row["sv_err"] < 1e-4, row
        assert abs(row["sv_err"] - err_o) < 2e-6, (row, err_o)


# curve tolerance per iteration dtype: bf16 two correct chains with different rounding
# points (the library's MFMA chain, the reference's eager bf16 ops), as for every
# polar factor; fp32 the same iteration in fp32 on both sides
CURVE_TOL = {"bf16": POLAR_TOL, "fp32": 1e-5}


@pytest.mark.parametrize("iter_dtype", ["fp32", "bf16"])
def test_polar_convergence(dump_dir, iter_dtype):
    """Rows in the reference's columns, and every point of every curve against the
    oracle: the same entry (the oracle's clip on the same sketch for the deflated
    arms) followed by the reference study's iteration, `_horner_iterate` one step at
    a time in the study's dtype with eager rounding (polar_convergence.py:61,177-185).
    The deflated arms choose k = 3 and end closer to the polar factor than their plain
    arms on spiked matrices."""
    from defmuon_amd.spectra import accuracy as SA
    from defmuon_amd.spectra.dumps import ROW_NAME, load_matrices
    data = load_matrices(dump_dir)
    rows = SA.polar_convergence(data, iter_dtype, tag="t")
    assert len(rows) == 2 * 6 * 4
    assert list(rows[0]) == (["tag", "step", "matrix", "method"]
                             + [f"rel_err_k{i}" for i in range(6)] + ["k_deflated", "iter_dtype"])
    by = {(r["step"], r["matrix"], r["method"]): r for r in rows}
    name = {ROW_NAME[l].replace("$", ""): l for l in ROW_NAME}
    dtype = SA.ITER_DTYPES[iter_dtype]
    worst = 0.0
    for (step, matrix, method), r in by.items():
        assert r["iter_dtype"] == iter_dtype
        curve = [float(r[f"rel_err_k{i}"]) for i in range(6)]
        if method.startswith("deflated"):
            assert r["k_deflated"] == K_DESIGN
            plain = "ns5" if method == "deflated_ns" else "polarexpress"
            assert curve[-1] < float(by[(step, matrix, plain)]["rel_err_k5"]), (step, matrix)
        A = data[step][name[matrix]]
        P = O.exact_polar(A)
        seed = SA.sketch_seed(step, name[matrix])
        if method.startswith("deflated"):
            m = A.shape[1]
            r_, _ = O.sketch_dims(m)
            g = torch.Generator(device=DEV).manual_seed(seed)
            Om = torch.randn(1, m, r_, device=DEV, generator=g).cpu()
            pad = 1.01 if method == "deflated_ns" else 1.1
            X0, k, _ = O.rmfro_clip(A[None], Om, pad=pad)
            assert int(k[0]) == K_DESIGN
            X = X0[0]
        else:
            X = A / ((1.01 if method == "polarexpress" else 1.0) * A.norm() + 1e-7)
        X = X.to(dtype)
        want = [O.rel_err(X, P)]
        for coef in SA.schedule(method):
            X = O.horner_iterate(X, [coef], rounding="eager")
            want.append(O.rel_err(X, P))
        dev = max(abs(a - b) for a, b in zip(curve, want))
        log_parity("convergence", f"{iter_dtype} {step} {matrix} {method}", max_curve_diff=dev)
        assert dev <= CURVE_TOL[iter_dtype], (step, matrix, method, curve, want)
        worst = max(worst, dev)
    print(f"polar convergence ({iter_dtype}): largest curve difference {worst:.2e}")


def test_collector_dumps_the_factorizer_input(tmp_path, monkeypatch):
    """The collector (spectra/collect.py) dumps the middle layer's post-Nesterov
    matrices at the chosen steps and writes singular-value quantiles every QSTEP
    steps; at step 1 (no momentum yet) A = (1 + mu) grad."""
    from defmuon_amd.optim import muon as M
    from defmuon_amd.spectra import dumps as SD
    monkeypatch.setattr(M.Muon, "__init__", M.Muon.__init__)   # restored afterwards
    monkeypatch.setattr(M.Muon, "step", M.Muon.step)
    monkeypatch.setattr(SD, "_INSTALLED", [False])
    monkeypatch.setenv("DEFMUON_SPECTRA_DIR", str(tmp_path))
    monkeypatch.setenv("DEFMUON_SPECTRA_TAG", "tiny")
    monkeypatch.setenv("DEFMUON_SPECTRA_STEPS", "1")
    monkeypatch.setenv("DEFMUON_SPECTRA_QSTEP", "2")
    SD.install()
    D = 64
    g = torch.Generator().manual_seed(3)
    shapes = {}
    for i in range(2):
        shapes[f"transformer.h.{i}.attn.c_attn.weight"] = (3 * D, D)
        shapes[f"transformer.h.{i}.attn.c_proj.weight"] = (D, D)
        shapes[f"transformer.h.{i}.mlp.c_fc.weight"] = (4 * D, D)
        shapes[f"transformer.h.{i}.mlp.c_proj.weight"] = (D, 4 * D)
    params = {k: torch.nn.Parameter((torch.randn(*v, generator=g) * 0.02).to(DEV))
              for k, v in shapes.items()}
    opt = M.Muon(params.items(), lr=0.01, momentum=0.95, nesterov=True, ns_steps=5,
                 polar_method="ns5")
    grads = []
    for step in range(2):
        gs = {k: torch.randn(*p.shape, generator=g).to(DEV) for k, p in params.items()}
        for k, p in params.items():
            p.grad = gs[k]
        grads.append(gs)
        opt.step()
    torch.cuda.synchronize()
    out = os.path.join(str(tmp_path), "tiny")
    files = sorted(f for f in os.listdir(out) if f.endswith(".pt"))
    assert files == [SD.dump_name(1, l) for l in sorted(["attn_qkv", "attn_o", "mlp_fc", "mlp_proj"])]
    lbl = {"attn_qkv": "attn.c_attn", "attn_o": "attn.c_proj", "mlp_fc": "mlp.c_fc",
           "mlp_proj": "mlp.c_proj"}
    for f in files:
        d = SD.load_dump(os.path.join(out, f))
        gname = f"transformer.h.1.{lbl[d['label']]}.weight"      # the middle layer
        assert torch.allclose(d["A"], 1.95 * grads[0][gname].cpu(), rtol=1e-6, atol=1e-7)
    q = json.load(open(os.path.join(out, "quantiles.json")))
    assert sorted({r["label"] for r in q}) == sorted(["attn_q", "attn_k", "attn_v", "attn_o",
                                                       "mlp_fc", "mlp_proj"])
    assert all(r["step"] == 2 for r in q)
