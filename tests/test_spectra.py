"""CPU checks of the spectra dump format, its loader and the harness's host logic
(defmuon_amd.spectra; reference: spectra/collect.py, spectra/polar_convergence.py,
spectra/rsvd_accuracy.py)."""

import os

import pytest
import torch

from defmuon_amd.spectra import dumps as D


def _write(tmp, step, E=16):
    g = torch.Generator().manual_seed(step)
    mats = {"attn_qkv": torch.randn(3 * E, E, generator=g),     # c_attn: rows Q | K | V
            "attn_o": torch.randn(E, E, generator=g),
            "mlp_fc": torch.randn(4 * E, E, generator=g),       # tall
            "mlp_proj": torch.randn(E, 4 * E, generator=g),     # wide: stored transposed
            "other": torch.randn(5, 5, generator=g)}            # not a projected matrix
    for lbl, A in mats.items():
        D.save_dump(tmp, step, lbl, A, 0.95, True)
    return mats


def test_dump_file_format(tmp_path):
    """One file per (step, label), named step{step:04d}_{label}.pt, holding exactly the
    reference's keys (collect.py:109-113); readable with the safe loader."""
    A = torch.randn(8, 4)
    path = D.save_dump(str(tmp_path), 12, "attn_o", A, 0.9, False)
    assert os.path.basename(path) == "step0012_attn_o.pt"
    d = torch.load(path, map_location="cpu", weights_only=True)
    assert set(d) == {"step", "label", "A", "momentum", "nesterov"}
    assert d["step"] == 12 and d["label"] == "attn_o" and d["momentum"] == 0.9
    assert d["nesterov"] is False
    assert d["A"].dtype == torch.float32 and torch.equal(d["A"], A)


def test_load_matrices_splits_and_transposes(tmp_path):
    """load_matrices follows polar_convergence.py:117-137: Q/K/V are the row blocks of
    the c_attn dump, wide matrices come back transposed (tall), other labels drop."""
    m1 = _write(str(tmp_path), 1)
    m2 = _write(str(tmp_path), 500)
    data = D.load_matrices(str(tmp_path))
    assert sorted(data) == [1, 500]
    for step, mats in ((1, m1), (500, m2)):
        ent = data[step]
        assert sorted(ent) == sorted(D.PANEL_COLS)
        E = 16
        for i, sub in enumerate(["attn_q", "attn_k", "attn_v"]):
            assert torch.equal(ent[sub], mats["attn_qkv"][i * E:(i + 1) * E])
        assert torch.equal(ent["mlp_proj"], mats["mlp_proj"].mT)
        assert torch.equal(ent["mlp_fc"], mats["mlp_fc"])
        for M in ent.values():
            assert M.shape[0] >= M.shape[1] and M.is_contiguous()


def test_momentum_A_is_the_nesterov_input():
    """The dumped matrix is what Muon's step feeds the factorizer: after
    buf <- mu buf + g, the Nesterov input g + mu buf (muon.py:266-272); without
    Nesterov, buf itself; on the first step (no buffer) (1 + mu) g."""
    g = torch.Generator().manual_seed(0)
    grad, buf = torch.randn(6, 5, generator=g), torch.randn(6, 5, generator=g)
    mu = 0.95
    b2 = buf.clone().mul_(mu).add_(grad)
    want = grad.add(b2, alpha=mu)
    assert torch.allclose(D.momentum_A(grad, buf, mu, True), want, rtol=1e-6, atol=1e-7)
    before = buf.clone()
    assert torch.equal(D.momentum_A(grad, buf, mu, False), b2)
    assert torch.equal(buf, before)                       # computed out of place
    assert torch.allclose(D.momentum_A(grad, None, mu, True), (1 + mu) * grad, rtol=1e-6)


def test_sv_quantiles_are_order_statistics():
    """sv_quantiles picks the ceil(q r)-th largest singular value over ||B||_F
    (collect.py:127-135): a diagonal matrix reads its own entries back."""
    s = torch.tensor([10.0, 8.0, 6.0, 4.0, 2.0, 1.0, 0.5, 0.25, 0.1, 0.05])
    rec = D.sv_quantiles(torch.diag(s))
    fro = float(s.norm())
    assert rec["sigma_max"] == pytest.approx(10.0, rel=1e-6)
    assert rec["fro"] == pytest.approx(fro, rel=1e-6)
    # r = 10: q = 0.1 -> 1st, 0.25 -> 3rd, 0.5 -> 5th, 0.75 -> 8th, 0.9 -> 9th largest
    for q, idx in ((0.1, 0), (0.25, 2), (0.5, 4), (0.75, 7), (0.9, 8)):
        assert rec["q"][str(q)] == pytest.approx(float(s[idx]) / fro, rel=1e-5)


def test_sketch_seed_distinguishes_matrices():
    """Per-matrix sketch seeds (polar_convergence.py:144-145): the base plus 7919 per
    step plus a label hash below 1000, so steps 1 apart never collide."""
    from defmuon_amd.spectra.accuracy import SEED, sketch_seed
    seeds = {(s, l): sketch_seed(s, l) for s in (1, 2, 500) for l in D.PANEL_COLS}
    assert len(set(seeds.values())) == len(seeds)
    for (s, l), v in seeds.items():
        assert 0 <= v - SEED - 7919 * s < 1000


def test_cli_refuses_without_gpu(tmp_path, capsys):
    from defmuon_amd.spectra.__main__ import main
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert main(["rsvd", "--dumps", str(tmp_path), "--out", str(tmp_path / "o")]) == 1
