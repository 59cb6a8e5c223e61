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


# ---------------------------------------------------------------------------
# the collector's hook logic on a CPU optimizer with the same momentum state
# (torch.optim.SGD keeps "momentum_buffer" and reads "momentum"/"nesterov" from its
# groups, as Muon does; with dampening 0 its buffer update is Muon's)
# ---------------------------------------------------------------------------

def _toy_model(D=8, layers=3, seed=0):
    g = torch.Generator().manual_seed(seed)
    shapes = {}
    for i in range(layers):
        shapes[f"transformer.h.{i}.ln_1.weight"] = (D,)
        shapes[f"transformer.h.{i}.attn.c_attn.weight"] = (3 * D, D)
        shapes[f"transformer.h.{i}.attn.c_proj.weight"] = (D, D)
        shapes[f"transformer.h.{i}.mlp.c_fc.weight"] = (4 * D, D)
        shapes[f"transformer.h.{i}.mlp.c_proj.weight"] = (D, 4 * D)
        shapes[f"transformer.h.{i}.mlp.c_proj.bias"] = (D,)
    shapes["transformer.wte.weight"] = (50, D)
    return {k: torch.nn.Parameter(torch.randn(*v, generator=g)) for k, v in shapes.items()}


def _expected_inputs(opt, params, names):
    """The factorizer inputs of the next step, from the state as it is now."""
    out = {}
    for lbl, name in names.items():
        p = params[name]
        buf = opt.state[p].get("momentum_buffer")
        g32 = p.grad.float()
        nb = g32.clone() if buf is None else buf * 0.9 + g32
        out[lbl] = g32 + 0.9 * nb
    return out


def test_middle_layer_targets():
    """The middle block of n_layer blocks is block n_layer // 2; its four dumped
    weights come back in parameter order (collect.py:64-76)."""
    for layers, mid in ((3, 1), (4, 2), (1, 0)):
        params = _toy_model(layers=layers)
        t = D.middle_layer_targets(params.items())
        assert [l for l, _ in t] == ["attn_qkv", "attn_o", "mlp_fc", "mlp_proj"]
        assert t[0][1] is params[f"transformer.h.{mid}.attn.c_attn.weight"]
        assert t[3][1] is params[f"transformer.h.{mid}.mlp.c_proj.weight"]
    assert D.middle_layer_targets([("wte.weight", torch.zeros(3, 3))]) == []


def test_collector_records_the_pre_step_inputs(tmp_path):
    """Dumps at the chosen steps hold the factorizer input computed from the state
    before that step (collect.py:89-113); quantiles every qstep steps, Q/K/V apart,
    rewritten in full each time (collect.py:115-139); training is unchanged."""
    params = _toy_model()
    ref = {k: torch.nn.Parameter(v.detach().clone()) for k, v in params.items()}
    opt = torch.optim.SGD(params.values(), lr=0.01, momentum=0.9, nesterov=True)
    opt_ref = torch.optim.SGD(ref.values(), lr=0.01, momentum=0.9, nesterov=True)
    col = D.SpectraCollector(D.middle_layer_targets(params.items()), str(tmp_path), [1, 3], 2,
                             writer=True)
    col.attach(opt)
    names = {"attn_qkv": "transformer.h.1.attn.c_attn.weight",
             "attn_o": "transformer.h.1.attn.c_proj.weight",
             "mlp_fc": "transformer.h.1.mlp.c_fc.weight",
             "mlp_proj": "transformer.h.1.mlp.c_proj.weight"}
    g = torch.Generator().manual_seed(1)
    want = {}
    for step in range(1, 5):
        for k in params:
            gr = torch.randn(params[k].shape, generator=g)
            params[k].grad, ref[k].grad = gr.clone(), gr.clone()
        want[step] = _expected_inputs(opt, params, names)
        opt.step()
        opt_ref.step()
    assert col.step_count == 4
    for k in params:                                   # read-only: same trajectory
        assert torch.equal(params[k], ref[k]), k
    files = sorted(f.name for f in tmp_path.iterdir() if f.suffix == ".pt")
    assert files == sorted(D.dump_name(s, l) for s in (1, 3) for l in names)
    for s in (1, 3):
        for lbl in names:
            d = D.load_dump(str(tmp_path / D.dump_name(s, lbl)))
            assert d["step"] == s and d["label"] == lbl
            assert d["momentum"] == 0.9 and d["nesterov"] is True
            assert torch.allclose(d["A"], want[s][lbl], rtol=1e-6, atol=1e-6), (s, lbl)
    import json
    recs = json.load(open(tmp_path / "quantiles.json"))
    assert [(r["step"], r["label"]) for r in recs] == [
        (s, l) for s in (2, 4) for l in D.PANEL_COLS]
    qkv = want[4]["attn_qkv"]
    rec = [r for r in recs if r["step"] == 4 and r["label"] == "attn_k"][0]
    assert rec == {"step": 4, "label": "attn_k", **D.sv_quantiles(qkv[8:16])}


def test_collector_counts_each_step_once(tmp_path):
    """Once a step function has been replaced after an optimizer of its class was
    built (as an install() hook does), torch wraps the new function again and the
    pre-hooks fire twice per step; the collector still counts one step per call.
    A step that raises is counted, and the next one is too."""
    class Opt(torch.optim.SGD):
        fail = False

        def step(self, closure=None):
            if self.fail:
                raise RuntimeError("planted failure")
            return super().step(closure)

    params = _toy_model()
    Opt(list(params.values()), lr=0.01, momentum=0.9)     # wraps Opt.step once
    inner = Opt.step

    def outer(self, closure=None):
        return inner(self, closure)

    Opt.step = outer
    opt = Opt(list(params.values()), lr=0.01, momentum=0.9, nesterov=True)  # wraps outer
    col = D.SpectraCollector(D.middle_layer_targets(params.items()), str(tmp_path), [2, 4], 0,
                             writer=True)
    col.attach(opt)
    calls = []
    opt.register_step_pre_hook(lambda o, a, k: calls.append(1))
    g = torch.Generator().manual_seed(2)
    for step in range(1, 5):
        for p in params.values():
            p.grad = torch.randn(p.shape, generator=g)
        opt.fail = step == 2
        if opt.fail:
            with pytest.raises(RuntimeError):
                opt.step()
        else:
            opt.step()
    assert len(calls) > 4            # the hooks did fire more than once per step
    assert col.step_count == 4
    files = sorted(f.name for f in tmp_path.iterdir() if f.suffix == ".pt")
    assert files == sorted(D.dump_name(s, l) for s in (2, 4)
                           for l in ("attn_qkv", "attn_o", "mlp_fc", "mlp_proj"))
