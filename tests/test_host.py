"""CPU checks of the host-side mirror of the reference interface (no GPU)."""

import math

import pytest
import torch


def test_constants_match_reference_defaults():
    from defmuon_amd.optim import deflation_batched as DB
    assert DB.DIVISOR_PAD == 1.01 and DB.RSVD_NITER == 1 and DB.CHOLQR_PASSES == 1
    assert DB.GRAM_DTYPE is torch.float64
    assert DB.GATE_WINDOW == DB.SKETCH_FRAC == DB.OVERSAMPLE_FRAC == 0.025
    assert DB.GATE_RATIO == DB.DEFLATE_THRESH == 0.10
    assert DB.DeflatedPEPolar.PAD == 1.1 and DB.DeflatedNSPolar.PAD == 1.01
    assert DB.DeflatedNSPolar.NS_ABC == (3.4445, -4.7750, 2.0315)


def test_pe_schedule_matches_oracle():
    from defmuon_amd.optim import polar_express as PE
    from oracle import polar_oracle as O
    assert PE.coeffs_list == O.PE_COEFFS
    assert PE.pe_schedule(11) == O.pe_schedule(11)


@pytest.mark.parametrize("m", [64, 80, 768, 1024, 1280])
def test_sketch_dims_match_oracle(m):
    from defmuon_amd.optim import deflation_batched as DB
    from oracle import polar_oracle as O
    assert DB.sketch_dims(m) == O.sketch_dims(m)


def test_polar_stats_schema():
    from defmuon_amd.optim import deflation_batched as DB
    DB._GATE_ACC[0] = torch.tensor([10, 4, 9])
    st = DB.polar_stats()
    assert st == dict(fired=4, total=10, k_mean=9 / 4, degenerate=0, parachute=0)
    DB._GATE_ACC[0] = None
    assert DB.polar_stats() == dict(fired=0, total=0, k_mean=0.0, degenerate=0, parachute=0)


def test_timing_accumulator():
    from defmuon_amd.optim import deflation_batched as DB

    class Ev:
        def __init__(self, t):
            self.t = t

        def elapsed_time(self, other):
            return other.t - self.t

    DB._PENDING.append((Ev(0.0), Ev(2.0), Ev(5.0)))
    st = DB.timing_stats()
    assert st == {"clip_ms": 2.0, "iter_ms": 3.0, "calls": 1}
    assert DB.timing_stats() == {"clip_ms": 0.0, "iter_ms": 0.0, "calls": 0}


def test_no_cpu_fallback():
    """The product path runs only through the HIP library."""
    from defmuon_amd import _native
    from defmuon_amd.optim import deflation_batched as DB
    from defmuon_amd.optim import muon
    G = torch.randn(16, 32)
    with pytest.raises(_native.NativeError):
        muon.zeropower_via_newtonschulz5(G, 5)
    with pytest.raises(_native.NativeError):
        DB.batched_rmfro_clip(torch.randn(1, 64, 32), Omega=torch.randn(1, 32, 2))


def test_muon_routing_and_arms(capsys):
    from defmuon_amd.optim import deflation_batched as DB
    from defmuon_amd.optim import deflation_cutoff as C
    from defmuon_amd.optim import muon
    C.install()
    C.install()           # idempotent
    params = [("wte.weight", torch.nn.Parameter(torch.zeros(10, 4))),
              ("h.0.attn.c_attn.weight", torch.nn.Parameter(torch.zeros(12, 4))),
              ("h.0.mlp.c_fc.weight", torch.nn.Parameter(torch.zeros(16, 4))),
              ("h.0.ln_1.weight", torch.nn.Parameter(torch.zeros(4)))]
    opt = muon.Muon(params, polar_method="deflated_ns_cut")
    assert isinstance(opt.polar_factorizer, C.CutoffDeflatedNSPolar)
    assert isinstance(opt.polar_factorizer, DB._DeflatedPolarBase)
    assert opt.batched_deflation and opt._bd_step == 0
    st = opt.state
    assert st[params[0][1]]["use_muon"] is False
    assert st[params[1][1]]["use_muon"] and st[params[1][1]]["is_W_QKV"]
    assert st[params[2][1]]["use_muon"] and "is_W_QKV" not in st[params[2][1]]
    assert st[params[3][1]]["use_muon"] is False
    assert opt._qkv_split(params[1][1], params[1][1]).shape == (3, 4, 4)
    opt2 = muon.Muon(params, polar_method="deflated_pe_cut")
    assert isinstance(opt2.polar_factorizer, C.CutoffDeflatedPEPolar)
    assert opt2.polar_factorizer.POST == "polarexpress"
    assert muon.Muon(params, polar_method="ns5").polar_factorizer is muon.zeropower_via_newtonschulz5
    with pytest.raises(ValueError):
        muon.Muon(params, polar_method="nope")
    # CPU parameters: the warm-up reports the missing GPU path and carries on
    assert "warm-up failed" in capsys.readouterr().out


def test_adjust_lr():
    from defmuon_amd.optim import muon
    opt = muon.Muon([("w", torch.nn.Parameter(torch.zeros(8, 2)))], polar_method="ns5")
    assert opt.adjust_lr_for_muon(0.1, True, False, (8, 2), None, None) == pytest.approx(0.2)
    assert opt.adjust_lr_for_muon(0.1, False, False, (8, 2), None, None) == 0.1
    g = torch.eye(3)
    assert opt.adjust_lr_for_muon(1.0, False, True, (3, 3), g, 2 * g) == pytest.approx(6.0)
