"""Pin the CPU oracle against the reference's own outputs (tests/golden, written by
tests/golden/make_golden.py from the reference's hot-path modules)."""

import numpy as np
import pytest
import torch

from conftest import bf16_from_bits, bits_of
from oracle import polar_oracle as O


def _rel(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("key", ["clip", "clip2"])
def test_clip_matches_reference(golden, key):
    ins, ref = golden["inputs"], golden["eager"]
    A = torch.from_numpy(ins[f"{key}_A"])
    Om = torch.from_numpy(ins[f"{key}_Omega"])
    U, s, V = O.rsvd_b(A, Om)
    np.testing.assert_allclose(s.numpy(), ref[f"{key}_s"], rtol=1e-5)
    proj = (U[..., :2] @ V[..., :2].mT).numpy()
    np.testing.assert_allclose(proj, ref[f"{key}_head_proj"], atol=1e-5)
    X0f, k, d = O.rmfro_clip(A, Om, pad=O.DIVISOR_PAD)
    np.testing.assert_array_equal(k.numpy(), ref[f"{key}_k"])
    np.testing.assert_allclose(d.numpy(), ref[f"{key}_d"], rtol=1e-6)
    np.testing.assert_allclose(X0f.numpy(), ref[f"{key}_X0f32"], atol=1e-6)
    X0, _, _ = O.rmfro_clip(A, Om, pad=O.DIVISOR_PAD, out_dtype=torch.bfloat16)
    np.testing.assert_array_equal(bits_of(X0), ref[f"{key}_X0"])
    X0pe, kpe, _ = O.rmfro_clip(A, Om, pad=O.PE_PAD, out_dtype=torch.bfloat16)
    np.testing.assert_array_equal(bits_of(X0pe), ref[f"{key}_X0pe"])
    np.testing.assert_array_equal(kpe.numpy(), ref[f"{key}_kpe"])


def test_gate_decisions_in_fixtures(golden):
    """The fixtures cover a fired gate (k=2, k=1) and a declined one (k=0)."""
    ref = golden["eager"]
    assert ref["clip_k"].tolist() == [2, 2]
    assert ref["clip2_k"].tolist() == [1, 0]


def test_orth_matches_reference(golden):
    ins, ref = golden["inputs"], golden["eager"]
    A = torch.from_numpy(ins["clip_A"])
    Om = torch.from_numpy(ins["clip_Omega"])
    Q = O.orth_b(A @ Om)
    np.testing.assert_allclose(Q.numpy(), ref["orth_Q"], atol=1e-6)


@pytest.mark.parametrize("key", ["clip", "clip2"])
@pytest.mark.parametrize("arm", ["ns", "pe"])
def test_horner_eager_bit_exact(golden, key, arm):
    ref = golden["eager"]
    X0 = bf16_from_bits(ref[f"{key}_X0" if arm == "ns" else f"{key}_X0pe"])
    hs = O.ns_schedule(5) if arm == "ns" else O.pe_schedule(5)
    out = O.horner_iterate(X0, hs, rounding="eager")
    np.testing.assert_array_equal(bits_of(out), ref[f"{key}_iter_{arm}"])


@pytest.mark.parametrize("name", ["wide_G", "tall_G", "qkv_G"])
def test_plain_arms_eager_bit_exact(golden, name):
    G = torch.from_numpy(golden["inputs"][name])
    ref = golden["eager"]
    np.testing.assert_array_equal(bits_of(O.ns5(G, 5, rounding="eager")), ref[f"{name}_ns5"])
    np.testing.assert_array_equal(bits_of(O.polar_express(G, 5, rounding="eager")),
                                  ref[f"{name}_pe"])


@pytest.mark.parametrize("name", ["wide_G", "tall_G"])
def test_plain_arms_compiled_2d_bit_exact(golden, name):
    """2-D operands: the oracle's model of the inductor graph (addmm with a bf16
    bias, entry norm over the un-rounded input) reproduces torch.compile bit for
    bit."""
    G = torch.from_numpy(golden["inputs"][name])
    ref = golden["compiled"]
    np.testing.assert_array_equal(bits_of(O.ns5(G, 5)), ref[f"{name}_ns5"])
    np.testing.assert_array_equal(bits_of(O.polar_express(G, 5)), ref[f"{name}_pe"])


def test_compiled_3d_within_rounding_spread(golden):
    """3-D operands: inductor's choice of where it stops inlining the running
    axpy depends on its fusion heuristics, so the oracle's compiled mode agrees
    only to bf16-rounding level there.  Bound: the reference's own eager-vs-
    compiled spread on the same inputs (a few 1e-2)."""
    ins, ce, ee = golden["inputs"], golden["compiled"], golden["eager"]
    for key in ("clip", "clip2"):
        for arm in ("ns", "pe"):
            X0 = bf16_from_bits(ee[f"{key}_X0" if arm == "ns" else f"{key}_X0pe"])
            hs = O.ns_schedule(5) if arm == "ns" else O.pe_schedule(5)
            mine = O.horner_iterate(X0, hs)
            r_ref = bf16_from_bits(ce[f"{key}_iter_{arm}"])
            spread = _rel(bf16_from_bits(ee[f"{key}_iter_{arm}"]), r_ref)
            assert _rel(mine, r_ref) <= max(spread, 1e-3) + 1e-3
    G = torch.from_numpy(ins["qkv_G"])
    r_ref = bf16_from_bits(ce["qkv_G_ns5"])
    assert _rel(O.ns5(G), r_ref) <= _rel(bf16_from_bits(ee["qkv_G_ns5"]), r_ref) + 1e-3
