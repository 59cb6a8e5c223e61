"""GPU parity of the bf16 MFMA chain (dmh_ns_chain) against the CPU oracle."""

import numpy as np
import pytest
import torch

from conftest import bf16_from_bits
from oracle import polar_oracle as O
from parity import assert_polar_parity, rel

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def N():
    from defmuon_amd import _native
    _native.load()
    assert torch.cuda.is_available()
    return _native


def _bf(t):
    return t.to(torch.bfloat16)


@pytest.mark.parametrize("shape", [(1, 256, 512), (2, 320, 96), (3, 100, 300), (1, 512, 256)])
def test_single_products_match_fp64(N, shape):
    """(a,b,c) = (0,1,0): X' = T (T^T T); (0,0,1): X' = T (T^T T)^2 (tall form).
    Checks the MFMA operand/output layouts of all three GEMM phases."""
    g = torch.Generator().manual_seed(sum(shape))
    X = _bf(torch.randn(*shape, generator=g) / (shape[1] * shape[2]) ** 0.25)
    Xd = X.double()
    G = Xd.mT @ Xd
    for coeffs, want in [((0.0, 1.0, 0.0), Xd @ G), ((0.0, 0.0, 1.0), Xd @ (G @ G))]:
        out = N.ns_chain(X.to(DEV), True, 0, [coeffs])
        err = rel(out, want)
        assert err < 2e-2, (coeffs, err)
    # wide convention: X' = (X X^T) X
    A = Xd @ Xd.mT
    out = N.ns_chain(X.to(DEV), False, 0, [(0.0, 1.0, 0.0)])
    assert rel(out, A @ Xd) < 2e-2


TILE_CHOICES = ["256,256,256", "128,128,128", "128,128,256"]


@pytest.mark.parametrize("tiles", TILE_CHOICES[1:])
@pytest.mark.parametrize("shape", [(1, 256, 512), (2, 320, 96), (1, 512, 256), (2, 768, 384)])
def test_single_products_match_fp64_small_tiles(N, shape, tiles, monkeypatch):
    """The 128 x 128-tile GEMMs (the m x m products of small matrices) read and write
    the same layouts as the 256 x 256 ones: the single products of each phase against
    fp64."""
    monkeypatch.setenv("DMH_CHAIN_TILES", tiles)
    test_single_products_match_fp64(N, shape)


@pytest.mark.parametrize("shape", [(4, 1024, 512), (6, 768, 768), (3, 520, 264)])
def test_tile_sizes_agree(N, shape, monkeypatch):
    """The chain on 256 x 256 and on 128 x 128 output tiles (which only changes each
    output's K-walk order) gives the same polar factor to the oracle's parity bounds,
    and the two agree with each other within bf16 rounding of the chain."""
    from defmuon_amd import synthetic as S
    B, n, m = shape
    A = torch.stack([S.spiked_matrix(n, m, seed=31 * b + n, n_spikes=3, hi=50.0, lo=20.0)
                     for b in range(B)])
    X0 = (A / (A.norm(dim=(-2, -1), keepdim=True) + 1e-7)).bfloat16()
    want = O.horner_iterate(X0, O.ns_schedule(5))
    outs = {}
    for tiles in TILE_CHOICES:
        monkeypatch.setenv("DMH_CHAIN_TILES", tiles)
        outs[tiles] = N.ns_chain(X0.to(DEV), True, 0, O.ns_schedule(5)).cpu()
        for b in range(B):
            assert_polar_parity(outs[tiles][b], want[b], A[b], tag=f"tiles {tiles} {shape} {b}")
    for tiles in TILE_CHOICES[1:]:
        assert rel(outs[tiles], outs[TILE_CHOICES[0]]) < 6e-2, tiles


def test_zero_steps_and_entry(N):
    G = torch.randn(2, 96, 160, generator=torch.Generator().manual_seed(3))
    for mode, scale in ((1, 1.0), (2, 1.01)):
        out = N.ns_chain(G.to(DEV), False, mode, [])
        want = (G / (G.norm(dim=(-2, -1), keepdim=True) * scale + 1e-7)).bfloat16()
        assert rel(out, want) < 1e-3
    out = N.ns_chain(G.to(DEV), True, 1, [])
    want = (G / (G.norm(dim=(-2, -1), keepdim=True) + 1e-7)).bfloat16()
    assert rel(out, want) < 1e-3


def test_zeros_fixed_point(N):
    Z = torch.zeros(3, 256, 128, dtype=torch.bfloat16, device=DEV)
    out = N.ns_chain(Z, True, 0, O.ns_schedule(5))
    assert int(torch.count_nonzero(out.float())) == 0


def test_config1_ns5(N):
    """ns5 on one fp32 768x3072 N(0,1) matrix, seed 0."""
    G = torch.randn(768, 3072, generator=torch.Generator().manual_seed(0))
    want = O.ns5(G, 5)
    got = N.ns_chain(G[None].to(DEV), False, 1, O.ns_schedule(5))[0]
    assert_polar_parity(got, want, G, "config1 ns5")


@pytest.mark.parametrize("shape", [(3072, 768), (300, 700), (700, 300)])
def test_polar_express_2d(N, shape):
    G = torch.randn(*shape, generator=torch.Generator().manual_seed(5))
    tall = G.size(-2) > G.size(-1)
    want = O.polar_express(G, 5)
    got = N.ns_chain(G[None].to(DEV), tall, 2, O.pe_schedule(5))[0]
    assert_polar_parity(got, want, G, f"pe {shape}")


def test_qkv_stack_ns5(N):
    """W_QKV is processed as its three square blocks, batch 3 (muon.py:160-165)."""
    G = torch.randn(3, 512, 512, generator=torch.Generator().manual_seed(6))
    want = O.ns5(G, 5)
    got = N.ns_chain(G.to(DEV), False, 1, O.ns_schedule(5))
    for i in range(3):
        assert_polar_parity(got[i], want[i], G[i], f"qkv block {i}")


@pytest.mark.parametrize("key", ["clip", "clip2"])
@pytest.mark.parametrize("arm", ["ns", "pe"])
def test_horner_against_reference_vectors(N, golden, key, arm):
    """The deflated arms' iteration on the reference's own X0, compared with the
    reference's compiled output (tests/golden) and with the oracle."""
    ref = golden["compiled"]
    X0 = bf16_from_bits(golden["eager"][f"{key}_X0" if arm == "ns" else f"{key}_X0pe"])
    hs = O.ns_schedule(5) if arm == "ns" else O.pe_schedule(5)
    got = N.ns_chain(X0.to(DEV), True, 0, hs).cpu()
    want = O.horner_iterate(X0, hs)
    A = torch.from_numpy(golden["inputs"][f"{key}_A"])
    for b in range(X0.shape[0]):
        assert_polar_parity(got[b], want[b], A[b], f"{key}/{arm}[{b}] vs oracle")
        assert_polar_parity(got[b], bf16_from_bits(ref[f"{key}_iter_{arm}"])[b], A[b],
                            f"{key}/{arm}[{b}] vs reference")


def test_config2_shape_deflated_iteration(N):
    """Tall (3072, 768) deflated iteration from an oracle clip of a spiked matrix."""
    from defmuon_amd import synthetic as S
    A = S.spiked_matrix(3072, 768, seed=0)
    r, _ = O.sketch_dims(768)
    X0, k, _ = O.rmfro_clip(A[None], O.draw_omega(1, 768, r, 1), out_dtype=torch.bfloat16)
    assert int(k[0]) == 8
    want = O.horner_iterate(X0, O.ns_schedule(5))
    got = N.ns_chain(X0.to(DEV), True, 0, O.ns_schedule(5))
    assert_polar_parity(got[0], want[0], A, "config2 deflated ns")


@pytest.mark.parametrize("shape,sched", [((2, 320, 96), "ns"), ((1, 768, 256), "pe"),
                                         ((2, 203, 67), "ns"), ((1, 1030, 130), "pe"),
                                         ((3, 96, 200), "ns")])
def test_horner_fp32_keeps_dtype(N, shape, sched):
    """_horner_iterate keeps X's dtype (deflation_batched.py:196-204): fp32 input runs
    the fp32 chain and comes back fp32, within 1e-5 of the oracle's fp32 chain (the
    reference's convergence study runs this function in fp32).  The shapes cover
    partial 128 x 128 output tiles, sizes that are not multiples of 4 (element-wise
    staging loads instead of 16-byte ones), a partial last 16-deep K slice and a wide
    input (n < m: G = X^T X is m x m of rank n)."""
    from defmuon_amd.optim import deflation_batched as DB
    g = torch.Generator().manual_seed(sum(shape))
    X = torch.randn(*shape, generator=g)
    X = X / X.norm(dim=(-2, -1), keepdim=True)
    hs = O.ns_schedule(5) if sched == "ns" else O.pe_schedule(5)
    want = O.horner_iterate(X, hs)
    got = DB._horner_iterate(X.to(DEV), hs)
    assert got.dtype == torch.float32 and got.shape == X.shape
    assert rel(got, want) <= 1e-5
    got2 = DB._horner_iterate(X[0].to(DEV), hs)
    assert got2.dtype == torch.float32 and got2.shape == X[0].shape
    assert rel(got2, want[0]) <= 1e-5
    with pytest.raises(N.NativeError):
        DB._horner_iterate(X.to(DEV).half(), hs)
