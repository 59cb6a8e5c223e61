"""GPU parity at the full BASELINE.json shapes of configs 3, 4 and 5.

Config 3: GPT-2 small, one Muon polar step per arm over 48 x (768, 768) and
24 x (3072, 768) tall matrices (12 layers x {3 QKV blocks, attn proj} and
{c_fc, mlp proj^T}), 8 spikes 50x..10x over a Marchenko-Pastur bulk.
Config 4: GPT-2 medium, deflated_pe_cut over 96 x (1024, 1024) and
48 x (4096, 1024), 16 spikes 100x..5x (expected k = 12) with every 4th matrix
left unspiked (expected k = 0).
Config 5: GPT-2 large, deflated_ns_cut over 144 x (1280, 1280) and 72 x (5120, 1280)
(the bench workload), 8 spikes 50x..10x (expected k = 8).

Every gate decision is checked exactly; the polar factors are checked against
the oracle (same sketch, drawn with the reference's seed formula, muon.py:290-291)
on 8 matrices spread over each group, with the tolerances of tests/parity.py.
"""

import pytest
import torch

from oracle import polar_oracle as O
from parity import assert_polar_parity

pytestmark = pytest.mark.gpu

DEV = "cuda"
SMALL = [(48, 768, 768), (24, 3072, 768)]
MEDIUM = [(96, 1024, 1024), (48, 4096, 1024)]
LARGE = [(144, 1280, 1280), (72, 5120, 1280)]


@pytest.fixture(scope="module")
def mods():
    from defmuon_amd import _native
    from defmuon_amd import synthetic as S
    from defmuon_amd.optim import deflation_cutoff as C
    from defmuon_amd.optim import muon as M
    from defmuon_amd.optim import polar_express as PE
    _native.load()
    return S, C, M, PE


def _deflated_group(C, arm, A, gi, bd_step=1):
    """One shape group through the arm's polar_group, with the sketch drawn the
    way the optimizer draws it; returns (U, k, Omega)."""
    fac = C.ARMS[arm]()
    B, n, m = A.shape
    r, _ = O.sketch_dims(m)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(O.group_seed(bd_step, gi))
    Om = torch.randn(B, m, r, device=DEV, dtype=torch.float32, generator=gen)
    U, k, _ = fac.polar_group(A, steps=5, Omega=Om)
    torch.cuda.synchronize()
    return U, k, Om


def _spread(B, count=8):
    """`count` matrix indices spread over a batch of B (first and last included)."""
    if B <= count:
        return list(range(B))
    return sorted({round(i * (B - 1) / (count - 1)) for i in range(count)})


def _check_deflated_sample(arm, A, Om, U, idx):
    pad = O.DIVISOR_PAD if arm == "deflated_ns_cut" else O.PE_PAD
    hs = O.ns_schedule(5) if arm == "deflated_ns_cut" else O.pe_schedule(5)
    for i in idx:
        Ai = A[i:i + 1].cpu()
        X0, _, _ = O.rmfro_clip(Ai, Om[i:i + 1].cpu(), pad=pad, out_dtype=torch.bfloat16)
        Uo = O.horner_iterate(X0, hs)
        assert_polar_parity(U[i].cpu(), Uo[0], Ai[0], tag=f"{arm} {tuple(A.shape)} #{i}")


@pytest.mark.parametrize("arm", ["deflated_ns_cut", "deflated_pe_cut"])
def test_config3_gpt2_small_deflated(mods, arm):
    S, C, _, _ = mods
    for gi, (B, n, m) in enumerate(SMALL):
        A = S.spiked_batch(B, n, m, seed=300 + gi, n_spikes=8, hi=50.0, lo=10.0, device=DEV)
        U, k, Om = _deflated_group(C, arm, A, gi)
        assert k.tolist() == [8] * B, k.tolist()
        assert torch.isfinite(U.float()).all()
        _check_deflated_sample(arm, A, Om, U, range(B))   # every matrix


@pytest.mark.parametrize("arm", ["ns5", "polarexpress"])
def test_config3_gpt2_small_plain(mods, arm):
    """The plain arms run per parameter (muon.py:361-402): one GPT-2-small layer's
    four parameters, in nn.Linear (out, in) layout, W_QKV as its (3, d, d) split."""
    S, _, M, PE = mods
    fn = M.zeropower_via_newtonschulz5 if arm == "ns5" else PE.PolarExpress
    ofn = O.ns5 if arm == "ns5" else O.polar_express
    d = 768
    params = {
        "attn.c_attn": S.spiked_batch(3, d, d, seed=31, device=DEV),
        "attn.c_proj": S.spiked_batch(1, d, d, seed=32, device=DEV)[0],
        "mlp.c_fc": S.spiked_batch(1, 4 * d, d, seed=33, device=DEV)[0],
        "mlp.c_proj": S.spiked_batch(1, d, 4 * d, seed=34, device=DEV)[0],
    }
    for name, G in params.items():
        u = fn(G, 5)
        torch.cuda.synchronize()
        assert u.shape == G.shape and u.dtype == torch.bfloat16
        uo = ofn(G.cpu(), 5)
        Gs = G if G.ndim == 3 else G[None]
        us, uos = (u if u.ndim == 3 else u[None]), (uo if uo.ndim == 3 else uo[None])
        for b in range(Gs.shape[0]):
            assert_polar_parity(us[b].cpu(), uos[b], Gs[b].cpu(), tag=f"{arm} {name}[{b}]")


def test_config4_gpt2_medium_pe(mods):
    S, C, _, _ = mods
    for gi, (B, n, m) in enumerate(MEDIUM):
        unspiked = tuple(range(0, B, 4))
        A = S.spiked_batch(B, n, m, seed=400 + gi, n_spikes=16, hi=100.0, lo=5.0,
                           device=DEV, unspiked=unspiked)
        U, k, Om = _deflated_group(C, "deflated_pe_cut", A, gi)
        want = [0 if i in unspiked else S.expected_k(16, 100.0, 5.0) for i in range(B)]
        assert want.count(12) == B - len(unspiked)
        assert k.tolist() == want, k.tolist()
        assert torch.isfinite(U.float()).all()
        _check_deflated_sample("deflated_pe_cut", A, Om, U, _spread(B, 24))


def test_config5_gpt2_large_deflated(mods):
    """The bench workload itself: every gate fires with k = 8, and 24 matrices spread
    over each group (the first and last included; 48 of the 216) match the oracle on
    their own sketches."""
    S, C, _, _ = mods
    for gi, (B, n, m) in enumerate(LARGE):
        A = S.spiked_batch(B, n, m, seed=500 + gi, n_spikes=8, hi=50.0, lo=10.0, device=DEV)
        U, k, Om = _deflated_group(C, "deflated_ns_cut", A, gi)
        assert S.expected_k(8, 50.0, 10.0) == 8
        assert k.tolist() == [8] * B, k.tolist()
        assert torch.isfinite(U.float()).all()
        _check_deflated_sample("deflated_ns_cut", A, Om, U, _spread(B, 24))
        del A, U, Om
        torch.cuda.empty_cache()


@pytest.mark.parametrize("arm", ["ns5", "polarexpress"])
def test_config3_grouped_plain_matches_oracle(mods, arm):
    """The grouped plain-arm launch (grouped_plain.install(), one launch per (shape,
    dtype, orientation) group) over GPT-2 small's full Muon parameter set -- 12
    layers x {attn.c_attn as its (3, 768, 768) split, attn.c_proj, mlp.c_fc,
    mlp.c_proj}, 72 matrices -- against the oracle's ns5 / PolarExpress on every
    matrix (muon.py:361-386: the factorizer of each parameter's Nesterov momentum)."""
    S, _, M, PE = mods
    from defmuon_amd import _native
    from defmuon_amd.optim import grouped_plain
    d = 768
    params, grads = {}, {}
    for layer in range(12):
        for name, shape in (("attn.c_attn", (3 * d, d)), ("attn.c_proj", (d, d)),
                            ("mlp.c_fc", (4 * d, d)), ("mlp.c_proj", (d, 4 * d))):
            key = f"h.{layer}.{name}.weight"
            params[key] = torch.nn.Parameter(torch.zeros(shape, device=DEV))
            seed = 3000 + 10 * layer + len(grads)
            if name == "attn.c_attn":
                g = torch.cat([S.spiked_matrix(d, d, seed=seed + j) for j in range(3)])
            else:
                g = S.spiked_matrix(*shape, seed=seed)
            grads[key] = g.to(DEV)
    launches = []
    real = _native.ns_chain

    def spy(X, tall, mode, sched, out=None):
        res = real(X, tall, mode, sched, out)
        launches.append((X.detach().clone(), tall, res.detach().clone()))
        return res

    grouped_plain.install()
    try:
        opt = M.Muon(list(params.items()), lr=0.01, weight_decay=0.0, momentum=0.95,
                     nesterov=True, ns_steps=5, polar_method=arm)   # (its warm-up unspied)
        _native.ns_chain = spy
        for k, p in params.items():
            p.grad = grads[k]
        opt.step()
        torch.cuda.synchronize()
    finally:
        _native.ns_chain = real
        grouped_plain.uninstall()
    # one launch per (shape, orientation) group: (768, 768) x 48, c_fc x 12, c_proj x 12
    assert sorted(X.shape[0] for X, _, _ in launches) == [12, 12, 48]
    ofn = O.ns5 if arm == "ns5" else O.polar_express
    checked = 0
    for X, tall, U in launches:
        for i in range(X.shape[0]):
            G = X[i].cpu()
            assert_polar_parity(U[i].cpu(), ofn(G, 5), G, tag=f"grouped {arm} {tuple(G.shape)} #{i}")
            checked += 1
    assert checked == 72
