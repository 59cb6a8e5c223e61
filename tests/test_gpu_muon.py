"""GPU parity of the drop-in Muon optimizer (all four arms) against a CPU
restatement of the reference's step built from the oracle (muon.py:251-402)."""

import math

import pytest
import torch

from oracle import polar_oracle as O
from parity import DIRECT_TOL, assert_polar_parity, rel

pytestmark = pytest.mark.gpu

DEV = "cuda"
D = 128          # model width: m = 128 -> r = 8, kw = 4
LAYERS = 2


def _named_params(seed):
    """A GPT-2-shaped parameter set (nn.Linear (out, in) layout, gpt_model.py)."""
    g = torch.Generator().manual_seed(seed)
    shapes = {"wte.weight": (512, D), "wpe.weight": (64, D)}
    for i in range(LAYERS):
        shapes[f"h.{i}.ln_1.weight"] = (D,)
        shapes[f"h.{i}.attn.c_attn.weight"] = (3 * D, D)
        shapes[f"h.{i}.attn.c_proj.weight"] = (D, D)
        shapes[f"h.{i}.mlp.c_fc.weight"] = (4 * D, D)
        shapes[f"h.{i}.mlp.c_proj.weight"] = (D, 4 * D)
    return {k: torch.nn.Parameter((torch.randn(*v, generator=g) * 0.02).to(DEV))
            for k, v in shapes.items()}


def _grads(params, seed):
    """Spiked gradients for the Muon matrices (2 spikes each: k = 2 where the
    gate sees them), Gaussian for the rest.  QKV blocks are spiked per block."""
    from defmuon_amd import synthetic as S
    g = torch.Generator().manual_seed(seed)
    out = {}
    for i, (name, p) in enumerate(params.items()):
        if p.ndim < 2 or "wte" in name or "wpe" in name:
            out[name] = torch.randn(*p.shape, generator=g) * 1e-2
        elif "c_attn" in name:
            out[name] = torch.cat([S.spiked_matrix(D, D, seed=seed * 100 + 10 * i + j,
                                                   n_spikes=2, hi=50.0, lo=20.0)
                                   for j in range(3)])
        else:
            rows, cols = p.shape
            out[name] = S.spiked_matrix(rows, cols, seed=seed * 100 + i, n_spikes=2,
                                        hi=50.0, lo=20.0)
    return {k: v.to(DEV) for k, v in out.items()}


def _expected_updates(params, grads, arm, bd_step, momentum=0.95, steps=5):
    """The reference's Muon update directions u per parameter (muon.py:266-318 for
    the deflated arms, :361-386 for the plain ones), computed with the oracle on
    the CPU.  Sketches are drawn on the GPU with the reference's seed formula."""
    entries = []
    for name, p in params.items():
        if p.ndim < 2 or any(x in name for x in ("wte", "wpe")):
            continue
        gr = grads[name].cpu()
        buf = gr.clone()                       # first step: buf = 0 * m + g
        g = gr + momentum * buf                # nesterov
        entries.append((name, p, g))
    ups = {}
    if arm in ("ns5", "polarexpress"):
        for name, p, g in entries:
            gq = g.reshape(3, D, D) if name.endswith("attn.c_attn.weight") else g
            fn = O.ns5 if arm == "ns5" else O.polar_express
            ups[name] = fn(gq, steps).reshape(p.shape), g
        return ups, None
    groups = {}
    for name, p, g in entries:
        A = g.reshape(3, D, D) if name.endswith("attn.c_attn.weight") else g[None]
        tr = A.shape[-2] < A.shape[-1]
        if tr:
            A = A.mT
        groups.setdefault(tuple(A.shape[-2:]), []).append((name, p, g, A, tr))
    stats = [0, 0, 0]
    pad = O.DIVISOR_PAD if arm == "deflated_ns_cut" else O.PE_PAD
    hs = O.ns_schedule(steps) if arm == "deflated_ns_cut" else O.pe_schedule(steps)
    for gi, (shape, es) in enumerate(sorted(groups.items())):
        A = torch.cat([e[3] for e in es])
        r, _ = O.sketch_dims(shape[1])
        Om = O.draw_omega(A.shape[0], shape[1], r, O.group_seed(bd_step, gi), device=DEV).cpu()
        X0, k, _ = O.rmfro_clip(A, Om, pad=pad, out_dtype=torch.bfloat16)
        stats[0] += A.shape[0]
        stats[1] += int((k > 0).sum())
        stats[2] += int(k.sum())
        Ug = O.horner_iterate(X0, hs)
        off = 0
        for name, p, g, Ae, tr in es:
            u = Ug[off:off + Ae.shape[0]]
            off += Ae.shape[0]
            ups[name] = ((u.mT if tr else u).reshape(p.shape), g)
    return ups, stats


@pytest.fixture(scope="module")
def muon_mod():
    from defmuon_amd.optim import deflation_batched as DB
    from defmuon_amd.optim import deflation_cutoff
    from defmuon_amd.optim import muon
    deflation_cutoff.install()
    return muon, DB


@pytest.mark.parametrize("arm", ["ns5", "polarexpress", "deflated_ns_cut", "deflated_pe_cut"])
def test_muon_step_matches_reference(muon_mod, arm):
    muon, DB = muon_mod
    params = _named_params(1)
    grads = _grads(params, 2)
    before = {k: v.detach().clone() for k, v in params.items()}
    DB._GATE_ACC[0] = None
    opt = muon.Muon(list(params.items()), lr=0.01, weight_decay=0.0, momentum=0.95,
                    nesterov=True, ns_steps=5, polar_method=arm)
    assert opt.batched_deflation == arm.startswith("deflated")
    for k, p in params.items():
        p.grad = grads[k]
    opt.step()
    torch.cuda.synchronize()
    ups, stats = _expected_updates(params, grads, arm, bd_step=1)
    for name, (u_ref, g) in ups.items():
        p = params[name]
        fan_out, fan_in = p.shape
        alr = 0.01 * math.sqrt(fan_out / fan_in)
        u_got = ((before[name] - p.detach()) / alr).cpu()
        src = g.reshape(3, D, D) if name.endswith("attn.c_attn.weight") else g
        got = u_got.reshape(src.shape) if src.ndim == 3 else u_got
        want = u_ref.reshape(src.shape).float() if src.ndim == 3 else u_ref.float()
        if src.ndim == 3:
            for j in range(3):
                assert_polar_parity(got[j], want[j], src[j], f"{arm} {name}[{j}]")
        else:
            assert_polar_parity(got, want, src, f"{arm} {name}")
    if stats is not None:
        st = DB.polar_stats()
        assert [st["total"], st["fired"]] == stats[:2]
        assert st["k_mean"] == stats[2] / max(stats[1], 1)
        assert st["degenerate"] == 0 and st["parachute"] == 0
    # AdamW parameters moved by the AdamW rule
    assert not torch.equal(before["wte.weight"], params["wte.weight"].detach())


def test_timing_and_second_step(muon_mod):
    """Event timing records clip vs iteration; a second step uses bd_step 2."""
    muon, DB = muon_mod
    params = _named_params(3)
    grads = _grads(params, 4)
    opt = muon.Muon(list(params.items()), lr=0.01, polar_method="deflated_ns_cut")
    DB.enable_polar_timing(True)
    try:
        for _ in range(2):
            for k, p in params.items():
                p.grad = grads[k]
            opt.step()
        torch.cuda.synchronize()
        t = DB.timing_stats()
    finally:
        DB.enable_polar_timing(False)
    assert opt._bd_step == 2
    assert t["calls"] == 4 and t["clip_ms"] > 0 and t["iter_ms"] > 0


def test_cutoff_switches_to_plain_arm(muon_mod, monkeypatch):
    muon, DB = muon_mod
    from defmuon_amd.optim import deflation_cutoff as C
    monkeypatch.setattr(C, "CUTOFF_STEPS", 1)
    params = _named_params(5)
    grads = _grads(params, 6)
    opt = muon.Muon(list(params.items()), lr=0.01, polar_method="deflated_pe_cut")
    assert opt.batched_deflation
    for _ in range(2):
        for k, p in params.items():
            p.grad = grads[k]
        opt.step()
    assert not opt.batched_deflation
    from defmuon_amd.optim.polar_express import PolarExpress
    assert opt.polar_factorizer is PolarExpress


@pytest.mark.parametrize("arm", ["deflated_ns_cut", "deflated_pe_cut"])
def test_polar_groups_equal_per_group_calls(arm):
    """polar_groups (one stream per shape group; the chains either on the groups'
    streams, or with chain events in turn on the current stream, or with a chain
    window together after every front-end) gives bit for bit the per-group
    polar_group results: polar factors, gate widths k and divisors d."""
    from defmuon_amd import synthetic as S
    from defmuon_amd.optim import deflation_cutoff as C
    fac = C.ARMS[arm]()
    shapes = [(5, 256, 256), (3, 1024, 256), (2, 520, 264)]
    As = [torch.stack([S.spiked_matrix(n, m, seed=100 * gi + b, n_spikes=3, hi=50.0, lo=20.0)
                       for b in range(B)]).to(DEV) for gi, (B, n, m) in enumerate(shapes)]

    def gens():
        out = []
        for gi, A in enumerate(As):
            g = torch.Generator(device=A.device)
            g.manual_seed((7 * 1009 + gi * 9176867) % (2 ** 62))
            out.append(g)
        return out

    evs = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(2)) for _ in As]
    got_seq = fac.polar_groups(As, gens(), steps=5, chain_events=evs)   # chains in turn
    got = fac.polar_groups(As, gens(), steps=5)                          # chains per stream
    win = tuple(torch.cuda.Event(enable_timing=True) for _ in range(2))
    got_win = fac.polar_groups(As, gens(), steps=5, chain_window=win)    # chains together
    want = [fac.polar_group(A, generator=g, steps=5) for A, g in zip(As, gens())]
    torch.cuda.synchronize()
    assert win[0].elapsed_time(win[1]) > 0.0
    for res in (got_seq, got, got_win):
        for gi, ((u1, k1, d1), (u2, k2, d2)) in enumerate(zip(res, want)):
            assert torch.equal(k1, k2), (gi, k1, k2)
            assert torch.equal(d1, d2), (gi, d1, d2)
            assert torch.equal(u1.view(torch.int16), u2.view(torch.int16)), gi
            assert k1.min().item() == 3, (gi, k1)
    for gi in range(len(As)):
        assert evs[gi][0].elapsed_time(evs[gi][1]) > 0.0


@pytest.mark.parametrize("arm", ["ns5", "polarexpress"])
def test_grouped_plain_step_equals_per_parameter_loop(muon_mod, arm):
    """grouped_plain.install(): one launch per (shape, dtype, orientation) group
    moves every parameter bit for bit like the per-parameter loop
    (muon.py:361-386), over two steps (momentum buffers included)."""
    muon, DB = muon_mod
    from defmuon_amd.optim import grouped_plain
    results = {}
    for grouped in (False, True):
        if grouped:
            grouped_plain.install()
        else:
            grouped_plain.uninstall()
        try:
            params = _named_params(7)
            grads = _grads(params, 8)
            opt = muon.Muon(list(params.items()), lr=0.01, weight_decay=0.1, momentum=0.95,
                            nesterov=True, ns_steps=5, polar_method=arm)
            for _ in range(2):
                for k, p in params.items():
                    p.grad = grads[k]
                opt.step()
            torch.cuda.synchronize()
            results[grouped] = {k: v.detach().clone() for k, v in params.items()}
        finally:
            grouped_plain.uninstall()
    for k in results[False]:
        assert torch.equal(results[False][k], results[True][k]), k


@pytest.mark.parametrize("nesterov", [True, False])
def test_fused_glue_equals_torch_ops(muon_mod, nesterov):
    """dmh_momentum_stack / dmh_apply_update (one launch per shape group) leave
    every parameter and momentum buffer bit for bit where the reference's torch
    ops (muon.py:266-289, 316-332) do, over two deflated steps: W_QKV blocks,
    square, tall and wide (transposed) parameters, weight decay."""
    muon, DB = muon_mod
    results = {}
    for fused in (False, True):
        params = _named_params(9)
        grads = _grads(params, 10)
        opt = muon.Muon(list(params.items()), lr=0.02, weight_decay=0.1, momentum=0.9,
                        nesterov=nesterov, ns_steps=5, polar_method="deflated_ns_cut")
        opt.FUSED_GLUE = fused
        for step in range(2):
            for k, p in params.items():
                p.grad = grads[k] * (1.0 + 0.5 * step)
            opt.step()
        torch.cuda.synchronize()
        bufs = {k: opt.state[p]["momentum_buffer"].clone() for k, p in params.items()
                if "momentum_buffer" in opt.state[p]}
        results[fused] = ({k: v.detach().clone() for k, v in params.items()}, bufs)
    (p0, b0), (p1, b1) = results[False], results[True]
    assert b0.keys() == b1.keys() and len(b0) == 4 * LAYERS
    for k in b0:
        assert torch.equal(b0[k], b1[k]), ("momentum", k)
    for k in p0:
        assert torch.equal(p0[k], p1[k]), ("param", k, (p0[k] - p1[k]).abs().max().item())


@pytest.mark.parametrize("betas", [(0.95, 0.95), (0.3, 0.6)])
def test_fused_adamw_equals_torch_ops(muon_mod, betas):
    """dmh_adamw_step (one launch for every non-Muon parameter) leaves the parameters
    and both moments bit for bit where the reference's per-parameter loop
    (muon.py:408-436) does, over three steps with weight decay.  betas (0.3, 0.6)
    take torch's other lerp branch (weight >= 0.5); sizes that are not multiples of
    4, and one spanning several 4096-element chunks, take the element tail and the
    chunk boundaries."""
    muon, _ = muon_mod
    shapes = {"wte.weight": (1031, 67), "wpe.weight": (33, 7), "h.0.ln_1.weight": (5,),
              "h.0.ln_1.bias": (4099,), "h.0.mlp.c_fc.bias": (3 * 4096 + 5,)}
    results = {}
    for fused in (False, True):
        g = torch.Generator().manual_seed(3)
        params = {k: torch.nn.Parameter((torch.randn(*v, generator=g) * 0.02).to(DEV))
                  for k, v in shapes.items()}
        grads = {k: (torch.randn(*v, generator=g) * 1e-2).to(DEV) for k, v in shapes.items()}
        opt = muon.Muon(list(params.items()), lr=0.02, weight_decay=0.1, momentum=0.9,
                        adamw_betas=betas, adamw_eps=1e-8, ns_steps=5, polar_method="ns5")
        opt.FUSED_GLUE = fused
        for step in range(3):
            for k, p in params.items():
                p.grad = grads[k] * (1.0 + 0.5 * step) - 0.003 * step
            opt.step()
        torch.cuda.synchronize()
        results[fused] = ({k: v.detach().clone() for k, v in params.items()},
                          {k: (opt.state[p]["moment1"].clone(), opt.state[p]["moment2"].clone(),
                               opt.state[p]["step"]) for k, p in params.items()})
    (p0, m0), (p1, m1) = results[False], results[True]
    for k in shapes:
        assert m0[k][2] == m1[k][2] == 3, k
        assert torch.equal(m0[k][0], m1[k][0]), ("moment1", k)
        assert torch.equal(m0[k][1], m1[k][1]), ("moment2", k)
        assert torch.equal(p0[k], p1[k]), ("param", k, (p0[k] - p1[k]).abs().max().item())


def test_fused_adamw_reuses_its_table(muon_mod, monkeypatch):
    """The fused AdamW's device table is built on the first step and reused while the
    tensors stay put: steps 2 and 3 build no AdamwTable (the same object, the same
    device memory), and the parameters and moments stay bit for bit where the
    reference's per-parameter loop (muon.py:408-436) leaves them.  Gradients are
    written in place, so they keep their addresses as a training loop's do."""
    muon, _ = muon_mod
    from defmuon_amd import _native
    built = []
    base_init = _native.AdamwTable.__init__

    def counting_init(self, quads):
        built.append(len(quads))
        base_init(self, quads)

    monkeypatch.setattr(_native.AdamwTable, "__init__", counting_init)
    shapes = {"wte.weight": (257, 31), "wpe.weight": (33, 7), "h.0.ln_1.bias": (4099,)}
    results = {}
    for fused in (False, True):
        g = torch.Generator().manual_seed(5)
        params = {k: torch.nn.Parameter((torch.randn(*v, generator=g) * 0.02).to(DEV))
                  for k, v in shapes.items()}
        grads = {k: (torch.randn(*v, generator=g) * 1e-2).to(DEV) for k, v in shapes.items()}
        for k, p in params.items():
            p.grad = torch.empty_like(p)
        opt = muon.Muon(list(params.items()), lr=0.02, weight_decay=0.1, momentum=0.9,
                        adamw_betas=(0.9, 0.95), adamw_eps=1e-8, ns_steps=5,
                        polar_method="ns5")
        opt.FUSED_GLUE = fused
        built.clear()
        seen = []
        for step in range(3):
            for k, p in params.items():
                p.grad.copy_(grads[k] * (1.0 + 0.5 * step) - 0.003 * step)
            opt.step()
            if fused:
                tabs = list(opt._adamw_tables[id(opt.param_groups[0])].values())
                assert len(tabs) == 1, step
                seen.append((tabs[0], tabs[0].table.data_ptr(), tabs[0].chunks.data_ptr()))
        torch.cuda.synchronize()
        if fused:
            assert built == [len(shapes)], built          # one table, built on step 1
            assert all(s[0] is seen[0][0] and s[1:] == seen[0][1:] for s in seen), seen
        else:
            assert built == []
        results[fused] = ({k: v.detach().clone() for k, v in params.items()},
                          {k: (opt.state[p]["moment1"].clone(), opt.state[p]["moment2"].clone())
                           for k, p in params.items()})
    (p0, m0), (p1, m1) = results[False], results[True]
    for k in shapes:
        assert torch.equal(m0[k][0], m1[k][0]) and torch.equal(m0[k][1], m1[k][1]), k
        assert torch.equal(p0[k], p1[k]), k


def test_fused_adamw_declines_foreign_moments(muon_mod):
    """Moments the fused kernel cannot index flat (here a non-contiguous moment, as a
    fallback loop or load_state_dict could leave) send the group to the torch loop,
    whose result the fused path would otherwise have to match."""
    muon, _ = muon_mod
    g = torch.Generator().manual_seed(6)
    p = torch.nn.Parameter((torch.randn(24, 16, generator=g) * 0.02).to(DEV))
    opt = muon.Muon([("wte.weight", p)], lr=0.02, weight_decay=0.1, momentum=0.9,
                    adamw_betas=(0.9, 0.95), adamw_eps=1e-8, ns_steps=5, polar_method="ns5")
    p.grad = (torch.randn(24, 16, generator=g) * 1e-2).to(DEV)
    st = opt.state[p]
    st["step"] = 1
    st["moment1"] = torch.zeros(16, 24, device=DEV).mT          # non-contiguous view
    st["moment2"] = torch.zeros(24, 16, device=DEV)
    group = opt.param_groups[0]
    assert not opt._adamw_fused(group, [p], 0.02, 0.1, 0.9, 0.95, 1e-8)
    assert st["step"] == 1                                       # nothing was touched
