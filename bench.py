#!/usr/bin/env python
"""Polar steps per second of deflated Muon's polar-factor path on one MI355X.

A polar step is what Muon._muon_step_batched does between stacking the momenta
and applying the update (muon.py:288-315): for every tall-shape group, seed the
sketch generator from (step, group), run BATCHED_CLIP (Gaussian sketch, rSVD,
gate, deflate/restore to bf16), tick the gate counters, and run the arm's 5-step
bf16 iteration over the whole group.  Inputs are synthetic spiked-spectrum fp32
momenta already resident in HBM (8 spikes 50x..10x over a Marchenko-Pastur
bulk, Haar singular vectors).

    python bench.py [--steps K] [--warmup W] [--workload gpt2-large] [--arm deflated_ns_cut]

prints one JSON line.  `roofline` covers the NS chain (the dominant work): its
canonical dense bf16 FLOPs per polar step over the time of its launches, taken
with HIP events on the launch stream inside the timed region.  `cpu_baseline`
times the CPU restatement of the reference arithmetic (oracle/) on a bounded
sample of the same workload and extrapolates to the full step.
"""

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "spectral-deflation_amd"))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0

# tall-shape groups (batch, n, m) of one polar step, after the W_QKV split and the
# wide -> tall transpose (muon.py:275-285); GPT-2 Linear weights are (out, in)
WORKLOADS = {
    # config 2: one spiked 768 x 3072 momentum, transposed to tall by Muon
    "config2": [(1, 3072, 768)],
    "gpt2-small": [(48, 768, 768), (24, 3072, 768)],
    "gpt2-medium": [(96, 1024, 1024), (48, 4096, 1024)],
    "gpt2-large": [(144, 1280, 1280), (72, 5120, 1280)],
}


# plain arms: the Muon parameters' matrices after the W_QKV split, nn.Linear
# (out, in) layout, grouped as the grouped plain step launches them:
# (count, rows, cols, tall) -- tall: the factorizer runs on the transpose
PLAIN_GROUPS = {
    # config 1: ns5 on one 768 x 3072 matrix with N(0, 1) entries (seed 0)
    "config1": [(1, 768, 3072, False)],
    "gpt2-small": [(48, 768, 768, False), (12, 3072, 768, True), (12, 768, 3072, False)],
    "gpt2-medium": [(96, 1024, 1024, False), (24, 4096, 1024, True), (24, 1024, 4096, False)],
    "gpt2-large": [(144, 1280, 1280, False), (36, 5120, 1280, True), (36, 1280, 5120, False)],
}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


CHAIN_SOURCES = ("common.h", "ns_chain.h", "ns_chain.hip")


def chain_sources_sha256():
    """sha256 over the NS chain's sources (csrc/common.h, ns_chain.h, ns_chain.hip, in
    that order): stamps counter measurements of the chain's kernels, so a measurement
    is used only with the kernels it was taken on."""
    import hashlib
    d = os.path.join(ROOT, "spectral-deflation_amd", "csrc")
    h = hashlib.sha256()
    for name in CHAIN_SOURCES:
        h.update(name.encode())
        with open(os.path.join(d, name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def ns_flops(groups, steps=5):
    """Canonical dense NS FLOPs: 4 m^2 n + 2 m^3 per matrix and iteration."""
    return sum(B * steps * (4 * m * m * n + 2 * m ** 3) for B, n, m in groups)


def make_inputs(groups, device, seed=1234, kind="spiked"):
    """Synthetic momenta per group.  "spiked": generated on the GPU; "spiked-cpu":
    the same construction on the host (its QRs run in the CPU solver), then copied
    to the GPU -- for hardware-counter runs, which should not run the GPU solver
    library; "gaussian": i.i.d. N(0, 1/n) entries (the gate declines every matrix)."""
    import torch
    from defmuon_amd import synthetic as S
    out = []
    for gi, (B, n, m) in enumerate(groups):
        if kind == "spiked-cpu":
            out.append(S.spiked_batch(B, n, m, seed=seed + gi, n_spikes=8, hi=50.0, lo=10.0,
                                      device="cpu").to(device))
        elif kind == "gaussian":
            g = torch.Generator(device=device)
            g.manual_seed(seed + gi)
            out.append(torch.randn(B, n, m, device=device, generator=g) / math.sqrt(n))
        else:
            out.append(S.spiked_batch(B, n, m, seed=seed + gi, n_spikes=8, hi=50.0, lo=10.0,
                                      device=device))
    return out


def polar_step(fac, stacks, bd_step, ns_steps, events=None, ns_timing="sequential"):
    """One polar step over all groups, as the optimizer runs it
    (_DeflatedPolarBase.polar_groups: the groups' clips, then their iterations);
    returns per-group (U, k).  With `events`, appends a list of (start, end) HIP
    event pairs recorded on the launch stream: ns_timing "sequential", one pair
    around each group's NS chain, the chains one after the other once every
    front-end has finished; "concurrent", one pair around the chain phase, every
    group's chain on its own stream once every front-end has finished."""
    import torch
    from defmuon_amd.optim import deflation_batched as DB
    gens = []
    for gi, A in enumerate(stacks):
        gen = torch.Generator(device=A.device)
        gen.manual_seed((bd_step * 1009 + gi * 9176867) % (2 ** 62))
        gens.append(gen)
    evs = window = None
    if events is not None and ns_timing == "concurrent" and len(stacks) > 1:
        window = tuple(torch.cuda.Event(enable_timing=True) for _ in range(2))
        events.append([window])
    elif events is not None:
        evs = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(2)) for _ in stacks]
        events.append(evs)
    res = fac.polar_groups(stacks, gens, steps=ns_steps, chain_events=evs, chain_window=window)
    outs = []
    for A, (U, kvec, _) in zip(stacks, res):
        if DB._GATE_ACC[0] is None:
            DB._GATE_ACC[0] = torch.zeros(3, dtype=torch.int64, device=A.device)
        DB._GATE_ACC[0][0] += A.shape[0]   # host scalar: no host->device copy, no wait
        DB._GATE_ACC[0][1:] += torch.stack([(kvec > 0).sum(), kvec.sum().to(torch.int64)])
        outs.append((U, kvec))
    return outs


def make_plain_inputs(pgroups, device, seed=4321, gaussian=False):
    """Spiked-spectrum momenta per plain group, in the parameters' own layout
    (gaussian: N(0, 1) entries from torch.Generator().manual_seed(0), config 1)."""
    import torch
    from defmuon_amd import synthetic as S
    out = []
    if gaussian:
        g = torch.Generator().manual_seed(0)
        return [torch.randn(B, rows, cols, generator=g).to(device)
                for B, rows, cols, _ in pgroups]
    for gi, (B, rows, cols, tall) in enumerate(pgroups):
        n, m = max(rows, cols), min(rows, cols)
        X = S.spiked_batch(B, n, m, seed=seed + gi, n_spikes=8, hi=50.0, lo=10.0, device=device)
        out.append(X if rows >= cols else X.mT.contiguous())
    return out


def plain_step(arm, stacks, pgroups, ns_steps, events=None):
    """One plain-arm polar step (muon.py:361-386 factorizer calls over every Muon
    parameter) with one launch per group, the groups on side streams of their own, as
    Muon._muon_step_plain_grouped runs it (plain_group_chains)."""
    import torch
    from defmuon_amd import _native
    from defmuon_amd.optim.muon import NS_ABC
    from defmuon_amd.optim.polar_express import pe_schedule
    from defmuon_amd.optim.muon import plain_group_chains
    mode, sched = (1, [NS_ABC] * ns_steps) if arm == "ns5" else (2, pe_schedule(ns_steps))
    ev = tuple(torch.cuda.Event(enable_timing=True) for _ in range(2))
    ev[0].record()
    outs = plain_group_chains(stacks, [tall for _, _, _, tall in pgroups], mode, sched)
    ev[1].record()
    if events is not None:
        events.append([ev])
    return outs


def _gpt2(vocab, ctx, d, layers, heads):
    """GPT-2 with nn.Linear weights named as the reference's model names them
    (attn.c_attn, attn.c_proj, mlp.c_fc, mlp.c_proj; wte, wpe, tied lm_head), so
    Muon routes and splits them the same way; bf16 autocast in the forward."""
    import torch
    import torch.nn as nn
    import torch.nn.functional as F

    class Attn(nn.Module):
        def __init__(self):
            super().__init__()
            self.c_attn, self.c_proj = nn.Linear(d, 3 * d), nn.Linear(d, d)

        def forward(self, x):
            B, T, _ = x.shape
            q, k, v = (t.view(B, T, heads, d // heads).transpose(1, 2)
                       for t in self.c_attn(x).split(d, dim=2))
            y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
            return self.c_proj(y.transpose(1, 2).reshape(B, T, d))

    class Mlp(nn.Module):
        def __init__(self):
            super().__init__()
            self.c_fc, self.c_proj = nn.Linear(d, 4 * d), nn.Linear(4 * d, d)

        def forward(self, x):
            return self.c_proj(F.gelu(self.c_fc(x), approximate="tanh"))

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.ln_1, self.attn, self.ln_2, self.mlp = nn.LayerNorm(d), Attn(), nn.LayerNorm(d), Mlp()

        def forward(self, x):
            x = x + self.attn(self.ln_1(x))
            return x + self.mlp(self.ln_2(x))

    class GPT(nn.Module):
        def __init__(self):
            super().__init__()
            self.wte, self.wpe = nn.Embedding(vocab, d), nn.Embedding(ctx, d)
            self.h = nn.ModuleList(Block() for _ in range(layers))
            self.ln_f = nn.LayerNorm(d)
            self.lm_head = nn.Linear(d, vocab, bias=False)
            self.lm_head.weight = self.wte.weight

        def forward(self, idx, targets):
            x = self.wte(idx) + self.wpe(torch.arange(idx.shape[1], device=idx.device))
            for blk in self.h:
                x = blk(x)
            logits = self.lm_head(self.ln_f(x))
            return F.cross_entropy(logits.float().view(-1, vocab), targets.reshape(-1))

    return GPT()


def train_step_report(args, dev):
    """Config 5: a GPT-2-large training step (batch 8 x 1024 random tokens, random
    init), Muon deflated_ns_cut on the 144 hidden matrices (216 after the W_QKV
    split), AdamW on embeddings, norms and biases.  Reports the step time, its
    forward+backward and optimizer parts, the polar path inside the optimizer step
    (events around the groups' clips + iterations) and its share, and the optimizer
    step with the reference's torch glue instead of the fused glue."""
    import torch
    from defmuon_amd.optim import deflation_cutoff
    from defmuon_amd.optim.muon import Muon
    deflation_cutoff.install()
    torch.manual_seed(0)
    model = _gpt2(50257, 1024, 1280, 36, 20).to(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    tok = torch.randint(0, 50257, (8, 1025), device=dev, generator=g)
    x, y = tok[:, :-1], tok[:, 1:]
    opt = Muon(model.named_parameters(), lr=0.01, weight_decay=0.0, momentum=0.95, nesterov=True,
               ns_steps=5, polar_method="deflated_ns_cut")
    fac = opt.polar_factorizer
    orig = fac.polar_groups
    marks = []

    def timed_groups(As, gens, steps=5, chain_events=None):
        e = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        e[0].record()
        out = orig(As, gens, steps=steps, chain_events=chain_events)
        e[1].record()
        marks.append(e)
        return out
    fac.polar_groups = timed_groups

    def one(evs):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = model(x, y)
        loss.backward()
        e[1].record()
        opt.step()
        opt.zero_grad(set_to_none=True)
        e[2].record()
        evs.append(e)

    res = {}
    for fused in (True, False):
        opt.FUSED_GLUE = fused
        for _ in range(args.warmup):
            one([])
        torch.cuda.synchronize()
        marks.clear()
        evs = []
        for _ in range(args.steps):
            one(evs)
        torch.cuda.synchronize()
        step = sum(e[0].elapsed_time(e[2]) for e in evs) / args.steps
        fb = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
        optm = sum(e[1].elapsed_time(e[2]) for e in evs) / args.steps
        polar = sum(m[0].elapsed_time(m[1]) for m in marks) / args.steps
        res[fused] = dict(step_ms=step, fwd_bwd_ms=fb, optimizer_ms=optm, polar_ms=polar)
        log(f"bench train: fused glue {fused}: {res[fused]}")
    f = res[True]
    return {"metric": "GPT-2-large training step (config 5): polar-factor share of step time",
            "value": f["polar_ms"] / f["step_ms"], "unit": "fraction of step time",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": f["step_ms"], "higher_is_better": False,
            "tokens_per_s": 8 * 1024 / (f["step_ms"] * 1e-3),
            "fwd_bwd_ms": f["fwd_bwd_ms"], "optimizer_ms": f["optimizer_ms"],
            "polar_ms": f["polar_ms"], "optimizer_ms_torch_glue": res[False]["optimizer_ms"],
            "dtype": "bf16 autocast (model), bf16/fp32/fp64 (polar path)",
            "data": "random init, random token ids uniform over 50257, batch 8 x 1024",
            "config": {"workload": "gpt2-large train step: d=1280, 36 layers, 20 heads, MLP "
                                   "5120; Muon deflated_ns_cut on 144 hidden matrices, AdamW "
                                   "on the rest"}}


def cpu_baseline(groups, arm, min_s=12.0, max_reps=20):
    """Time the oracle (CPU restatement of the reference arithmetic) on single
    matrices of each group -- one warm-up, then repeats until about min_s seconds
    of CPU work -- and extrapolate by batch size to the full step."""
    import torch
    from defmuon_amd import synthetic as S
    from oracle import polar_oracle as O
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    hs = O.ns_schedule(5) if arm in ("deflated_ns_cut", "ns5") else O.pe_schedule(5)
    pad = O.DIVISOR_PAD if arm == "deflated_ns_cut" else O.PE_PAD
    plain = arm in ("ns5", "polarexpress")
    per_matrix, reps = [], []
    for gi, (B, n, m) in enumerate(groups):
        A = S.spiked_batch(1, n, m, seed=99 + gi)
        r, _ = O.sketch_dims(m)
        Om = O.draw_omega(1, m, r, 7)
        times, spent = [], 0.0
        for rep in range(max_reps + 1):
            t0 = time.perf_counter()
            if plain:
                (O.ns5 if arm == "ns5" else O.polar_express)(A[0], 5)
            else:
                X0, _, _ = O.rmfro_clip(A, Om, pad=pad, out_dtype=torch.bfloat16)
                O.horner_iterate(X0, hs)
            dt = time.perf_counter() - t0
            if rep > 0:
                times.append(dt)
                spent += dt
            if rep >= 3 and spent > min_s / len(groups):
                break
        times.sort()
        per_matrix.append(times[len(times) // 2])
        reps.append(len(times))
        log(f"cpu_baseline: group {gi} ({n}x{m}) median {per_matrix[-1]:.3f} s per matrix "
            f"over {len(times)} runs")
    t_step = sum(B * t for (B, _, _), t in zip(groups, per_matrix))
    return {"value": 1.0 / t_step, "unit": "polar_steps/s", "cores": cores, "kind": "port",
            "sample": ("oracle/ (torch CPU restatement of the reference arithmetic, "
                       f"arm {arm}, torch.set_num_threads({cores})): single matrices of "
                       f"each shape group, median of {reps} runs after a warm-up, "
                       f"extrapolated by batch size to the full step ({t_step:.2f} s per "
                       "step)"),
            "cpu": _cpu_model()}


# Algorithmic bytes per element of a group's (n x m) matrices for the memory-bound
# kernels, per launch: fp32 reads 4 B, bf16 reads/writes 2 B, fp32 writes 4 B.
KERNEL_BYTES = {
    "sk_rows": 4,            # A read (A Omega, A Z)
    "sk_cols": 4,            # A read (A^T Q)
    "deflate_restore": 6,    # A read fp32, the chain's packed bf16 T written
    "entry_norm_partials": 4,  # X read fp32
    "entry_pack": 6,         # X read fp32, packed bf16 T written
    "momentum_stack": 16,    # grad and buffer read, buffer and fp32 stack written
    "apply_update": 10,      # parameter read and written fp32, bf16 update read
}
# (read, written) bytes per element of the same kernels
KERNEL_RW = {"sk_rows": (4, 0), "sk_cols": (4, 0), "deflate_restore": (4, 2),
             "entry_norm_partials": (4, 0), "entry_pack": (4, 2), "momentum_stack": (8, 8),
             "apply_update": (6, 4)}


def kernels_report(args, dev):
    """--mode kernels: the memory-bound kernels of the path, each group's launches
    one after the other on one stream (nothing overlapping), `args.steps` rounds,
    for rocprofv3 --kernel-trace --stats; then --summarize-trace turns the stats
    into GB/s.  Per round and shape group: the deflated front-end
    (dmh_deflated_polar_front: sk_rows x2, sk_cols x2, deflate_restore), the plain
    arms' fp32 entry (dmh_ns_chain with zero steps: entry_norm_partials, entry_pack,
    copy_out) and the optimizer glue (dmh_momentum_stack, dmh_apply_update)."""
    import torch
    from defmuon_amd import _native
    from defmuon_amd.optim import deflation_batched as DB
    groups = WORKLOADS[args.workload]
    stacks = make_inputs(groups, dev, kind=args.inputs)
    glue = []
    for (B, n, m), A in zip(groups, stacks):
        g = torch.randn(B, n, m, device=dev) * 1e-2
        buf = torch.zeros(B, n, m, device=dev)
        par = torch.randn(B, n, m, device=dev) * 2e-2
        stack = torch.empty(B, n, m, device=dev)
        u = torch.empty(B, n, m, dtype=torch.bfloat16, device=dev)
        ps = []
        for b in range(B):
            d = _native.GlueParam()
            d.grad, d.momentum, d.param = g[b].data_ptr(), buf[b].data_ptr(), par[b].data_ptr()
            d.rows, d.cols, d.blocks, d.transpose = n, m, 1, 0
            d.offset, d.alpha, d.decay = b * n * m, -1e-3, 1.0
            ps.append(d)
        glue.append((ps, stack, u, (g, buf, par)))
    torch.cuda.synchronize()
    for rnd in range(args.warmup + args.steps):
        for gi, ((B, n, m), A) in enumerate(zip(groups, stacks)):
            r, kw = DB.sketch_dims(m)
            gen = torch.Generator(device=dev)
            gen.manual_seed(rnd * 1009 + gi)
            Om = torch.randn(B, m, r, device=dev, generator=gen)
            _native.deflated_polar_front(A, Om, kw, DB.GATE_RATIO, DB.DEFLATE_THRESH,
                                         DB.DIVISOR_PAD, DB.RSVD_NITER, DB.CHOLQR_PASSES)
            _native.ns_chain(A, True, 1, [])
            ps, stack, u, _ = glue[gi]
            _native.momentum_stack(ps, 0.95, True, stack)
            _native.apply_update(ps, u)
        torch.cuda.synchronize()
    log(f"bench kernels: {args.warmup} + {args.steps} rounds over {groups}")
    return {"mode": "kernels", "workload": args.workload, "groups": groups,
            "rounds": args.warmup + args.steps}


def horner_f32_report(args, dev):
    """--mode horner-f32: the fp32 iteration (`_horner_iterate` on fp32 input, the
    path the reference's convergence study runs; dmh_horner_f32 on the fp32 matrix
    cores) over the workload's shape groups, 5 NS steps per matrix, the groups one
    after the other on the launch stream; `args.steps` timed rounds after
    `args.warmup`.  FLOP: the canonical 4m^2n + 2m^3 per matrix and step."""
    import torch
    from defmuon_amd.optim import deflation_batched as DB
    groups = WORKLOADS[args.workload]
    hs = [DB.DeflatedNSPolar.NS_ABC] * 5
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    xs = []
    for B, n, m in groups:
        X = torch.randn(B, n, m, device=dev, generator=gen)
        xs.append(X / X.norm(dim=(-2, -1), keepdim=True))
    for _ in range(args.warmup):
        for X in xs:
            DB._horner_iterate(X, hs)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        for X in xs:
            DB._horner_iterate(X, hs)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    flop = sum(B * (4 * m * m * n + 2 * m ** 3) * len(hs) for B, n, m in groups)
    tflops = flop / ms / 1e9
    log(f"bench horner-f32: {args.warmup} + {args.steps} rounds over {groups}")
    return {"mode": "horner-f32", "workload": args.workload, "groups": groups,
            "ms_per_step": round(ms, 3), "flop_per_step": flop, "tflops": round(tflops, 1),
            "frac_fp32_mfma_peak": round(tflops / 157.3, 3), "steps": args.steps,
            "warmup": args.warmup}


def summarize_trace(path, workload, rounds):
    """GB/s of the memory-bound kernels from a rocprofv3 --stats kernel_stats.csv of
    `bench.py --mode kernels` (algorithmic bytes KERNEL_BYTES per element, summed
    over the groups of every round, over the kernels' total duration)."""
    import csv
    groups = WORKLOADS[workload]
    elems = sum(B * n * m for B, n, m in groups)
    per_round_launches = {"sk_rows": 2, "sk_cols": 2}
    rows = list(csv.DictReader(open(path)))
    print("| kernel | launches | avg us | algorithmic GB per launch | achieved GB/s | "
          "fraction of 8 TB/s |")
    print("|---|---|---|---|---|---|")
    for name, bpe in KERNEL_BYTES.items():
        hit = [r for r in rows if name in r["Name"]]
        if not hit:
            continue
        calls = sum(int(r["Calls"]) for r in hit)
        tot_ns = sum(float(r["TotalDurationNs"]) for r in hit)
        nbytes = rounds * per_round_launches.get(name, 1) * bpe * elems
        gbs = nbytes / tot_ns
        print(f"| `{name}` | {calls} | {tot_ns / calls / 1e3:.1f} | {nbytes / calls / 1e9:.3f} | "
              f"{gbs:.0f} | {gbs / PEAK_HBM_GBS:.2f} |")


def summarize_kernel_traffic(paths, workload, rounds, copy_mib):
    """HBM bytes the memory-bound kernels moved, from two rocprofv3 --pmc runs of
    `bench.py --mode kernels --copy-calibration MIB` (FETCH_SIZE, then WRITE_SIZE, KiB per
    dispatch, each scaled by what it reads for torch's copy kernel of known size),
    against the algorithmic bytes (KERNEL_RW per element) of the same launches."""
    import collections
    import csv
    groups = WORKLOADS[workload]
    elems = sum(B * n * m for B, n, m in groups)
    per_round_launches = {"sk_rows": 2, "sk_cols": 2}
    sums = collections.defaultdict(lambda: collections.defaultdict(float))
    for path in paths:
        for r in csv.DictReader(open(path)):
            name = r["Kernel_Name"]
            if "copy" in name.lower() and "dmh" not in name:
                key = "copy"
            else:
                key = next((k for k in KERNEL_RW if k in name), None)
            if key:
                sums[key][r["Counter_Name"]] += float(r["Counter_Value"]) * 1024
    scale = {}
    cal = sums.get("copy", {})
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        if copy_mib and cal.get(c):
            scale[c] = 3 * copy_mib * 2 ** 20 / cal[c]
    print("| kernel | algorithmic GB read / written per round | measured GB fetched / written "
          "per round | fetched / algorithmic read | written / algorithmic write |")
    print("|---|---|---|---|---|")
    for name, (rd, wr) in KERNEL_RW.items():
        if name not in sums:
            continue
        n = rounds * per_round_launches.get(name, 1)
        a_rd, a_wr = rd * elems * n / rounds / 1e9, wr * elems * n / rounds / 1e9
        f = sums[name].get("FETCH_SIZE", 0.0) * scale.get("FETCH_SIZE", 1.0) / rounds / 1e9
        w = sums[name].get("WRITE_SIZE", 0.0) * scale.get("WRITE_SIZE", 1.0) / rounds / 1e9
        fr = f"{f / a_rd:.2f}" if a_rd else "-"
        wrr = f"{w / a_wr:.2f}" if a_wr else "-"
        print(f"| `{name}` | {a_rd:.3f} / {a_wr:.3f} | {f:.3f} / {w:.3f} | {fr} | {wrr} |")
    if scale:
        print()
        print("scale factors from the copy calibration: " +
              ", ".join(f"{c} x{v:.3f}" for c, v in scale.items()))


GEMM_LABELS = {}
for _tl in (256, 128):
    GEMM_LABELS.update({
        f"dmh::gemm_nt_bf16<0, 0, {_tl}>": f"K3 T' = T B', {_tl}x{_tl} tiles",
        f"dmh::gemm_nt_bf16<0, 1, {_tl}>": f"K1 A = T^T T, K-major, {_tl}x{_tl} tiles",
        f"dmh::gemm_nt_bf16<1, 0, {_tl}>": f"K2 B' = bA + cA^2 + aI, {_tl}x{_tl} tiles",
    })


def _dmh_kernel(name):
    """Short name of one of the library's kernels (None for any other kernel)."""
    import re
    name = name.replace("void ", "")
    m = re.match(r"(dmh::[A-Za-z_0-9]+(<[^>]*>)?)", name)
    if m:
        return m.group(1)
    m = re.match(r"_ZN3dmh(\d+)", name)
    if m:
        n = int(m.group(1))
        return "dmh::" + name[len("_ZN3dmh") + len(m.group(1)):][:n]
    return None


def summarize_step_trace(path, steps, warmup):
    """Per-polar-step table of the library's kernels from a rocprofv3 --kernel-trace
    kernel_trace.csv (plain or .gz) of `bench.py --steps S --warmup W`: the chain's
    GEMMs over the S steps of the sequential pass (launch stream, Stream_Id 0), every
    other kernel over all W + 3S steps (warm-up, timed steps, the two NS-chain
    passes)."""
    import collections
    import csv
    import gzip
    opener = gzip.open if path.endswith(".gz") else open
    with opener(path, "rt") as f:
        rows = list(csv.DictReader(f))
    all_steps = warmup + 3 * steps
    agg = collections.OrderedDict()
    for r in rows:
        k = _dmh_kernel(r["Kernel_Name"])
        if not k:
            continue
        gemm = "gemm_nt" in k
        if gemm and r["Stream_Id"] != "0":
            continue
        a = agg.setdefault(k, [0, 0, gemm])
        a[0] += 1
        a[1] += int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    per_step = {k: t / (steps if g else all_steps) for k, (c, t, g) in agg.items()}
    print("| kernel | calls | total ms | avg us | ms per polar step |")
    print("|---|---|---|---|---|")
    ns_t = ns_c = 0
    for k in sorted(agg, key=lambda k: -per_step[k]):
        c, t, gemm = agg[k]
        label = f"`{k}`" + (f" ({GEMM_LABELS[k]})" if k in GEMM_LABELS else "")
        print(f"| {label} | {c} | {t / 1e6:.2f} | {t / 1e3 / c:.1f} | {per_step[k] / 1e6:.2f} |")
        if gemm:
            ns_t += t
            ns_c += c
    print(f"| **NS chain (gemm_nt_bf16)** | {ns_c} | {ns_t / 1e6:.2f} | | "
          f"**{ns_t / 1e6 / steps:.2f}** |")
    print(f"| **all library kernels** | | | | {sum(per_step.values()) / 1e6:.2f} |")


def summarize_pmc(paths, steps_in_trace, copy_mib=0, traffic_json=None):
    """Per-kernel sums of rocprofv3 --pmc counter_collection.csv files taken over
    `bench.py --steps S --warmup W` (steps_in_trace = W + S + the 2 S steps of the two
    NS-chain passes), per polar step.  FETCH_SIZE / WRITE_SIZE (KiB per dispatch) are
    scaled by what they read for torch's copy kernel over --copy-calibration MiB
    (3 copies: FETCH should see the bytes read, WRITE the bytes written); with
    traffic_json the NS chain's traffic per step is written there, stamped with
    the NS chain sources' sha256.  MFMA utilisation = SQ_VALU_MFMA_BUSY_CYCLES /
    (4 SIMDs x SQ_BUSY_CU_CYCLES) per kernel."""
    import collections
    import csv
    sums = collections.OrderedDict()
    disp = collections.defaultdict(set)     # per kernel: (file, dispatch) pairs
    for path in paths:
        for r in csv.DictReader(open(path)):
            name = r["Kernel_Name"]
            short = ("copy (calibration)" if "copy" in name.lower() and "dmh" not in name else
                     _dmh_kernel(name) or name.split("(")[0].replace("void ", "").strip())
            key = short
            sums.setdefault(key, collections.defaultdict(float))
            sums[key][r["Counter_Name"]] += float(r["Counter_Value"])
            disp[key].add((path, r["Dispatch_Id"]))
    scale = {}
    if copy_mib and "copy (calibration)" in sums:
        cal = sums["copy (calibration)"]
        nbytes = 3 * copy_mib * 2 ** 20
        if cal.get("FETCH_SIZE"):
            scale["FETCH_SIZE"] = nbytes / (cal["FETCH_SIZE"] * 1024)
        if cal.get("WRITE_SIZE"):
            scale["WRITE_SIZE"] = nbytes / (cal["WRITE_SIZE"] * 1024)
    counters = sorted({c for v in sums.values() for c in v})
    print("| kernel | dispatches per step | " + " | ".join(
        c + (" (GB/step)" if c in ("FETCH_SIZE", "WRITE_SIZE") else " (/step)") for c in counters)
        + (" | MFMA util |" if "SQ_VALU_MFMA_BUSY_CYCLES" in counters else " |"))
    print("|---|---|" + "---|" * len(counters) + ("---|" if "SQ_VALU_MFMA_BUSY_CYCLES" in counters else ""))
    chain = collections.defaultdict(float)
    for key, v in sums.items():
        if key == "copy (calibration)":
            continue
        cells = []
        for c in counters:
            x = v.get(c, 0.0) / steps_in_trace
            if c in ("FETCH_SIZE", "WRITE_SIZE"):
                x = x * 1024 * scale.get(c, 1.0) / 1e9
                if "gemm" in key:
                    chain[c] += x
                cells.append(f"{x:.2f}")
            else:
                cells.append(f"{x:.4g}")
        util = ""
        if "SQ_VALU_MFMA_BUSY_CYCLES" in counters:
            busy = v.get("SQ_BUSY_CU_CYCLES", 0.0)
            util = f" {v.get('SQ_VALU_MFMA_BUSY_CYCLES', 0.0) / (4 * busy):.3f} |" if busy else " - |"
        per_file = max(sum(1 for p, _ in disp[key] if p == path) for path in paths)
        label = f"`{key}`" + (f" ({GEMM_LABELS[key]})" if key in GEMM_LABELS else "")
        print(f"| {label} | {per_file / steps_in_trace:.1f} | " + " | ".join(cells) + " |" + util)
    if scale:
        print()
        print("scale factors from the copy calibration: " +
              ", ".join(f"{c} x{v:.3f}" for c, v in scale.items()))
    if chain:
        print("NS chain (gemm) per step: " + ", ".join(f"{c} {v:.2f} GB" for c, v in chain.items()))
    if traffic_json and chain:
        rec = {}
        if os.path.exists(traffic_json):
            with open(traffic_json) as f:
                rec = json.load(f)
        if rec.get("ns_chain_sources_sha256") != chain_sources_sha256():
            rec = {}
        if "FETCH_SIZE" in chain:
            rec["ns_chain_read_bytes_per_step"] = chain["FETCH_SIZE"] * 1e9
            rec["fetch_scale"] = scale.get("FETCH_SIZE")
        if "WRITE_SIZE" in chain:
            rec["ns_chain_write_bytes_per_step"] = chain["WRITE_SIZE"] * 1e9
            rec["write_scale"] = scale.get("WRITE_SIZE")
        if "ns_chain_read_bytes_per_step" in rec and "ns_chain_write_bytes_per_step" in rec:
            rec["ns_chain_hbm_bytes_per_step"] = (rec["ns_chain_read_bytes_per_step"] +
                                                  rec["ns_chain_write_bytes_per_step"])
        rec["ns_chain_sources_sha256"] = chain_sources_sha256()
        rec["source"] = "profiles/polar_step_gpt2_large_hbm_traffic.md"
        with open(traffic_json, "w") as f:
            json.dump(rec, f, indent=1)


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="gpt2-large",
                    choices=sorted(set(WORKLOADS) | set(PLAIN_GROUPS)),
                    help="config1: ns5 on one 768x3072 matrix; config2: one deflated "
                         "3072x768 matrix; gpt2-small / -medium / -large: every Muon matrix "
                         "of the model (configs 3, 4, 5)")
    ap.add_argument("--arm", default="deflated_ns_cut",
                    choices=["deflated_ns_cut", "deflated_pe_cut", "ns5", "polarexpress"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--ns-timing", default="sequential", choices=["sequential", "concurrent"],
                    help="the deflated arms' NS-chain pass: the groups' chains one after the "
                         "other (sequential) or together, each on its group's stream "
                         "(concurrent), once every front-end has finished")
    ap.add_argument("--inputs", default="spiked", choices=["spiked", "spiked-cpu", "gaussian"],
                    help="synthetic momenta: spiked spectra generated on the GPU (default), "
                         "the same generated on the host (counter runs: no GPU solver "
                         "call), or i.i.d. Gaussian")
    ap.add_argument("--mode", default="polar",
                    choices=["polar", "train", "kernels", "horner-f32"],
                    help="polar: the polar-step bench (default); train: the GPT-2-large "
                         "training step of config 5, with the polar-factor share; kernels: "
                         "the memory-bound kernels one after the other, for a rocprofv3 "
                         "kernel trace (see --summarize-trace); horner-f32: the fp32 "
                         "iteration (the convergence study's path) over the workload's "
                         "shape groups")
    ap.add_argument("--summarize-pmc", nargs="+", metavar="COUNTER_CSV",
                    help="print per-kernel counter sums per polar step of rocprofv3 --pmc "
                         "counter_collection.csv files taken over this bench with the same "
                         "--steps/--warmup (and --copy-calibration)")
    ap.add_argument("--traffic-json", metavar="PATH",
                    help="with --summarize-pmc: write the NS chain's FETCH/WRITE bytes per "
                         "step there, stamped with the NS chain sources' sha256")
    ap.add_argument("--summarize-trace", metavar="KERNEL_STATS_CSV",
                    help="print the GB/s table of a rocprofv3 --stats kernel_stats.csv taken "
                         "over --mode kernels with the same --workload/--steps/--warmup")
    ap.add_argument("--summarize-step-trace", metavar="KERNEL_TRACE_CSV",
                    help="print the per-polar-step table of the library's kernels from a "
                         "rocprofv3 --kernel-trace kernel_trace.csv (or .csv.gz) taken over "
                         "this bench with the same --steps/--warmup")
    ap.add_argument("--summarize-kernel-traffic", nargs="+", metavar="COUNTER_CSV",
                    help="tabulate rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of --mode kernels "
                         "against the memory-bound kernels' algorithmic bytes (with the same "
                         "--workload/--steps/--warmup/--copy-calibration)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="before the steps, copy a MIB-MiB fp32 buffer three times with "
                         "torch's copy kernel: a known-size reference for HBM byte "
                         "counters (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.summarize_pmc:
        summarize_pmc(args.summarize_pmc, args.warmup + 3 * args.steps, args.copy_calibration,
                      args.traffic_json)
        return
    if args.summarize_trace:
        summarize_trace(args.summarize_trace, args.workload, args.warmup + args.steps)
        return
    if args.summarize_kernel_traffic:
        summarize_kernel_traffic(args.summarize_kernel_traffic, args.workload,
                                 args.warmup + args.steps, args.copy_calibration)
        return
    if args.summarize_step_trace:
        summarize_step_trace(args.summarize_step_trace, args.steps, args.warmup)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the polar path "
              "shards by matrix across GPUs, which this build does not run.", file=sys.stderr)
        sys.exit(2)

    import torch
    from defmuon_amd import _native
    from defmuon_amd.optim import deflation_batched as DB
    from defmuon_amd.optim import deflation_cutoff as C

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    _native.load()
    dev = torch.device("cuda", 0)
    if args.copy_calibration:
        src = torch.ones(args.copy_calibration * 2 ** 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"bench: copy calibration: 3 x {args.copy_calibration} MiB read + written")
        del src, dst
    if args.mode == "train":
        print(json.dumps(train_step_report(args, dev)), flush=True)
        return
    if args.mode == "kernels":
        print(json.dumps(kernels_report(args, dev)), flush=True)
        return
    if args.mode == "horner-f32":
        print(json.dumps(horner_f32_report(args, dev)), flush=True)
        return
    plain = args.arm in ("ns5", "polarexpress")
    if (plain and args.workload not in PLAIN_GROUPS) or (not plain and args.workload not in WORKLOADS):
        print(f"bench.py: workload {args.workload} has no {args.arm} configuration", file=sys.stderr)
        sys.exit(2)
    groups = WORKLOADS.get(args.workload)
    fac = None if plain else C.ARMS[args.arm]()
    if plain:
        pgroups = PLAIN_GROUPS[args.workload]
        log(f"bench: generating inputs for {args.workload} ({args.arm}): {pgroups}")
        stacks = make_plain_inputs(pgroups, dev, gaussian=args.workload == "config1")

        def step(i, events=None):
            return plain_step(args.arm, stacks, pgroups, 5, events)
    else:
        log(f"bench: generating inputs for {args.workload}: {groups}")
        stacks = make_inputs(groups, dev, kind=args.inputs)

        def step(i, events=None):
            return polar_step(fac, stacks, i, 5, events, args.ns_timing)
    torch.cuda.synchronize()

    log(f"bench: warmup {args.warmup}")
    for w in range(args.warmup):
        step(w + 1)
    torch.cuda.synchronize()
    DB._GATE_ACC[0] = None

    log(f"bench: timing {args.steps} steps")
    events = []
    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for s in range(args.steps):
        step(args.warmup + s + 1, None if not plain else events)
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start.elapsed_time(stop)
    ms_per_step = gpu_ms / args.steps
    st = DB.polar_stats()   # gate statistics of the timed steps
    if not plain:
        # The timed steps run every group's chain on its own stream, overlapping the
        # other group's work, so the chains' own time is measured in a second pass of
        # the same steps with the chains one after the other on the launch stream
        # (HIP events around each chain call) once both front-ends have finished.
        log(f"bench: NS-chain pass, {args.steps} steps")
        events = []
        seq0 = torch.cuda.Event(enable_timing=True)
        seq1 = torch.cuda.Event(enable_timing=True)
        seq0.record()
        for s in range(args.steps):
            step(args.warmup + s + 1, events)
        seq1.record()
        torch.cuda.synchronize()
        seq_ms = seq0.elapsed_time(seq1) / args.steps
        # the other NS-chain timing, reported beside the primary one
        other = "concurrent" if args.ns_timing == "sequential" else "sequential"
        log(f"bench: NS-chain pass ({other} chains), {args.steps} steps")
        events2 = []
        for s in range(args.steps):
            polar_step(fac, stacks, args.warmup + s + 1, 5, events2, other)
        torch.cuda.synchronize()
        ns_ms_other = sum(e0.elapsed_time(e1) for evs in events2 for e0, e1 in evs) / args.steps
    ns_ms = sum(e0.elapsed_time(e1) for evs in events for e0, e1 in evs) / args.steps
    # plain arms: the chain is the whole step; deflated arms: the front-ends (with the
    # chains of the sequential pass subtracted) and the gate ticks
    front_ms = ms_per_step - ns_ms if plain else seq_ms - ns_ms
    if plain:   # the chain is the whole step: same matrices, plain-arm layout
        groups = [(B, max(r_, c_), min(r_, c_)) for B, r_, c_, _ in PLAIN_GROUPS[args.workload]]
    flops = ns_flops(groups)
    achieved = flops / (ns_ms * 1e-3) / 1e12
    log(f"bench: {ms_per_step:.3f} ms/step (wall {1e3 * wall / args.steps:.3f}), NS chain "
        f"{ns_ms:.3f} ms" + ("" if plain else f" (sequential pass {seq_ms:.3f} ms/step)")
        + f", gate {st}")

    cpu = None
    if not args.no_cpu_baseline:
        log("bench: cpu baseline")
        cpu = cpu_baseline(groups, args.arm)

    nmat = sum(B for B, _, _ in groups)
    # HBM traffic of the NS chain from the committed counter runs, used only when they
    # were measured on this build (same workload and arm, same NS chain sources)
    traffic = {}
    tpath = os.path.join(ROOT, "profiles", "ns_chain_traffic.json")
    if args.workload == "gpt2-large" and args.arm == "deflated_ns_cut" and os.path.exists(tpath):
        with open(tpath) as f:
            rec = json.load(f)
        if rec.get("ns_chain_sources_sha256") == chain_sources_sha256():
            traffic = rec
        else:
            log("bench: profiles/ns_chain_traffic.json was measured on other NS chain sources; "
                "roofline.traffic is null")
    out = {
        "metric": "polar steps/sec (GPT-2-large all matrices, 1 GPU) + % bf16 MFMA peak",
        "value": 1e3 / ms_per_step,
        "unit": "polar_steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 (NS chain) / fp32+fp64 (rSVD front-end)",
        "data": ("synthetic: one 768x3072 fp32 matrix with N(0, 1) entries (seed 0), "
                 "resident in HBM" if args.workload == "config1" else
                 "synthetic: spiked-spectrum fp32 momenta (8 spikes 50x..10x over a "
                 "Marchenko-Pastur bulk, Haar singular vectors), resident in HBM"),
        "config": {"workload": f"{args.workload} {args.arm} polar step: "
                               + " + ".join(f"{B}x({n},{m})" for B, n, m in groups)
                               + " (tall convention: wide matrices run as their transpose)",
                   "matrices": nmat, "ns_steps": 5, "arm": args.arm},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / PEAK_BF16_TFLOPS,
                     "traffic": traffic.get("ns_chain_hbm_bytes_per_step"),
                     "traffic_scope": ("bytes per polar step the L2 fetched from and wrote to "
                                       "the memory fabric (MALL or HBM) over the NS chain "
                                       "launches, measured with rocprofv3 --pmc FETCH_SIZE "
                                       "(x2) and WRITE_SIZE (x1), scales from torch's copy "
                                       "kernel; " + traffic.get("source", "not measured"))
                     if traffic else None,
                     "kernel": "NS chain (gemm_nt_bf16 K1/K2/K3 launches of a polar step), "
                               "canonical dense 4m^2n+2m^3 FLOP per matrix-iteration",
                     "flops_per_step": flops, "ns_ms_per_step": ns_ms,
                     "ns_timing": ("HIP events on the launch stream around the plain "
                                   "arm's group chains (entry normalisation included; the "
                                   "groups on side streams of their own, as the optimizer "
                                   "runs them)") if plain else
                                  ("HIP events on the launch stream, in a pass of the same "
                                   "steps once both front-ends have finished (the timed "
                                   "steps overlap the chains with the other group's work): "
                                   + ("one pair around each group's chain, the chains one "
                                      "after the other" if args.ns_timing == "sequential" else
                                      "one pair around the chain phase, every group's chain "
                                      "on its own stream"))},
        "frontend_ms_per_step": None if plain else front_ms,
        "ns_other_timing": None if plain else {
            "ns_timing": other, "ns_ms_per_step": ns_ms_other,
            "achieved": flops / (ns_ms_other * 1e-3) / 1e12,
            "frac": flops / (ns_ms_other * 1e-3) / 1e12 / PEAK_BF16_TFLOPS},
        "gate": None if plain else st,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
