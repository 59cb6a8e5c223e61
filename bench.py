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
    "gpt2-small": [(48, 768, 768), (24, 3072, 768)],
    "gpt2-medium": [(96, 1024, 1024), (48, 4096, 1024)],
    "gpt2-large": [(144, 1280, 1280), (72, 5120, 1280)],
}


# plain arms: the Muon parameters' matrices after the W_QKV split, nn.Linear
# (out, in) layout, grouped as the grouped plain step launches them:
# (count, rows, cols, tall) -- tall: the factorizer runs on the transpose
PLAIN_GROUPS = {
    "gpt2-small": [(48, 768, 768, False), (12, 3072, 768, True), (12, 768, 3072, False)],
    "gpt2-medium": [(96, 1024, 1024, False), (24, 4096, 1024, True), (24, 1024, 4096, False)],
    "gpt2-large": [(144, 1280, 1280, False), (36, 5120, 1280, True), (36, 1280, 5120, False)],
}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def ns_flops(groups, steps=5):
    """Canonical dense NS FLOPs: 4 m^2 n + 2 m^3 per matrix and iteration."""
    return sum(B * steps * (4 * m * m * n + 2 * m ** 3) for B, n, m in groups)


def make_inputs(groups, device, seed=1234, kind="spiked"):
    """Synthetic momenta per group.  "gaussian": i.i.d. N(0, 1/n) entries (no QR, so
    nothing from the solver library runs; the gate declines every matrix), for
    hardware-counter runs whose NS-chain traffic does not depend on the values."""
    import torch
    from defmuon_amd import synthetic as S
    out = []
    for gi, (B, n, m) in enumerate(groups):
        if kind == "gaussian":
            g = torch.Generator(device=device)
            g.manual_seed(seed + gi)
            out.append(torch.randn(B, n, m, device=device, generator=g) / math.sqrt(n))
        else:
            out.append(S.spiked_batch(B, n, m, seed=seed + gi, n_spikes=8, hi=50.0, lo=10.0,
                                      device=device))
    return out


def polar_step(fac, stacks, bd_step, ns_steps, events=None):
    """One polar step over all groups, as the optimizer runs it
    (_DeflatedPolarBase.polar_groups: the groups' clips, then their iterations);
    returns per-group (U, k).  With `events`, appends a list of (start, end) HIP
    event pairs recorded on the launch stream around each group's NS chain."""
    import torch
    from defmuon_amd.optim import deflation_batched as DB
    gens = []
    for gi, A in enumerate(stacks):
        gen = torch.Generator(device=A.device)
        gen.manual_seed((bd_step * 1009 + gi * 9176867) % (2 ** 62))
        gens.append(gen)
    evs = None
    if events is not None:
        evs = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(2)) for _ in stacks]
        events.append(evs)
    res = fac.polar_groups(stacks, gens, steps=ns_steps, chain_events=evs)
    outs = []
    for A, (U, kvec, _) in zip(stacks, res):
        if DB._GATE_ACC[0] is None:
            DB._GATE_ACC[0] = torch.zeros(3, dtype=torch.int64, device=A.device)
        DB._GATE_ACC[0][0] += A.shape[0]   # host scalar: no host->device copy, no wait
        DB._GATE_ACC[0][1:] += torch.stack([(kvec > 0).sum(), kvec.sum().to(torch.int64)])
        outs.append((U, kvec))
    return outs


def make_plain_inputs(pgroups, device, seed=4321):
    """Spiked-spectrum momenta per plain group, in the parameters' own layout."""
    from defmuon_amd import synthetic as S
    out = []
    for gi, (B, rows, cols, tall) in enumerate(pgroups):
        n, m = max(rows, cols), min(rows, cols)
        X = S.spiked_batch(B, n, m, seed=seed + gi, n_spikes=8, hi=50.0, lo=10.0, device=device)
        out.append(X if rows >= cols else X.mT.contiguous())
    return out


def plain_step(arm, stacks, pgroups, ns_steps, events=None):
    """One plain-arm polar step (muon.py:361-386 factorizer calls over every Muon
    parameter) with one launch per group, as Muon._muon_step_plain_grouped runs it."""
    import torch
    from defmuon_amd import _native
    from defmuon_amd.optim.muon import NS_ABC
    from defmuon_amd.optim.polar_express import pe_schedule
    mode, sched = (1, [NS_ABC] * ns_steps) if arm == "ns5" else (2, pe_schedule(ns_steps))
    evs = []
    outs = []
    for X, (_, _, _, tall) in zip(stacks, pgroups):
        ev = tuple(torch.cuda.Event(enable_timing=True) for _ in range(2))
        ev[0].record()
        outs.append(_native.ns_chain(X, tall, mode, sched))
        ev[1].record()
        evs.append(ev)
    if events is not None:
        events.append(evs)
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
    ap.add_argument("--workload", default="gpt2-large", choices=sorted(WORKLOADS))
    ap.add_argument("--arm", default="deflated_ns_cut",
                    choices=["deflated_ns_cut", "deflated_pe_cut", "ns5", "polarexpress"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--inputs", default="spiked", choices=["spiked", "gaussian"],
                    help="synthetic momenta: spiked spectra (default) or i.i.d. Gaussian "
                         "(for counter runs; no solver call)")
    ap.add_argument("--mode", default="polar", choices=["polar", "train"],
                    help="polar: the polar-step bench (default); train: the GPT-2-large "
                         "training step of config 5, with the polar-factor share")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="before the steps, copy a MIB-MiB fp32 buffer three times with "
                         "torch's copy kernel: a known-size reference for HBM byte "
                         "counters (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
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
    if args.mode == "train":
        print(json.dumps(train_step_report(args, dev)), flush=True)
        return
    groups = WORKLOADS[args.workload]
    plain = args.arm in ("ns5", "polarexpress")
    fac = None if plain else C.ARMS[args.arm]()
    if args.copy_calibration:
        src = torch.ones(args.copy_calibration * 2 ** 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"bench: copy calibration: 3 x {args.copy_calibration} MiB read + written")
        del src, dst
    if plain:
        pgroups = PLAIN_GROUPS[args.workload]
        log(f"bench: generating inputs for {args.workload} ({args.arm}): {pgroups}")
        stacks = make_plain_inputs(pgroups, dev)

        def step(i, events=None):
            return plain_step(args.arm, stacks, pgroups, 5, events)
    else:
        log(f"bench: generating inputs for {args.workload}: {groups}")
        stacks = make_inputs(groups, dev, kind=args.inputs)

        def step(i, events=None):
            return polar_step(fac, stacks, i, 5, events)
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
    # HBM traffic of the NS chain from the committed counter runs (same workload and arm)
    traffic = {}
    tpath = os.path.join(ROOT, "profiles", "ns_chain_traffic.json")
    if args.workload == "gpt2-large" and args.arm == "deflated_ns_cut" and os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f)
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
        "data": "synthetic: spiked-spectrum fp32 momenta (8 spikes 50x..10x over a "
                "Marchenko-Pastur bulk, Haar singular vectors), resident in HBM",
        "config": {"workload": f"{args.workload} {args.arm} polar step: "
                               + " + ".join(f"{B}x({n},{m})" for B, n, m in groups),
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
                     "ns_timing": "HIP events around each chain call on the launch stream"
                                  + ("" if plain else ", in a pass of the same steps with "
                                     "the chains one after the other (the timed steps "
                                     "overlap them with the other group's work)")},
        "frontend_ms_per_step": None if plain else front_ms,
        "gate": None if plain else st,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
