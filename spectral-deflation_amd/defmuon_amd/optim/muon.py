"""Muon with the polar factor on the HIP library.

Drop-in for defmuon/optim/muon.py: the same `zeropower_via_newtonschulz5(G, steps)`
contract (muon.py:16-44) and the same `Muon` optimizer API, parameter routing,
W_QKV split, batched deflated step, sketch seeding, gate statistics, learning
rate scaling and AdamW backup (muon.py:47-438).

Execution differences, with identical per-matrix results: the deflated step runs
the bf16 iteration once per tall-shape group (one grouped launch per GEMM phase
over every matrix of the group) instead of once per parameter (muon.py:309-312);
for the built-in arms the clip hands X0 to the chain in its packed layout, and
the groups' clips run concurrently on separate streams before their chains
(`_DeflatedPolarBase.polar_groups`).  Each matrix's computation is independent
of the others in the batch and of the order the groups run in.
"""

import math
import os

import torch

from defmuon_amd import _native
from defmuon_amd.optim.deflation_batched import (_DeflatedPolarBase, _GATE_ACC, _PENDING,
                                                 _TIMING_ON)
from defmuon_amd.optim.polar_express import PolarExpress, as_batch, pe_schedule

NS_ABC = (3.4445, -4.7750, 2.0315)


def zeropower_via_newtonschulz5(G, steps):
    """Quintic Newton-Schulz polar factor: bf16 output of G's shape.  Entry
    X / (||X||_F + 1e-7); the chain runs on the transposed matrix when
    G.size(0) > G.size(1), the reference's own test (muon.py:30)."""
    assert len(G.shape) >= 2
    tall = G.size(0) > G.size(1)
    out = _native.ns_chain(as_batch(G), tall, 1, [NS_ABC] * steps)
    return out.reshape(G.shape)


def plain_group_chains(stacks, talls, entry_mode, sched):
    """The plain arm's chain (ns_chain with entry normalisation) over each stacked
    group, [polar factors] in group order.  With several groups on a GPU every group
    runs on a side stream of its own, the largest first: a small group's launches
    leave most compute units idle, which the other groups' launches fill.  Each result
    equals that of ns_chain on its group alone."""
    if len(stacks) < 2 or not stacks[0].is_cuda:
        return [_native.ns_chain(X, t, entry_mode, sched) for X, t in zip(stacks, talls)]
    from defmuon_amd.optim.deflation_batched import _side_streams
    dev = stacks[0].device
    main = torch.cuda.current_stream(dev)
    order = sorted(range(len(stacks)), key=lambda i: -stacks[i].numel())
    outs = [None] * len(stacks)
    side = _side_streams(dev, len(stacks))
    for s in side:
        s.wait_stream(main)
    for s, i in zip(side, order):
        with torch.cuda.stream(s):
            outs[i] = _native.ns_chain(stacks[i], talls[i], entry_mode, sched)
        stacks[i].record_stream(s)
        outs[i].record_stream(main)
    for s in side:
        main.wait_stream(s)
    return outs


_EXCLUDED = ("embeddings", "embed_tokens", "wte", "lm_head", "wpe")


class Muon(torch.optim.Optimizer):
    """MomentUm Orthogonalized by Newton-Schulz, with the polar factor computed by
    the HIP library.

    Arguments (muon.py:78-92): named_params, lr, weight_decay, momentum,
    nesterov, ns_steps, rms_scaling, nuclear_scaling, polar_method ("ns5" or
    "polarexpress"; the deflated arms are added by deflation_cutoff.install()),
    adamw_betas, adamw_eps, polar_args, batched_deflation (accepted and ignored:
    the batched path is chosen from the factorizer, as in the reference).
    """

    def __init__(self, named_params, lr=1e-3, weight_decay=0, momentum=0.95, nesterov=True,
                 ns_steps=5, rms_scaling=True, nuclear_scaling=False, polar_method="ns5",
                 adamw_betas=(0.95, 0.95), adamw_eps=1e-8, polar_args={},
                 batched_deflation=False):
        defaults = dict(lr=lr, weight_decay=weight_decay, momentum=momentum,
                        nesterov=nesterov, ns_steps=ns_steps, rms_scaling=rms_scaling,
                        nuclear_scaling=nuclear_scaling, adamw_betas=adamw_betas,
                        adamw_eps=adamw_eps)
        muon, muon_names, adamw = [], [], []
        for name, p in named_params:
            if p.ndim >= 2 and not any(x in name for x in _EXCLUDED):
                muon.append(p)
                muon_names.append(name)
            else:
                adamw.append(p)
        super().__init__(muon + adamw, defaults)
        for p, name in zip(muon, muon_names):
            assert p.ndim == 2, p.ndim
            self.state[p]["use_muon"] = True
            if name.endswith("attn.c_attn.weight"):
                self.state[p]["is_W_QKV"] = True
        for p in adamw:
            self.state[p]["use_muon"] = False

        self.polar_factorizer = self._initialize_polar_factorizer(polar_method, polar_args)
        self.batched_deflation = isinstance(self.polar_factorizer, _DeflatedPolarBase)
        if self.batched_deflation:
            self._bd_step = 0
        if os.environ.get("DEFMUON_WARM_POLAR", "1") == "1":
            self._warm_polar_compile()

    # -- helpers --------------------------------------------------------------
    def _qkv_split(self, p, g):
        """A W_QKV gradient (3d x d) is processed as its three d x d blocks."""
        if self.state[p].get("is_W_QKV", False):
            return g.reshape(3, g.shape[0] // 3, g.shape[1])
        return g

    def _warm_polar_compile(self):
        """Construction-time warm-up (muon.py:167-240): load the library and run
        each kernel family once on every shape the step will feed it, so first-call
        costs land before the clock starts.  Zeros for the iteration, randn from a
        dedicated generator for the clip; the global RNG is never touched."""
        fac = self.polar_factorizer
        steps = self.defaults["ns_steps"]
        try:
            _native.load()
            if isinstance(fac, _DeflatedPolarBase):
                groups, dev = {}, None
                for group in self.param_groups:
                    for p in group["params"]:
                        if self.state[p].get("use_muon"):
                            A = self._qkv_split(p, p)
                            nb = A.shape[0] if A.ndim == 3 else 1
                            n, m = max(A.shape[-2:]), min(A.shape[-2:])
                            groups[(n, m)] = groups.get((n, m), 0) + nb
                            dev = p.device
                for (n, m), cnt in sorted(groups.items()):
                    g_ = torch.Generator(device=dev)
                    g_.manual_seed(0)
                    A = torch.randn((cnt, n, m), dtype=torch.float32, device=dev, generator=g_)
                    X0, _, _ = fac.BATCHED_CLIP(A, generator=g_, pad=fac.PAD,
                                                out_dtype=torch.bfloat16)
                    fac._iterate(torch.zeros_like(X0), steps)
                    del A, X0
                if groups:
                    print(f"warm_polar: warmed the deflated clip and iteration for "
                          f"{len(groups)} tall-shape groups at construction")
            else:
                seen = set()
                for group in self.param_groups:
                    for p in group["params"]:
                        if not self.state[p].get("use_muon"):
                            continue
                        shape = tuple(self._qkv_split(p, p).shape)
                        key = (shape, p.dtype, p.device)
                        if key not in seen:
                            seen.add(key)
                            fac(torch.zeros(shape, dtype=p.dtype, device=p.device), steps)
                if seen:
                    print(f"warm_polar: warmed the polar factorizer for {len(seen)} shapes")
        except Exception as e:   # a failed warm-up only moves first-call cost into step 1
            print(f"warm_polar: warm-up failed ({e}); step 1 pays the first-call cost")

    def _initialize_polar_factorizer(self, polar_method, polar_args):
        if polar_method == "ns5":
            return zeropower_via_newtonschulz5
        elif polar_method == "polarexpress":
            return PolarExpress
        else:
            raise ValueError(f"Unknown polar method: {polar_method}")

    def adjust_lr_for_muon(self, lr, rms_scaling, nuclear_scaling, param_shape, grad,
                           grad_sign):
        scale = 1.0
        if rms_scaling:
            fan_out, fan_in = param_shape[:2]
            scale *= math.sqrt(fan_out / fan_in)
        if nuclear_scaling:
            scale *= torch.trace(grad.T @ grad_sign)
        return lr * scale

    # -- the batched deflated step (muon.py:251-323) ---------------------------
    # momentum -> stack and the update as one library launch per shape group
    # (dmh_momentum_stack / dmh_apply_update); False: the reference's torch ops
    FUSED_GLUE = True

    def _fused_glue_ok(self, group, params):
        """The fused glue covers rms scaling on contiguous fp32 GPU tensors."""
        if not self.FUSED_GLUE or group["nuclear_scaling"]:
            return False
        for p in params:
            g = p.grad
            if g is None:
                continue
            buf = self.state[p].get("momentum_buffer")
            ts = (p.data, g) if buf is None else (p.data, g, buf)
            if any(not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous()
                   for t in ts) or p.ndim != 2:
                return False
        return True

    def _muon_step_batched(self, group, params, lr, weight_decay, momentum):
        fac = self.polar_factorizer
        ns_steps = group["ns_steps"]
        fused = self._fused_glue_ok(group, params)
        entries = []
        for p in params:
            if p.grad is None:
                continue
            state = self.state[p]
            if "momentum_buffer" not in state:
                state["momentum_buffer"] = torch.zeros_like(p.grad)
            if fused:
                # the same tall blocks as below, described instead of materialised
                rows, cols = p.shape
                nb = 3 if state.get("is_W_QKV", False) else 1
                tr = rows // nb < cols
                shape = (cols, rows // nb) if tr else (rows // nb, cols)
                entries.append({"p": p, "tr": tr, "nb": nb, "shape": shape})
                continue
            buf = state["momentum_buffer"]
            buf.mul_(momentum).add_(p.grad)
            g = p.grad.add(buf, alpha=momentum) if group["nesterov"] else buf
            A = self._qkv_split(p, g).float()
            if A.ndim == 2:
                A = A[None]
            tr = A.shape[-2] < A.shape[-1]
            if tr:
                A = A.mT
            entries.append({"p": p, "g": g, "A": A, "tr": tr, "nb": A.shape[0],
                            "shape": tuple(A.shape[-2:])})

        shapes = {}
        for e in entries:
            shapes.setdefault(e["shape"], []).append(e)

        self._bd_step += 1
        groups = sorted(shapes.items())
        As, gens = [], []
        for gi, (shape, es) in enumerate(groups):
            if fused:
                A = torch.empty((sum(e["nb"] for e in es),) + shape, dtype=torch.float32,
                                device=es[0]["p"].device)
                _native.momentum_stack(self._glue_params(es, shape), momentum,
                                       group["nesterov"], A)
            else:
                A = torch.cat([e["A"] for e in es], dim=0)
            gen = torch.Generator(device=A.device)
            gen.manual_seed((self._bd_step * 1009 + gi * 9176867) % (2 ** 62))
            As.append(A)
            gens.append(gen)
        timed = _TIMING_ON[0] and bool(As) and As[0].is_cuda
        if timed:
            # one group after the other, with separate clip and iteration calls so
            # that the events can split them
            results, marks = [], []
            for A, gen in zip(As, gens):
                e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
                e0.record()
                X0, kvec, d = fac.BATCHED_CLIP(A, generator=gen, pad=fac.PAD,
                                               out_dtype=torch.bfloat16)
                e1.record()
                Ug = fac._iterate(X0, ns_steps)      # one grouped launch per GEMM phase
                e2.record()
                results.append((Ug, kvec, d))
                marks.append((e0, e1, e2))
            _PENDING.extend(marks)
        else:
            results = fac.polar_groups(As, gens, steps=ns_steps)
        for (shape, es), A, (Ug, kvec, _) in zip(groups, As, results):
            if _GATE_ACC[0] is None or _GATE_ACC[0].device != kvec.device:
                _GATE_ACC[0] = torch.zeros(3, dtype=torch.int64, device=kvec.device)
            # the same tick as muon.py:306-308, with the matrix count added as a host
            # scalar: a torch.tensor(..., device=gpu) copy would block the host until
            # the stream drains (the whole polar step), every optimizer step
            _GATE_ACC[0][0] += A.shape[0]
            _GATE_ACC[0][1:] += torch.stack([(kvec > 0).sum(), kvec.sum().to(torch.int64)])
            if fused:
                _native.apply_update(self._glue_params(es, shape, lr, weight_decay, group), Ug)
                continue
            off = 0
            for e in es:
                e["u"] = Ug[off:off + e["nb"]]
                off += e["nb"]
            for e in es:
                p, g = e["p"], e["g"]
                u = (e["u"].mT if e["tr"] else e["u"]).reshape(p.shape).bfloat16()
                adjusted_lr = self.adjust_lr_for_muon(lr, group["rms_scaling"],
                                                      group["nuclear_scaling"], p.shape,
                                                      g.bfloat16(), u)
                p.data.mul_(1 - lr * weight_decay)
                p.data.add_(u, alpha=-adjusted_lr)

    def _glue_params(self, es, shape, lr=None, weight_decay=0.0, group=None):
        """dmh_glue_param descriptors of a shape group's parameters, in stack order;
        with lr, the update's alpha = -lr * sqrt(fan_out / fan_in) (rms scaling, as
        adjust_lr_for_muon) and decay = 1 - lr * wd."""
        n, m = shape
        out, off = [], 0
        for e in es:
            p = e["p"]
            d = _native.GlueParam()
            d.grad = p.grad.data_ptr()
            d.momentum = self.state[p]["momentum_buffer"].data_ptr()
            d.param = p.data.data_ptr()
            d.rows, d.cols = p.shape
            d.blocks = e["nb"]
            d.transpose = int(e["tr"])
            d.offset = off * n * m
            if lr is not None:
                d.alpha = -self.adjust_lr_for_muon(lr, group["rms_scaling"], False, p.shape,
                                                   None, None)
                d.decay = 1 - lr * weight_decay
            off += e["nb"]
            out.append(d)
        return out

    # -- the plain arms, grouped by matrix shape (grouped_plain.install()) -------
    GROUPED_PLAIN = False

    def _muon_step_plain_grouped(self, group, params, lr, weight_decay, momentum):
        """The plain-arm update (muon.py:361-386) with one library launch per
        (matrix shape, dtype, orientation) instead of one factorizer call per
        parameter.  The orientation is the one the factorizer itself would pick
        for the parameter (size(0) > size(1) for ns5, muon.py:30; size(-2) >
        size(-1) for PolarExpress, polar_express.py:25), the entry normalisation
        is per matrix, and the matrices of a launch do not interact, so every
        update equals the per-parameter one.  Returns False (nothing done) for a
        factorizer other than the built-in two."""
        fac = self.polar_factorizer
        steps = group["ns_steps"]
        if fac is zeropower_via_newtonschulz5:
            mode, sched = 1, [NS_ABC] * steps
        elif fac is PolarExpress:
            mode, sched = 2, pe_schedule(steps)
        else:
            return False
        groups = {}
        for p in params:
            g = p.grad
            if g is None:
                continue
            state = self.state[p]
            if "momentum_buffer" not in state:
                state["momentum_buffer"] = torch.zeros_like(g)
            buf = state["momentum_buffer"]
            buf.mul_(momentum).add_(g)
            g = g.add(buf, alpha=momentum) if group["nesterov"] else buf
            gq = self._qkv_split(p, g)
            tall = gq.size(0) > gq.size(1) if mode == 1 else gq.size(-2) > gq.size(-1)
            X = as_batch(gq)
            groups.setdefault((tuple(X.shape[1:]), X.dtype, tall), []).append((p, g, X))
        keys = list(groups)
        stacks = [groups[k][0][2] if len(groups[k]) == 1 else torch.cat([X for _, _, X in groups[k]])
                  for k in keys]
        outs = plain_group_chains(stacks, [k[2] for k in keys], mode, sched)
        for key, out in zip(keys, outs):
            es = groups[key]
            off = 0
            for p, g, X in es:
                u = out[off:off + X.shape[0]].reshape(g.shape)
                off += X.shape[0]
                adjusted_lr = self.adjust_lr_for_muon(lr, group["rms_scaling"],
                                                      group["nuclear_scaling"], p.shape,
                                                      g.bfloat16(), u)
                p.data.mul_(1 - lr * weight_decay)
                p.data.add_(u, alpha=-adjusted_lr)
        return True

    # -- the AdamW backup as one library launch per group (FUSED_GLUE) ----------
    ADAMW_TABLES_KEPT = 4   # device tables kept per parameter group
    def _adamw_fused(self, group, params, lr, weight_decay, beta1, beta2, eps):
        """The AdamW loop below (muon.py:408-436) in one dmh_adamw_step launch per
        distinct step count: the same fp32 operations per element, the moments
        created and the step counts kept exactly as the loop does.  Returns False
        (nothing done) when a parameter, its gradient or an existing moment is not a
        contiguous fp32 GPU tensor of the parameter's shape (the kernel indexes all
        four flat).

        The device table of a group's tensors is built once and reused while the
        tensors stay at the same addresses: tables are cached per group by those
        addresses (not by the step count, which only enters the scalar alpha), the
        few most recent kept, so gradients that alternate between a couple of
        buffers do not rebuild it either."""
        if not self.FUSED_GLUE:
            return False
        live = [p for p in params if p.grad is not None]
        if not live:
            return True
        for p in live:
            st = self.state[p]
            ts = [p.data, p.grad] + [st[k] for k in ("moment1", "moment2") if k in st]
            if any(not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous()
                   or t.shape != p.shape for t in ts):
                return False
        by_step = {}
        for p in live:
            state = self.state[p]
            if "step" not in state:
                state["step"] = 0
                state["moment1"] = torch.zeros_like(p.grad)
                state["moment2"] = torch.zeros_like(p.grad)
            state["step"] += 1
            by_step.setdefault(state["step"], []).append(
                (p.data, p.grad, state["moment1"], state["moment2"]))
        tables = self.__dict__.setdefault("_adamw_tables", {}).setdefault(id(group), {})
        for step, quads in by_step.items():
            key = _native.AdamwTable.key_of(quads)
            tab = tables.pop(key, None)
            if tab is None:
                tab = _native.AdamwTable(quads)
                while len(tables) >= self.ADAMW_TABLES_KEPT:
                    tables.pop(next(iter(tables)))      # the least recently used
            tables[key] = tab                           # most recently used last
            scale = (1 - beta1 ** step) / (1 - beta2 ** step) ** 0.5
            _native.adamw_step(tab, 1 - beta1, 1 - beta2, eps, 1 - lr * weight_decay,
                               -lr / scale)
        return True

    # -- step (muon.py:334-438) ------------------------------------------------
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self.param_groups:
            params = [p for p in group["params"] if self.state[p]["use_muon"]]
            lr = group["lr"]
            weight_decay = group["weight_decay"]
            momentum = group["momentum"]
            if self.batched_deflation and params:
                self._muon_step_batched(group, params, lr, weight_decay, momentum)
                params = []
            if (self.GROUPED_PLAIN and params
                    and self._muon_step_plain_grouped(group, params, lr, weight_decay,
                                                      momentum)):
                params = []
            for p in params:
                g = p.grad
                if g is None:
                    continue
                state = self.state[p]
                if "momentum_buffer" not in state:
                    state["momentum_buffer"] = torch.zeros_like(g)
                buf = state["momentum_buffer"]
                buf.mul_(momentum).add_(g)
                g = g.add(buf, alpha=momentum) if group["nesterov"] else buf
                old_shape = g.shape
                g = self._qkv_split(p, g)
                u = self.polar_factorizer(g, group["ns_steps"])
                g = g.reshape(old_shape)
                u = u.reshape(old_shape)
                adjusted_lr = self.adjust_lr_for_muon(lr, group["rms_scaling"],
                                                      group["nuclear_scaling"], p.shape,
                                                      g.bfloat16(), u)
                p.data.mul_(1 - lr * weight_decay)
                p.data.add_(u, alpha=-adjusted_lr)

            params = [p for p in group["params"] if not self.state[p]["use_muon"]]
            beta1, beta2 = group["adamw_betas"]
            eps = group["adamw_eps"]
            if self._adamw_fused(group, params, lr, weight_decay, beta1, beta2, eps):
                params = []
            for p in params:
                g = p.grad
                if g is None:
                    continue
                state = self.state[p]
                if "step" not in state:
                    state["step"] = 0
                    state["moment1"] = torch.zeros_like(g)
                    state["moment2"] = torch.zeros_like(g)
                state["step"] += 1
                step = state["step"]
                buf1, buf2 = state["moment1"], state["moment2"]
                buf1.lerp_(g, 1 - beta1)
                buf2.lerp_(g.square(), 1 - beta2)
                g = buf1 / (eps + buf2.sqrt())
                scale = (1 - beta1 ** step) / (1 - beta2 ** step) ** 0.5
                p.data.mul_(1 - lr * weight_decay)
                p.data.add_(g, alpha=-lr / scale)
        return loss
