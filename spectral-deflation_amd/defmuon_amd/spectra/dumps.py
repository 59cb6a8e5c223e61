"""Momentum dumps of the deflated polar path: file format, loader and collector.

File format (the interface of spectra/collect.py:109-113 and :134-139, kept so that
dumps written by either side load in the other):
  * one file per (optimizer step, dumped parameter), `step{step:04d}_{label}.pt`,
    holding torch.save({"step", "label", "A", "momentum", "nesterov"}); "A" is the fp32
    post-Nesterov matrix the polar factorizer consumes that step (collect.py:89-97);
  * labels attn_qkv (the whole c_attn weight: Q, K and V stacked by rows), attn_o,
    mlp_fc and mlp_proj of the middle transformer layer;
  * `quantiles.json`: a list of {"step", "label", "fro", "sigma_max", "q": {str(q): v}}
    records, one per orthogonalized matrix (attn_qkv as attn_q / attn_k / attn_v), with
    v the ceil(q r)-th largest singular value over the Frobenius norm (collect.py:127-135).

Dumps are read with torch.load(weights_only=True): a dump holds tensors and plain
Python scalars only, so nothing in the file is executed.
"""

import glob
import json
import os
import re

import torch

# the six matrices Muon orthogonalizes, each with its own Frobenius entry (plot_spectra.py:76)
PANEL_COLS = ["attn_q", "attn_k", "attn_v", "attn_o", "mlp_fc", "mlp_proj"]
ROW_NAME = {"attn_q": "Attn $Q$", "attn_k": "Attn $K$", "attn_v": "Attn $V$",
            "attn_qkv": "Attn $QKV$", "attn_o": "Attn $O$",
            "mlp_fc": "MLP in", "mlp_proj": "MLP out"}           # plot_spectra.py:68-70
QUANTILES = (0.1, 0.25, 0.5, 0.75, 0.9)                           # collect.py:43

# dumped parameters: module path inside a transformer block -> dump label
LABEL_OF_MODULE = {"attn.c_attn": "attn_qkv", "attn.c_proj": "attn_o",
                   "mlp.c_fc": "mlp_fc", "mlp.c_proj": "mlp_proj"}
_BLOCK_PARAM = re.compile(r"\.h\.(\d+)\.(.+)$")       # "<prefix>.h.<layer>.<rest>"
_QKV_PARTS = ("attn_q", "attn_k", "attn_v")


def momentum_A(grad, buf, momentum, nesterov):
    """The matrix the factorizer consumes this step, out of place (collect.py:89-97):
    buf' = momentum * buf + grad (grad where there is no buffer yet);
    A = grad + momentum * buf' with Nesterov, else buf'."""
    g32 = grad.float()
    newbuf = g32 if buf is None else buf.float().mul(momentum).add_(g32)
    return g32 + momentum * newbuf if nesterov else newbuf


def split_blocks(label, A):
    """[(name, matrix)] of the matrices Muon orthogonalizes inside one dumped
    parameter: the c_attn weight is its three row blocks of E rows, E its width
    (muon.py:160-165 splits W_QKV the same way); any other parameter is itself."""
    if label != "attn_qkv":
        return [(label, A)]
    E = A.shape[1]
    return [(part, A[i * E:(i + 1) * E]) for i, part in enumerate(_QKV_PARTS)]


def tall(M):
    """M in the tall convention (n >= m), contiguous."""
    return (M.mT if M.shape[0] < M.shape[1] else M).contiguous()


def dump_name(step, label):
    return f"step{int(step):04d}_{label}.pt"


def save_dump(out_dir, step, label, A, momentum, nesterov):
    """Write one dump file; returns its path."""
    os.makedirs(out_dir, exist_ok=True)
    path = os.path.join(out_dir, dump_name(step, label))
    torch.save({"step": int(step), "label": str(label), "A": A.detach().float().cpu(),
                "momentum": float(momentum), "nesterov": bool(nesterov)}, path)
    return path


def load_dump(path):
    """One dump as its dict (safe loader)."""
    return torch.load(path, map_location="cpu", weights_only=True)


def load_matrices(dump_dir):
    """{step: {name: A}} over every dump in dump_dir, for the names of PANEL_COLS,
    each A a tall fp32 CPU tensor (the study's input, polar_convergence.py:117-137)."""
    out = {}
    for path in sorted(glob.glob(os.path.join(dump_dir, "step*_*.pt"))):
        rec = load_dump(path)
        mats = out.setdefault(int(rec["step"]), {})
        for name, M in split_blocks(rec["label"], rec["A"].float()):
            if name in PANEL_COLS:
                mats[name] = tall(M)
    return out


def sv_quantiles(B, quantiles=QUANTILES):
    """Singular-value quantiles of one matrix over its Frobenius norm: for each q,
    the ceil(q r)-th largest of its r singular values (collect.py:127-135)."""
    fro = B.norm().item()
    s = torch.linalg.svdvals(B.float())
    r = s.numel()
    q_of = {}
    for q in quantiles:
        rank = min(max(1, int(-(-q * r // 1))), r)      # ceil(q r), at least the first
        q_of[str(q)] = (s[rank - 1] / (fro + 1e-30)).item()
    return {"fro": fro, "sigma_max": s[0].item(), "q": q_of}


# ---------------------------------------------------------------------------
# collector
# ---------------------------------------------------------------------------

def _is_rank0():
    return int(os.environ.get("RANK", "0") or 0) <= 0


def middle_layer_targets(named_params):
    """[(label, param)] of the middle transformer block's four dumped weights, in
    parameter order.  Blocks are the `<prefix>.h.<i>.` names; the middle one is
    block n_layer // 2 of n_layer = 1 + the largest index (collect.py:64-76)."""
    by_layer = {}
    for name, p in named_params:
        m = _BLOCK_PARAM.search(name)
        if m:
            by_layer.setdefault(int(m.group(1)), []).append((m.group(2), p))
    if not by_layer:
        return []
    mid = (1 + max(by_layer)) // 2
    out = []
    for rest, p in by_layer.get(mid, []):
        module, _, leaf = rest.rpartition(".")
        if leaf == "weight" and module in LABEL_OF_MODULE:
            out.append((LABEL_OF_MODULE[module], p))
    return out


class SpectraCollector:
    """Records the polar factorizer's inputs of one optimizer, read-only.

    Registered as a step pre-hook of the optimizer: before optimizer step n (counted
    from 1) it computes, out of place, the matrix each target parameter's update
    will orthogonalize (`momentum_A` on the gradient and the momentum buffer as they
    are before the step mutates them) and
      * at the steps in `dump_steps` writes one dump per target;
      * every `qstep` steps (0: never) appends the singular-value quantiles of every
        orthogonalized matrix and rewrites quantiles.json.
    It touches no optimizer state and no RNG, so training is unchanged.  Only rank 0
    writes.  Nested step wrappers (a step function wrapped twice by torch's hook
    machinery) fire the hook once per step: a depth count skips the inner calls,
    and a step that raised (no post-hook) is recognised by the changed gradient and
    momentum state at the next step."""

    def __init__(self, targets, out_dir, dump_steps, qstep, writer=None):
        self.targets = list(targets)
        self.out_dir = out_dir
        self.dump_steps = frozenset(int(s) for s in dump_steps)
        self.qstep = int(qstep)
        self.writer = _is_rank0() if writer is None else bool(writer)
        self.step_count = 0
        self.records = []
        self._depth = 0
        self._key = None

    @classmethod
    def from_env(cls, named_params):
        """A collector for the middle layer of `named_params`, configured as the
        reference's collector is (collect.py:19-43): DEFMUON_SPECTRA_DIR (output
        root, default spectra/dumps), DEFMUON_SPECTRA_TAG (run folder; default
        gpt-large for n_embd 1280, else nembd<n_embd>), DEFMUON_SPECTRA_STEPS (steps
        to dump, default 1,500,1000,1500), DEFMUON_SPECTRA_QSTEP (quantile cadence,
        default 10).  None when there is no transformer block to watch."""
        targets = middle_layer_targets(named_params)
        if not targets:
            return None
        root = os.environ.get("DEFMUON_SPECTRA_DIR", "spectra/dumps")
        n_embd = min(min(p.shape) for _, p in targets)
        tag = os.environ.get("DEFMUON_SPECTRA_TAG") or (
            "gpt-large" if n_embd == 1280 else f"nembd{n_embd}")
        steps = [int(s) for s in os.environ.get("DEFMUON_SPECTRA_STEPS",
                                                "1,500,1000,1500").split(",") if s.strip()]
        qstep = int(os.environ.get("DEFMUON_SPECTRA_QSTEP", "10"))
        return cls(targets, os.path.join(root, tag), steps, qstep)

    def attach(self, optimizer):
        """Register on `optimizer`; returns the hook handles (pre, post)."""
        if self.writer:
            os.makedirs(self.out_dir, exist_ok=True)
        return (optimizer.register_step_pre_hook(self._before_step),
                optimizer.register_step_post_hook(self._after_step))

    def _inputs(self, optimizer):
        """(label, A) for every target with a gradient, A the factorizer's input."""
        group_of = {id(p): g for g in optimizer.param_groups for p in g["params"]}
        out = []
        for label, p in self.targets:
            group = group_of.get(id(p))
            if group is not None and p.grad is not None:
                buf = optimizer.state[p].get("momentum_buffer")
                out.append((label, momentum_A(p.grad, buf, group["momentum"],
                                              group["nesterov"])))
        return out

    def _state_key(self, optimizer):
        """Identity and in-place version of every target's gradient and momentum
        buffer: unchanged between the nested hook calls of one step, changed by the
        step itself."""
        key = []
        for _, p in self.targets:
            g, buf = p.grad, optimizer.state[p].get("momentum_buffer")
            key.append((id(g), g._version if g is not None else -1,
                        id(buf), buf._version if buf is not None else -1))
        return tuple(key)

    def _before_step(self, optimizer, args, kwargs):
        key = self._state_key(optimizer)
        if self._depth > 0 and key != self._key:
            self._depth = 0            # the last step raised before its post-hook ran
        self._depth += 1
        if self._depth > 1:
            return None
        self._key = key
        self.step_count += 1
        n = self.step_count
        dump_now = n in self.dump_steps
        quant_now = self.qstep > 0 and n % self.qstep == 0
        if not self.writer or not (dump_now or quant_now):
            return None
        inputs = self._inputs(optimizer)
        for label, A in inputs:
            if dump_now:
                save_dump(self.out_dir, n, label, A, optimizer.defaults["momentum"],
                          optimizer.defaults["nesterov"])
            if quant_now:
                for name, B in split_blocks(label, A):
                    self.records.append({"step": n, "label": name, **sv_quantiles(B)})
        if quant_now:
            with open(os.path.join(self.out_dir, "quantiles.json"), "w") as f:
                json.dump(self.records, f)
        return None

    def _after_step(self, optimizer, args, kwargs):
        self._depth = max(0, self._depth - 1)


_INSTALLED = [False]


def install():
    """Make every Muon constructed from now on carry a SpectraCollector (idempotent):
    the drop-in for spectra/collect.py's install(), with the same environment
    variables and outputs.  Only the constructor is wrapped (to see the parameter
    names); the collection itself runs as an optimizer step pre-hook."""
    if _INSTALLED[0]:
        return
    _INSTALLED[0] = True
    from defmuon_amd.optim.muon import Muon

    base_init = Muon.__init__

    def init_and_attach(self, named_params, *args, **kwargs):
        named = list(named_params)                  # the constructor consumes it too
        base_init(self, named, *args, **kwargs)
        col = SpectraCollector.from_env(named)
        self._spectra = col
        if col is not None:
            col.attach(self)
            if col.writer:
                print(f"[spectra] tracking {[l for l, _ in col.targets]} -> {col.out_dir} "
                      f"(dump at {sorted(col.dump_steps)}, quantiles every {col.qstep} steps)")

    Muon.__init__ = init_and_attach
