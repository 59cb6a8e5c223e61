"""Momentum dumps in the reference's format (spectra/collect.py).

A dump is one file per (optimizer step, matrix), `step{step:04d}_{label}.pt`, holding
torch.save({"step", "label", "A", "momentum", "nesterov"}) (collect.py:109-113).  "A" is
the fp32 post-Nesterov matrix the polar factorizer consumes that step, computed out of
place before the step updates the momentum buffer (collect.py:89-97).  Labels are
attn_qkv (the whole c_attn weight; its row blocks are the Q, K and V matrices), attn_o,
mlp_fc and mlp_proj of the middle layer.

Dumps are read with torch.load(weights_only=True): a dump holds tensors and plain
Python scalars only, so nothing in the file is executed.
"""

import glob
import json
import os
import re

import torch

# the six matrices Muon projects, each with its own Frobenius entry (plot_spectra.py:76)
PANEL_COLS = ["attn_q", "attn_k", "attn_v", "attn_o", "mlp_fc", "mlp_proj"]
ROW_NAME = {"attn_q": "Attn $Q$", "attn_k": "Attn $K$", "attn_v": "Attn $V$",
            "attn_qkv": "Attn $QKV$", "attn_o": "Attn $O$",
            "mlp_fc": "MLP in", "mlp_proj": "MLP out"}           # plot_spectra.py:68-70
QUANTILES = (0.1, 0.25, 0.5, 0.75, 0.9)                           # collect.py:43


def momentum_A(grad, buf, momentum, nesterov):
    """The matrix the factorizer consumes this step, out of place (collect.py:89-97):
    buf' = momentum * buf + grad (grad where there is no buffer yet);
    A = grad + momentum * buf' with Nesterov, else buf'."""
    g32 = grad.float()
    newbuf = g32 if buf is None else buf.float().mul(momentum).add_(g32)
    return g32 + momentum * newbuf if nesterov else newbuf


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
    """{step: {label: A}} with A a tall (n >= m) contiguous fp32 CPU tensor, as
    polar_convergence.py:117-137 builds it: the attn_qkv dump is cut by rows into
    attn_q / attn_k / attn_v (E rows each, E = its column count), wide matrices are
    transposed, and only the labels of PANEL_COLS are kept."""
    out = {}
    for path in sorted(glob.glob(os.path.join(dump_dir, "step*_*.pt"))):
        d = load_dump(path)
        A = d["A"].float()
        step, lbl = int(d["step"]), d["label"]
        ent = out.setdefault(step, {})
        blocks = {lbl: A}
        if lbl == "attn_qkv":                       # rows: Q | K | V
            E = A.shape[1]
            blocks = {sub: A[i * E:(i + 1) * E]
                      for i, sub in enumerate(["attn_q", "attn_k", "attn_v"])}
        for name, M in blocks.items():
            if name in PANEL_COLS:
                ent[name] = (M.mT if M.shape[0] < M.shape[1] else M).contiguous()
    return out


def sv_quantiles(B, quantiles=QUANTILES):
    """Singular-value quantiles of one matrix, normalised by its Frobenius norm, as
    collect.py:127-135 records them: the ceil(q r)-th largest singular value."""
    fro = B.norm().item()
    s = torch.linalg.svdvals(B.float())
    r = s.numel()
    qv = {str(q): (s[min(int(-(-q * r // 1)), r) - 1] / (fro + 1e-30)).item()
          for q in quantiles}
    return {"fro": fro, "sigma_max": s[0].item(), "q": qv}


# ---------------------------------------------------------------------------
# collector (spectra/collect.py:46-143): patches Muon so that chosen optimizer steps
# dump the middle layer's post-Nesterov matrices and every QSTEP steps record their
# singular-value quantiles; the training run itself is unchanged
# ---------------------------------------------------------------------------

_INSTALLED = [False]
_EMBD_TAG = {1280: "gpt-large"}


def _config():
    return (os.environ.get("DEFMUON_SPECTRA_DIR", "spectra/dumps"),
            {int(s) for s in os.environ.get("DEFMUON_SPECTRA_STEPS", "1,500,1000,1500").split(",")},
            int(os.environ.get("DEFMUON_SPECTRA_QSTEP", "10")))


def _master():
    return int(os.environ.get("RANK", "0") or 0) <= 0


def install():
    """Patch defmuon_amd.optim.muon.Muon to collect spectra (idempotent).  Environment:
    DEFMUON_SPECTRA_DIR, DEFMUON_SPECTRA_TAG, DEFMUON_SPECTRA_STEPS,
    DEFMUON_SPECTRA_QSTEP, as collect.py reads them."""
    if _INSTALLED[0]:
        return
    _INSTALLED[0] = True
    from defmuon_amd.optim.muon import Muon

    orig_init = Muon.__init__
    orig_step = Muon.step

    def init_with_capture(self, named_params, *args, **kwargs):
        named = list(named_params)
        orig_init(self, named, *args, **kwargs)
        spectra_dir, dump_steps, qstep = _config()
        self._spectra_steps, self._spectra_qstep = dump_steps, qstep
        layers = [int(m.group(1)) for name, _ in named
                  for m in [re.search(r"\.h\.(\d+)\.", name)] if m]
        if not layers:
            self._spectra_targets = []
            return
        mid = (max(layers) + 1) // 2
        suffixes = {f"h.{mid}.attn.c_attn.weight": "attn_qkv",
                    f"h.{mid}.attn.c_proj.weight": "attn_o",
                    f"h.{mid}.mlp.c_fc.weight": "mlp_fc",
                    f"h.{mid}.mlp.c_proj.weight": "mlp_proj"}
        self._spectra_targets = [(lbl, p) for name, p in named
                                 for sfx, lbl in suffixes.items() if name.endswith(sfx)]
        if not self._spectra_targets:
            return
        n_embd = min(min(p.shape) for _, p in self._spectra_targets)
        tag = os.environ.get("DEFMUON_SPECTRA_TAG") or _EMBD_TAG.get(n_embd, f"nembd{n_embd}")
        self._spectra_out = os.path.join(spectra_dir, tag)
        self._spectra_qrecs = []
        if _master():
            os.makedirs(self._spectra_out, exist_ok=True)

    def _A(self, p):
        group = next(g for g in self.param_groups if any(q is p for q in g["params"]))
        return momentum_A(p.grad, self.state[p].get("momentum_buffer"), group["momentum"],
                          group["nesterov"])

    def step_with_spectra(self, closure=None):
        n = getattr(self, "_spectra_n", 0) + 1      # this call = optimizer step n
        self._spectra_n = n
        targets = getattr(self, "_spectra_targets", None)
        if _master() and targets:
            if n in self._spectra_steps:
                for lbl, p in targets:
                    if p.grad is not None:
                        save_dump(self._spectra_out, n, lbl, _A(self, p),
                                  self.defaults["momentum"], self.defaults["nesterov"])
            if self._spectra_qstep and n % self._spectra_qstep == 0:
                for lbl, p in targets:
                    if p.grad is None:
                        continue
                    A = _A(self, p)
                    if lbl == "attn_qkv":
                        E = A.shape[1]
                        blocks = [("attn_q", A[:E]), ("attn_k", A[E:2 * E]), ("attn_v", A[2 * E:])]
                    else:
                        blocks = [(lbl, A)]
                    for bl, B in blocks:
                        rec = sv_quantiles(B)
                        self._spectra_qrecs.append({"step": n, "label": bl, **rec})
                with open(os.path.join(self._spectra_out, "quantiles.json"), "w") as f:
                    json.dump(self._spectra_qrecs, f)
        return orig_step(self, closure)

    Muon.__init__ = init_with_capture
    Muon.step = step_with_spectra
