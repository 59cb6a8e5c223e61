"""Deflated Muon arms with an optional early-stage cutoff.

Drop-in for defmuon/optim/deflation_cutoff.py.  `install()` adds the arm names
"deflated_ns_cut" and "deflated_pe_cut" to Muon by wrapping
Muon._initialize_polar_factorizer and Muon.step (deflation_cutoff.py:46-112).
With DEFMUON_DEFL_CUTOFF=N set, the optimizer hard-switches to the plain arm
(ns5 / polarexpress) after N steps; unset (the default) it never switches.
"""

import os

import torch

from defmuon_amd.optim.deflation_batched import DeflatedNSPolar, DeflatedPEPolar

_env = os.environ.get("DEFMUON_DEFL_CUTOFF")
CUTOFF_STEPS = int(_env) if _env else None
_INSTALLED = [False]


class CutoffDeflatedNSPolar(DeflatedNSPolar):
    """deflated_ns; the class marks the arm for the step-counter switch."""
    IS_CUTOFF_ARM = True
    POST = "ns5"


class CutoffDeflatedPEPolar(DeflatedPEPolar):
    """Deflated Polar Express; switches to plain PolarExpress at the cutoff."""
    IS_CUTOFF_ARM = True
    POST = "polarexpress"


ARMS = {"deflated_ns_cut": CutoffDeflatedNSPolar, "deflated_pe_cut": CutoffDeflatedPEPolar}


def install():
    if _INSTALLED[0]:
        return
    _INSTALLED[0] = True
    from defmuon_amd.optim.muon import Muon, zeropower_via_newtonschulz5
    from defmuon_amd.optim.polar_express import PolarExpress

    post_fns = {"ns5": zeropower_via_newtonschulz5, "polarexpress": PolarExpress}
    orig_init = Muon._initialize_polar_factorizer

    def warm_post(muon, post):
        """Run the post-cutoff factorizer once per shape at construction (zeros:
        the global RNG stays untouched)."""
        fn = post_fns[post]
        steps = muon.defaults["ns_steps"]
        seen = set()
        for group in muon.param_groups:
            for p in group["params"]:
                if not muon.state[p].get("use_muon"):
                    continue
                shape = tuple(muon._qkv_split(p, p).shape)
                key = (shape, p.dtype, p.device)
                if key not in seen:
                    seen.add(key)
                    fn(torch.zeros(shape, dtype=p.dtype, device=p.device), steps)
        print(f"[deflation_cutoff] warmed {post} for {len(seen)} shapes")

    def init_with_cutoff(self, polar_method, polar_args):
        arm = ARMS.get(polar_method)
        if arm is None:
            return orig_init(self, polar_method, polar_args)
        if CUTOFF_STEPS is None:
            print("[deflation_cutoff] no cutoff set: deflation on for the whole run")
            return arm()
        try:
            warm_post(self, arm.POST)
        except Exception as e:
            print(f"[deflation_cutoff] {arm.POST} warm-up failed ({e}); "
                  f"the switch step pays the first-call cost instead")
        return arm()

    Muon._initialize_polar_factorizer = init_with_cutoff
    orig_step = Muon.step

    def step_with_cutoff(self, closure=None):
        n = getattr(self, "_cut_steps", 0)
        if (CUTOFF_STEPS is not None and n == CUTOFF_STEPS
                and getattr(self.polar_factorizer, "IS_CUTOFF_ARM", False)):
            post = self.polar_factorizer.POST
            self.batched_deflation = False
            self.polar_factorizer = post_fns[post]
            print(f"[deflation_cutoff] optimizer step {n}: deflation OFF -> plain {post}")
        out = orig_step(self, closure)
        self._cut_steps = n + 1
        return out

    Muon.step = step_with_cutoff
