"""Momentum dumps and the accuracy harness of the deflated polar path.

Drop-in for the reference's spectra tooling on the hot path's data:
  dumps     the dump format of spectra/collect.py (one torch.save per optimizer step and
            matrix), its loader (spectra/polar_convergence.py:117-137) and the collector
            that writes dumps and singular-value quantiles from a training run
  accuracy  the rSVD head accuracy study (spectra/rsvd_accuracy.py) and the polar-factor
            convergence study (spectra/polar_convergence.py) run through this library's
            kernels, writing the reference's CSV columns

Run as `python -m defmuon_amd.spectra {rsvd,convergence} --dumps DIR --out DIR`.
"""
