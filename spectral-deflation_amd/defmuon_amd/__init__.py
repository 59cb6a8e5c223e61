"""MI355X-native polar-factor path of deflated Muon.

Mirrors the reference package layout (defmuon.optim.{muon, polar_express,
deflation_batched, deflation_cutoff}) under defmuon_amd.optim; the numerical work
runs in the HIP C-ABI library loaded by defmuon_amd._native.
"""
