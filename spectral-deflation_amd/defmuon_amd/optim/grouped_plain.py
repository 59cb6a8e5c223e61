"""Grouped launches for the plain polar arms ("ns5", "polarexpress").

The reference's plain Muon step calls the factorizer once per parameter
(muon.py:361-386): at GPT-2 sizes that is a stream of small, occupancy-bound
launches.  `install()` switches Muon to one library launch per (matrix shape,
dtype, orientation), the way deflation_cutoff.install() (deflation_cutoff.py:46-112)
changes Muon's behaviour from outside; every parameter's update is unchanged
(Muon._muon_step_plain_grouped).  The deflated arms batch by shape already.
"""

_INSTALLED = [False]


def install():
    """Enable the grouped plain-arm step for every Muon instance (idempotent)."""
    if _INSTALLED[0]:
        return
    _INSTALLED[0] = True
    from defmuon_amd.optim.muon import Muon
    Muon.GROUPED_PLAIN = True


def uninstall():
    """Back to one factorizer call per parameter (the reference's loop)."""
    from defmuon_amd.optim.muon import Muon
    Muon.GROUPED_PLAIN = False
    _INSTALLED[0] = False
