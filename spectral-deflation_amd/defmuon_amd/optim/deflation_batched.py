"""Batched, gated randomized-SVD deflation front-end and the deflated arms, on the
HIP C-ABI library.

Drop-in for defmuon/optim/deflation_batched.py.  For a tall momentum batch
A (B, n, m), n >= m (deflation_batched.py:1-27):

    W   = A - U_k S_k V_k^T          remove the leading outlier directions
    X0  = W / (||W||_F + 1e-7)       Frobenius entry on the remainder
    X0 += U_k (1/pad) V_k^T          restore the head at height 1/pad

with (U, s, V) from a Gaussian-sketch subspace iteration (CholeskyQR with an fp64
Gram, Rayleigh-Ritz) and a gate that declines matrices without outlier
structure (X0 = A / (||A||_F + 1e-7) there).  The sketch is drawn here with
torch.randn from the caller's generator, exactly as the reference draws it
(deflation_batched.py:172-174), so the random stream is torch's; everything
after the sketch runs in the library on the current stream with no host sync.

Module-level names, environment variables and defaults match the reference
(deflation_batched.py:42-110) so logs and ablation scripts keep working.

Behaviour the reference leaves undefined: a rank-deficient sketch Gram (e.g. an
all-zero momentum) makes the reference's cholesky_ex fail silently and its
output non-finite.  Here such a matrix is declined by the gate (k = 0) and gets
the plain entry A / (||A||_F + 1e-7), which is finite.
"""

import math
import os

import torch

from defmuon_amd import _native

# ---------------------------------------------------------------------------
# deflation constants (deflation_batched.py:42-59; same env names and defaults)
# ---------------------------------------------------------------------------
DIVISOR_PAD = float(os.environ.get("DEFMUON_DEFL_PAD", "1.01"))
RSVD_NITER = int(os.environ.get("DEFMUON_DEFL_NITER", "1"))
CHOLQR_PASSES = int(os.environ.get("DEFMUON_DEFL_QR_PASSES", "1"))
GRAM_DTYPE = torch.float64
GATE_WINDOW = float(os.environ.get("DEFMUON_DEFL_WINDOW", "0.025"))
SKETCH_FRAC = float(os.environ.get("DEFMUON_DEFL_SKETCH", str(GATE_WINDOW)))
OVERSAMPLE_FRAC = float(os.environ.get("DEFMUON_DEFL_OS", "0.025"))
GATE_RATIO = float(os.environ.get("DEFMUON_DEFL_RATIO", "0.10"))
DEFLATE_THRESH = float(os.environ.get("DEFMUON_DEFL_THRESH", str(GATE_RATIO)))

# gate statistics: device int64[3] (total, fired, k_sum) ticked by the optimizer
_GATE_ACC = [None]
_DEGENERATE = [0]
_PARACHUTE = [0]

# optional per-call timing, clip vs iteration (DEFMUON_TIME_POLAR=1)
_TIMING = {"clip_ms": 0.0, "iter_ms": 0.0, "calls": 0}
_PENDING = []
_TIMING_ON = [bool(int(os.environ.get("DEFMUON_TIME_POLAR", "0")))]


def enable_polar_timing(on=True):
    _TIMING_ON[0] = bool(on)


def flush_timings():
    """Drain recorded events into the accumulator.  Call only after a sync."""
    if not _PENDING:
        return
    for e0, e1, e2 in _PENDING:
        _TIMING["clip_ms"] += e0.elapsed_time(e1)
        _TIMING["iter_ms"] += e1.elapsed_time(e2)
        _TIMING["calls"] += 1
    _PENDING.clear()


def timing_stats(reset=True):
    """(clip_ms, iter_ms, calls) accumulated since the last reset."""
    flush_timings()
    out = dict(_TIMING)
    if reset:
        _TIMING.update(clip_ms=0.0, iter_ms=0.0, calls=0)
    return out


def polar_stats():
    """Gate firing rate and mean deflation width; the one host read of the
    device-side accumulator."""
    if _GATE_ACC[0] is not None:
        total, fired, k_sum = _GATE_ACC[0].tolist()
    else:
        total = fired = k_sum = 0
    return dict(fired=fired, total=total, k_mean=(k_sum / max(fired, 1)),
                degenerate=_DEGENERATE[0], parachute=_PARACHUTE[0])


# ---------------------------------------------------------------------------
# batched randomized SVD (library kernels)
# ---------------------------------------------------------------------------

def sketch_dims(m):
    """(r, kw): sketch width and gate window (deflation_batched.py:170-171)."""
    r = min(int(math.ceil(SKETCH_FRAC * m)) + int(math.ceil(OVERSAMPLE_FRAC * m)), m)
    kw = min(max(1, int(math.ceil(GATE_WINDOW * m))), r)
    return r, kw


def _orth_b(X):
    """Batched CholeskyQR (CHOLQR_PASSES passes): X (B, n, r) -> Q."""
    return _native.orth(X, CHOLQR_PASSES)


def _project_b(Q, A):
    """Batched Rayleigh-Ritz: U = Q Ub, s, V from the thin SVD of Q^T A."""
    return _native.project(Q, A)


def _rsvd_b(A, Omega, n_iter):
    """Batched subspace iteration with `n_iter` power steps, then Rayleigh-Ritz."""
    return _native.rsvd(A, Omega, n_iter, CHOLQR_PASSES)


# ---------------------------------------------------------------------------
# the deflation front-end (batched remove-then-restore), fp32
# ---------------------------------------------------------------------------

def batched_rmfro_clip(A, generator=None, Omega=None, out_dtype=None, pad=DIVISOR_PAD):
    """Remove-then-restore deflation for a batch A (B, n, m), n >= m.

    Returns (X0, k (B,) int64, d (B,) fp32): the deflation entry, the deflation
    width (0 where the gate declined) and the Frobenius divisor used."""
    Bn, n, m = A.shape
    r, kw = sketch_dims(m)
    if Omega is None:
        Omega = torch.randn(Bn, m, r, device=A.device, dtype=A.dtype, generator=generator)
    if r > _native.MAX_SKETCH:
        raise _native.NativeError(f"sketch width r={r} exceeds the library's {_native.MAX_SKETCH}")
    return _native.rmfro_clip(A, Omega, kw, GATE_RATIO, DEFLATE_THRESH, pad, RSVD_NITER,
                              CHOLQR_PASSES, out_dtype)


# ---------------------------------------------------------------------------
# the deflated arms: the setup above, plus a per-arm pad and bf16 iteration
# ---------------------------------------------------------------------------

def _horner_iterate(X, hs):
    """X <- aX + bX^3 + cX^5 per (a, b, c) in hs, tall convention
    (G = X^T X, X <- aX + X(bG + cG^2)), on a (B, n, m) or (n, m) batch in one
    grouped launch per GEMM phase, in X's dtype (deflation_batched.py:196-204):
    bf16 through the bf16 MFMA chain (the training path), fp32 through the fp32
    chain (the reference's convergence study runs this function in fp32).  Other
    dtypes raise NativeError."""
    squeeze = X.ndim == 2
    Xb = X[None] if squeeze else X
    hs = [tuple(h) for h in hs]
    if X.dtype == torch.bfloat16:
        out = _native.ns_chain(Xb, True, 0, hs)
    elif X.dtype == torch.float32:
        out = _native.horner_f32(Xb, hs)
    else:
        raise _native.NativeError(f"_horner_iterate: {X.dtype} input is not supported "
                                  "(bf16 or fp32)")
    return out[0] if squeeze else out


class _DeflatedPolarBase:
    """A deflated arm: the batched fp32 setup, then a subclass-chosen bf16
    iteration.  Subclasses supply `_iterate` (and, for the fused path,
    `schedule`)."""
    PAD = DIVISOR_PAD
    BATCHED_CLIP = staticmethod(batched_rmfro_clip)

    def _iterate(self, X, steps):
        raise NotImplementedError

    def schedule(self, steps):
        """The (a, b, c) triples `_iterate` applies, or None if unknown."""
        return None

    def _fused(self, steps):
        """The schedule when this arm's clip and iteration are the library's own
        (so both can run as one library call), else None."""
        cls = type(self)
        hs = self.schedule(steps)
        if (hs is not None and cls.BATCHED_CLIP is _DeflatedPolarBase.BATCHED_CLIP
                and cls._iterate in (DeflatedNSPolar._iterate, DeflatedPEPolar._iterate)):
            return hs
        return None

    def polar_group(self, A, generator=None, steps=5, Omega=None, chain_event=None):
        """BATCHED_CLIP(A, bf16) then `_iterate` for one tall shape group, as
        muon.py:298,310-312 run them.  For the built-in arms both run in one
        library call (dmh_deflated_polar) that hands X0 to the chain in its packed
        layout; an arm that overrides BATCHED_CLIP or `_iterate` gets exactly its
        own two calls.  Returns (polar factors (B, n, m) bf16, k, d).  chain_event
        (fused path only): a torch.cuda.Event recorded between the two phases."""
        hs = self._fused(steps)
        if hs is None:
            X0, k, d = self.BATCHED_CLIP(A, generator=generator, Omega=Omega, pad=self.PAD,
                                         out_dtype=torch.bfloat16)
            return self._iterate(X0, steps), k, d
        Bn, n, m = A.shape
        r, kw = sketch_dims(m)
        if Omega is None:
            Omega = torch.randn(Bn, m, r, device=A.device, dtype=A.dtype, generator=generator)
        return _native.deflated_polar(A, Omega, kw, GATE_RATIO, DEFLATE_THRESH, self.PAD, hs,
                                      RSVD_NITER, CHOLQR_PASSES, chain_event)

    def polar_groups(self, As, generators, steps=5, chain_events=None, chain_window=None):
        """polar_group over the tall shape groups of one optimizer step, with one
        generator per group; returns [(polar factors, k, d)] in group order.

        For the built-in arms every group runs on a stream of its own, its chain right
        after its front-end: the front-ends are chains of small latency-bound launches
        that alone leave most of the GPU idle, and the GEMM launches of one group's
        chain leave partial last rounds of tiles that the other group's work fills.
        With chain_events (a list of (start, end) torch.cuda.Event pairs, one per group)
        the chains instead run one after the other on the current stream once every
        front-end has finished, with pair g recorded around group g's chain, so that
        the chains' time can be measured alone.  With chain_window (one (start, end)
        pair) every front-end finishes first, then the chains run together, each on
        its group's stream, with start recorded on the current stream before them and
        end after all of them: the time of the chain phase of the step with the
        groups' chains overlapping each other but no front-end.  Every group's sketch
        comes from its own generator and every result equals that of a polar_group
        call."""
        hs = self._fused(steps)
        if hs is None or len(As) < 2 or not As[0].is_cuda:
            # one group after the other (an arm with its own clip or iteration: the
            # start event then marks the start of the group, not of its chain)
            outs = []
            for gi, (A, gen) in enumerate(zip(As, generators)):
                ev = chain_events[gi] if chain_events else None
                if ev is not None:
                    ev[0].record()   # creates the HIP event; the fused call re-records it
                outs.append(self.polar_group(A, generator=gen, steps=steps,
                                             chain_event=ev[0] if ev is not None else None))
                if ev is not None:
                    ev[1].record()
            return outs
        dev = As[0].device
        main = torch.cuda.current_stream(dev)
        side = _side_streams(dev, len(As))
        concurrent_chains = not chain_events and chain_window is None
        # the largest group (the critical path) is enqueued first
        order = sorted(range(len(As)), key=lambda gi: -As[gi].numel())
        fronts = [None] * len(As)
        outs = [None] * len(As)
        for s, gi in zip(side, order):
            A, gen = As[gi], generators[gi]
            s.wait_stream(main)
            with torch.cuda.stream(s):
                Bn, n, m = A.shape
                r, kw = sketch_dims(m)
                Omega = torch.randn(Bn, m, r, device=dev, dtype=A.dtype, generator=gen)
                fr = _native.deflated_polar_front(A, Omega, kw, GATE_RATIO, DEFLATE_THRESH,
                                                  self.PAD, RSVD_NITER, CHOLQR_PASSES)
                if concurrent_chains:
                    U = _native.deflated_polar_chain(fr, hs)
                    U.record_stream(main)
                    outs[gi] = (U, fr.k, fr.d)
            A.record_stream(s)
            for t in (fr.ws, fr.k, fr.d):
                t.record_stream(main)
            fronts[gi] = fr
        for s in side:
            main.wait_stream(s)
        if concurrent_chains:
            return outs
        if chain_window is not None:
            chain_window[0].record(main)
            for s, gi in zip(side, order):
                s.wait_stream(main)
                with torch.cuda.stream(s):
                    U = _native.deflated_polar_chain(fronts[gi], hs)
                U.record_stream(main)
                outs[gi] = (U, fronts[gi].k, fronts[gi].d)
            for s in side:
                main.wait_stream(s)
            chain_window[1].record(main)
            return outs
        for gi, fr in enumerate(fronts):
            ev = chain_events[gi]
            ev[0].record(main)
            U = _native.deflated_polar_chain(fr, hs)
            ev[1].record(main)
            outs[gi] = (U, fr.k, fr.d)
        return outs


_SIDE_STREAMS = {}


def _side_streams(device, count):
    """`count` streams of `device` for concurrent group front-ends (created once,
    default priority)."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    lst = _SIDE_STREAMS.setdefault(key, [])
    while len(lst) < count:
        lst.append(torch.cuda.Stream(device=device))
    return lst[:count]


class DeflatedNSPolar(_DeflatedPolarBase):
    """The standard Newton-Schulz quintic behind the deflation."""
    NS_ABC = (3.4445, -4.7750, 2.0315)

    def schedule(self, steps):
        return [self.NS_ABC] * steps

    def _iterate(self, X, steps):
        return _horner_iterate(X, [self.NS_ABC] * steps)


class DeflatedPEPolar(_DeflatedPolarBase):
    """The Polar Express schedule behind the deflation; PAD defaults to 1.1
    (DEFMUON_DEFL_PE_PAD)."""
    PAD = float(os.environ.get("DEFMUON_DEFL_PE_PAD", "1.1"))

    def schedule(self, steps):
        from defmuon_amd.optim.polar_express import pe_schedule
        return pe_schedule(steps)

    def _iterate(self, X, steps):
        from defmuon_amd.optim.polar_express import pe_schedule
        return _horner_iterate(X, pe_schedule(steps))
