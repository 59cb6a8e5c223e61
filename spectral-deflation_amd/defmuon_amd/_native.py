"""ctypes binding of the HIP C-ABI library (include/defmuon_hip.h).

The library is the only compute path: if it is missing, or no GPU is visible,
every entry point raises.  There is no CPU fallback.

Device memory comes from torch's caching allocator (outputs and workspaces are
plain torch tensors); kernels are enqueued on torch's current HIP stream and
nothing here synchronises.
"""

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libdefmuon_hip.so")

_lib = None

c_int, c_ll, c_sz, c_vp, c_float = (ctypes.c_int, ctypes.c_longlong, ctypes.c_size_t,
                                    ctypes.c_void_p, ctypes.c_float)

# name -> (restype, argtypes)
_SIGS = {
    "dmh_last_error": (ctypes.c_char_p, []),
    "dmh_ns_workspace_size": (c_int, [c_int, c_int, c_int, c_int, ctypes.POINTER(c_sz)]),
    "dmh_ns_chain": (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_int, c_ll, c_ll, c_ll, c_vp,
                             c_int, c_int, ctypes.POINTER(ctypes.c_double), c_int, c_vp, c_sz]),
    "dmh_ns_chain_noalloc": (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_int, c_ll, c_ll, c_ll,
                                     c_vp, c_int, c_int, ctypes.POINTER(ctypes.c_double),
                                     c_int]),
    "dmh_horner_f32_workspace_size": (c_int, [c_int, c_int, c_int, ctypes.POINTER(c_sz)]),
    "dmh_horner_f32": (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_vp,
                               ctypes.POINTER(ctypes.c_double), c_int, c_vp, c_sz]),
    "dmh_rsvd_workspace_size": (c_int, [c_int, c_int, c_int, c_int, ctypes.POINTER(c_sz)]),
    "dmh_rmfro_workspace_size": (c_int, [c_int, c_int, c_int, c_int, ctypes.POINTER(c_sz)]),
    "dmh_orth": (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_int, c_vp, c_vp, c_sz]),
    "dmh_project": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_vp, c_vp, c_vp,
                            c_vp, c_sz]),
    "dmh_rsvd": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_vp, c_vp,
                         c_vp, c_vp, c_sz]),
    "dmh_rmfro_clip": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_float,
                               c_float, c_float, c_int, c_int, c_vp, c_int, c_vp, c_vp, c_vp,
                               c_sz]),
    "dmh_deflated_polar_workspace_size": (c_int, [c_int, c_int, c_int, c_int,
                                                  ctypes.POINTER(c_sz)]),
    "dmh_deflated_polar": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_float,
                                   c_float, c_float, c_int, c_int,
                                   ctypes.POINTER(ctypes.c_double), c_int, c_vp, c_vp, c_vp,
                                   c_vp, c_sz, c_vp]),
    "dmh_deflated_polar_front": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int,
                                         c_float, c_float, c_float, c_int, c_int, c_vp, c_vp,
                                         c_vp, c_sz]),
    "dmh_deflated_polar_chain": (c_int, [c_vp, c_int, c_int, c_int,
                                         ctypes.POINTER(ctypes.c_double), c_int, c_vp, c_vp,
                                         c_sz]),
    "dmh_momentum_stack": (c_int, [c_vp, c_vp, c_int, c_float, c_int, c_vp]),
    "dmh_apply_update": (c_int, [c_vp, c_vp, c_int, c_vp]),
    "dmh_adamw_chunks": (c_int, [c_ll]),
    "dmh_adamw_step": (c_int, [c_vp, c_vp, c_int, c_vp, c_int, c_float, c_float, c_float,
                               c_float, c_float]),
}


class GlueParam(ctypes.Structure):
    """dmh_glue_param (include/defmuon_hip.h)."""
    _fields_ = [("grad", c_vp), ("momentum", c_vp), ("param", c_vp), ("rows", c_int),
                ("cols", c_int), ("blocks", c_int), ("transpose", c_int),
                ("offset", c_ll), ("alpha", c_float), ("decay", c_float)]

# largest sketch width the front-end kernels carry (include/defmuon_hip.h)
MAX_SKETCH = 64

EXPORTS = tuple(_SIGS)


class NativeError(RuntimeError):
    pass


def load(path=None):
    """Load (once) and return the library handle (from `path`, else the module's
    LIB_PATH as it is at the first call)."""
    global _lib
    if _lib is not None:
        return _lib
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise NativeError(
            f"HIP library not built: {path} is missing.  Build it with "
            "`python spectral-deflation_amd/build.py` (or __graft_entry__.build()).")
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _check(rc, what):
    if rc != 0:
        msg = load().dmh_last_error().decode(errors="replace")
        raise NativeError(f"{what} failed (status {rc}): {msg}")


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_gpu(t, what):
    if not t.is_cuda:
        raise NativeError(f"{what}: the HIP path needs a GPU tensor (got {t.device})")


def _workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def ns_chain(X, orient_tall, entry_mode, coeffs, out=None):
    """Run the bf16 polynomial chain on a (batch, rows, cols) stack.

    orient_tall: the input is the tall operand T of the tall convention
        (G = X^T X, X <- aX + XB); otherwise it is the wide W (A = X X^T,
        X <- aX + BX).
    entry_mode: 0 none (input already normalised), 1 divide by ||X||_F + 1e-7,
        2 divide by 1.01 ||X||_F + 1e-7 (norm over the un-rounded input).
    coeffs: list of (a, b, c) triples, one per step.
    Returns a contiguous bf16 tensor of the input's shape.
    """
    _require_gpu(X, "ns_chain")
    if X.ndim != 3:
        raise NativeError(f"ns_chain expects (batch, rows, cols), got {tuple(X.shape)}")
    if X.dtype not in (torch.float32, torch.bfloat16):
        X = X.float()
    lib = load()
    B, R, C = X.shape
    if out is None:
        out = torch.empty((B, R, C), dtype=torch.bfloat16, device=X.device)
    if B == 0:
        return out
    steps = len(coeffs)
    flat = (ctypes.c_double * max(3 * steps, 1))(*[float(v) for t in coeffs for v in t])
    nbytes = c_sz()
    _check(lib.dmh_ns_workspace_size(B, R, C, int(bool(orient_tall)), ctypes.byref(nbytes)),
           "dmh_ns_workspace_size")
    ws = _workspace(nbytes.value, X.device)
    bs, rs, cs = X.stride()
    rc = lib.dmh_ns_chain(_stream(X.device), c_vp(X.data_ptr()), 0 if X.dtype == torch.float32 else 1,
                          B, R, C, bs, rs, cs, c_vp(out.data_ptr()), int(bool(orient_tall)),
                          int(entry_mode), flat, steps, c_vp(ws.data_ptr()), nbytes.value)
    _check(rc, "dmh_ns_chain")
    return out


def _ptr(t):
    return c_vp(t.data_ptr())


def horner_f32(X, coeffs):
    """The tall-convention chain in fp32 on a (batch, n, m) stack: per (a, b, c),
    G = X^T X, B = bG + (cG)G, X <- aX + XB.  Returns a new fp32 tensor."""
    _require_gpu(X, "horner_f32")
    if X.ndim != 3:
        raise NativeError(f"horner_f32 expects (batch, n, m), got {tuple(X.shape)}")
    X = X.float().contiguous()
    B, n, m = X.shape
    out = torch.empty_like(X)
    if B == 0:
        return out
    lib = load()
    nbytes = c_sz()
    _check(lib.dmh_horner_f32_workspace_size(B, n, m, ctypes.byref(nbytes)),
           "dmh_horner_f32_workspace_size")
    ws = _workspace(nbytes.value, X.device)
    steps = len(coeffs)
    flat = (ctypes.c_double * max(3 * steps, 1))(*[float(v) for t in coeffs for v in t])
    _check(lib.dmh_horner_f32(_stream(X.device), _ptr(X), B, n, m, _ptr(out), flat, steps,
                              _ptr(ws), nbytes.value), "dmh_horner_f32")
    return out


def _f32c(t, what):
    _require_gpu(t, what)
    return t.contiguous() if t.dtype == torch.float32 else t.float().contiguous()


def _rsvd_ws(B, n, m, r, device):
    nbytes = c_sz()
    _check(load().dmh_rsvd_workspace_size(B, n, m, r, ctypes.byref(nbytes)),
           "dmh_rsvd_workspace_size")
    return _workspace(nbytes.value, device), nbytes.value


def orth(X, passes=1):
    """Batched CholeskyQR of X (B, rows, r) fp32 -> Q (B, rows, r)."""
    X = _f32c(X, "orth")
    B, rows, r = X.shape
    Q = torch.empty_like(X)
    if B == 0:
        return Q
    ws, nb = _rsvd_ws(B, rows, r, r, X.device)
    _check(load().dmh_orth(_stream(X.device), _ptr(X), B, rows, r, int(passes), _ptr(Q),
                           _ptr(ws), nb), "dmh_orth")
    return Q


def project(Q, A):
    """Rayleigh-Ritz: thin SVD of Q^T A.  Q (B, n, r), A (B, n, m) fp32 ->
    U (B, n, r), s (B, r) descending, V (B, m, r)."""
    Q, A = _f32c(Q, "project"), _f32c(A, "project")
    B, n, m = A.shape
    r = Q.shape[-1]
    U = torch.empty((B, n, r), dtype=torch.float32, device=A.device)
    s = torch.empty((B, r), dtype=torch.float32, device=A.device)
    V = torch.empty((B, m, r), dtype=torch.float32, device=A.device)
    if B == 0:
        return U, s, V
    ws, nb = _rsvd_ws(B, n, m, r, A.device)
    _check(load().dmh_project(_stream(A.device), _ptr(Q), _ptr(A), B, n, m, r, _ptr(U), _ptr(s),
                              _ptr(V), _ptr(ws), nb), "dmh_project")
    return U, s, V


def rsvd(A, Omega, niter=1, passes=1):
    """Subspace iteration + Rayleigh-Ritz on A (B, n, m) with sketch Omega (B, m, r)."""
    A, Omega = _f32c(A, "rsvd"), _f32c(Omega, "rsvd")
    B, n, m = A.shape
    r = Omega.shape[-1]
    U = torch.empty((B, n, r), dtype=torch.float32, device=A.device)
    s = torch.empty((B, r), dtype=torch.float32, device=A.device)
    V = torch.empty((B, m, r), dtype=torch.float32, device=A.device)
    if B == 0:
        return U, s, V
    ws, nb = _rsvd_ws(B, n, m, r, A.device)
    _check(load().dmh_rsvd(_stream(A.device), _ptr(A), _ptr(Omega), B, n, m, r, int(niter),
                           int(passes), _ptr(U), _ptr(s), _ptr(V), _ptr(ws), nb), "dmh_rsvd")
    return U, s, V


def rmfro_clip(A, Omega, kw, ratio, thresh, pad, niter=1, passes=1, out_dtype=None):
    """Deflation front-end on A (B, n, m), n >= m: returns (X0, k int64, d fp32).
    X0 is bf16 when out_dtype is torch.bfloat16, else fp32."""
    A, Omega = _f32c(A, "rmfro_clip"), _f32c(Omega, "rmfro_clip")
    B, n, m = A.shape
    r = Omega.shape[-1]
    bf = out_dtype == torch.bfloat16
    X0 = torch.empty((B, n, m), dtype=torch.bfloat16 if bf else torch.float32, device=A.device)
    k = torch.empty((B,), dtype=torch.int64, device=A.device)
    d = torch.empty((B,), dtype=torch.float32, device=A.device)
    if B == 0:
        return X0, k, d
    ws, nb = _rsvd_ws(B, n, m, r, A.device)
    _check(load().dmh_rmfro_clip(_stream(A.device), _ptr(A), _ptr(Omega), B, n, m, r, int(kw),
                                 float(ratio), float(thresh), float(pad), int(niter),
                                 int(passes), _ptr(X0), int(bf), _ptr(k), _ptr(d), _ptr(ws), nb),
           "dmh_rmfro_clip")
    if out_dtype is not None and not bf and out_dtype != torch.float32:
        X0 = X0.to(out_dtype)
    return X0, k, d


def deflated_polar(A, Omega, kw, ratio, thresh, pad, coeffs, niter=1, passes=1,
                   chain_event=None):
    """Front-end + bf16 chain in one call on a tall group A (B, n, m): returns the
    polar factors (B, n, m) bf16, k (B,) int64 and d (B,) fp32.  chain_event: a
    torch.cuda.Event (already recorded once, so that its HIP event exists) that the
    library re-records between the front-end and the chain."""
    A, Omega = _f32c(A, "deflated_polar"), _f32c(Omega, "deflated_polar")
    B, n, m = A.shape
    r = Omega.shape[-1]
    out = torch.empty((B, n, m), dtype=torch.bfloat16, device=A.device)
    k = torch.empty((B,), dtype=torch.int64, device=A.device)
    d = torch.empty((B,), dtype=torch.float32, device=A.device)
    if B == 0:
        return out, k, d
    lib = load()
    nbytes = c_sz()
    _check(lib.dmh_deflated_polar_workspace_size(B, n, m, r, ctypes.byref(nbytes)),
           "dmh_deflated_polar_workspace_size")
    ws = _workspace(nbytes.value, A.device)
    steps = len(coeffs)
    flat = (ctypes.c_double * max(3 * steps, 1))(*[float(v) for t in coeffs for v in t])
    _check(lib.dmh_deflated_polar(_stream(A.device), _ptr(A), _ptr(Omega), B, n, m, r, int(kw),
                                  float(ratio), float(thresh), float(pad), int(niter),
                                  int(passes), flat, steps, _ptr(out), _ptr(k), _ptr(d),
                                  _ptr(ws), nbytes.value,
                                  c_vp(chain_event.cuda_event if chain_event is not None else 0)),
           "dmh_deflated_polar")
    return out, k, d


class PolarFront:
    """A deflated front-end result waiting for its chain: the workspace (holding
    the packed bf16 entry X0), the gate widths k and divisors d, and the shape."""
    __slots__ = ("ws", "nbytes", "k", "d", "shape", "device")

    def __init__(self, ws, nbytes, k, d, shape, device):
        self.ws, self.nbytes, self.k, self.d, self.shape, self.device = ws, nbytes, k, d, shape, device


def deflated_polar_front(A, Omega, kw, ratio, thresh, pad, niter=1, passes=1):
    """Front-end half of deflated_polar on the current stream: returns a
    PolarFront for deflated_polar_chain."""
    A, Omega = _f32c(A, "deflated_polar_front"), _f32c(Omega, "deflated_polar_front")
    B, n, m = A.shape
    r = Omega.shape[-1]
    k = torch.empty((B,), dtype=torch.int64, device=A.device)
    d = torch.empty((B,), dtype=torch.float32, device=A.device)
    lib = load()
    nbytes = c_sz()
    _check(lib.dmh_deflated_polar_workspace_size(B, n, m, r, ctypes.byref(nbytes)),
           "dmh_deflated_polar_workspace_size")
    ws = _workspace(max(nbytes.value, 1), A.device)
    if B:
        _check(lib.dmh_deflated_polar_front(_stream(A.device), _ptr(A), _ptr(Omega), B, n, m, r,
                                            int(kw), float(ratio), float(thresh), float(pad),
                                            int(niter), int(passes), _ptr(k), _ptr(d), _ptr(ws),
                                            nbytes.value),
               "dmh_deflated_polar_front")
    return PolarFront(ws, nbytes.value, k, d, (B, n, m), A.device)


def deflated_polar_chain(front, coeffs):
    """Chain half of deflated_polar on the current stream: the polar factors
    (B, n, m) bf16 from a PolarFront."""
    B, n, m = front.shape
    out = torch.empty((B, n, m), dtype=torch.bfloat16, device=front.device)
    if B == 0:
        return out
    steps = len(coeffs)
    flat = (ctypes.c_double * max(3 * steps, 1))(*[float(v) for t in coeffs for v in t])
    _check(load().dmh_deflated_polar_chain(_stream(front.device), B, n, m, flat, steps,
                                           _ptr(out), _ptr(front.ws), front.nbytes),
           "dmh_deflated_polar_chain")
    return out


def momentum_stack(params, momentum, nesterov, stack):
    """Nesterov momentum of every parameter in place and its tall fp32 blocks into
    `stack` (B, n, m): `params` is a list of GlueParam (grad, momentum, rows, cols,
    blocks, transpose, offset set).  Enqueued on the current stream."""
    arr = (GlueParam * max(len(params), 1))(*params)
    _check(load().dmh_momentum_stack(_stream(stack.device), ctypes.cast(arr, c_vp), len(params),
                                     float(momentum), int(bool(nesterov)), _ptr(stack)),
           "dmh_momentum_stack")


def apply_update(params, ustack):
    """p <- p * decay + alpha * u for every parameter, u read from the bf16 polar
    factors `ustack` (B, n, m) in the stack layout.  Enqueued on the current stream."""
    arr = (GlueParam * max(len(params), 1))(*params)
    _check(load().dmh_apply_update(_stream(ustack.device), ctypes.cast(arr, c_vp), len(params),
                                   _ptr(ustack)),
           "dmh_apply_update")


class AdamwTable:
    """The device-side parameter table and chunk boundaries of dmh_adamw_step for a
    list of (param, grad, moment1, moment2) fp32 tensors.  It holds raw addresses:
    reuse it only for tensors at the same addresses (`key`), in the same order.
    The moments and parameters stay put between steps; gradients that come back at
    the same addresses (torch's caching allocator) keep the table valid, otherwise
    the caller builds a new one."""
    __slots__ = ("key", "table", "chunks", "count", "nchunks")

    def __init__(self, quads):
        lib = load()
        dev = quads[0][0].device
        words, starts, total = [], [0], 0
        for p, g, m1, m2 in quads:
            words += [p.data_ptr(), g.data_ptr(), m1.data_ptr(), m2.data_ptr(), p.numel()]
            total += lib.dmh_adamw_chunks(p.numel())
            starts.append(total)
        self.key = AdamwTable.key_of(quads)
        # pinned staging so the copies are ordered on the stream without a host wait
        self.table = torch.tensor(words, dtype=torch.int64).pin_memory().to(dev, non_blocking=True)
        self.chunks = torch.tensor(starts, dtype=torch.int32).pin_memory().to(dev,
                                                                              non_blocking=True)
        self.count, self.nchunks = len(quads), total

    @staticmethod
    def key_of(quads):
        """Addresses of every tensor and each parameter's size, in table order."""
        return tuple((t.data_ptr(), t.numel()) for q in quads for t in q)


def adamw_step(tab, w1, w2, eps, decay, alpha):
    """One AdamW step (muon.py:408-436) over every parameter of `tab` (AdamwTable),
    enqueued on the current stream."""
    if tab.count == 0:
        return
    _check(load().dmh_adamw_step(_stream(tab.table.device), _ptr(tab.table), tab.count,
                                 _ptr(tab.chunks), tab.nchunks, float(w1), float(w2),
                                 float(eps), float(decay), float(alpha)),
           "dmh_adamw_step")
