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
}

EXPORTS = tuple(_SIGS)


class NativeError(RuntimeError):
    pass


def load(path=LIB_PATH):
    """Load (once) and return the library handle."""
    global _lib
    if _lib is not None:
        return _lib
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
