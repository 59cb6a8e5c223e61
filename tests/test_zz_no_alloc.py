"""GPU check of the allocation-free chain entry dmh_ns_chain_noalloc: through the
C ABI it must give dmh_ns_chain's output bit for bit, on two calls in a row (the
second on a smaller input, so stale scratch contents from the first would show),
and refuse a shape whose workspace exceeds its static scratch."""

import ctypes
import os
import re

import pytest
import torch

from conftest import ROOT

NS = (3.4445, -4.7750, 2.0315)


def _scratch_bytes_from(path, pattern):
    text = open(os.path.join(ROOT, path)).read()
    m = re.fullmatch(r"(\d+)u << (\d+)", re.search(pattern, text).group(1))
    return int(m.group(1)) << int(m.group(2))


def test_scratch_size_matches_header():
    pat = r"#define DMH_NS_SCRATCH_BYTES \((.+?)\)"
    assert _scratch_bytes_from("include/defmuon_hip.h", pat) == \
        _scratch_bytes_from("spectral-deflation_amd/csrc/ns_chain.h", pat) == 64 << 20


def _noalloc(lib, X, out, tall, mode, coeffs):
    flat = (ctypes.c_double * (3 * len(coeffs)))(*[v for t in coeffs for v in t])
    B, R, C = X.shape
    bs, rs, cs = X.stride()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return lib.dmh_ns_chain_noalloc(stream, ctypes.c_void_p(X.data_ptr()),
                                    0 if X.dtype == torch.float32 else 1, B, R, C, bs, rs, cs,
                                    ctypes.c_void_p(out.data_ptr()), int(tall), mode, flat,
                                    len(coeffs))


@pytest.mark.gpu
def test_noalloc_matches_ns_chain_twice():
    from defmuon_amd import _native
    lib = _native.load()
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    cases = [
        # (batch, rows, cols, tall, entry mode, coefficients): the second is smaller
        (2, 768, 3072, False, 1, [NS] * 5),
        (3, 300, 200, True, 2, [(8.2872, -23.5959, 17.3004), NS, NS]),
    ]
    for B, R, C, tall, mode, co in cases:
        print(f"noalloc case B={B} {R}x{C} tall={tall} mode={mode}", flush=True)
        X = torch.randn(B, R, C, device="cuda", generator=g)
        ref = _native.ns_chain(X, tall, mode, co)
        out = torch.full_like(ref, float("nan"))
        rc = _noalloc(lib, X, out, tall, mode, co)
        assert rc == 0, lib.dmh_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


@pytest.mark.gpu
def test_noalloc_rejects_oversize_shape():
    from defmuon_amd import _native
    lib = _native.load()
    X = torch.zeros(8, 5120, 1280, device="cuda")   # ~262 MiB of workspace
    out = torch.empty(8, 5120, 1280, dtype=torch.bfloat16, device="cuda")
    assert _noalloc(lib, X, out, True, 1, [NS]) == 2
    assert b"static scratch" in lib.dmh_last_error()
