"""CPU checks of the C-ABI library: it loads, exports every entry point that
include/defmuon_hip.h declares, and its host-side argument checks work (no
kernel is launched here)."""

import ctypes
import os
import re

import pytest

from conftest import ROOT


def _declared():
    text = open(os.path.join(ROOT, "include", "defmuon_hip.h")).read()
    return sorted(set(re.findall(r"\b(dmh_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from defmuon_amd import _native
    return _native.load()


def test_exports_match_header(lib):
    from defmuon_amd import _native
    declared = _declared()
    assert declared, "no declarations found"
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(_native.EXPORTS) == declared


def test_ns_workspace_size(lib):
    n = ctypes.c_size_t()
    assert lib.dmh_ns_workspace_size(2, 300, 700, 0, ctypes.byref(n)) == 0
    mp, np_ = 512, 768          # 300 -> 512, 700 -> 768 (256 tiles)
    # T double-buffered (2 x np x mp), A and B' (mp x mp), bf16; fp64 norm partials
    want = 2 * 2 * np_ * mp * 2 + 2 * 2 * mp * mp * 2 + 256 * ((2 * 64 * 8 + 255) // 256)
    assert n.value == want
    assert lib.dmh_ns_workspace_size(1, 0, 5, 0, ctypes.byref(n)) == 1
    assert b"bad arguments" in lib.dmh_last_error()


def test_rsvd_workspace_limits(lib):
    n = ctypes.c_size_t()
    assert lib.dmh_rsvd_workspace_size(3, 5120, 1280, 64, ctypes.byref(n)) == 0
    assert n.value > 3 * 5120 * 64 * 4
    assert lib.dmh_rsvd_workspace_size(3, 5120, 1280, 65, ctypes.byref(n)) == 1
    assert b"unsupported shape" in lib.dmh_last_error()
    assert lib.dmh_rsvd_workspace_size(3, 100, 200, 8, ctypes.byref(n)) == 1   # n < m
    # sketch-width panels (n x 64 fp32) are addressed with 32-bit offsets: n < 2^23
    assert lib.dmh_rsvd_workspace_size(1, (1 << 23) - 1, 64, 64, ctypes.byref(n)) == 0
    assert lib.dmh_rsvd_workspace_size(1, 1 << 23, 64, 64, ctypes.byref(n)) == 1
    assert b"unsupported shape" in lib.dmh_last_error()


def test_entry_points_reject_bad_arguments_without_launching(lib):
    from defmuon_amd import _native
    v = ctypes.c_void_p(0)
    # null pointers / bad shapes are refused before any HIP call
    assert lib.dmh_rmfro_clip(v, None, None, 1, 10, 5, 2, 1, 0.1, 0.1, 1.01, 1, 1, None, 1,
                              None, None, None, 0) == 1
    coeffs = (ctypes.c_double * 3)(1, 0, 0)
    assert lib.dmh_ns_chain(v, None, 0, 1, 8, 8, 64, 8, 1, None, 0, 1, coeffs, 1, None, 0) == 1
    dummy = ctypes.c_void_p(16)
    assert lib.dmh_ns_chain(v, dummy, 0, 1, 8, 8, 64, 8, 1, dummy, 0, 1, coeffs, 1, dummy,
                            16) == 2
    assert b"workspace" in lib.dmh_last_error()
    # batch 0 is a no-op
    assert lib.dmh_orth(v, None, 0, 10, 2, 1, None, None, 0) == 0


def test_workspace_sizes_for_empty_batch(lib):
    """An empty shape group (batch 0) sizes its workspaces without faulting."""
    n = ctypes.c_size_t()
    for fn in ("dmh_rsvd_workspace_size", "dmh_rmfro_workspace_size",
               "dmh_deflated_polar_workspace_size"):
        assert getattr(lib, fn)(0, 512, 256, 14, ctypes.byref(n)) == 0, fn
    assert lib.dmh_ns_workspace_size(0, 512, 256, 1, ctypes.byref(n)) == 0


def test_chain_refuses_operands_beyond_32bit_addressing(lib):
    """The bf16 chain addresses each padded operand through 32-bit buffer descriptors
    and offsets: a matrix whose padded bf16 iterate reaches 2^31 bytes is refused with
    status 1 by every entry that runs the chain, before any HIP call; one just below
    the limit is accepted."""
    n = ctypes.c_size_t()
    v, dummy = ctypes.c_void_p(0), ctypes.c_void_p(16)
    coeffs = (ctypes.c_double * 3)(3.4445, -4.7750, 2.0315)
    big, ok = (32768, 32768), (32768, 32512)     # 2^31 and 2^31 - 2^24 bytes of bf16
    assert lib.dmh_ns_workspace_size(1, *ok, 1, ctypes.byref(n)) == 0
    assert lib.dmh_ns_workspace_size(1, *big, 1, ctypes.byref(n)) == 1
    assert b"32-bit" in lib.dmh_last_error()
    assert lib.dmh_ns_chain(v, dummy, 1, 1, *big, 1 << 30, big[1], 1, dummy, 1, 0, coeffs, 1,
                            dummy, 16) == 1
    assert b"32-bit" in lib.dmh_last_error()
    assert lib.dmh_ns_chain_noalloc(v, dummy, 1, 1, *big, 1 << 30, big[1], 1, dummy, 1, 0,
                                    coeffs, 1) == 1
    assert b"32-bit" in lib.dmh_last_error()
    assert lib.dmh_deflated_polar_workspace_size(1, *ok, 64, ctypes.byref(n)) == 0
    assert lib.dmh_deflated_polar_workspace_size(1, *big, 64, ctypes.byref(n)) == 1
    assert b"32-bit" in lib.dmh_last_error()
    assert lib.dmh_deflated_polar_chain(v, 1, *big, coeffs, 1, dummy, dummy, 16) == 1
    assert b"32-bit" in lib.dmh_last_error()
    assert lib.dmh_deflated_polar_front(v, dummy, dummy, 1, *big, 64, 32, 0.1, 0.1, 1.01, 1,
                                        1, dummy, dummy, dummy, 16) == 1
    assert b"32-bit" in lib.dmh_last_error()
