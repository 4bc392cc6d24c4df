"""The C-ABI library loads on a CPU-only host and exports every declared symbol."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    inc = os.path.join(ROOT, "include")
    for f in os.listdir(inc):
        if f.endswith(".h"):
            src = open(os.path.join(inc, f)).read()
            names |= set(re.findall(r"^(?:int|int64_t|const char\*)\s+(a8_\w+)\s*\(", src, re.M))
    return sorted(names)


def test_header_declares_entry_points():
    names = _declared()
    assert "a8_fused_update_1d" in names and len(names) >= 8, names


def test_library_exports_declared_symbols():
    from adafactor8bit import _native as nat
    L = nat.lib()
    for n in _declared():
        assert hasattr(L, n), f"symbol {n} declared in include/ but not exported"
    assert L.a8_version().startswith(b"adafactor8bit_amd")


def test_ctypes_signatures_cover_header():
    from adafactor8bit import _native as nat
    assert set(_declared()) <= set(nat.exported_symbols())


def test_argument_errors_without_gpu():
    """Shape/dtype validation happens on the host and returns an error code."""
    from adafactor8bit import _native as nat
    L = nat.lib()
    rc = L.a8_fused_update_1d(0, 0, 0, None, None, None, None, None, None, None, None, None, None,
                              None, None, None, 0, 0, 0.9, 0.001, 1e-8, 1, -126.0, 0.0, 1e-16, 10, 100,
                              256, 8, 0, 0.0, 8, 0, 1e-4, 1.0, 0, None)
    assert rc == -3, rc  # block_size 100 rejected
    assert b"block_size" in L.a8_last_error()
    rc = L.a8_fused_update_1d(0, 0, 7, None, None, None, None, None, None, None, None, None, None,
                              None, None, None, 0, 0, 0.9, 0.001, 1e-8, 1, -126.0, 0.0, 1e-16, 10, 2048,
                              256, 8, 0, 0.0, 8, 0, 1e-4, 1.0, 0, None)
    assert rc == -2, rc


def test_module_signatures_match_reference():
    """Every name the reference-named module provides has the reference's positional parameters
    (fixture written from kernels.cu:3089-3150 by tests/golden/gen_signatures.py)."""
    import inspect
    import json
    import os
    from adafactor8bit import adafactor8bit_cuda as K
    path = os.path.join(os.path.dirname(__file__), "golden", "module_signatures.json")
    with open(path) as f:
        ref = json.load(f)
    assert len(ref) == 61
    for name in K.__all__:
        assert name in ref, name
        assert list(inspect.signature(getattr(K, name)).parameters) == ref[name], name
    assert sorted(set(ref) - {"qmaps"}) == sorted(set(K.__all__)), sorted(set(ref) ^ set(K.__all__))


def test_apollo_lowrank_and_phase_argument_errors_without_gpu():
    """The APOLLO low-rank stage and the phased group call check their records on
    the host before any launch."""
    import ctypes
    from adafactor8bit import _native as nat
    L = nat.lib()
    a = nat.ApolloXArgs()
    a.rows_low, a.cols_low = 16, 8
    assert L.a8_apollo_lowrank_x(ctypes.byref(a), None) == -1            # null g_low / u / workspace
    a.g_low = a.u = a.xws = 256
    assert L.a8_apollo_lowrank_x(ctypes.byref(a), None) == -1            # plain stage without its V state
    assert b"low-rank V state" in L.a8_last_error()
    a.came, a.has_m = 1, 0
    assert L.a8_apollo_lowrank_x(ctypes.byref(a), None) == -1            # CAME without momentum
    assert b"beta1" in L.a8_last_error()
    a.has_m, a.m_fp32, a.v_bits, a.block_size, a.c_bits = 1, 256, 8, 100, 8
    assert L.a8_apollo_lowrank_x(ctypes.byref(a), None) == -3            # AL block 100
    a.rows_low = 0
    assert L.a8_apollo_lowrank_x(ctypes.byref(a), None) == -4            # empty matrix
    a.rows_low, a.cols_low, a.u_rowsums = 16, 12, 1
    assert L.a8_apollo_lowrank_x(ctypes.byref(a), None) == -4            # row sums of 12-element rows
    assert b"u_rowsums" in L.a8_last_error()
    a.u_rowsums = 0
    assert L.a8_apollo_x_workspace_floats(0, 8) == 0
    assert L.a8_apollo_x_workspace_floats(5632, 256) > 4 * 5632 * 256
    rc = L.a8_apollo_step_multi_phase(4, 0, 0, None, 1, None, 0, 0.001, 0.9, 1, 1e-6, -39.9, 0, 2048, 8, 0, 1,
                                      256, 1, 1.0, 0, 1, 0.01, 0.0, 1e-3, 1e-3, 0, 0, 0.0, 0, 1, None, None)
    assert rc == -1 and b"phase" in L.a8_last_error()
    assert L.a8_vema_fp32(None, None, 0, 0.001, 0.0, 4, None) == -1
    assert L.a8_vema_fp32(256, 256, 9, 0.001, 0.0, 4, None) == -2


def test_noalloc_rejects_more_tensors_than_its_scratch_holds():
    """The no-allocation multi-tensor step holds its table in a fixed 64 KiB device
    array: a launch over more tensors fails on the host with A8_ERR_SIZE."""
    from adafactor8bit import _native as nat
    L = nat.lib()
    cap = L.a8_noalloc_max_tensors_1d()
    assert cap * int(L.a8_table_bytes_1d(1)) <= 64 * 1024 < (cap + 1) * int(L.a8_table_bytes_1d(1))
    n = cap + 1
    arr = (nat.Tensor1D * n)()
    rc = L.a8_fused_update_1d_multi_noalloc(0, 0, 0, arr, n, 0.9, 0.001, 1e-8, 1, -126.0, 0.0, 1e-16, 2048, 256, 8,
                                            0, 0.0, 8, 0, 1, 1e-4, 1.0, 0, 1, None, None)
    assert rc == -4, rc
    assert b"scratch" in L.a8_last_error()
    assert L.a8_fused_update_1d_multi_noalloc(0, 0, 0, arr, 0, 0.9, 0.001, 1e-8, 1, -126.0, 0.0, 1e-16, 2048, 256,
                                              8, 0, 0.0, 8, 0, 1, 1e-4, 1.0, 0, 1, None, None) == 0
