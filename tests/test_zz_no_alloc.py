"""sampler_argmax_noalloc (the argmax staged in one statically allocated
device array, no hipMalloc) against sampler_argmax (device buffers
allocated per call), through the C-ABI: the same index, bit for bit, on
consecutive calls whose sizes shrink and grow, with planted maxima, ties
and NaNs, and at the size limit."""
import ctypes
import subprocess
import sys
import textwrap

import numpy as np
import pytest

from conftest import REPO

pytestmark = pytest.mark.gpu


def lib():
    from strasgpt_amd import runtime as rt
    L = rt.lib()
    fp = ctypes.POINTER(ctypes.c_float)
    L.sampler_argmax_noalloc.restype = ctypes.c_size_t
    L.sampler_argmax_noalloc.argtypes = [fp, ctypes.c_size_t]
    return L


def call(fn, x):
    x = np.ascontiguousarray(x, np.float32)
    return int(fn(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), x.size))


def scan(x):
    """The reference sample_argmax (source/sampler.c:92-102)."""
    best, bv = 0, x[0]
    for i in range(1, len(x)):
        if x[i] > bv:
            best, bv = i, x[i]
    return best


def test_noalloc_argmax_matches_allocating_entry_point():
    L = lib()
    rng = np.random.default_rng(11)
    cases = []
    a = rng.standard_normal(201088).astype(np.float32)
    a[150000] = 20.0
    cases.append(("vocab 201088, max late", a))
    b = rng.standard_normal(5000).astype(np.float32)  # smaller than the call before
    b[[4000, 4500]] = 15.0
    cases.append(("5000, tie", b))
    c = rng.standard_normal(262144).astype(np.float32)  # the size limit
    c[1::9] = np.nan  # from index 1: a NaN at index 0 would win by itself
    c[262143] = 30.0  # the last element of the full staging copy
    cases.append(("limit 262144, NaNs", c))
    d = np.array([np.nan, 1.0, 2.0], np.float32)
    cases.append(("3, NaN first", d))
    e = rng.standard_normal(131072).astype(np.float32)
    cases.append(("131072", e))
    cases.append(("1", np.array([-3.0], np.float32)))
    for what, x in cases:
        want = call(L.sampler_argmax, x)
        got = call(L.sampler_argmax_noalloc, x)
        print(f"[noalloc] {what}: noalloc {got} allocating {want}", flush=True)
        assert got == want, what
        assert got == scan(x.tolist()), what


def test_noalloc_argmax_rejects_oversize():
    """n above SAMPLER_ARGMAX_NOALLOC_MAX dies with a message, before any
    device work."""
    code = textwrap.dedent(f"""
        import ctypes, sys
        sys.path.insert(0, {REPO!r})
        import numpy as np
        from strasgpt_amd import runtime as rt
        L = rt.lib()
        L.sampler_argmax_noalloc.restype = ctypes.c_size_t
        L.sampler_argmax_noalloc.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
        x = np.zeros(262145, np.float32)
        L.sampler_argmax_noalloc(x.ctypes.data, x.size)
        print("NOT REACHED")
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "NOT REACHED" not in r.stdout
    assert "exceeds SAMPLER_ARGMAX_NOALLOC_MAX" in r.stderr
