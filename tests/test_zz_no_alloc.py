"""tlh_matmul_noalloc -- the allocation-free form of tlh_matmul_ws, whose
K-chunk partials live in the library's own per-GPU device array -- through
the C-ABI against tlh_matmul_ws given tlh_matmul_workspace_size's scratch:
bit for bit, on calls in a row whose second is smaller than the first (the
array keeps the last call's contents), for every plan that uses scratch
(split-K, the tail split, the one-row GEMV) and for one that uses none; a
product whose scratch would exceed the array is refused without a launch.
"""
import ctypes

import numpy as np
import pytest

import oracle_lib as O
from gpu_util import Gpu, assert_rel, u32
from templit_amd.native import check

pytestmark = pytest.mark.gpu

SCRATCH_FLOATS = 8 * 1024 * 1024  # TLH_NOALLOC_SCRATCH_FLOATS


@pytest.fixture(scope="module")
def g():
    return Gpu()


def args(M, K, N):
    return (M, K, N, K, 1, N, 1, N, 1, 0, u32([1]), u32([0]), u32([0]), u32([0]))


def workspace_elems(g, M, K, N):
    n = ctypes.c_size_t()
    check(g.lib.tlh_matmul_workspace_size(*args(M, K, N), ctypes.byref(n)), "workspace_size")
    return n.value


def both(g, a, b, seed_out):
    """(tlh_matmul_noalloc result, tlh_matmul_ws result, scratch floats)."""
    M, K = a.shape
    N = b.shape[1]
    da, db = g.dev(a), g.dev(b)
    n = workspace_elems(g, M, K, N)
    ws = g.empty((max(n, 1),))
    ref = g.dev(O.normal((M, N), seed_out))  # garbage the product must overwrite
    g.call("tlh_matmul_ws", da, db, ref, *args(M, K, N), ws if n else None, n)
    out = g.dev(O.normal((M, N), seed_out + 1))
    g.call("tlh_matmul_noalloc", da, db, out, *args(M, K, N))
    return g.host(out), g.host(ref), n


# (first, second): the second call is the smaller one
CASES = [
    ((384, 6144, 2048), (384, 6144, 384)),   # split-K: 4 then 8 splits of [384, N]
    ((6144, 1536, 448), (384, 6144, 384)),   # tail split (672 tiles of 64x64), then split-K
    ((1, 4096, 1024), (1, 1024, 512)),       # one-row GEMV chunks
    ((384, 6144, 384), (256, 256, 256)),     # split-K, then a plan without scratch
]


@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_matches_workspace_form_on_consecutive_calls(g, first, second):
    for i, (M, K, N) in enumerate((first, second)):
        a = O.normal((M, K), 900 + 10 * i, 0, 0.5)
        b = O.normal((K, N), 901 + 10 * i, 0, 0.5)
        out, ref, n = both(g, a, b, 902 + 10 * i)
        assert n <= SCRATCH_FLOATS
        if (M, K, N) != (256, 256, 256):
            assert n > 0, (M, K, N)  # the case exercises the scratch array
        np.testing.assert_array_equal(out, ref)
        assert_rel(out, O.matmul(a, b), 1e-3, f"noalloc {M}x{K}x{N}")


def test_noalloc_refuses_products_beyond_its_scratch(g):
    # A^T.B with A stored [K, M], 3456 x 4352 on 128x128 tiles: 918 tiles on
    # 256 CUs, so 150 tail tiles are cut into 16 K chunks, 39.3 M floats of
    # partials: more than the array holds. The call returns an error and
    # writes nothing.
    M, K, N = 3456, 1024, 4352
    ta = (M, K, N, 1, M, N, 1, N, 1, 0, u32([1]), u32([0]), u32([0]), u32([0]))
    n = ctypes.c_size_t()
    check(g.lib.tlh_matmul_workspace_size(*ta, ctypes.byref(n)), "workspace_size")
    assert n.value > SCRATCH_FLOATS
    a, b = g.zeros((K, M)), g.zeros((K, N))
    out = g.dev(np.full((M, N), 7.0, np.float32))
    st = g.lib.tlh_matmul_noalloc(a.data_ptr(), b.data_ptr(), out.data_ptr(), *ta, g.stream)
    assert st != 0
    assert np.all(g.host(out) == 7.0)
