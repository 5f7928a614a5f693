"""CPU oracle vs the reference CPU runtime itself.

oracle/_ref/libref_cpu.so is the reference's src/CPU/cpu.cpp compiled from
its own source (oracle/Makefile, target `ref`) behind a small C shim. On
random inputs the oracle's rank-N restatement must reproduce the
reference's rank-2 results bit for bit where both use the same loop order
(i-k-j matmul, serial row sums, max/exp/sum/divide softmax, strided
transpose) -- a transposed operand, a wrong broadcast stride or a different
summation order shows up as a mismatch.
"""
import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.skipif(not O.ref_available(),
                                reason="oracle/_ref not built (needs the reference tree)")


def ref_call(name, *args):
    rc = getattr(O.ref(), name)(*args)
    assert rc == 0, f"{name} raised inside the reference runtime"


@pytest.mark.parametrize("M,K,N", [(7, 5, 3), (64, 32, 48), (96, 384, 160)])
def test_mult_matches_reference(M, K, N):
    a = O.normal((M, K), 1, 0, 0.5)
    b = O.normal((K, N), 2, 0, 0.5)
    out = np.empty((M, N), np.float32)
    ref_call("ref_mult", O.p(a), O.p(b), O.p(out), M, K, N)
    np.testing.assert_array_equal(O.matmul(a, b), out)


# (a_shape, b_shape) covering every branch of binary_transform (cpu.cpp:37-147)
BROADCASTS = [((5, 7), (5, 7)), ((5, 7), (5, 1)), ((5, 7), (1, 7)), ((5, 7), (1, 1)),
              ((5, 1), (1, 7)), ((1, 7), (5, 1)), ((5, 1), (5, 7)), ((1, 7), (5, 7)),
              ((1, 1), (5, 7))]


@pytest.mark.parametrize("op", ["add", "sub", "hadamard", "divide"])
@pytest.mark.parametrize("sa,sb", BROADCASTS)
def test_binary_matches_reference(op, sa, sb):
    a = O.normal(sa, 3, 0, 1)
    b = O.normal(sb, 4, 2, 1)  # mean 2 keeps divide away from 0
    out_shape = O.broadcast_shape(sa, sb)
    out = np.empty(out_shape, np.float32)
    ref_call("ref_binary", O.BIN_OPS[op], O.p(a), sa[0], sa[1], O.p(b), sb[0], sb[1], O.p(out))
    np.testing.assert_array_equal(O.binary(op, a, b), out)


@pytest.mark.parametrize("rows,cols", [(1, 1), (6, 11), (64, 2048)])
def test_softmax_matches_reference(rows, cols):
    x = O.normal((rows, cols), 5, 0, 3)
    out = np.empty_like(x)
    ref_call("ref_softmax", O.p(x), O.p(out), rows, cols)
    np.testing.assert_array_equal(O.softmax(x), out)


@pytest.mark.parametrize("rows,cols", [(3, 5), (64, 130)])
def test_transpose_matches_reference(rows, cols):
    x = O.normal((rows, cols), 6)
    out = np.empty((cols, rows), np.float32)
    ref_call("ref_transpose", O.p(x), O.p(out), rows, cols)
    np.testing.assert_array_equal(O.transpose(x), out)


@pytest.mark.parametrize("target", [(9, 13), (9, 1), (1, 13), (1, 1)])
def test_sum_to_shape_matches_reference(target):
    x = O.normal((9, 13), 7)
    out = np.empty(target, np.float32)
    ref_call("ref_sum_to_shape", O.p(x), 9, 13, O.p(out), target[0], target[1])
    np.testing.assert_array_equal(O.sum_to_shape(x, list(target)), out)


def test_sum_matches_reference():
    x = O.normal((33, 17), 8)
    out = np.empty(1, np.float32)
    ref_call("ref_sum", O.p(x), 33, 17, O.p(out))
    assert O.total_sum(x) == out[0]


@pytest.mark.parametrize("op,name", [(0, "sqrt"), (1, "sigmoid")])
def test_unary_matches_reference(op, name):
    x = np.abs(O.normal((7, 9), 9)) if name == "sqrt" else O.normal((7, 9), 9)
    out = np.empty_like(x)
    ref_call("ref_unary", op, O.p(x), O.p(out), 7, 9)
    np.testing.assert_array_equal(O.unary(name, x), out)


def test_argmax_matches_reference():
    x = O.normal((40, 50), 10)
    out = np.zeros(1, np.uint32)
    ref_call("ref_argmax", O.p(x), 40, 50, O.p(out))
    assert O.argmax(x) == int(out[0])
