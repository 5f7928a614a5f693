"""CPU oracle vs the reference's own known-answer tests.

Every expected value below is the one tests/test_metal_runtime.cpp (and
tests/test_meta.cpp) of the reference asserts for the Metal runtime; the
line numbers are cited per test. These pin the oracle's restatement of the
runtime semantics (broadcasting, eps inside the RMS sqrt, lowest-index
argmax, CE/+INF handling, scatter, clipping, AdamW).
"""
import math

import numpy as np
import pytest

import oracle_lib as O

EPS = 1e-5  # test_metal_runtime.cpp:22


def close(actual, expected, eps=EPS):
    actual = np.asarray(actual, dtype=np.float64).ravel()
    expected = np.asarray(expected, dtype=np.float64).ravel()
    assert actual.shape == expected.shape
    assert np.all(np.abs(actual - expected) < eps), (actual, expected)


def test_binary_and_chained():  # test_metal_runtime.cpp:131-158
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[5, 6], [7, 8]], np.float32)
    added = O.binary("add", a, b)
    close(added, [6, 8, 10, 12])
    close(O.binary("sub", a, b), [-4, -4, -4, -4])
    close(O.binary("hadamard", a, b), [5, 12, 21, 32])
    close(O.binary("divide", a, b), [0.2, 1 / 3, 3 / 7, 0.5])
    close(O.binary("hadamard", added, a), [6, 16, 30, 48])


def test_broadcasting():  # test_metal_runtime.cpp:160-174
    m = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    row = np.array([10, 20, 30], np.float32)
    out = O.binary("add", m, row)
    assert out.shape == (2, 3)
    close(out, [11, 22, 33, 14, 25, 36])


def test_scalar_ops():  # test_metal_runtime.cpp:176-199
    x = np.array([[2, 4], [6, 8]], np.float32)
    close(O.scalar("add", x, 3.0), [5, 7, 9, 11])
    close(O.scalar("divide", x, 2.0), [1, 2, 3, 4])
    close(O.scalar("pow", x, 3.0), [8, 64, 216, 512], 1e-3)
    close(O.scalar("pow", O.scalar("divide", x, 2.0), 2.0), [1, 4, 9, 16], 1e-3)


def test_unary_ops():  # test_metal_runtime.cpp:201-226
    x = np.array([0, 1, -1, 2], np.float32)
    sig = [1 / (1 + math.exp(-v)) for v in (0, 1, -1, 2)]
    close(O.unary("sigmoid", x), sig)
    close(O.unary("exp", x), [1, math.e, math.exp(-1), math.exp(2)], 1e-5 * 8)
    close(O.unary("sqrt", np.array([0, 1, 4, 9], np.float32)), [0, 1, 2, 3])


def test_rms_and_rms_norm():  # test_metal_runtime.cpp:228-244 (eps 1e-6 inside sqrt)
    x = np.array([[3, 4], [0, 0]], np.float32)
    first = math.sqrt(12.5 + 1e-6)
    close(O.rms(x), [first, 1e-3])
    close(O.rms_norm(x), [3 / first, 4 / first, 0, 0])


def test_gelu():  # test_metal_runtime.cpp:246-279
    x = np.array([-2, -1, 0, 1, 2], np.float32)
    a, b = 0.7978845608, 0.044715

    def g(v):
        return 0.5 * v * (1 + math.tanh(a * (v + b * v ** 3)))

    def gd(v):
        t = math.tanh(a * (v + b * v ** 3))
        return 0.5 * (1 + t) + 0.5 * v * (1 - t * t) * a * (1 + 3 * b * v * v)

    close(O.unary("gelu", x), [g(v) for v in x])
    close(O.unary("gelu_derivative", x), [gd(v) for v in x])


def test_matmul():  # test_metal_runtime.cpp:281-305
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    close(O.matmul(a, b), [58, 64, 139, 154])
    ba = np.array([1, 2, 3, 4, 2, 0, 1, 2], np.float32).reshape(2, 2, 2)
    bb = np.array([5, 6, 7, 8, 1, 3, 4, 2], np.float32).reshape(2, 2, 2)
    out = O.matmul(ba, bb)
    assert out.shape == (2, 2, 2)
    close(out, [19, 22, 43, 50, 2, 6, 9, 7])


def test_tiled_identity_matmul():  # test_metal_runtime.cpp:307-342
    size, batches = 64, 2
    ident = np.zeros((batches, size, size), np.float32)
    for bt in range(batches):
        ident[bt] = np.eye(size)
    vals = (np.arange(batches * size * size) % 31 - 15).astype(np.float32).reshape(
        batches, size, size)
    close(O.matmul(ident, vals), vals)


def test_reductions_and_transpose():  # test_metal_runtime.cpp:344-374
    x = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    assert O.total_sum(x) == 21
    close(O.sum_to_shape(x, [2, 1]), [6, 15])
    close(O.sum_to_shape(x, [1, 3]), [5, 7, 9])
    close(O.max_to_shape(x, [2, 1]), [3, 6])
    t = O.transpose(x)
    assert t.shape == (3, 2)
    close(t, [1, 4, 2, 5, 3, 6])


def test_sum_to_shape_multiple_dims():  # test_metal_runtime.cpp:376-413
    x = np.arange(1, 25, dtype=np.float32).reshape(2, 3, 4)
    close(O.sum_to_shape(x, [1, 3, 1]), [68, 100, 132])
    close(O.sum_to_shape(x, [2, 1, 1]), [78, 222])
    close(O.sum_to_shape(x, [1, 1, 1]), [300])
    close(O.sum_to_shape(x, [4]), [66, 72, 78, 84])


def test_sum_to_shape_leading_singleton():  # test_metal_runtime.cpp:415-430
    x = np.array([[1, 2, 3, 4]], np.float32)
    out = O.sum_to_shape(x, [4])
    assert out.shape == (4,)
    close(out, [1, 2, 3, 4])


def test_softmax():  # test_metal_runtime.cpp:432-472
    den = math.exp(-2) + math.exp(-1) + 1
    low, mid, high = math.exp(-2) / den, math.exp(-1) / den, 1 / den
    close(O.softmax(np.array([[1, 2, 3], [1, 1, 1]], np.float32)),
          [low, mid, high, 1 / 3, 1 / 3, 1 / 3])
    close(O.softmax(np.array([1, 2, 3], np.float32)), [low, mid, high])
    r4 = np.array([1, 2, 3, 3, 2, 1, 1000, 1001, 1002, -1000, -1000, -1000],
                  np.float32).reshape(2, 2, 1, 3)
    close(O.softmax(r4), [low, mid, high, high, mid, low, low, mid, high, 1 / 3, 1 / 3, 1 / 3])
    close(O.softmax(np.array([[4], [-7]], np.float32)), [1, 1])


def test_cross_entropy():  # test_metal_runtime.cpp:474-507
    logits = np.array([1, 2, 3, 1, 1, 1, 1000, 1001, 1002, -1, -2, -3],
                      np.float32).reshape(2, 2, 3)
    targets = np.array([[2, 0], [1, 2]], np.uint32)
    den = math.exp(-2) + math.exp(-1) + 1
    low, mid, high = math.exp(-2) / den, math.exp(-1) / den, 1 / den
    ld = math.log(den)
    losses = O.cross_entropy(logits, targets)
    assert losses.shape == (2, 2, 1)
    close(losses, [ld, math.log(3), 1 + ld, 2 + ld], 1e-4)
    close(O.cross_entropy_backward(logits, targets),
          [low, mid, high - 1, -2 / 3, 1 / 3, 1 / 3, low, mid - 1, high, high, mid, low - 1],
          1e-4)


def test_cross_entropy_invalid_target_is_inf():  # math.metal:893-896, 921-926
    logits = np.zeros((2, 3), np.float32)
    targets = np.array([3, 1], np.uint32)
    losses = O.cross_entropy(logits, targets)
    assert np.isinf(losses[0, 0]) and losses[0, 0] > 0
    grads = O.cross_entropy_backward(logits, targets)
    assert np.all(np.isinf(grads[0])) and np.all(np.isfinite(grads[1]))


def test_argmax():  # test_metal_runtime.cpp:509-531
    assert O.argmax(np.array([[1, 4, 2], [9, 3, 5]], np.float32)) == 3
    big = np.zeros(5000, np.float32)
    big[4097] = 100
    assert O.argmax(big) == 4097


def test_argmax_ties_pick_lowest_index():  # math.metal:715-777 (strict '>')
    x = np.zeros(3000, np.float32)
    x[[17, 500, 2999]] = 7.0
    assert O.argmax(x) == 17


def test_embedding_lookup():  # test_metal_runtime.cpp:533-549
    w = np.arange(1, 13, dtype=np.float32).reshape(4, 3)
    ids = np.array([[2, 0], [3, 1]], np.uint32)
    close(O.embedding_lookup(w, ids), [7, 8, 9, 1, 2, 3, 10, 11, 12, 4, 5, 6])


def test_scatter_index():  # test_metal_runtime.cpp:551-569 (zero-fill then scatter)
    values = np.array([1, 2, 3, 4, 5, 6, 10, 20, 30, 7, 8, 9], np.float32).reshape(2, 2, 3)
    ids = np.array([[2, 0], [2, 1]], np.uint32)
    out = O.scatter_add_rows(np.zeros((4, 3), np.float32), ids, values)
    close(out, [4, 5, 6, 7, 8, 9, 11, 22, 33, 0, 0, 0])


def test_scatter_add_rows():  # test_metal_runtime.cpp:571-593
    base = np.arange(100, 112, dtype=np.float32).reshape(4, 3)
    values = np.array([1, 2, 3, 4, 5, 6, 10, 20, 30, 7, 8, 9], np.float32).reshape(2, 2, 3)
    ids = np.array([[2, 0], [2, 1]], np.uint32)
    close(O.scatter_add_rows(base, ids, values),
          [104, 106, 108, 110, 112, 114, 117, 129, 141, 109, 110, 111])


def test_gradient_clipping():  # test_metal_runtime.cpp:595-615
    first = np.array([3, 4, 0], np.float32)
    second = np.array([12], np.float32)
    s = O.grad_norm_accumulate([first, second])
    close([s], [169])
    close(O.clip_gradient(first, s, 1.0), [3 / 13, 4 / 13, 0])
    close(O.clip_gradient(second, s, 1.0), [12 / 13])


def test_adamw_two_steps():  # test_metal_runtime.cpp:617-658
    param = np.array([1, -2, 3, -4], np.float32)
    grad = np.array([0.5, -0.25, 1, -0.75], np.float32)
    m1 = np.zeros(4, np.float32)
    m2 = np.zeros(4, np.float32)
    lr, wd = 0.01, 0.01
    decay = np.float32(1) - np.float32(lr) * np.float32(wd)  # AdamW.h:28-29
    exp_p = param.astype(np.float64).copy()
    em1 = np.zeros(4)
    em2 = np.zeros(4)
    for step in (1, 2):
        param, m1, m2 = O.adamw(param, grad, m1, m2, 0.9, 0.999, float(decay), lr, 1e-8, step)
        c1 = 1 - 0.9 ** step
        c2 = 1 - 0.999 ** step
        em1 = 0.9 * em1 + 0.1 * grad
        em2 = 0.999 * em2 + 0.001 * grad * grad
        exp_p = exp_p * 0.9999 - 0.01 * (em1 / c1) / (np.sqrt(em2 / c2) + 1e-8)
        close(param, exp_p, 1e-5)
