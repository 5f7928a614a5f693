"""Parity of every C-ABI kernel entry point with the CPU oracle, on seeded
inputs, at the benchmark's shapes where the oracle is fast enough and at the
reference's edge cases (ragged sizes, broadcasting, ties, invalid targets,
in-place use). Tolerances: rtol 1e-4 / atol 1e-5 for elementwise and
reduction ops, 1e-3 relative for matmul and attention, bit-exact for
gathers and argmax.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle_lib as O
from gpu_util import Gpu, assert_close, assert_rel, rel_err, u32
from templit_amd.native import EPI_GELU, EPI_GELU_BWD, GemmDesc, check

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def g():
    return Gpu()


# ---------------------------------------------------------------------------
# elementwise
# ---------------------------------------------------------------------------
BROADCASTS = [
    ((6144, 384), (6144, 384)),          # same shape
    ((6144, 384), (1, 384)),             # bias row
    ((32, 6, 192, 192), (1, 1, 192, 192)),  # causal mask
    ((32, 6, 192, 192), (1, 1)),         # divide by sqrt(64)
    ((32, 192, 384), (32, 192, 1)),      # RMSNorm' column broadcast
    ((32, 192, 1), (32, 192, 2048)),     # CE upstream scale
    ((2, 3), (3,)),                      # rank mismatch (test_metal_runtime.cpp:160)
    ((5, 1, 7), (1, 3, 1)),              # both broadcast
    ((3, 1, 4, 1, 2), (1, 5, 1, 6, 2)),  # generic rank-5 decode
]


@pytest.mark.parametrize("op", ["add", "sub", "hadamard", "divide"])
@pytest.mark.parametrize("sa,sb", BROADCASTS)
def test_binary_broadcast(g, op, sa, sb):
    a = O.normal(sa, 1, 0, 1)
    b = O.normal(sb, 2, 3, 1)
    out_shape = O.broadcast_shape(sa, sb)
    expect = O.binary(op, a, b)
    da, db, do = g.dev(a), g.dev(b), g.empty(out_shape)
    g.call(f"tlh_{op}", da, db, do, len(out_shape), u32(out_shape),
           u32(O.broadcast_strides(sa, out_shape)), u32(O.broadcast_strides(sb, out_shape)))
    assert_close(g.host(do), expect, what=op)


def test_binary_in_place(g):
    # LINEAR's add(destination, bias, destination) (execute.h:249)
    a = O.normal((512, 384), 3)
    b = O.normal((1, 384), 4)
    expect = O.binary("add", a, b)
    da, db = g.dev(a), g.dev(b)
    g.call("tlh_add", da, db, da, 2, u32([512, 384]), u32([384, 1]), u32([0, 1]))
    assert_close(g.host(da), expect)


@pytest.mark.parametrize("name,orc,pos", [("sqrt", "sqrt", True), ("exp", "exp", False),
                                         ("sigmoid", "sigmoid", False), ("gelu", "gelu", False),
                                         ("gelu_derivative", "gelu_derivative", False),
                                         ("copy", "copy", False)])
@pytest.mark.parametrize("n", [1, 1023, 6144 * 1536])
def test_unary(g, name, orc, pos, n):
    x = O.normal((n,), 5, 0, 2)
    if pos:
        x = np.abs(x)
    out = g.empty((n,))
    g.call(f"tlh_{name}", g.dev(x), out, n)
    assert_close(g.host(out), O.unary(orc, x), what=name)


@pytest.mark.parametrize("name,orc,s", [("add_scalar", "add", 1e-6), ("divide_scalar", "divide", 384.0),
                                       ("pow_scalar", "pow", 3.0)])
def test_scalar_ops(g, name, orc, s):
    x = np.abs(O.normal((100003,), 6)) + 0.1
    out = g.empty(x.shape)
    g.call(f"tlh_{name}", g.dev(x), s, out, x.size)
    assert_close(g.host(out), O.scalar(orc, x, s), what=name)


def test_gelu_backward(g):
    x = O.normal((6144 * 1536 + 3,), 7, 0, 2)
    gr = O.normal(x.shape, 8)
    out = g.empty(x.shape)
    g.call("tlh_gelu_backward", g.dev(gr), g.dev(x), out, x.size)
    expect = O.binary("hadamard", gr, O.unary("gelu_derivative", x))
    assert_close(g.host(out), expect)


TRANSPOSES = [((6144, 1536), -2, -1), ((32, 192, 6, 64), 1, 2), ((32, 6, 192, 64), -2, -1),
              ((4, 100, 70), -2, -1), ((3, 4, 5, 6), 0, 3), ((1, 384), 0, 1),
              ((32, 6, 192, 64), 0, 1), ((2, 3, 5, 4, 8), 1, 3),  # float4 gathers
              ((4, 5, 6), 0, 1)]                                  # last dim not float4


@pytest.mark.parametrize("shape,da,db", TRANSPOSES)
def test_transpose(g, shape, da, db):
    x = O.normal(shape, 9)
    expect = O.transpose(x, da, db)
    nd = len(shape)
    a, b = da % nd, db % nd
    ist = O.contiguous_strides(shape)
    ist[a], ist[b] = ist[b], ist[a]
    out = g.empty(expect.shape)
    g.call("tlh_transpose", g.dev(x), out, nd, u32(expect.shape), u32(ist))
    np.testing.assert_array_equal(g.host(out), expect)  # a permutation is exact


@pytest.mark.parametrize("shape,perm", [
    ((4, 96, 6, 64), (0, 2, 3, 1)),    # K^T of a head split: [B,T,H,D] -> [B,H,D,T]
    ((2, 70, 3, 33), (0, 2, 3, 1)),    # ragged tiles
    ((5, 7, 9, 11), (2, 0, 3, 1)),     # leading dims permuted as well
    ((4, 6, 64, 96), (0, 3, 1, 2)),    # head merge [B,H,D,T] -> [B,T,H,D]: H,D fold to one dim
    ((3, 1, 40, 70), (0, 3, 1, 2)),    # a size-1 dim dropped
    ((3, 64, 130), (2, 0, 1)),         # folds to a plain 2-D transpose
    ((3, 64, 130), (2, 1, 0)),         # input-contiguous dim leading: the gather path
])
def test_transpose_general_permutations(g, shape, perm):
    # adjacent output dims that the input walks as one run are folded
    # together; permutations whose input is then contiguous along the
    # output's second-to-last dim take the batched tiled kernel (the others
    # a gather); every element moves exactly
    x = O.normal(shape, 19)
    expect = np.ascontiguousarray(np.transpose(x, perm))
    ist = [O.contiguous_strides(shape)[p] for p in perm]
    out = g.empty(expect.shape)
    g.call("tlh_transpose", g.dev(x), out, len(shape), u32(expect.shape), u32(ist))
    np.testing.assert_array_equal(g.host(out), expect)


JOB = np.dtype([("src", "<u8"), ("dst", "<u8"), ("rows", "<u4"), ("cols", "<u4"),
                ("first_tile", "<u4"), ("reserved", "<u4")])


def test_transpose_multi(g):
    # ragged shapes (partial 64x64 tiles, a single row, a single column),
    # destinations in another order than the sources
    shapes = [(384, 384), (384, 1536), (1536, 384), (100, 70), (1, 5), (65, 129), (7, 1)]
    offs, off = [], 0
    for r, c in shapes:
        offs.append(off)
        off += (r * c + 63) // 64 * 64
    src = O.normal((off,), 31)
    dst_offs, off2 = [], 0  # the destinations laid out in reverse order
    for r, c in reversed(shapes):
        dst_offs.append(off2)
        off2 += (r * c + 63) // 64 * 64
    dst_offs = list(reversed(dst_offs))
    jobs = np.zeros(len(shapes), JOB)
    tiles = 0
    for i, ((r, c), so, do) in enumerate(zip(shapes, offs, dst_offs)):
        jobs[i] = (so, do, r, c, tiles, 0)
        tiles += ((r + 63) // 64) * ((c + 63) // 64)
    dev_jobs = torch.from_numpy(jobs.view(np.uint8).copy()).to("cuda")
    out = g.zeros((off2,))
    g.call("tlh_transpose_multi", g.dev(src), out, dev_jobs, len(shapes), tiles)
    got = g.host(out)
    for (r, c), so, do in zip(shapes, offs, dst_offs):
        want = src[so:so + r * c].reshape(r, c).T
        np.testing.assert_array_equal(got[do:do + r * c].reshape(c, r), want)


def _transpose_jobs(shapes):
    offs, off = [], 0
    for r, c in shapes:
        offs.append(off)
        off += (r * c + 63) // 64 * 64
    jobs = np.zeros(len(shapes), JOB)
    tiles = 0
    for i, ((r, c), o) in enumerate(zip(shapes, offs)):
        jobs[i] = (o, o, r, c, tiles, 0)
        tiles += ((r + 63) // 64) * ((c + 63) // 64)
    return jobs, offs, off, tiles


def test_transpose_multi_extra_tiles_and_inconsistent_tables(g):
    # blocks past the last job's tiles write nothing; a table whose
    # first_tile values descend makes the whole launch a no-op
    shapes = [(100, 70), (64, 64), (3, 200)]
    jobs, offs, n, tiles = _transpose_jobs(shapes)
    src = O.normal((n,), 32)
    sentinel = np.float32(-12345.0)
    out = g.dev(np.full(n + 4096, sentinel, np.float32))
    dev_jobs = torch.from_numpy(jobs.view(np.uint8).copy()).to("cuda")
    g.call("tlh_transpose_multi", g.dev(src), out, dev_jobs, len(shapes), tiles + 37)
    got = g.host(out)
    written = np.zeros(got.size, bool)
    for (r, c), o in zip(shapes, offs):
        np.testing.assert_array_equal(got[o:o + r * c].reshape(c, r), src[o:o + r * c].reshape(r, c).T)
        written[o:o + r * c] = True
    assert np.all(got[~written] == sentinel)
    bad = jobs.copy()
    bad["first_tile"][1], bad["first_tile"][2] = bad["first_tile"][2], bad["first_tile"][1]
    out2 = g.dev(np.full(n, sentinel, np.float32))
    dev_bad = torch.from_numpy(bad.view(np.uint8).copy()).to("cuda")
    g.call("tlh_transpose_multi", g.dev(src), out2, dev_bad, len(shapes), tiles)
    assert np.all(g.host(out2) == sentinel)


# ---------------------------------------------------------------------------
# matmul
# ---------------------------------------------------------------------------
def mult(g, a, b):
    M, K = a.shape[-2], a.shape[-1]
    N = b.shape[-1]
    ab, bb = list(a.shape[:-2]), list(b.shape[:-2])
    batch = O.broadcast_shape(ab, bb) if (ab or bb) else []
    sa = [s * M * K for s in O.broadcast_strides(ab, batch)] if ab else [0] * len(batch)
    sb = [s * K * N for s in O.broadcast_strides(bb, batch)] if bb else [0] * len(batch)
    sc = [s * M * N for s in O.contiguous_strides(batch)]
    out = g.empty(batch + [M, N])
    g.call("tlh_matmul", g.dev(a), g.dev(b), out, M, K, N, K, 1, N, 1, N, 1, len(batch),
           u32(batch or [1]), u32(sa or [0]), u32(sb or [0]), u32(sc or [0]))
    return g.host(out)


MATMULS = [
    ((768, 384), (384, 1536)),                 # config 1
    ((2, 3), (3, 2)),                          # KAT shape
    ((32, 192, 384), (384, 384)),              # linear, weight broadcast over batch
    ((32, 6, 192, 64), (32, 6, 64, 192)),      # attention scores
    ((32, 6, 192, 192), (32, 6, 192, 64)),     # attention output
    ((32, 384, 192), (32, 192, 384)),          # per-sample weight grad
    ((2, 1, 33, 17), (1, 3, 17, 29)),          # broadcast both batch dims, ragged
    ((1, 65), (65, 1)),                        # vector dot
]


@pytest.mark.parametrize("sa,sb", MATMULS)
def test_matmul(g, sa, sb):
    a = O.normal(sa, 10, 0, 0.5)
    b = O.normal(sb, 11, 0, 0.5)
    assert_rel(mult(g, a, b), O.matmul(a, b), 1e-3, "matmul")


@pytest.mark.parametrize("sa,sb,splits", [
    ((6144, 1536), (1536, 448), True),          # 672 tiles of 64x64: tail split over K chunks
    ((32, 192, 1536), (1536, 448), True),       # weight broadcast, folded into one product
    ((6144, 1536), (1536, 384), False),         # 256 tiles of 96x96: no scratch
    ((384, 6144), (6144, 384), True),           # 36 tiles: split-K
    ((32, 384, 192), (32, 192, 384), False),    # per-sample weight grad: no scratch
    ((1, 1024), (1024, 512), True),             # one row: GEMV chunks
])
def test_matmul_workspace(g, sa, sb, splits):
    # tlh_matmul_ws with the scratch tlh_matmul_workspace_size asks for equals
    # the oracle and tlh_matmul; a null workspace runs tlh_matmul's plan
    # (bit for bit)
    a = O.normal(sa, 12, 0, 0.5)
    b = O.normal(sb, 13, 0, 0.5)
    M, K, N = sa[-2], sa[-1], sb[-1]
    batch = list(sa[:-2])
    sa_ = [M * K] if batch else [0]
    sb_ = [K * N] if len(sb) > 2 else [0]  # 0: B broadcast over the batch
    sc = [M * N] if batch else [0]
    shape = u32(batch or [1])
    args = (M, K, N, K, 1, N, 1, N, 1, len(batch), shape, u32(sa_), u32(sb_), u32(sc))
    n = ctypes.c_size_t()
    check(g.lib.tlh_matmul_workspace_size(*args, ctypes.byref(n)), "matmul_workspace_size")
    assert (n.value > 0) == splits
    da, db = g.dev(a), g.dev(b)
    ws = g.empty((max(1, n.value),))
    outs = []
    for workspace, elems in ((ws.data_ptr(), n.value), (None, 0)):
        out = g.empty(batch + [M, N])
        g.call("tlh_matmul_ws", da, db, out, *args, workspace, elems)
        outs.append(g.host(out))
    plain = mult(g, a, b)
    np.testing.assert_array_equal(outs[1], plain)
    assert_rel(outs[0], O.matmul(a, b), 1e-3, "matmul_ws")
    assert_rel(outs[0], plain, 1e-5, "matmul_ws vs matmul")


@pytest.mark.parametrize("sa,sb", [((6144, 384), (384, 384)), ((192, 1536), (1536, 384)),
                                   ((3, 40, 24), (24, 33)), ((3, 16, 8), (3, 8, 12))])
def test_matmul_bias(g, sa, sb):
    # the product with a bias row in its epilogue (with the workspace the
    # plan asks for, and without) is bit for bit the product followed by the
    # broadcast add
    a = O.normal(sa, 14, 0, 0.5)
    b = O.normal(sb, 15, 0, 0.5)
    M, K, N = sa[-2], sa[-1], sb[-1]
    batch = list(sa[:-2])
    sa_ = [M * K] if batch else [0]
    sb_ = [K * N] if len(sb) > 2 else [0]
    sc = [M * N] if batch else [0]
    shape = u32(batch or [1])
    args = (M, K, N, K, 1, N, 1, N, 1, len(batch), shape, u32(sa_), u32(sb_), u32(sc))
    n = ctypes.c_size_t()
    check(g.lib.tlh_matmul_workspace_size(*args, ctypes.byref(n)), "matmul_workspace_size")
    bias = O.normal((N,), 16)
    da, db, dbias = g.dev(a), g.dev(b), g.dev(bias)
    ws = g.empty((max(1, n.value),))
    for workspace, elems in ((ws.data_ptr(), n.value), (None, 0)):
        prod = g.empty(batch + [M, N])  # the same plan without the bias
        g.call("tlh_matmul_ws", da, db, prod, *args, workspace, elems)
        expect = g.host(prod) + bias  # fp32 adds, as the add kernel does
        out = g.empty(batch + [M, N])
        g.call("tlh_matmul_bias_ws", da, db, out, dbias, None, *args, workspace, elems)
        np.testing.assert_array_equal(g.host(out), expect)
    assert_rel(g.host(out), O.matmul(a, b) + bias, 1e-3, "matmul + bias")


def test_matmul_kat_and_identity(g):
    # test_metal_runtime.cpp:281-342
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    np.testing.assert_allclose(mult(g, a, b), [[58, 64], [139, 154]], atol=1e-5)
    ident = np.stack([np.eye(64, dtype=np.float32)] * 2)
    vals = (np.arange(2 * 64 * 64) % 31 - 15).astype(np.float32).reshape(2, 64, 64)
    np.testing.assert_allclose(mult(g, ident, vals), vals, atol=1e-5)


def gemm(g, a, b, ta=False, tb=False, bias=None, residual=None, epi=0, aux=None, beta=0.0,
         c_init=None, remap=None, split=True, bias_grad_init=None):
    M = a.shape[1] if ta else a.shape[0]
    K = a.shape[0] if ta else a.shape[1]
    N = b.shape[0] if tb else b.shape[1]
    d = GemmDesc()
    da, db = g.dev(a), g.dev(b)
    dc = g.dev(c_init) if c_init is not None else g.zeros((M * N,))
    keep = [da, db, dc]
    d.a, d.b, d.c = da.data_ptr(), db.data_ptr(), dc.data_ptr()
    if bias is not None:
        t = g.dev(bias); keep.append(t); d.bias = t.data_ptr()
    if residual is not None:
        t = g.dev(residual); keep.append(t); d.residual = t.data_ptr()
    daux = None
    if aux is not None:
        daux = g.dev(aux); keep.append(daux); d.aux = daux.data_ptr()
    elif epi == EPI_GELU:
        daux = g.zeros((M * N,)); keep.append(daux); d.aux = daux.data_ptr()
    d.m, d.n, d.k = M, N, K
    d.lda = M if ta else K
    d.ldb = K if tb else N
    d.ldc = N
    d.trans_a, d.trans_b = int(ta), int(tb)
    d.beta = beta
    d.epilogue = epi
    if remap:
        d.remap_t, d.remap_h, d.remap_d = remap
    dbg = None
    if bias_grad_init is not None:
        dbg = g.dev(bias_grad_init); keep.append(dbg); d.bias_grad = dbg.data_ptr()
    if split:
        n = ctypes.c_size_t()
        g.lib.tlh_gemm_workspace_size(ctypes.byref(d), ctypes.byref(n))
        if n.value:
            ws = g.empty((n.value,)); keep.append(ws); d.workspace = ws.data_ptr()
    g.call("tlh_gemm", ctypes.byref(d))
    if dbg is not None:
        return g.host(dc), g.host(dbg)
    return g.host(dc), (g.host(daux) if daux is not None else None)


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(6144, 384, 384), (384, 384, 6144), (100, 70, 37)])
def test_gemm_layouts(g, ta, tb, M, N, K):
    a = O.normal((K, M) if ta else (M, K), 12, 0, 0.5)
    b = O.normal((N, K) if tb else (K, N), 13, 0, 0.5)
    out, _ = gemm(g, a, b, ta, tb)
    expect = O.matmul(a.T if ta else a, b.T if tb else b)
    assert_rel(out.reshape(M, N), expect, 1e-3, "gemm")


@pytest.mark.parametrize("M,N,K,split", [(384, 384, 6144, True), (384, 2048, 6144, True),
                                         (100, 70, 37, True), (384, 384, 6144, False)])
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_gemm_weight_grad_fused_bias_grad(g, M, N, K, split, beta):
    # dW = X^T.dY with db = column sums of dY from the same launch
    x = O.normal((K, M), 130, 0, 0.5)   # X stored [rows=K, in=M]
    dy = O.normal((K, N), 131, 0, 0.5)
    w0, b0 = O.normal((M, N), 132), O.normal((N,), 133)
    dw, db = gemm(g, x, dy, ta=True, beta=beta, c_init=w0, bias_grad_init=b0, split=split)
    assert_rel(dw.reshape(M, N), O.matmul(x.T, dy) + beta * w0, 1e-3, "dW")
    assert_close(db, O.sum_to_shape(dy, [N]) + beta * b0, rtol=1e-4, atol=1e-3, what="db")


@pytest.fixture
def forced_plan(g):
    """tlh_gemm_set_plan is process-wide: restore the planner afterwards."""
    yield lambda *plan: check(g.lib.tlh_gemm_set_plan(*plan), "set_plan")
    check(g.lib.tlh_gemm_set_plan(0, 0, 0, 16), "set_plan")
    check(g.lib.tlh_gemm_set_plan(0, 0, 0, -4), "set_plan")
    check(g.lib.tlh_gemm_set_plan(0, 0, 0, -6), "set_plan")
    check(g.lib.tlh_gemm_set_plan(0, 0, 0, -8), "set_plan")
    check(g.lib.tlh_gemm_set_plan(0, 0, 0, -10), "set_plan")
    check(g.lib.tlh_gemm_set_plan(0, 0, 0, -12), "set_plan")
    check(g.lib.tlh_gemm_set_plan(0, 0, 0, -14), "set_plan")
    check(g.lib.tlh_gemm_set_plan(0, 0, 0, -16), "set_plan")
    check(g.lib.tlh_gemm_set_plan(0, 0, 0, -18), "set_plan")


@pytest.mark.parametrize("K,N", [(1024, 1024), (4096, 1024), (1024, 4096), (384, 2048), (100, 68),
                                 (64, 4)])
@pytest.mark.parametrize("variant", ["plain", "bias_residual", "gelu", "beta"])
def test_gemm_one_row(g, forced_plan, K, N, variant):
    # m = 1 with a workspace runs the GEMV path (K chunks summed in a fixed
    # order); it matches the oracle and the MFMA tile path.
    a, b = O.normal((1, K), 50, 0, 0.5), O.normal((K, N), 51, 0, 0.5)
    ref = O.matmul(a, b)
    kw = {}
    if variant == "bias_residual":
        bias, res = O.normal((N,), 52), O.normal((1, N), 53)
        kw = dict(bias=bias, residual=res)
        ref = O.binary("add", O.binary("add", ref, bias.reshape(1, -1)), res)
    elif variant == "gelu":
        bias = O.normal((N,), 54)
        kw = dict(bias=bias, epi=EPI_GELU)
        pre = O.binary("add", ref, bias.reshape(1, -1))
        ref = O.unary("gelu", pre)
    elif variant == "beta":
        c0 = O.normal((1, N), 55)
        kw = dict(beta=0.5, c_init=c0)
        ref = ref + np.float32(0.5) * c0
    out, aux = gemm(g, a, b, **kw)
    assert_rel(out.reshape(1, N), ref, 1e-3, "gemv")
    if variant == "gelu":
        assert_rel(aux.reshape(1, N), pre, 1e-3, "gemv pre-activation")
    forced_plan(0, 0, 0, -7)  # the MFMA tile path
    out_tiles, _ = gemm(g, a, b, **kw)
    assert_rel(out.reshape(1, N), out_tiles.reshape(1, N), 1e-4, "gemv vs tiles")


@pytest.mark.parametrize("M,N,K,ta", [(384, 2048, 6144, True), (384, 1536, 6144, True),
                                      (6144, 2048, 384, False), (2048, 1024, 256, False)])
def test_gemm_xcd_rectangles(g, forced_plan, M, N, K, ta):
    # The XCD rectangles change which block computes a tile, not how it is
    # computed: the results are bitwise equal to the contiguous block order.
    a = O.normal((K, M) if ta else (M, K), 40, 0, 0.5)
    b = O.normal((K, N), 41, 0, 0.5)
    outs = []
    for toggle in (-6, -5):
        forced_plan(0, 0, 0, toggle)
        out, _ = gemm(g, a, b, ta, False)
        outs.append(out)
    np.testing.assert_array_equal(outs[0], outs[1])
    assert_rel(outs[0].reshape(M, N), O.matmul(a.T if ta else a, b), 1e-3, "gemm")


@pytest.mark.parametrize("M,N,batch", [(384, 384, 1), (1536, 384, 1), (384, 2048, 1),
                                         (384, 384, 3)])
def test_gemm_split_major_xcd_order(g, forced_plan, M, N, batch):
    # Split-K weight gradients (K = 6144; three entries for the batched
    # Q/K/V form): the split-major XCD order changes which block computes a
    # (tile, split), not how: weights and bias gradients are bitwise equal
    # with the order off, and match the oracle.
    K = 6144
    x = O.normal((K, M), 42, 0, 0.5)
    dys = O.normal((batch, K, N), 43, 0, 0.5)
    gap = M * N + N + 64
    outs = []
    for toggle in (-14, -13):
        forced_plan(0, 0, 0, toggle)
        keep = []
        dx_, ddy, dout = g.dev(x), g.dev(dys), g.zeros((batch * gap,))
        d = _batched_desc(dx_, ddy, dout, True, False, M, N, K, batch, 0, K * N, gap)
        d.bias_grad = dout.data_ptr() + 4 * M * N
        d.bias_batch_stride = gap
        _with_workspace(g, keep, d)
        g.call("tlh_gemm", ctypes.byref(d))
        outs.append(g.host(dout))
    np.testing.assert_array_equal(outs[0], outs[1])
    for j in range(batch):
        w = outs[0][j * gap:j * gap + M * N].reshape(M, N)
        assert_rel(w, O.matmul(x.T, dys[j]), 1e-3, f"dW[{j}]")
        bg = outs[0][j * gap + M * N:j * gap + M * N + N]
        assert_close(bg, O.sum_to_shape(dys[j], [N]), rtol=1e-4, atol=1e-3, what=f"db[{j}]")


def _every_layout(g, forced_plan, bm, bn, bk, M=256):
    # A tile plan on a tile-aligned shape (the bounds-free path), every
    # operand layout, and the weight-gradient form with its bias gradient,
    # unsplit and split over K; then ragged edges (the bounds-checked path).
    N, K = 384, 512
    for ta in (False, True):
        for tb in (False, True):
            forced_plan(bm, bn, 1, bk)
            a = O.normal((K, M) if ta else (M, K), 150, 0, 0.5)
            b = O.normal((N, K) if tb else (K, N), 151, 0, 0.5)
            out, _ = gemm(g, a, b, ta, tb)
            expect = O.matmul(a.T if ta else a, b.T if tb else b)
            assert_rel(out.reshape(M, N), expect, 1e-3, f"gemm ta={ta} tb={tb}")
    x, dy = O.normal((K, M), 152, 0, 0.5), O.normal((K, N), 153, 0, 0.5)
    for splits in (1, 4):
        forced_plan(bm, bn, splits, bk)
        dw, db = gemm(g, x, dy, ta=True, bias_grad_init=np.zeros(N, np.float32))
        assert_rel(dw.reshape(M, N), O.matmul(x.T, dy), 1e-3, f"dW splits={splits}")
        assert_close(db, O.sum_to_shape(dy, [N]), rtol=1e-4, atol=1e-3, what="db")
    forced_plan(bm, bn, 1, bk)
    for ta in (False, True):
        for tb in (False, True):
            a = O.normal((100, 200) if ta else (200, 100), 154, 0, 0.5)
            b = O.normal((300, 100) if tb else (100, 300), 155, 0, 0.5)
            out, _ = gemm(g, a, b, ta, tb)
            expect = O.matmul(a.T if ta else a, b.T if tb else b)
            assert_rel(out.reshape(200, 300), expect, 1e-3, f"ragged ta={ta} tb={tb}")


@pytest.mark.parametrize("bm,bn", [(64, 64), (64, 128), (128, 64), (128, 128)])
@pytest.mark.parametrize("bk", [16, 32])
def test_gemm_every_tile_plan(g, forced_plan, bm, bn, bk):
    _every_layout(g, forced_plan, bm, bn, bk)


@pytest.mark.parametrize("tile", [64, 128])
def test_gemm_tile16_square_plans(g, forced_plan, tile):
    # The 16x16x4 MFMA kernel at 64x64 and 128x128 tiles (set_plan bm = 16):
    # its row-contiguous operand tiles (A transposed, B not) are read with
    # interleaved subtiles (b64 / b128 LDS reads), and it carries the bias
    # gradient of the weight-gradient form.
    _every_layout(g, forced_plan, 16, tile, 32)


@pytest.mark.parametrize("bk", [32, 64])
def test_gemm_96x64_tiles(g, forced_plan, bk):
    # 96x64 tiles on the 16x16x4 kernel (4 waves of 48x32, or 8 in two K
    # groups): every layout on a tile-aligned shape (288 = 3 x 96 rows), the
    # weight-gradient form with its bias gradient (4 waves), split over K,
    # and ragged edges
    _every_layout(g, forced_plan, 96, 64, bk, M=288)


def test_gemm_matmul_bias_configuration(g):
    # [768,384].[384,1536] + bias (the matmul + bias configuration): 192
    # tiles of 96x64, one round on the CUs; against fp64
    M, K, N = 768, 384, 1536
    a, b = O.normal((M, K), 156, 0, 0.02), O.normal((K, N), 157, 0, 0.02)
    bias = O.normal((N,), 158, 0, 0.02)
    out, _ = gemm(g, a, b, False, False, bias=bias)
    expect = a.astype(np.float64) @ b.astype(np.float64) + bias
    assert_rel(out.reshape(M, N), expect, 1e-3, "matmul + bias")


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("K", [384, 1536])
def test_gemm_tail_split(g, forced_plan, ta, tb, K):
    # 6144 x 384 is 576 tiles of 64x64: 512 whole-K blocks (2 per CU) and
    # 64 tiles cut into K chunks summed afterwards. Same result with the
    # tail split off, bit-identical run to run, every epilogue input. (The
    # planner's 96x96 tiles, one per CU, are switched off.)
    forced_plan(0, 0, 0, -11)
    M, N = 6144, 384
    a = O.normal((K, M) if ta else (M, K), 160, 0, 0.5)
    b = O.normal((N, K) if tb else (K, N), 161, 0, 0.5)
    bias, res, c0 = O.normal((N,), 162), O.normal((M, N), 163), O.normal((M, N), 164)
    expect = O.matmul(a.T if ta else a, b.T if tb else b) + bias + c0 + res
    outs = []
    for on in (True, True, False):
        forced_plan(0, 0, 0, -4 if on else -3)
        out, _ = gemm(g, a, b, ta, tb, bias=bias, residual=res, beta=1.0, c_init=c0)
        assert_rel(out.reshape(M, N), expect, 1e-3, f"tail split {on}")
        outs.append(out)
    np.testing.assert_array_equal(outs[0], outs[1])


def test_gemm_tail_split_gelu_epilogues(g, forced_plan):
    # the tail tiles' reduction applies the GELU forward (writing the
    # pre-activation) and the GELU' epilogue like the whole-K blocks do
    forced_plan(0, 0, 0, -11)  # 64x64 tiles (576, so a tail split)
    M, N, K = 6144, 384, 1536
    a, b = O.normal((M, K), 165, 0, 0.05), O.normal((K, N), 166, 0, 0.05)
    bias = O.normal((N,), 167)
    pre = O.matmul(a, b) + bias
    out, aux = gemm(g, a, b, bias=bias, epi=EPI_GELU)
    assert_rel(aux.reshape(M, N), pre, 1e-3, "pre-activation")
    assert_rel(out.reshape(M, N), O.unary("gelu", pre), 1e-3, "gelu")
    out, _ = gemm(g, a, b, epi=EPI_GELU_BWD, aux=pre)
    assert_rel(out.reshape(M, N), O.matmul(a, b) * O.unary("gelu_derivative", pre), 1e-3, "gelu'")


@pytest.mark.parametrize("N", [4096, 1024])
def test_gemm_d1024_shapes(g, N):
    # The d=1024 products of the scaled configuration, [8192,1024].[1024,N],
    # N = 4096 (FFN up) and 1024 (attention projections), through the same
    # call the benchmark times (tlh_gemm, planner's choice, no workspace).
    # Oracle-free checks against float64 on the host: 96 sampled rows in
    # full, and every column's sum over all 8192 rows, which equals
    # (1^T A) B and so covers every output row.
    M, K = 8192, 1024
    a = O.normal((M, K), 170, 0, 0.02)
    b = O.normal((K, N), 171, 0, 0.02)
    out, _ = gemm(g, a, b, split=False)
    out = out.reshape(M, N)
    rows = np.sort(np.concatenate([[0, 63, 64, M - 1], O.uniform_u32((92,), 172, M)]))
    ref = a[rows].astype(np.float64) @ b.astype(np.float64)
    assert_rel(out[rows], ref, 1e-3, "sampled rows")
    col = a.astype(np.float64).sum(axis=0) @ b.astype(np.float64)
    got = out.astype(np.float64).sum(axis=0)
    # |sum| of 8192 terms of size ~|ref| cancels; bound by the summed magnitudes
    scale = np.abs(out.astype(np.float64)).sum(axis=0)
    assert np.all(np.abs(got - col) <= 1e-4 * scale), float(np.max(np.abs(got - col) / scale))


def test_gemm_bias_residual_beta(g):
    M, N, K = 1000, 384, 384
    a, b = O.normal((M, K), 14, 0, 0.1), O.normal((K, N), 15, 0, 0.1)
    bias, res, c0 = O.normal((N,), 16), O.normal((M, N), 17), O.normal((M, N), 18)
    out, _ = gemm(g, a, b, bias=bias, residual=res, beta=1.0, c_init=c0)
    expect = O.matmul(a, b) + bias + c0 + res
    assert_rel(out.reshape(M, N), expect, 1e-3)


def test_gemm_gelu_and_gelu_backward(g):
    M, N, K = 768, 1536, 384
    a, b = O.normal((M, K), 19, 0, 0.1), O.normal((K, N), 20, 0, 0.1)
    bias = O.normal((N,), 21, 0, 0.1)
    out, pre = gemm(g, a, b, bias=bias, epi=EPI_GELU)
    u = O.binary("add", O.matmul(a, b), bias.reshape(1, N))
    assert_rel(pre.reshape(M, N), u, 1e-3)
    assert_rel(out.reshape(M, N), O.unary("gelu", u), 1e-3)
    # backward epilogue: C = (dY . W^T) * GELU'(u) with W stored [N, K]
    uu = O.normal((M, N), 24)
    dy = O.normal((M, K), 25)
    w = O.normal((N, K), 26, 0, 0.1)
    out2, _ = gemm(g, dy, w, tb=True, epi=EPI_GELU_BWD, aux=uu)
    expect = O.binary("hadamard", O.matmul(dy, w.T), O.unary("gelu_derivative", uu))
    assert_rel(out2.reshape(M, N), expect, 1e-3)


def _batched_desc(a, b, c, ta, tb, M, N, K, batch, sa, sb, sc):
    d = GemmDesc()
    d.a, d.b, d.c = a.data_ptr(), b.data_ptr(), c.data_ptr()
    d.m, d.n, d.k = M, N, K
    d.lda, d.ldb, d.ldc = (M if ta else K), (K if tb else N), N
    d.trans_a, d.trans_b = int(ta), int(tb)
    d.batch, d.batch_stride_a, d.batch_stride_b, d.batch_stride_c = batch, sa, sb, sc
    return d


def _with_workspace(g, keep, d):
    n = ctypes.c_size_t()
    check(g.lib.tlh_gemm_workspace_size(ctypes.byref(d), ctypes.byref(n)), "ws")
    if n.value:
        ws = g.empty((n.value,))
        keep.append(ws)
        d.workspace = ws.data_ptr()


@pytest.mark.parametrize("K", [6144, 96])
def test_gemm_batched_weight_grads_with_bias_grads(g, K):
    # dW_j = X^T.dY_j and db_j = column sums of dY_j for three dY planes, one
    # launch (the Q/K/V weight gradients), with split-K when K is long
    M = N = 128
    x = O.normal((K, M), 140, 0, 0.5)
    dys = O.normal((3, K, N), 141, 0, 0.5)
    gap = M * N + N + 64  # weight, bias and padding of one entry
    out = np.zeros(3 * gap, np.float32)
    keep = []
    dx_, ddy, dout = g.dev(x), g.dev(dys), g.dev(out)
    d = _batched_desc(dx_, ddy, dout, True, False, M, N, K, 3, 0, K * N, gap)
    d.bias_grad = dout.data_ptr() + 4 * M * N
    d.bias_batch_stride = gap
    _with_workspace(g, keep, d)
    g.call("tlh_gemm", ctypes.byref(d))
    got = g.host(dout)
    for j in range(3):
        w = got[j * gap:j * gap + M * N].reshape(M, N)
        bg = got[j * gap + M * N:j * gap + M * N + N]
        assert_rel(w, O.matmul(x.T, dys[j]), 1e-3, f"dW[{j}]")
        assert_close(bg, O.sum_to_shape(dys[j], [N]), rtol=1e-4, atol=1e-3, what=f"db[{j}]")


@pytest.mark.parametrize("splits", [3, 8, 16])
@pytest.mark.parametrize("beta", [0.0, 1.0])
@pytest.mark.parametrize("M", [384, 2])
def test_gemm_split_k_reducers_agree(g, forced_plan, splits, beta, M):
    # The split-K partials are summed by a float4 kernel over a (plane,
    # entry) grid or by the grid-stride kernel; both add in the same fixed
    # order, so the weights and bias gradients agree bit for bit. M = 2:
    # fewer float4 groups in a plane than bias-gradient columns.
    N, K = 256, 6144
    x = O.normal((K, M), 147, 0, 0.5)
    dys = O.normal((3, K, N), 148, 0, 0.5)
    gap = M * N + N + 64
    init = O.normal((3 * gap,), 149, 0, 0.1)
    outs = []
    for toggle in (-9, -10):
        forced_plan(0, 0, 0, toggle)
        forced_plan(64, 64, splits, 32)
        keep = []
        dx_, ddy, dout = g.dev(x), g.dev(dys), g.dev(init)
        d = _batched_desc(dx_, ddy, dout, True, False, M, N, K, 3, 0, K * N, gap)
        d.bias_grad = dout.data_ptr() + 4 * M * N
        d.bias_batch_stride = gap
        d.beta = beta
        _with_workspace(g, keep, d)
        g.call("tlh_gemm", ctypes.byref(d))
        outs.append(g.host(dout))
    np.testing.assert_array_equal(outs[0], outs[1])
    for j in range(3):
        w = outs[1][j * gap:j * gap + M * N].reshape(M, N)
        w0 = init[j * gap:j * gap + M * N].reshape(M, N)
        bg = outs[1][j * gap + M * N:j * gap + M * N + N]
        bg0 = init[j * gap + M * N:j * gap + M * N + N]
        assert_rel(w, O.matmul(x.T, dys[j]) + beta * w0, 1e-3, f"dW[{j}]")
        assert_close(bg, O.sum_to_shape(dys[j], [N]) + beta * bg0, rtol=1e-4, atol=1e-3,
                     what=f"db[{j}]")


@pytest.mark.parametrize("M,N,K", [(6144, 384, 384), (100, 70, 64)])
def test_gemm_summed_batches(g, M, N, K):
    # C = beta*C0 + residual + bias + sum_j A_j.W_j^T (the Q/K/V input gradient)
    a = O.normal((3, M, K), 142, 0, 0.5)
    w = O.normal((3, N, K), 143, 0, 0.5)
    c0, res, bias = O.normal((M, N), 144), O.normal((M, N), 145), O.normal((N,), 146)
    keep = []
    da, dw, dc = g.dev(a), g.dev(w), g.dev(c0)
    d = _batched_desc(da, dw, dc, False, True, M, N, K, 3, M * K, N * K, 0)
    d.sum_batches = 1
    d.beta = 1.0
    dres, dbias = g.dev(res), g.dev(bias)
    d.residual, d.bias = dres.data_ptr(), dbias.data_ptr()
    _with_workspace(g, keep, d)
    g.call("tlh_gemm", ctypes.byref(d))
    expect = sum(O.matmul(a[j], w[j].T) for j in range(3)) + c0 + res + bias
    assert_rel(g.host(dc).reshape(M, N), expect, 1e-3, "summed")


@pytest.mark.parametrize("bn", [96, 64])
@pytest.mark.parametrize("bk", [32, 64])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_tile96(g, forced_plan, ta, tb, bk, bn):
    # 96x96 and 96x64 tiles on the 16x16x4 MFMA: every operand layout on the
    # step's [6144,384] product (exactly 256 tiles of 96x96), every epilogue,
    # the head-layout store (96-column tiles straddle the 64-wide heads), the
    # batched and summed-batch (K-segmented) forms and the bounds-checked
    # ragged path. bk 32: 4 waves; bk 64: 8 waves in two K groups over K
    # tiles of 64.
    forced_plan(96, bn, 1, bk)
    M, N, K = 6144, 384, 384
    a = O.normal((K, M) if ta else (M, K), 180, 0, 0.5)
    b = O.normal((N, K) if tb else (K, N), 181, 0, 0.5)
    prod = O.matmul(a.T if ta else a, b.T if tb else b)
    out, _ = gemm(g, a, b, ta, tb)
    assert_rel(out.reshape(M, N), prod, 1e-3, "plain")
    bias, res, c0 = O.normal((N,), 182), O.normal((M, N), 183), O.normal((M, N), 184)
    out, _ = gemm(g, a, b, ta, tb, bias=bias, residual=res, beta=1.0, c_init=c0)
    assert_rel(out.reshape(M, N), prod + bias + c0 + res, 1e-3, "bias+residual+beta")
    out, pre = gemm(g, a, b, ta, tb, bias=bias, epi=EPI_GELU)
    u = O.binary("add", prod, bias.reshape(1, N))
    assert_rel(pre.reshape(M, N), u, 1e-3, "gelu pre-activation")
    assert_rel(out.reshape(M, N), O.unary("gelu", u), 1e-3, "gelu")
    out, _ = gemm(g, a, b, ta, tb, epi=EPI_GELU_BWD, aux=u)
    assert_rel(out.reshape(M, N), prod * O.unary("gelu_derivative", u), 1e-3, "gelu'")
    if not ta:
        T, H, D = 192, 6, 64
        out, _ = gemm(g, a, b, ta, tb, bias=bias, remap=(T, H, D))
        y = O.binary("add", prod, bias.reshape(1, -1)).reshape(M // T, T, H, D)
        assert_rel(out.reshape(M // T, H, T, D), y.transpose(0, 2, 1, 3), 1e-3, "head remap")
    # ragged edges: bounds-checked loads and stores
    a2 = O.normal((100, 200) if ta else (200, 100), 185, 0, 0.5)
    b2 = O.normal((300, 100) if tb else (100, 300), 186, 0, 0.5)
    out, _ = gemm(g, a2, b2, ta, tb)
    assert_rel(out.reshape(200, 300), O.matmul(a2.T if ta else a2, b2.T if tb else b2), 1e-3,
               "ragged")


@pytest.mark.parametrize("bn", [96, 64])
@pytest.mark.parametrize("bk", [32, 64])
def test_gemm_tile96_batched_and_summed(g, forced_plan, bk, bn):
    forced_plan(96, bn, 1, bk)
    M, N, K = 960, 192, 384
    a = O.normal((3, M, K), 187, 0, 0.5)
    w = O.normal((3, N, K), 188, 0, 0.5)
    keep = []
    da, dw, dc = g.dev(a), g.dev(w), g.zeros((3 * M * N,))
    d = _batched_desc(da, dw, dc, False, True, M, N, K, 3, M * K, N * K, M * N)
    g.call("tlh_gemm", ctypes.byref(d))
    got = g.host(dc).reshape(3, M, N)
    for j in range(3):
        assert_rel(got[j], O.matmul(a[j], w[j].T), 1e-3, f"batched[{j}]")
    c0, res, bias = O.normal((M, N), 189), O.normal((M, N), 190), O.normal((N,), 191)
    dc = g.dev(c0)
    d = _batched_desc(da, dw, dc, False, True, M, N, K, 3, M * K, N * K, 0)
    d.sum_batches = 1
    d.beta = 1.0
    dres, dbias = g.dev(res), g.dev(bias)
    d.residual, d.bias = dres.data_ptr(), dbias.data_ptr()
    _with_workspace(g, keep, d)
    g.call("tlh_gemm", ctypes.byref(d))
    expect = sum(O.matmul(a[j], w[j].T) for j in range(3)) + c0 + res + bias
    assert_rel(g.host(dc).reshape(M, N), expect, 1e-3, "summed")


def test_gemm_head_remap(g):
    B, T, H, D = 4, 48, 6, 64
    a, b = O.normal((B * T, H * D), 27, 0, 0.1), O.normal((H * D, H * D), 28, 0, 0.1)
    bias = O.normal((H * D,), 29)
    out, _ = gemm(g, a, b, bias=bias, remap=(T, H, D))
    y = O.binary("add", O.matmul(a, b), bias.reshape(1, -1)).reshape(B, T, H, D)
    assert_rel(out.reshape(B, H, T, D), y.transpose(0, 2, 1, 3), 1e-3)


# ---------------------------------------------------------------------------
# reductions
# ---------------------------------------------------------------------------
REDUCTIONS = [
    ((2, 3), [1, 3]), ((2, 3), [2, 1]), ((2, 3, 4), [1, 3, 1]), ((2, 3, 4), [2, 1, 1]),
    ((2, 3, 4), [1, 1, 1]), ((2, 3, 4), [4]), ((1, 4), [4]),          # KATs 344-430
    ((32, 384, 384), [384, 384]), ((32, 192, 384), [1, 384]),        # weight / bias grads
    ((32, 192, 384), [32, 192, 1]), ((32, 6, 192, 192), [32, 6, 192, 1]),  # sum(axis)
    ((5, 7, 9, 11), [5, 1, 9, 1]), ((6144, 384), [6144, 384]),      # generic, identity copy
]


@pytest.mark.parametrize("shape,target", REDUCTIONS)
def test_sum_to_shape(g, shape, target):
    x = O.normal(shape, 30)
    al = O.aligned_shape(shape, target)
    out = g.empty(al)
    g.call("tlh_sum_to_shape", g.dev(x), out, len(shape), u32(shape), u32(al))
    assert_close(g.host(out).reshape(target), O.sum_to_shape(x, target), rtol=1e-4, atol=1e-4)


# Tall column sums (bias gradients) take row-chunk partials in a workspace;
# the others need none and run the single-pass kernels.
TWO_PASS = [
    ((32, 192, 384), [1, 1, 384], True), ((6144, 2048), [1, 2048], True),
    ((300, 1536), [1, 1536], True),      # last chunk shorter than the rest
    ((8192, 4096), [1, 4096], True),     # d = 1024 FFN bias gradient
    ((6144, 386), [1, 386], False),      # columns not float4-aligned
    ((200, 384), [1, 384], False),       # too few rows to split
    ((32, 192, 384), [32, 192, 1], False),
]


@pytest.mark.parametrize("shape,target,split", TWO_PASS)
def test_sum_to_shape_workspace(g, shape, target, split):
    x = O.normal(shape, 33)
    al = O.aligned_shape(shape, target)
    elems = ctypes.c_size_t(123)
    check(g.lib.tlh_sum_to_shape_workspace(len(shape), u32(shape), u32(al), ctypes.byref(elems)),
          "workspace")
    assert (elems.value > 0) == split
    # float64 sums: at 8192 rows the float32 sequential oracle's own rounding
    # reaches the tolerance on near-zero sums
    axes = tuple(d for d in range(len(shape)) if al[d] == 1 and shape[d] != 1)
    want = x.astype(np.float64).sum(axis=axes, keepdims=True).reshape(target)
    ws = g.empty((max(1, elems.value),))
    xd = g.dev(x)
    outs = []
    for _ in range(2):
        out = g.empty(al)
        g.call("tlh_sum_to_shape_ws", xd, out, len(shape), u32(shape), u32(al), ws, elems.value)
        outs.append(g.host(out))
    assert_close(outs[0].reshape(target), want, rtol=1e-4, atol=1e-4)
    np.testing.assert_array_equal(outs[0], outs[1])  # deterministic
    rows = x.size // int(np.prod(target))
    # too little scratch: the single-pass kernel (its per-thread sequential
    # float32 sums drift past atol 1e-4 beyond ~6k rows; the two-pass ones do not)
    if split and rows <= 6144:
        out = g.empty(al)
        g.call("tlh_sum_to_shape_ws", xd, out, len(shape), u32(shape), u32(al), ws,
               elems.value - 1)
        assert_close(g.host(out).reshape(target), want, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("shape,target", [((2, 3), [2, 1]), ((32, 6, 192, 192), [32, 6, 192, 1]),
                                          ((7, 9, 5), [1, 9, 5]), ((4, 5, 6), [4, 1, 6])])
def test_max_to_shape(g, shape, target):
    x = O.normal(shape, 31)
    al = O.aligned_shape(shape, target)
    out = g.empty(al)
    g.call("tlh_max_to_shape", g.dev(x), out, len(shape), u32(shape), u32(al))
    np.testing.assert_array_equal(g.host(out).reshape(target), O.max_to_shape(x, target))


@pytest.mark.parametrize("n", [1, 6, 5000, 6144 * 384])
def test_sum_all(g, n):
    x = O.normal((n,), 32)
    out = g.empty((1,))
    g.call("tlh_sum", g.dev(x), n, out)
    np.testing.assert_allclose(g.host(out)[0], x.astype(np.float64).sum(), rtol=1e-4, atol=1e-3)


def test_argmax_kats(g):
    # test_metal_runtime.cpp:509-531 + lowest index on ties + -inf/NaN rows
    cases = [np.array([1, 4, 2, 9, 3, 5], np.float32)]
    big = np.zeros(5000, np.float32); big[4097] = 100; cases.append(big)
    ties = np.zeros(3000, np.float32); ties[[17, 500, 2999]] = 7; cases.append(ties)
    cases.append(np.full(300, -np.inf, np.float32))
    nan = O.normal((2048,), 33); nan[5] = np.nan; cases.append(nan)
    for x in cases + [O.normal((2048,), 34), O.normal((6144 * 2048,), 35)]:
        out = g.empty((1,), torch.int32)
        g.call("tlh_argmax", g.dev(x), x.size, out)
        assert int(g.host(out)[0]) == O.argmax(x)


# ---------------------------------------------------------------------------
# top-k sampling (inference.h:14-43, 80-84)
# ---------------------------------------------------------------------------
def sample(g, x, top_k, temperature, seed=0, counter=0, uniforms=None, eos=0, resample=False,
           max_draws=1):
    x = np.ascontiguousarray(x, np.float32)
    rows, V = (1, x.size) if x.ndim == 1 else x.shape
    dx = g.dev(x)
    tokens, draws = g.empty((rows,), torch.int32), g.empty((rows,), torch.int32)
    du = g.dev_f64(uniforms) if uniforms is not None else None
    g.call("tlh_sample_top_k", dx, rows, V, V, top_k, temperature, seed, counter, du, eos,
           int(resample), max_draws, tokens, draws)
    return g.host(tokens).view(np.uint32), g.host(draws).view(np.uint32)


@pytest.mark.parametrize("rows,V,top_k,temperature", [
    (1, 2048, 40, 0.6), (7, 2048, 5, 1.3), (3, 97, 12, 0.35), (2, 4096, 4096, 0.9),
    (4, 300, 0, 0.5), (5, 256, 1000, 2.0), (1, 1, 1, 1.0)])
def test_sample_top_k_matches_oracle(g, rows, V, top_k, temperature):
    # bit-exact tokens and draw counts against the oracle on the same logits
    # and the same SplitMix64 draws, with and without the EOS re-draw
    x = O.normal((rows, V), 1200 + V, 0.0, 2.0)
    for seed, counter in ((3, 0), (4, 1000)):
        got = sample(g, x, top_k, temperature, seed, counter)
        ref = O.sample_top_k(x, top_k, temperature, seed, counter)
        np.testing.assert_array_equal(got[0], ref[0])
        np.testing.assert_array_equal(got[1], ref[1])
    eos = int(O.argmax(x[0]))  # the most likely token of row 0
    got = sample(g, x, top_k, temperature, 5, 0, eos=eos, resample=True, max_draws=32)
    ref = O.sample_top_k(x, top_k, temperature, 5, 0, eos=eos, resample_eos=True, max_draws=32)
    np.testing.assert_array_equal(got[0], ref[0])
    np.testing.assert_array_equal(got[1], ref[1])


def test_sample_top_k_ties_nan_and_many_draws(g):
    x = O.normal((64, 512), 1300, 0.0, 1.0)
    x[:, 17] = x[:, 300] = x.max(axis=1) + 0.5  # ties at the top
    x[::3, 5] = np.nan                           # NaN ranks as -INF
    for k in (1, 2, 9):
        got = sample(g, x, k, 0.8, seed=11)
        ref = O.sample_top_k(x, k, 0.8, seed=11)
        np.testing.assert_array_equal(got[0], ref[0])
    assert np.all(sample(g, x, 1, 0.8)[0] == 17)
    # 2000 rows of one row's logits: frequencies and the oracle, token for token
    y = np.tile(O.normal((2048,), 1301, 0.0, 2.0), (2000, 1))
    got = sample(g, y, 40, 0.6, seed=12)
    np.testing.assert_array_equal(got[0], O.sample_top_k(y, 40, 0.6, seed=12)[0])


def test_sample_top_k_reproduces_the_reference_draws(g):
    # Fed the uniforms the reference's std::discrete_distribution drew
    # (tests/golden/sampler_reference.json, from the reference's own
    # inference::sample_top_k on std::mt19937), the kernel returns the
    # reference's tokens.
    import json
    from pathlib import Path
    gold = json.loads((Path(__file__).parent / "golden" / "sampler_reference.json").read_text())
    for i, c in enumerate(gold["cases"]):
        x = O.normal((c["vocab"],), gold["logit_seed"] + i, 0.0, 2.0)
        u = np.array([float.fromhex(h) for h in c["uniforms"]])
        rows = np.tile(x, (len(u), 1))
        got = sample(g, rows, c["top_k"], c["temperature"], uniforms=u)
        np.testing.assert_array_equal(got[0], c["tokens"], err_msg=f"case {i}")


def test_sample_top_k_rejects_bad_arguments(g):
    x, out = g.dev(np.zeros((2, 5000), np.float32)), g.empty((2,), torch.int32)
    for args in ((2, 5000, 5000, 5, 1.0, 1), (2, 64, 64, 5, 0.0, 1), (2, 64, 64, 5, np.inf, 1),
                 (2, 64, 32, 5, 1.0, 1), (2, 64, 64, 5, 1.0, 0)):
        rows, V, stride, k, t, draws = args
        st = g.lib.tlh_sample_top_k(x.data_ptr(), rows, V, stride, k, float(t), 0, 0, None, 0, 0,
                                    draws, out.data_ptr(), None, g.stream)
        assert st != 0, args


def test_argmax_rows(g):
    x = O.normal((64, 2048), 36)
    x[3, [10, 20]] = 99.0
    out = g.empty((64,), torch.int32)
    g.call("tlh_argmax_rows", g.dev(x), 64, 2048, out)
    got = g.host(out)
    for r in range(64):
        assert got[r] == O.argmax(x[r])


def test_gradient_norm_single_and_multi(g):
    # KAT 169 (test_metal_runtime.cpp:595-615) + GPT-sized multi-tensor
    first, second = np.array([3, 4, 0], np.float32), np.array([12], np.float32)
    s = g.zeros((1,))
    g.call("tlh_accumulate_gradient_squared_norm", g.dev(first), 3, s)
    g.call("tlh_accumulate_gradient_squared_norm", g.dev(second), 1, s)
    assert abs(g.host(s)[0] - 169.0) < 1e-5
    # 16-byte aligned tensors (float4 path, n % 4 tails) and two that start
    # one float past an aligned address (scalar path)
    sizes = [384 * 384, 384, 1536 * 384, 1536, 2048 * 384, 7, 1, 9001, 5]
    skew = [0, 0, 0, 0, 0, 0, 0, 1, 1]
    grads = [g.dev(O.normal((n + k,), 40 + i)) for i, (n, k) in enumerate(zip(sizes, skew))]
    ptrs = torch.tensor([t.data_ptr() + 4 * k for t, k in zip(grads, skew)], dtype=torch.int64,
                        device="cuda")
    dsz = torch.tensor(sizes, dtype=torch.int64, device="cuda")
    partials = g.empty((1024,))
    out = g.empty((1,))
    g.call("tlh_gradient_squared_norm_multi", ptrs, dsz, len(sizes), partials, out)
    expect = sum(float((g.host(t)[k:].astype(np.float64) ** 2).sum())
                 for t, k in zip(grads, skew))
    assert abs(g.host(out)[0] - expect) / expect < 1e-5


def test_column_sum(g):
    x = O.normal((6144, 384), 50)
    old = O.normal((384,), 51)
    out = g.dev(old)
    g.call("tlh_column_sum", g.dev(x), 6144, 384, out, 1.0)
    assert_close(g.host(out), O.sum_to_shape(x, [384]) + old, rtol=1e-4, atol=1e-3)


# ---------------------------------------------------------------------------
# row ops
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rows,cols", [(6144, 2048), (36864, 192), (2, 3), (100, 2500), (7, 1)])
def test_softmax(g, rows, cols):
    x = O.normal((rows, cols), 52, 0, 3)
    out = g.empty((rows, cols))
    g.call("tlh_softmax", g.dev(x), out, rows, cols)
    assert_close(g.host(out), O.softmax(x))


def test_softmax_stability_kat(g):
    # test_metal_runtime.cpp:432-472 rank-4 with +-1000 rows
    x = np.array([1, 2, 3, 3, 2, 1, 1000, 1001, 1002, -1000, -1000, -1000], np.float32)
    out = g.empty((4, 3))
    g.call("tlh_softmax", g.dev(x.reshape(4, 3)), out, 4, 3)
    assert_close(g.host(out), O.softmax(x.reshape(4, 3)))


# cols 2048 / 1024 / 512 / 192 run the register kernels for 8 / 4 / 2 / 1
# float4 per lane and 77 the looped kernel; (6144, 2048) is the row-op
# configuration the benchmark times
@pytest.mark.parametrize("rows,cols", [(6144, 2048), (6144, 1024), (6144, 512), (36864, 192),
                                       (50, 77)])
def test_softmax_backward(g, rows, cols):
    y = O.softmax(O.normal((rows, cols), 53, 0, 2))
    gr = O.normal((rows, cols), 54)
    out = g.empty((rows, cols))
    g.call("tlh_softmax_backward", g.dev(gr), g.dev(y), out, rows, cols)
    assert_close(g.host(out), O.softmax_backward(gr, y), rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("rows,vocab", [(6144, 2048), (4, 3), (33, 1000)])
def test_cross_entropy(g, rows, vocab):
    logits = O.normal((rows, vocab), 55, 0, 2)
    t = O.uniform_u32((rows,), 56, vocab)
    t[0] = vocab  # invalid target -> +INF row
    loss = g.empty((rows,))
    g.call("tlh_cross_entropy_rows", g.dev(logits), g.dev(t), loss, rows, vocab)
    assert_close(g.host(loss), O.cross_entropy(logits, t)[:, 0])
    grad = g.empty((rows, vocab))
    g.call("tlh_cross_entropy_rows_backward", g.dev(logits), g.dev(t), grad, rows, vocab, None)
    assert_close(g.host(grad), O.cross_entropy_backward(logits, t), rtol=1e-4, atol=1e-6)
    scale = 1.0 / rows
    loss2, grad2 = g.empty((rows,)), g.empty((rows, vocab))
    g.call("tlh_cross_entropy_rows_fused", g.dev(logits), g.dev(t), loss2, grad2, rows, vocab,
           scale)
    assert_close(g.host(loss2), O.cross_entropy(logits, t)[:, 0])
    expect = O.cross_entropy_backward(logits, t) * np.float32(scale)
    assert_close(g.host(grad2), expect, rtol=1e-4, atol=1e-8)


@pytest.mark.parametrize("rows,cols", [(6144, 384), (8192, 1024), (2, 2), (10, 300)])
@pytest.mark.parametrize("with_gain", [False, True])
def test_rms_norm(g, rows, cols, with_gain):
    x = O.normal((rows, cols), 57)
    if rows == 2:
        x = np.array([[3, 4], [0, 0]], np.float32)  # KAT: zero row -> rms = 1e-3
    gain = O.normal((cols,), 58, 1, 0.02) if with_gain else None
    eps = 1e-5 if with_gain else 1e-6
    y, r = g.empty((rows, cols)), g.empty((rows,))
    g.call("tlh_rms_norm", g.dev(x), g.dev(gain) if with_gain else None, y, r, rows, cols, eps)
    assert_close(g.host(y), O.rms_norm(x, gain, eps))
    assert_close(g.host(r), O.rms(x, eps)[:, 0])
    r2 = g.empty((rows,))
    g.call("tlh_rms", g.dev(x), r2, rows, cols, eps)
    assert_close(g.host(r2), O.rms(x, eps)[:, 0])


@pytest.mark.parametrize("rows,cols", [(6144, 384), (9, 300)])
@pytest.mark.parametrize("with_gain", [False, True])
def test_rms_norm_backward(g, rows, cols, with_gain):
    x, gr = O.normal((rows, cols), 59), O.normal((rows, cols), 60)
    gain = O.normal((cols,), 61, 1, 0.02) if with_gain else None
    old = O.normal((rows, cols), 62)
    dx = g.dev(old)
    dgain = g.empty((cols,)) if with_gain else None
    g.call("tlh_rms_norm_backward", g.dev(gr), g.dev(x), g.dev(gain) if with_gain else None,
           dx, dgain, rows, cols, 1e-6, 1.0)
    edx, edgain = O.rms_norm_backward(gr, x, gain, 1e-6)
    assert_close(g.host(dx), edx + old, rtol=1e-4, atol=1e-5)
    if with_gain:
        assert_close(g.host(dgain), edgain, rtol=1e-4, atol=1e-3)


# ---------------------------------------------------------------------------
# embedding
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rows,dim,n", [(2048, 384, 6144), (4, 3, 4), (192, 1023, 50)])
def test_embedding_lookup_bit_exact(g, rows, dim, n):
    w = O.normal((rows, dim), 63)
    ids = O.uniform_u32((n,), 64, rows)
    out = g.empty((n, dim))
    g.call("tlh_embedding_lookup", g.dev(w), rows, dim, g.dev(ids), n, out)
    np.testing.assert_array_equal(g.host(out), O.embedding_lookup(w, ids))


def test_embedding_add_positions(g):
    B, T, D, V = 32, 192, 384, 2048
    tok, pos = O.normal((V, D), 65), O.normal((T, D), 66)
    ids = O.uniform_u32((B, T), 67, V)
    out = g.empty((B, T, D))
    g.call("tlh_embedding_add_positions", g.dev(tok), V, g.dev(pos), g.dev(ids), B, T, D, out)
    expect = O.embedding_lookup(tok, ids) + pos[None, :, :]
    np.testing.assert_array_equal(g.host(out), expect)


def test_embedding_out_of_range_ids(g):
    # The reference reads unchecked; an id past the table gives a NaN row
    # (gather) or is dropped (scatter), never an access outside the table.
    rows, dim = 5, 8
    w = O.normal((rows, dim), 70)
    ids = np.array([1, 5, 0, 1000000], np.uint32)
    out = g.empty((4, dim))
    g.call("tlh_embedding_lookup", g.dev(w), rows, dim, g.dev(ids), 4, out)
    got = g.host(out)
    np.testing.assert_array_equal(got[[0, 2]], w[[1, 0]])
    assert np.isnan(got[[1, 3]]).all()
    dst = g.zeros((rows, dim))
    values = O.normal((4, dim), 71)
    g.call("tlh_scatter_add_rows", g.dev(values), g.dev(ids), 4, dim, dst, rows)
    expect = np.zeros((rows, dim), np.float32)
    expect[1] += values[0]
    expect[0] += values[2]
    np.testing.assert_array_equal(g.host(dst), expect)


def test_scatter_add_rows(g):
    # KAT (test_metal_runtime.cpp:571-593) then the GPT shape
    base = np.arange(100, 112, dtype=np.float32).reshape(4, 3)
    values = np.array([1, 2, 3, 4, 5, 6, 10, 20, 30, 7, 8, 9], np.float32).reshape(4, 3)
    ids = np.array([2, 0, 2, 1], np.uint32)
    dst = g.dev(base)
    g.call("tlh_scatter_add_rows", g.dev(values), g.dev(ids), 4, 3, dst, 4)
    np.testing.assert_array_equal(g.host(dst), O.scatter_add_rows(base, ids, values))


@pytest.mark.parametrize("V,D,n,skew", [
    (2048, 384, 6144, None),      # the GPT token table
    (2048, 1024, 8192, None),     # the scaled one
    (50000, 64, 3000, None),      # several destination rows per block
    (3, 13000, 2500, None),       # rows longer than one block's LDS: column chunks
    (100, 7, 1, None), (100, 7, 1023, None), (100, 7, 1025, None),
    (64, 33, 5000, "one"),        # every id the same row
    (64, 33, 5000, "two"),        # two rows, interleaved
])
def test_scatter_add_rows_sequential_order(g, V, D, n, skew):
    # Adds happen in increasing index order per element, without atomics:
    # the result equals the sequential loop bit for bit.
    values = O.normal((n, D), 68)
    ids = O.uniform_u32((n,), 69, V)
    if skew == "one":
        ids[:] = 17
    elif skew == "two":
        ids = np.where(np.arange(n) % 3 == 0, 5, 60).astype(np.uint32)
    base = O.normal((V, D), 72)
    dst = g.dev(base)
    g.call("tlh_scatter_add_rows", g.dev(values), g.dev(ids), n, D, dst, V)
    np.testing.assert_array_equal(g.host(dst), O.scatter_add_rows(base, ids, values))


# ---------------------------------------------------------------------------
# optimiser
# ---------------------------------------------------------------------------
def test_clip_kat(g):
    s = g.dev(np.array([169.0], np.float32))
    x = g.dev(np.array([3, 4, 0], np.float32))
    g.call("tlh_clip_gradient", x, s, 1.0, x, 3)
    assert_close(g.host(x), [3 / 13, 4 / 13, 0])


def test_adamw_two_steps(g):
    n = 100003
    p, gr = O.normal((n,), 70), O.normal((n,), 71)
    m1 = np.zeros(n, np.float32); m2 = np.zeros(n, np.float32)
    lr, b1, b2, wd, eps = 3e-4, 0.9, 0.95, 0.1, 1e-8
    decay = float(np.float32(1) - np.float32(lr) * np.float32(wd))
    sc = [g.dev(np.array([v], np.float32)) for v in (b1, b2, decay, lr)]
    dp, dg, dm1, dm2 = g.dev(p), g.dev(gr), g.dev(m1), g.dev(m2)
    ep, em1, em2 = p, m1, m2
    for step in (1, 2):
        g.call("tlh_adamw", dp, dg, dp, dm1, dm2, *sc, eps, step, n)
        ep, em1, em2 = O.adamw(ep, gr, em1, em2, b1, b2, decay, lr, eps, step)
        assert_close(g.host(dp), ep, rtol=1e-4, atol=1e-6)
        assert_close(g.host(dm1), em1)
        assert_close(g.host(dm2), em2, rtol=1e-4, atol=1e-9)


def test_adamw_multi_matches_per_tensor(g):
    sizes = [384 * 384, 384, 4097, 1, 2048 * 384]
    lr, b1, b2, wd, eps, max_norm = 3e-4, 0.9, 0.95, 0.1, 1e-8, 1.0
    decay = float(np.float32(1) - np.float32(lr) * np.float32(wd))
    ps = [O.normal((n,), 80 + i) for i, n in enumerate(sizes)]
    gs = [O.normal((n,), 90 + i) for i, n in enumerate(sizes)]
    m1s = [O.normal((n,), 100 + i, 0, 0.01) for i, n in enumerate(sizes)]
    m2s = [np.abs(O.normal((n,), 110 + i, 0, 0.01)) for i, n in enumerate(sizes)]
    steps = [3, 3, 1, 7, 2]
    sq = sum(float((x.astype(np.float64) ** 2).sum()) for x in gs)
    dev = [[g.dev(x) for x in arr] for arr in (ps, gs, m1s, m2s)]
    tabs = [torch.tensor([t.data_ptr() for t in arr], dtype=torch.int64, device="cuda")
            for arr in dev]
    dsz = torch.tensor(sizes, dtype=torch.int64, device="cuda")
    dst = torch.tensor(steps, dtype=torch.int32, device="cuda")
    sc = [g.dev(np.array([v], np.float32)) for v in (b1, b2, decay, lr)]
    dsq = g.dev(np.array([sq], np.float32))
    g.call("tlh_adamw_multi", *tabs, dsz, dst, len(sizes), *sc, eps, dsq, max_norm)
    for i in range(len(sizes)):
        gc = O.clip_gradient(gs[i], np.float32(sq), max_norm)
        ep, em1, em2 = O.adamw(ps[i], gc, m1s[i], m2s[i], b1, b2, decay, lr, eps, steps[i])
        assert_close(g.host(dev[0][i]), ep, rtol=1e-4, atol=1e-6, what=f"param {i}")
        assert_close(g.host(dev[2][i]), em1, what=f"m1 {i}")
        assert_close(g.host(dev[3][i]), em2, rtol=1e-4, atol=1e-9, what=f"m2 {i}")


def test_clip_multi_matches_per_tensor(g):
    # one launch over ragged tensors (a partial 4096-element chunk, a single
    # element, a float4-misaligned start), in place and from another source,
    # gives each tensor exactly what tlh_clip_gradient gives it, and the
    # oracle's clip within rounding
    sizes = [384 * 384, 4101, 1, 2048 * 384, 7]
    gs = [O.normal((n,), 120 + i, 0, 3.0) for i, n in enumerate(sizes)]
    sq = np.float32(sum(float((x.astype(np.float64) ** 2).sum()) for x in gs))
    dsq = g.dev(np.array([sq], np.float32))
    multi = [g.dev(x) for x in gs]
    odd = g.dev(np.concatenate([np.zeros(1, np.float32), gs[4]]))  # starts 4 bytes in
    srcs = [t.data_ptr() for t in multi[:4]] + [odd.data_ptr() + 4]
    outs = [multi[0], g.empty((sizes[1],)), multi[2], g.empty((sizes[3],)), odd]
    dsts = [outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(), outs[3].data_ptr(),
            odd.data_ptr() + 4]
    ts = torch.tensor(srcs, dtype=torch.int64, device="cuda")
    td = torch.tensor(dsts, dtype=torch.int64, device="cuda")
    dsz = torch.tensor(sizes, dtype=torch.int64, device="cuda")
    g.call("tlh_clip_multi", ts, td, dsz, len(sizes), dsq, 1.0)
    got = [g.host(t) for t in outs[:4]] + [g.host(odd)[1:]]
    for i, x in enumerate(gs):
        one = g.dev(x)
        g.call("tlh_clip_gradient", one, dsq, 1.0, one, x.size)
        np.testing.assert_array_equal(got[i], g.host(one), err_msg=f"tensor {i}")
        assert_close(got[i], O.clip_gradient(x, sq, 1.0), rtol=1e-6, atol=1e-7, what=f"oracle {i}")
    assert g.lib.tlh_clip_multi(None, None, None, 0, None, 1.0, None) == 0  # nothing to do


@pytest.mark.parametrize("H,stride,t", [(2, 64, 0), (4, 1024, 1), (3, 100, 57), (16, 1024, 255),
                                        (16, 1024, 1023)])
def test_attention_decode(g, H, stride, t):
    # One query at position t over keys 0..t of [H, stride, 64] planes equals
    # row t of causal attention over the first t + 1 positions.
    q, k, v = (O.normal((1, H, stride, 64), s, 0, 0.125) for s in (130, 131, 132))
    o_ref, _ = O.attention_forward(q[:, :, :t + 1], k[:, :, :t + 1], v[:, :, :t + 1], True)
    o = g.empty((H * 64,))
    g.call("tlh_attention_decode", g.dev(q), g.dev(k), g.dev(v), o, H, stride, t, 64, 0.125)
    assert_rel(g.host(o).reshape(H, 64), o_ref[0, :, t, :], 1e-3, "decode O")


def test_attention_decode_rejects_bad_positions(g):
    q = g.empty((2 * 16 * 64,))
    for stride, t, hd in ((16, 16, 64), (16, 3, 32), (9000, 5, 64)):
        assert g.lib.tlh_attention_decode(q.data_ptr(), q.data_ptr(), q.data_ptr(), q.data_ptr(), 2,
                                          stride, t, hd, 0.125, g.stream) != 0


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("B,H,T,causal", [(4, 6, 192, True), (2, 3, 100, True),
                                          (2, 2, 130, False), (1, 1, 1, True),
                                          (2, 2, 65, True), (3, 1, 33, False),
                                          (1, 4, 257, True), (1, 2, 1024, True)])
@pytest.mark.parametrize("merged", [False, True])
def test_attention_forward_backward(g, B, H, T, causal, merged):
    D = 64
    q, k, v = (O.normal((B, H, T, D), s, 0, 0.125) for s in (120, 121, 122))
    dout_h = O.normal((B, H, T, D), 123)
    o_ref, probs = O.attention_forward(q, k, v, causal)
    dq_r, dk_r, dv_r = O.attention_backward(q, k, v, probs, dout_h)

    def to_layout(x):  # [B,H,T,D] -> merged [B,T,H*D]
        return np.ascontiguousarray(x.transpose(0, 2, 1, 3).reshape(B, T, H * D)) if merged else x

    dq_, dk_, dv_ = g.dev(q), g.dev(k), g.dev(v)
    o = g.empty((B * H * T * D,))
    lse = g.empty((B * H * T,))
    g.call("tlh_attention_forward", dq_, dk_, dv_, o, lse, B, H, T, D, 0.125, int(causal),
           int(merged))
    assert_rel(g.host(o).reshape(to_layout(o_ref).shape), to_layout(o_ref), 1e-3, "O")
    delta = g.empty((B * H * T,))
    dq, dk, dv = (g.empty((B * H * T * D,)) for _ in range(3))
    g.call("tlh_attention_backward", dq_, dk_, dv_, o, g.dev(to_layout(dout_h)), lse, delta, dq, dk,
           dv, B, H, T, D, 0.125, int(causal), int(merged), int(merged))
    # A gradient that is exactly zero (dQ, dK at T=1: softmax over one key)
    # is compared against the scale of the whole backward output.
    scale = max(float(np.abs(r).max()) for r in (dq_r, dk_r, dv_r))
    for got, ref, name in ((dq, dq_r, "dQ"), (dk, dk_r, "dK"), (dv, dv_r, "dV")):
        err = rel_err(g.host(got).reshape(to_layout(ref).shape), to_layout(ref),
                      floor=1e-3 * scale)
        assert err <= 1e-3, f"{name}: relative error {err:.3e}"
