"""Kernel microbenchmarks of libtemplit_hip.so at the GPT shapes.

Times each GEMM of the GPT training step (V 2048, T 192, d 384, 4 blocks,
batch 32: 12 distinct shapes), the fused causal attention at the
attention-benchmark and scaled shapes, and the memory-bound kernels of the
step (row ops, embedding gather/scatter, gradient norm, clip + AdamW over the
step's 52 parameter tensors) with HIP events on one stream. It is also the
program the rocprofv3 counter profiles under profiles/ run: before each case
it prints "[case i] <name>" and launches one single-element fill_u32_kernel
(value i), so that a profile's dispatches can be split into cases (cases
named "set-up ..." hold buffer initialisation and warm-up calls).

  python -m templit_amd.kernel_bench [--gemm] [--attention] [--memory]
                                     [--iters N]
                                     [--sweep]   (every tile/split plan)
"""
from __future__ import annotations

import argparse
import ctypes
import sys

from templit_amd.native import GemmDesc, check, load_hip

R, D, F, V = 6144, 384, 1536, 2048
GEMM_SHAPES = [  # name, M, N, K, trans_a, trans_b, bias gradient
    ("qkv/o fwd", R, D, D, 0, 1, 0), ("w1 fwd", R, F, D, 0, 1, 0),
    ("w2 fwd", R, D, F, 0, 1, 0), ("vocab fwd", R, V, D, 0, 1, 0),
    ("dX d->d", R, D, D, 0, 1, 0), ("dG d->f", R, F, D, 0, 1, 0),
    ("dN f->d", R, D, F, 0, 1, 0), ("dX vocab", R, D, V, 0, 1, 0),
    ("wgrad dd", D, D, R, 1, 0, 1), ("wgrad fd", F, D, R, 1, 0, 1),
    ("wgrad df", D, F, R, 1, 0, 1), ("wgrad dv", D, V, R, 1, 0, 1),
    ("d1024 up", 8192, 4096, 1024, 0, 0, 0), ("d1024 sq", 8192, 1024, 1024, 0, 0, 0),
    ("c1 matmul", 768, 1536, 384, 0, 0, 0),
    # the reference executor's forward products read W [in, out] as stored
    ("nn qkv/o fwd", R, D, D, 0, 0, 0), ("nn w1 fwd", R, F, D, 0, 0, 0),
    ("nn w2 fwd", R, D, F, 0, 0, 0), ("nn vocab fwd", R, V, D, 0, 0, 0),
]
BUF = 8192 * 4096  # largest operand of the shapes above
ATTENTION_SHAPES = [(32, 6, 192), (8, 16, 1024)]  # (B, H, T), head dim 64
BATCH, SEQ = 32, 192


def gpt_parameter_sizes() -> list[int]:
    """Element counts of the 52 parameter tensors of the GPT step (4 blocks of
    q/k/v/o [D,D]+[D], FFN [D,F]+[F] and [F,D]+[D]; token [V,D], position
    [T,D] and vocab [D,V]+[V]): 8,740,352 floats."""
    block = [D * D, D] * 4 + [D * F, F, F * D, D]
    return block * 4 + [V * D, SEQ * D, D * V, V]


# Algorithmic bytes per launch of the memory-bound cases: every tensor the
# operation must read or write once (fp32, u32 ids).
P_TOTAL = sum(gpt_parameter_sizes())
MEMORY_BYTES = {
    "rmsnorm fwd [6144,384]": 4 * (2 * R * D),
    "rmsnorm bwd [6144,384]": 4 * (3 * R * D),
    "gelu fwd [6144,1536]": 4 * 2 * R * F,
    "gelu bwd [6144,1536]": 4 * 3 * R * F,
    "softmax fwd [6144,2048]": 4 * 2 * R * V,
    "softmax bwd [6144,2048]": 4 * 3 * R * V,
    "cross-entropy fwd [6144,2048]": 4 * (R * V + 2 * R),
    "cross-entropy bwd scaled [6144,2048]": 4 * (2 * R * V + 2 * R),
    "cross-entropy fused fwd+bwd [6144,2048]": 4 * (2 * R * V + 2 * R),
    "embedding tok+pos gather [32x192,384]": 4 * (R + 2 * R * D + SEQ * D),
    "embedding scatter-add 6144 rows -> [2048,384]": 4 * (R * D + R + 2 * V * D),
    "gradient squared norm, 52 tensors": 4 * P_TOTAL,
    "clip + AdamW, 52 tensors": 4 * 7 * P_TOTAL,
}


class Bench:
    def __init__(self):
        self.hip = load_hip()
        check(self.hip.tlh_init(0), "init")
        s = ctypes.c_void_p()
        check(self.hip.tlh_stream_create(ctypes.byref(s)), "stream")
        self.stream = s.value
        self.ev = [ctypes.c_void_p(), ctypes.c_void_p()]
        for e in self.ev:
            check(self.hip.tlh_event_create(ctypes.byref(e)), "event")
        self.bufs = []
        self.cases = 0
        self.marker = self.alloc(1)

    def mark(self, name: str) -> None:
        """Case boundary for profiles: a printed line and one fill_u32_kernel."""
        print(f"[case {self.cases}] {name}", flush=True)
        check(self.hip.tlh_fill_u32(self.marker, self.cases, 1, self.stream), "marker")
        self.cases += 1

    def alloc(self, n, seed=None):
        p = ctypes.c_void_p()
        check(self.hip.tlh_malloc(ctypes.byref(p), max(n, 64) * 4), "malloc")
        self.bufs.append(p.value)
        if seed is not None:
            check(self.hip.tlh_fill_normal(p.value, n, seed, 0.0, 0.125, self.stream), "fill")
        return p.value

    def time_us(self, fn, iters):
        for _ in range(3):
            fn()
        check(self.hip.tlh_event_record(self.ev[0], self.stream), "record")
        for _ in range(iters):
            fn()
        check(self.hip.tlh_event_record(self.ev[1], self.stream), "record")
        check(self.hip.tlh_stream_synchronize(self.stream), "sync")
        ms = ctypes.c_float()
        check(self.hip.tlh_event_elapsed_ms(self.ev[0], self.ev[1], ctypes.byref(ms)), "elapsed")
        return ms.value * 1e3 / iters

    def close(self):
        for b in self.bufs:
            self.hip.tlh_free(b)
        for e in self.ev:
            self.hip.tlh_event_destroy(e)
        self.hip.tlh_stream_destroy(self.stream)


def run_gemm(b: Bench, iters: int, sweep: bool, only: str | None = None) -> None:
    b.mark("set-up gemm")
    a = b.alloc(BUF, 1)
    bb = b.alloc(BUF, 2)
    c = b.alloc(BUF)
    bias_grad = b.alloc(V)
    ws_elems = 16 * (F * V + V)
    ws = b.alloc(ws_elems)
    plans = [(0, 0, 0, 16)]
    if sweep:
        plans += [(bm, bn, s, bk) for bk in (16, 32) for bm in (64, 128) for bn in (64, 128)
                  for s in (1, 4, 8, 16)]
        plans += [(96, 96, s, 32) for s in (1, 4, 8, 16)] + [(96, 96, 1, 64)]
        plans += [(16, t, s, 32) for t in (64, 128) for s in (1, 2, 4, 8, 16)]
    for name, M, N, K, ta, tb, bgrad in GEMM_SHAPES:
        if only and only not in name:
            continue
        d = GemmDesc()
        d.a, d.b, d.c = a, bb, c
        d.m, d.n, d.k = M, N, K
        d.lda, d.ldb, d.ldc = (M if ta else K), (K if tb else N), N
        d.trans_a, d.trans_b = ta, tb
        d.workspace, d.workspace_elems = ws, ws_elems
        if bgrad:
            d.bias_grad = bias_grad
        results = []
        b.mark(f"gemm {name} M{M} N{N} K{K} ta{ta} tb{tb}")
        for plan in plans:
            if plan[2] > 1 and not bgrad and not name.startswith("c1"):
                continue
            check(b.hip.tlh_gemm_set_plan(*plan), "plan")
            need = ctypes.c_size_t()
            check(b.hip.tlh_gemm_workspace_size(ctypes.byref(d), ctypes.byref(need)), "ws")
            if need.value > ws_elems:
                continue
            us = b.time_us(lambda: check(b.hip.tlh_gemm(ctypes.byref(d), b.stream), "gemm"),
                           iters)
            results.append((us, plan))
        check(b.hip.tlh_gemm_set_plan(0, 0, 0, 16), "plan")
        us, plan = results[0]
        line = (f"gemm {name:10s} M{M:5d} N{N:5d} K{K:5d} ta{ta} tb{tb}: {us:8.1f} us "
                f"{2.0 * M * N * K / us / 1e6:6.1f} TFLOP/s")
        if sweep:
            best_us, best = min(results)
            line += f" | best {best_us:8.1f} us plan {best}"
            line += "\n    " + " ".join(f"{p_[0]}x{p_[1]}/s{p_[2]}/k{p_[3]}:{u:.1f}"
                                        for u, p_ in results[1:])
        print(line, flush=True)


def run_attention(b: Bench, iters: int) -> None:
    hd = 64
    for B, H, T in ATTENTION_SHAPES:
        b.mark(f"set-up attention B{B} H{H} T{T}")
        n = B * H * T * hd
        q, k, v, do = (b.alloc(n, 10 + i) for i in range(4))
        o, dq, dk, dv = (b.alloc(n) for _ in range(4))
        lse, delta = b.alloc(B * H * T), b.alloc(B * H * T)

        def fwd():
            check(b.hip.tlh_attention_forward(q, k, v, o, lse, B, H, T, hd, 0.125, 1, 0,
                                              b.stream), "attention forward")

        def bwd():
            check(b.hip.tlh_attention_backward(q, k, v, o, do, lse, delta, dq, dk, dv, B, H, T,
                                               hd, 0.125, 1, 0, 0, b.stream),
                  "attention backward")

        fwd()
        for name, fn, mult in (("fwd", fwd, 4), ("bwd", bwd, 10)):
            b.mark(f"attention {name} B{B} H{H} T{T}")
            us = b.time_us(fn, iters)
            flops = mult * B * H * T * T * hd / 2  # causal: half the dense work
            print(f"attention {name} B{B} H{H} T{T}: {us:9.1f} us "
                  f"{flops / us / 1e6:6.1f} TFLOP/s (causal-effective)", flush=True)


def run_memory(b: Bench, iters: int) -> None:
    """The memory-bound kernels of the GPT step at its shapes, against HBM."""
    hip, s = b.hip, b.stream
    b.mark("set-up memory")
    x, gx, dx, y = b.alloc(R * D, 20), b.alloc(R * D, 21), b.alloc(R * D), b.alloc(R * D)
    h, gh, dh, hy = b.alloc(R * F, 22), b.alloc(R * F, 23), b.alloc(R * F), b.alloc(R * F)
    lg, glg, ly = b.alloc(R * V, 24), b.alloc(R * V, 25), b.alloc(R * V)
    loss, scale = b.alloc(R), b.alloc(R, 26)
    ids = b.alloc(R)
    check(hip.tlh_fill_uniform_u32(ids, R, 27, V, s), "ids")
    tok, pos, emb = b.alloc(V * D, 28), b.alloc(SEQ * D, 29), b.alloc(R * D)
    eps = 1e-6

    sizes = gpt_parameter_sizes()
    tensors = {k: [b.alloc(n, 30 + i) if k != "m" else b.alloc(n) for i, n in enumerate(sizes)]
               for k in ("p", "g", "m")}
    m2 = [b.alloc(n) for n in sizes]
    for ptr, n in zip(tensors["m"] + m2, sizes + sizes):
        check(hip.tlh_fill_u32(ptr, 0, n, s), "zero")

    def table(values, ctype):
        arr = (ctype * len(values))(*values)
        dev = b.alloc(len(values) * ctypes.sizeof(ctype) // 4 + 1)
        check(hip.tlh_memcpy_h2d(dev, arr, ctypes.sizeof(arr), s), "table")
        check(hip.tlh_stream_synchronize(s), "sync")
        return dev

    u64 = ctypes.c_uint64
    tp, tg, tm1, tm2 = (table(v, u64) for v in (tensors["p"], tensors["g"], tensors["m"], m2))
    tsz = table(sizes, u64)
    steps = table([1] * len(sizes), ctypes.c_uint32)
    partials, sqn = b.alloc(1024), b.alloc(1)
    hyper = [b.alloc(1) for _ in range(4)]
    for ptr, val in zip(hyper, (0.9, 0.95, 0.1, 3e-4)):
        f = ctypes.c_float(val)
        check(hip.tlh_memcpy_h2d(ptr, ctypes.byref(f), 4, s), "hyper")
        check(hip.tlh_stream_synchronize(s), "sync")
    n_t = len(sizes)

    ops = {
        "rmsnorm fwd [6144,384]": lambda: hip.tlh_rms_norm(x, None, y, None, R, D, eps, s),
        "rmsnorm bwd [6144,384]": lambda: hip.tlh_rms_norm_backward(gx, x, None, dx, None, R, D,
                                                                    eps, 0.0, s),
        "gelu fwd [6144,1536]": lambda: hip.tlh_gelu(h, hy, R * F, s),
        "gelu bwd [6144,1536]": lambda: hip.tlh_gelu_backward(gh, h, dh, R * F, s),
        "softmax fwd [6144,2048]": lambda: hip.tlh_softmax(lg, ly, R, V, s),
        "softmax bwd [6144,2048]": lambda: hip.tlh_softmax_backward(glg, ly, lg, R, V, s),
        "cross-entropy fwd [6144,2048]": lambda: hip.tlh_cross_entropy_rows(lg, ids, loss, R, V,
                                                                            s),
        "cross-entropy bwd scaled [6144,2048]": lambda: hip.tlh_cross_entropy_rows_backward(
            lg, ids, ly, R, V, scale, s),
        "cross-entropy fused fwd+bwd [6144,2048]": lambda: hip.tlh_cross_entropy_rows_fused(
            lg, ids, loss, ly, R, V, 1.0 / R, s),
        "embedding tok+pos gather [32x192,384]": lambda: hip.tlh_embedding_add_positions(
            tok, V, pos, ids, BATCH, SEQ, D, emb, s),
        "embedding scatter-add 6144 rows -> [2048,384]": lambda: hip.tlh_scatter_add_rows(
            emb, ids, R, D, tok, V, s),
        "gradient squared norm, 52 tensors": lambda: hip.tlh_gradient_squared_norm_multi(
            tg, tsz, n_t, partials, sqn, s),
        "clip + AdamW, 52 tensors": lambda: hip.tlh_adamw_multi(
            tp, tg, tm1, tm2, tsz, steps, n_t, hyper[0], hyper[1], hyper[2], hyper[3], 1e-8,
            sqn, 1.0, s),
    }
    check(ops["gradient squared norm, 52 tensors"](), "norm")
    for name, fn in ops.items():
        b.mark(name)
        us = b.time_us(lambda: check(fn(), name), iters)
        gbs = MEMORY_BYTES[name] / us / 1e3
        print(f"memory {name:46s}: {us:8.2f} us {gbs:7.1f} GB/s "
              f"({MEMORY_BYTES[name] / 1e6:.1f} MB per launch)", flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gemm", action="store_true")
    ap.add_argument("--attention", action="store_true")
    ap.add_argument("--memory", action="store_true",
                    help="the memory-bound kernels (row ops, embedding, norm, AdamW)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="first, one device copy of MIB MiB, whose FETCH_SIZE / WRITE_SIZE "
                         "readings scale those counters to bytes")
    ap.add_argument("--sweep", action="store_true")
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--only", help="GEMM shapes whose name contains this text")
    ap.add_argument("--no-tail-split", action="store_true",
                    help="no K-chunked tail tiles for grids that do not spread evenly")
    ap.add_argument("--no-xcd-rects", action="store_true",
                    help="contiguous tile ranges per XCD instead of rectangular tile blocks")
    args = ap.parse_args()
    if not (args.gemm or args.attention or args.memory):
        args.gemm = args.attention = args.memory = True
    b = Bench()
    if args.no_tail_split:
        check(b.hip.tlh_gemm_set_plan(0, 0, 0, -3), "plan")
    if args.no_xcd_rects:
        check(b.hip.tlh_gemm_set_plan(0, 0, 0, -5), "plan")
    try:
        if args.copy_calibration:
            n = args.copy_calibration * (1 << 20) // 4
            b.mark("set-up copy calibration")
            src, dst = b.alloc(n), b.alloc(n)
            check(b.hip.tlh_fill_f32(src, 1.0, n, b.stream), "fill")
            b.mark(f"copy calibration {args.copy_calibration} MiB")
            check(b.hip.tlh_copy(src, dst, n, b.stream), "copy")
            check(b.hip.tlh_stream_synchronize(b.stream), "sync")
        if args.gemm:
            run_gemm(b, args.iters, args.sweep, args.only)
        if args.attention:
            run_attention(b, args.iters)
        if args.memory:
            run_memory(b, args.iters)
    finally:
        b.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
