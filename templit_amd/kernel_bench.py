"""Kernel microbenchmarks of libtemplit_hip.so at the GPT shapes.

Times each GEMM of the GPT training step (V 2048, T 192, d 384, 4 blocks,
batch 32: 12 distinct shapes) and the fused causal attention at the
attention-benchmark and scaled shapes, with HIP events on one stream. It is
also the program the rocprofv3 counter profiles under profiles/ run.

  python -m templit_amd.kernel_bench [--gemm] [--attention] [--iters N]
                                     [--sweep]   (every tile/split plan)
"""
from __future__ import annotations

import argparse
import ctypes
import sys

from templit_amd.native import GemmDesc, check, load_hip

R, D, F, V = 6144, 384, 1536, 2048
GEMM_SHAPES = [  # name, M, N, K, trans_a, trans_b, bias gradient
    ("qkv/o fwd", R, D, D, 0, 0, 0), ("w1 fwd", R, F, D, 0, 0, 0),
    ("w2 fwd", R, D, F, 0, 0, 0), ("vocab fwd", R, V, D, 0, 0, 0),
    ("dX d->d", R, D, D, 0, 1, 0), ("dG d->f", R, F, D, 0, 1, 0),
    ("dN f->d", R, D, F, 0, 1, 0), ("dX vocab", R, D, V, 0, 1, 0),
    ("wgrad dd", D, D, R, 1, 0, 1), ("wgrad fd", F, D, R, 1, 0, 1),
    ("wgrad df", D, F, R, 1, 0, 1), ("wgrad dv", D, V, R, 1, 0, 1),
    ("d1024 up", 8192, 4096, 1024, 0, 0, 0), ("d1024 sq", 8192, 1024, 1024, 0, 0, 0),
]
BUF = 8192 * 4096  # largest operand of the shapes above
ATTENTION_SHAPES = [(32, 6, 192), (8, 16, 1024)]  # (B, H, T), head dim 64


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
        for plan in plans:
            if plan[2] > 1 and not bgrad:
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
        print(line, flush=True)


def run_attention(b: Bench, iters: int) -> None:
    hd = 64
    for B, H, T in ATTENTION_SHAPES:
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
            us = b.time_us(fn, iters)
            flops = mult * B * H * T * T * hd / 2  # causal: half the dense work
            print(f"attention {name} B{B} H{H} T{T}: {us:9.1f} us "
                  f"{flops / us / 1e6:6.1f} TFLOP/s (causal-effective)", flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gemm", action="store_true")
    ap.add_argument("--attention", action="store_true")
    ap.add_argument("--sweep", action="store_true")
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--only", help="GEMM shapes whose name contains this text")
    ap.add_argument("--no-tail-split", action="store_true",
                    help="no K-chunked tail tiles for grids that do not spread evenly")
    args = ap.parse_args()
    if not (args.gemm or args.attention):
        args.gemm = args.attention = True
    b = Bench()
    if args.no_tail_split:
        check(b.hip.tlh_gemm_set_plan(0, 0, 0, -3), "plan")
    try:
        if args.gemm:
            run_gemm(b, args.iters, args.sweep, args.only)
        if args.attention:
            run_attention(b, args.iters)
    finally:
        b.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
