#!/usr/bin/env python3
"""Benchmark: GPT training step on one MI355X (the reference's GPT example
config: vocab 2048, T=192, d=384, 4 blocks, 6 heads, FFN 4x, batch 32, fp32,
CE loss, global grad-norm clip 1.0, AdamW lr 3e-4 b1 0.9 b2 0.95 wd 0.1).

One step = forward + loss + backward + clip + AdamW over one batch of 6,144
tokens already resident in HBM, launched eagerly on the program's two
streams (input gradients on one, weight gradients on the other, ordered by
events). The same step replayed as one captured hipGraph is timed too and
reported under "other_execution": on ROCm 7.2 the graph's cross-stream
edges idle the GPU about 10 us each, so the eager launches are faster.
Prints one JSON line: tokens/s, the GEMM roofline fraction (fp32 MFMA), the
d=1024 GEMM rate, and the CPU oracle's rate on a bounded sample of the same
step.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--graph] [--no-cpu-baseline]

Profiling runs (rocprofv3 counters) use --skip-d1024 and --copy-calibration
MiB (one device copy of that size, whose FETCH_SIZE / WRITE_SIZE readings
scale the counters to bytes).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "train tokens/sec (GPT step, 1 GPU); matmul TFLOP/s & % fp32-MFMA peak"
FP32_MFMA_PEAK = 157.3  # TFLOP/s, MI355X dense fp32 matrix
HBM_PEAK = 8000.0       # GB/s

CFG = dict(vocab=2048, seq=192, dim=384, heads=6, layers=4, batch=32)
HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
MAX_NORM = 1.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemm_d1024(hip, stream) -> dict:
    """fp32 MFMA GEMM at the d=1024 FFN-up shape [8192,1024].[1024,4096]."""
    from templit_amd.native import GemmDesc, check

    M, N, K = 8192, 4096, 1024
    bufs = []
    for n in (M * K, K * N, M * N):
        p = ctypes.c_void_p()
        check(hip.tlh_malloc(ctypes.byref(p), n * 4), "malloc")
        bufs.append(p.value)
    try:
        check(hip.tlh_fill_normal(bufs[0], M * K, 11, 0.0, 0.02, stream), "fill")
        check(hip.tlh_fill_normal(bufs[1], K * N, 12, 0.0, 0.02, stream), "fill")
        d = GemmDesc()
        d.a, d.b, d.c = bufs
        d.m, d.n, d.k = M, N, K
        d.lda, d.ldb, d.ldc = K, N, N
        for _ in range(3):
            check(hip.tlh_gemm(ctypes.byref(d), stream), "gemm")
        ev = [ctypes.c_void_p(), ctypes.c_void_p()]
        for e in ev:
            check(hip.tlh_event_create(ctypes.byref(e)), "event")
        iters = 20
        check(hip.tlh_event_record(ev[0], stream), "record")
        for _ in range(iters):
            check(hip.tlh_gemm(ctypes.byref(d), stream), "gemm")
        check(hip.tlh_event_record(ev[1], stream), "record")
        check(hip.tlh_stream_synchronize(stream), "sync")
        ms = ctypes.c_float()
        check(hip.tlh_event_elapsed_ms(ev[0], ev[1], ctypes.byref(ms)), "elapsed")
        for e in ev:
            hip.tlh_event_destroy(e)
        per = ms.value / iters
        tflops = 2.0 * M * N * K / (per * 1e-3) / 1e12
        return {"shape": [M, K, N], "ms": round(per, 4), "tflops": round(tflops, 2),
                "frac_fp32_peak": round(tflops / FP32_MFMA_PEAK, 4)}
    finally:
        for b in bufs:
            hip.tlh_free(b)


class DeviceTimer:
    """Device buffers and HIP-event timing on one stream, for the kernel
    configurations below."""

    def __init__(self, hip, stream):
        from templit_amd.native import check

        self.hip, self.stream, self.check = hip, stream, check
        self.bufs = []
        self.ev = [ctypes.c_void_p(), ctypes.c_void_p()]
        for e in self.ev:
            check(hip.tlh_event_create(ctypes.byref(e)), "event")

    def buf(self, n, seed=None, mean=0.0, std=1.0, bound=None):
        ptr = ctypes.c_void_p()
        self.check(self.hip.tlh_malloc(ctypes.byref(ptr), max(n, 1) * 4), "malloc")
        self.bufs.append(ptr.value)
        if bound is not None:
            self.check(self.hip.tlh_fill_uniform_u32(ptr.value, n, seed, bound, self.stream), "fill")
        elif seed is not None:
            self.check(self.hip.tlh_fill_normal(ptr.value, n, seed, mean, std, self.stream), "fill")
        return ptr.value

    def us(self, fn, iters=50):
        for _ in range(3):
            fn()
        self.check(self.hip.tlh_event_record(self.ev[0], self.stream), "record")
        for _ in range(iters):
            fn()
        self.check(self.hip.tlh_event_record(self.ev[1], self.stream), "record")
        self.check(self.hip.tlh_stream_synchronize(self.stream), "sync")
        ms = ctypes.c_float()
        self.check(self.hip.tlh_event_elapsed_ms(self.ev[0], self.ev[1], ctypes.byref(ms)),
                   "elapsed")
        return ms.value * 1e3 / iters

    def close(self):
        for b in self.bufs:
            self.hip.tlh_free(b)
        for e in self.ev:
            self.hip.tlh_event_destroy(e)


# Row-op sizes: X [6144,384], H [6144,1536], logits [6144,2048]
R2, D2, F2, V2 = 6144, 384, 1536, 2048
# Minimum HBM bytes per launch (each operand read once, each result written once)
ROW_OP_BYTES = {
    "rmsnorm_fwd": 4 * (2 * R2 * D2 + D2), "rmsnorm_bwd": 4 * (3 * R2 * D2 + D2),
    "gelu_fwd": 4 * 2 * R2 * F2, "gelu_bwd": 4 * 3 * R2 * F2,
    "softmax_fwd": 4 * 2 * R2 * V2, "softmax_bwd": 4 * 3 * R2 * V2,
    "cross_entropy_fwd": 4 * (R2 * V2 + 2 * R2),
    "cross_entropy_bwd_scaled": 4 * (2 * R2 * V2 + 2 * R2),
}
C1 = (768, 384, 1536)           # A [768,384] . B [384,1536] + bias [1,1536]
C3 = (32, 6, 192, 64)           # attention Q, K, V, dO [B, H, T, 64], causal


def kernel_configs(hip, stream) -> dict:
    """The single-kernel configurations, each against its roofline:
    matmul + bias (fp32 MFMA), the row ops (HBM) and causal attention
    (fp32 MFMA, causal-effective flops)."""
    from templit_amd.native import GemmDesc, u32_array

    t = DeviceTimer(hip, stream)
    ck, s = t.check, stream
    out: dict = {}
    try:
        # c1: through the runtime's two calls (mult, then the broadcast add of
        # nn::Layer, execute.h:241-252) and as one GEMM with the bias fused
        M, K, N = C1
        a, b, bias, c = t.buf(M * K, 1, 0, 0.02), t.buf(K * N, 2, 0, 0.02), t.buf(N, 3, 0, 0.02), t.buf(M * N)
        shape, sa, sb = u32_array([M, N]), u32_array([N, 1]), u32_array([0, 1])
        flops = 2.0 * M * N * K + M * N

        def mult_add():
            ck(hip.tlh_matmul(a, b, c, M, K, N, K, 1, N, 1, N, 1, 0, None, None, None, None, s),
               "matmul")
            ck(hip.tlh_add(c, bias, c, 2, shape, sa, sb, s), "add")

        d = GemmDesc()
        d.a, d.b, d.c, d.bias = a, b, c, bias
        d.m, d.n, d.k = M, N, K
        d.lda, d.ldb, d.ldc = K, N, N
        rows = {}
        for name, fn in (("mult_then_add", mult_add),
                         ("fused_bias_gemm", lambda: ck(hip.tlh_gemm(ctypes.byref(d), s), "gemm"))):
            us = t.us(fn)
            tf = flops / us / 1e6
            rows[name] = {"us": round(us, 2), "tflops": round(tf, 2),
                          "frac": round(tf / FP32_MFMA_PEAK, 4)}
        out["matmul_bias_768x384x1536"] = {"bound": "mfma", "flops": flops, **rows}

        # c2: row ops at the GPT shapes
        x, gx, gain = t.buf(R2 * D2, 4), t.buf(R2 * D2, 5), t.buf(D2, 6, 1.0, 0.02)
        y = t.buf(R2 * D2)
        h, gh, hy = t.buf(R2 * F2, 7), t.buf(R2 * F2, 8), t.buf(R2 * F2)
        lg, glg, ly = t.buf(R2 * V2, 9), t.buf(R2 * V2, 10), t.buf(R2 * V2)
        tgt, loss, scale = t.buf(R2, 11, bound=V2), t.buf(R2), t.buf(R2, 12)
        eps = 1e-6
        ops = {
            "rmsnorm_fwd": lambda: hip.tlh_rms_norm(x, gain, y, None, R2, D2, eps, s),
            "rmsnorm_bwd": lambda: hip.tlh_rms_norm_backward(gx, x, gain, y, None, R2, D2, eps,
                                                             0.0, s),
            "gelu_fwd": lambda: hip.tlh_gelu(h, hy, R2 * F2, s),
            "gelu_bwd": lambda: hip.tlh_gelu_backward(gh, h, hy, R2 * F2, s),
            "softmax_fwd": lambda: hip.tlh_softmax(lg, ly, R2, V2, s),
            "softmax_bwd": lambda: hip.tlh_softmax_backward(glg, ly, glg, R2, V2, s),
            "cross_entropy_fwd": lambda: hip.tlh_cross_entropy_rows(lg, tgt, loss, R2, V2, s),
            "cross_entropy_bwd_scaled": lambda: hip.tlh_cross_entropy_rows_backward(
                lg, tgt, ly, R2, V2, scale, s),
        }
        rowops = {}
        for name, fn in ops.items():
            us = t.us(lambda: ck(fn(), name))
            gbs = ROW_OP_BYTES[name] / us / 1e3
            rowops[name] = {"us": round(us, 2), "bytes": ROW_OP_BYTES[name],
                            "gb_s": round(gbs, 1), "frac": round(gbs / HBM_PEAK, 4)}
        out["row_ops"] = {"bound": "hbm", "peak_gb_s": HBM_PEAK, **rowops}

        # c3: fused causal attention
        B, H, T, Dh = C3
        n = B * H * T * Dh
        q, k, v = (t.buf(n, 13 + i, 0.0, 0.125) for i in range(3))
        do = t.buf(n, 16)
        o, dq, dk, dv = (t.buf(n) for _ in range(4))
        lse, delta = t.buf(B * H * T), t.buf(B * H * T)
        sc = 1.0 / 8.0
        fwd = lambda: ck(hip.tlh_attention_forward(q, k, v, o, lse, B, H, T, Dh, sc, 1, 0, s),
                         "attention forward")
        bwd = lambda: ck(hip.tlh_attention_backward(q, k, v, o, do, lse, delta, dq, dk, dv, B,
                                                    H, T, Dh, sc, 1, 0, 0, s),
                         "attention backward")
        fwd()
        att = {}
        for name, fn, mult in (("forward", fwd, 4), ("backward", bwd, 10)):
            us = t.us(fn)
            causal = mult * B * H * T * T * Dh / 2
            tf = causal / us / 1e6
            att[name] = {"us": round(us, 2), "causal_flops": causal, "tflops": round(tf, 2),
                         "frac": round(tf / FP32_MFMA_PEAK, 4)}
        out["attention_b32_h6_t192"] = {"bound": "mfma", **att}
    finally:
        t.close()
    log(f"[bench] kernel configurations: {json.dumps(out)}")
    return out


SCALED = dict(vocab=2048, seq=1024, dim=1024, heads=16, layers=12, batch=8)
EOS = 256  # the BPE tokeniser's end-of-sequence id (dataset/ tokens split on it)


def time_steps(prog, step, warmup: int, steps: int) -> float:
    """Seconds per step of `steps` calls of `step` after `warmup` untimed ones,
    bracketed by device synchronisations."""
    for _ in range(warmup):
        step()
    prog.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    prog.synchronize()
    return (time.perf_counter() - t0) / steps


def scaled_gpt(steps: int, gen_tokens: int) -> dict:
    """The scaled configuration: d 1024, 16 heads, 12 blocks, T 1024, V 2048,
    batch 8 -- a training step (eager launches on the streams the program
    picks for this size; the hipGraph replay of the same step and the other
    stream choice are timed too) and greedy generation of
    `gen_tokens` tokens from a 32-token random prompt (batch 1: the reference's
    full-window recompute, the equivalent valid-prefix recompute, and a KV
    cache that runs each new position alone)."""
    import numpy as np

    from templit_amd.native import GptProgram

    out: dict = {"config": dict(SCALED), "data": "synthetic: random tokens, N(0,0.02) weights"}
    prog = GptProgram(**SCALED)
    try:
        tokens = SCALED["batch"] * SCALED["seq"]
        prog.init_params(seed=21, std=0.02)
        prog.set_optimizer(**HP)
        prog.random_batch(seed=22)
        eager = lambda: prog.train_step(1.0 / tokens, MAX_NORM)
        streams = lambda two: "two streams" if two else "one stream"
        two = prog.set_concurrency(-1)
        dt = time_steps(prog, eager, 2, steps)
        model_flops = 6.0 * prog.total * tokens  # excludes attention's T^2 term
        out["train"] = {"tokens_per_step": tokens, "ms_per_step": round(dt * 1e3, 3),
                        "tokens_per_s": round(tokens / dt, 1), "steps": steps,
                        "execution": f"eager launches on {streams(two)}",
                        "loss": round(float(prog.losses().mean()), 4),
                        "param_flops_tflops": round(model_flops / dt / 1e12, 2)}
        prog.capture(1.0 / tokens, MAX_NORM)
        dt = time_steps(prog, prog.replay, 2, steps)
        out["train_graph_replay"] = {"ms_per_step": round(dt * 1e3, 3),
                                     "tokens_per_s": round(tokens / dt, 1)}
        prog.set_concurrency(int(not two))
        dt = time_steps(prog, eager, 2, steps)
        out["train_other_streams"] = {"execution": f"eager launches on {streams(not two)}",
                                      "ms_per_step": round(dt * 1e3, 3),
                                      "tokens_per_s": round(tokens / dt, 1)}
    finally:
        prog.close()
    log(f"[bench] scaled train: {out['train']}")
    gen = GptProgram(**dict(SCALED, batch=1))
    try:
        gen.init_params(seed=21, std=0.02)
        prompt = np.random.default_rng(23).integers(0, SCALED["vocab"], 32, dtype=np.uint32)
        gen.generate_greedy(prompt, 2, EOS)  # warm-up
        for mode, prefix in (("full_window", 0), ("valid_prefix", 1), ("kv_cache", 2)):
            t0 = time.perf_counter()
            toks = gen.generate_greedy(prompt, gen_tokens, EOS, prefix_only=prefix)
            dt = time.perf_counter() - t0
            out[f"generate_{mode}"] = {"tokens": gen_tokens, "s": round(dt, 3),
                                       "tokens_per_s": round(gen_tokens / dt, 2),
                                       "first_tokens": [int(t) for t in toks[:8]]}
    finally:
        gen.close()
    log(f"[bench] scaled generation: {out['generate_full_window']}, {out['generate_valid_prefix']}, "
        f"{out['generate_kv_cache']}")
    return out


def gemm_traffic() -> float | None:
    """HBM bytes per GEMM launch from the committed counter profile (two
    rocprofv3 --pmc runs, FETCH_SIZE and WRITE_SIZE, scaled by a copy of
    known size; the file names the commands)."""
    path = ROOT / "profiles" / "gpt_step_b32_t192_d384_gemm_hbm_traffic.md"
    try:
        for line in path.read_text().splitlines():
            if line.startswith("machine-readable:"):
                fields = dict(kv.split("=") for kv in line.split(":", 1)[1].split())
                return float(fields["gemm_traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None
    return None


def copy_calibration(hip, stream, mib: int) -> None:
    """One device-to-device copy of `mib` MiB (tlh_copy): its FETCH_SIZE and
    WRITE_SIZE readings must equal the copy size, which calibrates the
    counters of the other kernels."""
    from templit_amd.native import check

    n = mib * (1 << 20) // 4
    bufs = []
    for _ in range(2):
        ptr = ctypes.c_void_p()
        check(hip.tlh_malloc(ctypes.byref(ptr), n * 4), "malloc")
        bufs.append(ptr.value)
    try:
        check(hip.tlh_fill_f32(bufs[0], 1.0, n, stream), "fill")
        check(hip.tlh_copy(bufs[0], bufs[1], n, stream), "copy")
        check(hip.tlh_stream_synchronize(stream), "sync")
    finally:
        for b in bufs:
            hip.tlh_free(b)
    log(f"[bench] calibration copy of {mib} MiB done")


def cpu_baseline(sample_batch: int, steps: int) -> dict:
    """The CPU oracle (single-threaded C++ restatement of the reference
    algorithms) running the same training step at a smaller batch."""
    sys.path.insert(0, str(ROOT / "tests"))
    import numpy as np
    import oracle_lib as O

    cfg = O.gpt_config(CFG["vocab"], CFG["seq"], CFG["dim"], CFG["heads"], CFG["layers"],
                       sample_batch)
    total = int(sum(O.gpt_param_sizes(cfg)))
    params = O.normal((total,), 1, 0, 0.02)
    rows = sample_batch * CFG["seq"]
    tok = O.uniform_u32((rows,), 2, CFG["vocab"])
    tgt = O.uniform_u32((rows,), 3, CFG["vocab"])
    m = np.zeros_like(params)
    v = np.zeros_like(params)
    t0 = time.perf_counter()
    for s in range(steps):
        out = O.gpt_train_step(cfg, params, m, v, s + 1, tok, tgt, 1.0 / rows, HP["lr"],
                               HP["beta1"], HP["beta2"], HP["eps"], HP["weight_decay"],
                               MAX_NORM)
        params, m, v = out["params"], out["m"], out["v"]
    dt = time.perf_counter() - t0
    return {"value": round(rows * steps / dt, 2), "unit": "tokens/s", "cores": 1,
            "kind": "port",
            "sample": f"{steps} oracle training steps of the same model at batch "
                      f"{sample_batch} ({rows} tokens/step, {dt:.1f} s), single thread",
            **host_cpu(),
            "kernel_configs": cpu_kernel_configs(),
            "reference_cpu_runtime": reference_cpu_kernels()}


def host_cpu() -> dict:
    """CPU model and core counts of the machine the baseline ran on."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = None
    return {"cpu_model": model, "nproc": usable, "cpu_count": os.cpu_count()}


def reference_cpu_kernels() -> dict | None:
    """The reference's own CPU runtime (src/CPU/cpu.cpp, compiled from its
    sources into oracle/_ref/libref_cpu.so at -O2, one thread) on the
    configurations it can run: matmul + bias (config 1, mult then the
    broadcast add) and the [6144,2048] softmax. Times include copying the
    operands into and out of its tensors (a few MB, well under 1 %)."""
    sys.path.insert(0, str(ROOT / "tests"))
    import numpy as np
    import oracle_lib as O

    if not O.ref_available():
        return None
    r = O.ref()
    M, K, N = C1
    a, b, bias = O.normal((M, K), 1, 0, 0.02), O.normal((K, N), 2, 0, 0.02), O.normal((1, N), 3)
    c, out = np.empty((M, N), np.float32), np.empty((M, N), np.float32)
    x, y = O.normal((R2, V2), 9), np.empty((R2, V2), np.float32)

    def best_of(fn, n=3):
        times = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return min(times)

    def mult_add():
        assert r.ref_mult(O.p(a), O.p(b), O.p(c), M, K, N) == 0
        assert r.ref_binary(0, O.p(c), M, N, O.p(bias), 1, N, O.p(out)) == 0

    mm = best_of(mult_add)
    sm = best_of(lambda: r.ref_softmax(O.p(x), O.p(y), R2, V2))
    res = {"kind": "reference", "cores": 1, "build": "clang++ -O2 (the reference's default)",
           "matmul_bias_768x384x1536": {"s": round(mm, 4),
                                        "gflops": round((2.0 * M * N * K + M * N) / mm / 1e9, 2)},
           "softmax_6144x2048": {"s": round(sm, 4),
                                 "gb_s": round(ROW_OP_BYTES["softmax_fwd"] / sm / 1e9, 2)},
           "timing": "best of 3 calls"}
    log(f"[bench] reference CPU runtime: {json.dumps(res)}")
    return res


def cpu_kernel_configs() -> dict:
    """The oracle (one thread) on the kernel configurations, full size."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O

    def timed(fn):
        t0 = time.perf_counter()
        fn()
        return time.perf_counter() - t0

    out = {}
    M, K, N = C1
    a, b, bias = O.normal((M, K), 1, 0, 0.02), O.normal((K, N), 2, 0, 0.02), O.normal((1, N), 3)
    dt = timed(lambda: O.binary("add", O.matmul(a, b), bias))
    out["matmul_bias_768x384x1536"] = {"s": round(dt, 3),
                                       "gflops": round((2.0 * M * N * K + M * N) / dt / 1e9, 2)}
    x, gx, gain = O.normal((R2, D2), 4), O.normal((R2, D2), 5), O.normal((D2,), 6, 1.0, 0.02)
    h, gh = O.normal((R2, F2), 7), O.normal((R2, F2), 8)
    lg, glg = O.normal((R2, V2), 9), O.normal((R2, V2), 10)
    tgt = O.uniform_u32((R2,), 11, V2)
    y = O.softmax(lg)
    ops = {
        "rmsnorm_fwd": lambda: O.rms_norm(x, gain),
        "rmsnorm_bwd": lambda: O.rms_norm_backward(gx, x, gain),
        "gelu_fwd": lambda: O.unary("gelu", h),
        "gelu_bwd": lambda: O.binary("hadamard", gh, O.unary("gelu_derivative", h)),
        "softmax_fwd": lambda: O.softmax(lg),
        "softmax_bwd": lambda: O.softmax_backward(glg, y),
        "cross_entropy_fwd": lambda: O.cross_entropy(lg, tgt),
        "cross_entropy_bwd_scaled": lambda: O.cross_entropy_backward(lg, tgt),
    }
    rowops = {}
    for name, fn in ops.items():
        dt = timed(fn)
        rowops[name] = {"s": round(dt, 4), "gb_s": round(ROW_OP_BYTES[name] / dt / 1e9, 2)}
    out["row_ops"] = rowops
    B, H, T, Dh = C3
    q, k, v = (O.normal((B, H, T, Dh), 13 + i, 0.0, 0.125) for i in range(3))
    do = O.normal((B, H, T, Dh), 16)
    t0 = time.perf_counter()
    o, probs = O.attention_forward(q, k, v)
    t1 = time.perf_counter()
    O.attention_backward(q, k, v, probs, do)
    t2 = time.perf_counter()
    out["attention_b32_h6_t192"] = {"forward_s": round(t1 - t0, 3), "backward_s": round(t2 - t1, 3)}
    log(f"[bench] CPU oracle kernel configurations: {json.dumps(out)}")
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-batch", type=int, default=4)
    ap.add_argument("--cpu-steps", type=int, default=6)
    ap.add_argument("--graph", action="store_true",
                    help="time hipGraph replays of the captured step instead of eager launches "
                         "(the other execution is timed afterwards either way)")
    ap.add_argument("--eager", action="store_true",
                    help="eager launches (the default; kept for existing command lines)")
    ap.add_argument("--skip-d1024", action="store_true")
    ap.add_argument("--skip-kernels", action="store_true",
                    help="skip the single-kernel configurations (matmul+bias, row ops, attention)")
    ap.add_argument("--skip-scaled", action="store_true",
                    help="skip the d=1024 / 12-block / T=1024 configuration")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="run one device copy of MIB MiB (counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the GPT step runs on a single MI355X; "
              "across GPUs it would shard along the batch (data parallel, one "
              "gradient all-reduce before the norm)", file=sys.stderr)
        return 2

    from templit_amd.native import GptProgram, load_hip

    hip = load_hip()
    prog = GptProgram(**CFG)
    tokens = CFG["batch"] * CFG["seq"]
    root = 1.0 / tokens
    prog.init_params(seed=1, std=0.02)
    prog.set_optimizer(**HP)
    prog.random_batch(seed=7)
    prog.synchronize()
    log(f"[bench] program ready: {prog.total} parameters, {tokens} tokens/step")

    if args.copy_calibration:
        copy_calibration(hip, prog.stream, args.copy_calibration)
    eager = lambda: prog.train_step(root, MAX_NORM)
    step = prog.replay if args.graph else eager
    if args.graph:
        prog.capture(root, MAX_NORM)
    for _ in range(args.warmup):
        step()
    prog.synchronize()
    log(f"[bench] {args.warmup} warmup steps done")

    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    prog.synchronize()
    dt = time.perf_counter() - t0
    ms_per_step = dt * 1e3 / args.steps
    tok_s = tokens * args.steps / dt
    loss = float(prog.losses().mean())
    log(f"[bench] {args.steps} timed steps: {ms_per_step:.3f} ms/step, "
        f"{tok_s:.0f} tokens/s, loss {loss:.4f}")
    # the other execution of the same step, for comparison
    if args.graph:
        other_name, other = "eager launches on two streams", eager
    else:
        other_name, other = "one hipGraph replay per step", prog.replay
        prog.capture(root, MAX_NORM)
    other_dt = time_steps(prog, other, args.warmup, args.steps)
    other_exec = {"execution": other_name, "ms_per_step": round(other_dt * 1e3, 4),
                  "tokens_per_s": round(tokens / other_dt, 1)}
    log(f"[bench] {other_name}: {other_exec['ms_per_step']} ms/step")

    prof = prog.profile_step(root, MAX_NORM)
    # kernel time: each GEMM launch of that step again, 10 times back to back
    gemm_ms = prog.time_gemms(10)
    gemm_tflops = prof["gemm_flops"] / (gemm_ms * 1e-3) / 1e12
    log(f"[bench] profiled step: {prof}")
    d1024 = None if args.skip_d1024 else gemm_d1024(hip, prog.stream)
    log(f"[bench] d=1024 GEMM: {d1024}")
    kernels = None if args.skip_kernels else kernel_configs(hip, prog.stream)
    prog.close()

    result = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: uniform random tokens in [0,2048), random-init weights N(0,0.02)",
        "config": {
            "workload": "GPT training step (fwd + CE + bwd + clip 1.0 + AdamW), "
                        "vocab 2048, T 192, d 384, 4 blocks, 6 heads, FFN 1536, batch 32",
            "global_batch": CFG["batch"], "seq_len": CFG["seq"], "tokens_per_step": tokens,
            "parallelism": "single GPU",
            "execution": "one hipGraph replay per step" if args.graph
                         else "eager launches on two streams",
        },
        "other_execution": other_exec,
        "roofline": {
            "bound": "mfma",
            "kernel": "gemm_mfma_kernel (every GEMM launch of one step)",
            "achieved": round(gemm_tflops, 2),
            "peak": FP32_MFMA_PEAK,
            "unit": "TFLOP/s",
            "frac": round(gemm_tflops / FP32_MFMA_PEAK, 4),
            "traffic": gemm_traffic(),
            "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0, "
                            "profiles/gpt_step_b32_t192_d384_gemm_hbm_traffic.md)",
            "algorithmic_bytes_per_launch": round(prof["gemm_bytes"] / max(1, prof["gemm_launches"])),
            "flops_per_step": prof["gemm_flops"],
            "launches_per_step": prof["gemm_launches"],
            "avg_launch_us": round(gemm_ms * 1e3 / max(1, prof["gemm_launches"]), 2),
            "gemm_ms_per_step": round(gemm_ms, 4),
            "timing": "HIP events on the program's stream around 10 back-to-back repeats of "
                      "each GEMM launch of one eager step",
            "gemm_ms_in_eager_step": round(prof["gemm_ms"], 4),
            "attention_ms_per_step": round(prof["attention_ms"], 4),
            "eager_step_ms": round(prof["step_ms"], 4),
        },
        "gemm_d1024": d1024,
        "kernel_configs": kernels,
        "scaled_gpt": None if args.skip_scaled else scaled_gpt(5, 256),
        "loss": round(loss, 4),
    }
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU oracle sample ...")
        result["cpu_baseline"] = cpu_baseline(args.cpu_sample_batch, args.cpu_steps)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
