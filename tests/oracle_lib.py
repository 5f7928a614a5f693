"""numpy front-end for the CPU oracle (oracle/liboracle.so) and for the
reference CPU runtime shim (oracle/_ref/libref_cpu.so).

The oracle is the checker: tests compare the HIP path against it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_float, c_int, c_size_t, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_DIR = ROOT / "oracle"
# TEMPLIT_ORACLE_LIB / TEMPLIT_REF_CPU_LIB select other builds of the same
# sources (the sanitizer builds of tests/test_sanitizers.py)
ORACLE_LIB = Path(os.environ.get("TEMPLIT_ORACLE_LIB", ORACLE_DIR / "liboracle.so"))
REF_LIB = Path(os.environ.get("TEMPLIT_REF_CPU_LIB", ORACLE_DIR / "_ref" / "libref_cpu.so"))

F32P = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
U32P = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")


class GptConfig(ctypes.Structure):
    _fields_ = [("vocab", c_uint32), ("seq", c_uint32), ("dim", c_uint32),
                ("heads", c_uint32), ("layers", c_uint32), ("batch", c_uint32),
                ("ffn", c_uint32)]


def _u32(values) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(values, dtype=np.uint32))


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _load_oracle() -> ctypes.CDLL:
    if not ORACLE_LIB.exists():
        subprocess.run(["make", "-C", str(ORACLE_DIR), "oracle"], check=True,
                       stdout=subprocess.DEVNULL)
    lib = ctypes.CDLL(str(ORACLE_LIB))
    V = c_void_p
    sig = {
        "orc_fill_normal": [V, c_size_t, c_uint64, c_float, c_float],
        "orc_fill_uniform_u32": [V, c_size_t, c_uint64, c_uint32],
        "orc_binary": [c_int, V, V, V, c_uint32, V, V, V],
        "orc_unary": [c_int, V, V, c_size_t],
        "orc_scalar": [c_int, V, c_float, V, c_size_t],
        "orc_transpose": [V, V, c_uint32, V, V],
        "orc_matmul": [V, V, V, c_uint32, c_uint32, c_uint32, c_uint32, V, V, V],
        "orc_sum_to_shape": [V, V, c_uint32, V, V],
        "orc_max_to_shape": [V, V, c_uint32, V, V],
        "orc_softmax": [V, V, c_size_t, c_uint32],
        "orc_softmax_backward": [V, V, V, c_size_t, c_uint32],
        "orc_cross_entropy_rows": [V, V, V, c_size_t, c_uint32],
        "orc_cross_entropy_rows_backward": [V, V, V, c_size_t, c_uint32],
        "orc_rms": [V, V, c_size_t, c_uint32, c_float],
        "orc_rms_norm": [V, V, V, V, c_size_t, c_uint32, c_float],
        "orc_rms_norm_backward": [V, V, V, V, V, c_size_t, c_uint32, c_float],
        "orc_embedding_lookup": [V, c_uint32, V, c_size_t, V],
        "orc_scatter_add_rows": [V, V, c_size_t, c_uint32, V],
        "orc_accumulate_gradient_squared_norm": [V, c_size_t, V],
        "orc_clip_gradient": [V, V, c_float, V, c_size_t],
        "orc_adamw": [V, V, V, V, V, c_float, c_float, c_float, c_float, c_float, c_uint32,
                      c_size_t],
        "orc_attention_forward": [V, V, V, V, V, c_uint32, c_uint32, c_uint32, c_uint32, c_int],
        "orc_attention_backward": [V, V, V, V, V, V, V, V, c_uint32, c_uint32, c_uint32,
                                   c_uint32],
        "orc_gpt_param_count": [POINTER(GptConfig)],
        "orc_gpt_param_size": [POINTER(GptConfig), c_uint32],
        "orc_gpt_total_params": [POINTER(GptConfig)],
        "orc_gpt_train_step": [POINTER(GptConfig), V, V, V, c_uint32, V, V, c_float, c_float,
                               c_float, c_float, c_float, c_float, c_float, V, V, V],
        "orc_gpt_forward": [POINTER(GptConfig), V, V, V],
        "orc_sample_top_k": [V, c_uint32, c_uint32, c_uint32, c_uint32, c_float, c_uint64,
                             c_uint64, V, c_uint32, c_int, c_uint32, V, V],
    }
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = c_int
    lib.orc_sum.argtypes = [c_void_p, c_size_t]
    lib.orc_sum.restype = c_float
    lib.orc_argmax.argtypes = [c_void_p, c_size_t]
    lib.orc_argmax.restype = c_uint32
    lib.orc_gpt_param_count.restype = c_uint32
    lib.orc_gpt_param_size.restype = c_uint64
    lib.orc_gpt_total_params.restype = c_uint64
    return lib


_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = _load_oracle()
    return _LIB


def p(a: np.ndarray) -> int:
    return a.ctypes.data


# ---- synthetic data --------------------------------------------------------
def normal(shape, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(int(np.prod(shape)) if len(shape) else 1, dtype=np.float32)
    lib().orc_fill_normal(p(out), out.size, seed, mean, std)
    return out.reshape(shape)


def uniform_u32(shape, seed: int, bound: int) -> np.ndarray:
    out = np.empty(int(np.prod(shape)), dtype=np.uint32)
    lib().orc_fill_uniform_u32(p(out), out.size, seed, bound)
    return out.reshape(shape)


# ---- broadcast helpers (runtime.cpp:18-39 broadcast_strides) ---------------
def contiguous_strides(shape) -> list[int]:
    st, s = [], 1
    for d in reversed(shape):
        st.append(s)
        s *= d
    return list(reversed(st))


def broadcast_shape(a, b) -> list[int]:
    rank = max(len(a), len(b))
    out = []
    for i in range(rank):
        x = a[len(a) - rank + i] if i >= rank - len(a) else 1
        y = b[len(b) - rank + i] if i >= rank - len(b) else 1
        if x != y and x != 1 and y != 1:
            raise ValueError("shapes cannot be broadcast")
        out.append(max(x, y))
    return out


def broadcast_strides(shape, out_shape) -> list[int]:
    strides = contiguous_strides(shape)
    res = [0] * len(out_shape)
    off = len(out_shape) - len(shape)
    for i, d in enumerate(shape):
        if d == out_shape[off + i]:
            res[off + i] = strides[i]
        elif d == 1:
            res[off + i] = 0
        else:
            raise ValueError("invalid broadcast")
    return res


BIN_OPS = {"add": 0, "sub": 1, "hadamard": 2, "divide": 3}


def binary(op: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    out_shape = broadcast_shape(a.shape, b.shape)
    out = np.empty(out_shape, dtype=np.float32)
    shp = _u32(out_shape)
    sa = _u32(broadcast_strides(a.shape, out_shape))
    sb = _u32(broadcast_strides(b.shape, out_shape))
    lib().orc_binary(BIN_OPS[op], p(a), p(b), p(out), len(out_shape), p(shp), p(sa), p(sb))
    return out


UN_OPS = {"sqrt": 0, "exp": 1, "sigmoid": 2, "gelu": 3, "gelu_derivative": 4, "copy": 5}


def unary(op: str, a: np.ndarray) -> np.ndarray:
    a = _f32(a)
    out = np.empty_like(a)
    lib().orc_unary(UN_OPS[op], p(a), p(out), a.size)
    return out


SC_OPS = {"add": 0, "divide": 1, "pow": 2}


def scalar(op: str, a: np.ndarray, s: float) -> np.ndarray:
    a = _f32(a)
    out = np.empty_like(a)
    lib().orc_scalar(SC_OPS[op], p(a), s, p(out), a.size)
    return out


def transpose(a: np.ndarray, dim_a: int = -2, dim_b: int = -1) -> np.ndarray:
    a = _f32(a)
    nd = a.ndim
    da, db = dim_a % nd, dim_b % nd
    out_shape = list(a.shape)
    out_shape[da], out_shape[db] = out_shape[db], out_shape[da]
    in_strides = contiguous_strides(a.shape)
    in_strides[da], in_strides[db] = in_strides[db], in_strides[da]
    out = np.empty(out_shape, dtype=np.float32)
    shp, ist = _u32(out_shape), _u32(in_strides)
    lib().orc_transpose(p(a), p(out), nd, p(shp), p(ist))
    return out


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Batched broadcasting matmul (Runtime::mult semantics)."""
    a, b = _f32(a), _f32(b)
    M, K = a.shape[-2], a.shape[-1]
    N = b.shape[-1]
    assert b.shape[-2] == K
    ab, bb = list(a.shape[:-2]), list(b.shape[:-2])
    batch = broadcast_shape(ab, bb) if (ab or bb) else []
    sa = broadcast_strides(ab, batch) if ab else [0] * len(batch)
    sb = broadcast_strides(bb, batch) if bb else [0] * len(batch)
    sa = [s * M * K for s in sa]
    sb = [s * K * N for s in sb]
    out = np.empty(batch + [M, N], dtype=np.float32)
    bs, bsa, bsb = _u32(batch or [1]), _u32(sa or [0]), _u32(sb or [0])
    lib().orc_matmul(p(a), p(b), p(out), M, K, N, len(batch), p(bs), p(bsa), p(bsb))
    return out


def aligned_shape(a_shape, out_shape) -> list[int]:
    off = len(a_shape) - len(out_shape)
    return [1] * off + list(out_shape)


def sum_to_shape(a: np.ndarray, out_shape) -> np.ndarray:
    a = _f32(a)
    al = aligned_shape(a.shape, out_shape)
    out = np.empty(al, dtype=np.float32)
    ash, alu = _u32(a.shape), _u32(al)
    lib().orc_sum_to_shape(p(a), p(out), a.ndim, p(ash), p(alu))
    return out.reshape(out_shape)


def max_to_shape(a: np.ndarray, out_shape) -> np.ndarray:
    a = _f32(a)
    al = aligned_shape(a.shape, out_shape)
    out = np.empty(al, dtype=np.float32)
    ash, alu = _u32(a.shape), _u32(al)
    lib().orc_max_to_shape(p(a), p(out), a.ndim, p(ash), p(alu))
    return out.reshape(out_shape)


def total_sum(a: np.ndarray) -> float:
    a = _f32(a)
    return lib().orc_sum(p(a), a.size)


def argmax(a: np.ndarray) -> int:
    a = _f32(a)
    return int(lib().orc_argmax(p(a), a.size))


def sample_top_k(logits: np.ndarray, top_k: int, temperature: float, seed: int = 0,
                 counter: int = 0, uniforms=None, eos: int = 0, resample_eos: bool = False,
                 max_draws: int = 1, row_stride: int | None = None):
    """orc_sample_top_k over the rows of `logits` ([rows, V], or [V] for one
    row): (tokens u32 [rows], draws u32 [rows])."""
    x = _f32(logits)
    V = x.shape[-1]
    rows = x.size // V if row_stride is None else len(uniforms) // max_draws
    stride = V if row_stride is None else row_stride
    tokens = np.zeros(rows, np.uint32)
    draws = np.zeros(rows, np.uint32)
    u = None if uniforms is None else np.ascontiguousarray(uniforms, dtype=np.float64)
    lib().orc_sample_top_k(p(x), rows, V, stride, top_k, temperature, seed, counter,
                           None if u is None else p(u), eos, int(resample_eos), max_draws,
                           p(tokens), p(draws))
    return tokens, draws


def softmax(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_softmax(p(x), p(out), x.size // x.shape[-1], x.shape[-1])
    return out


def softmax_backward(g: np.ndarray, y: np.ndarray) -> np.ndarray:
    g, y = _f32(g), _f32(y)
    out = np.empty_like(g)
    lib().orc_softmax_backward(p(g), p(y), p(out), g.size // g.shape[-1], g.shape[-1])
    return out


def cross_entropy(logits: np.ndarray, targets: np.ndarray) -> np.ndarray:
    logits, targets = _f32(logits), _u32(targets)
    V = logits.shape[-1]
    out = np.empty(list(targets.shape) + [1], dtype=np.float32)
    lib().orc_cross_entropy_rows(p(logits), p(targets), p(out), targets.size, V)
    return out


def cross_entropy_backward(logits: np.ndarray, targets: np.ndarray) -> np.ndarray:
    logits, targets = _f32(logits), _u32(targets)
    out = np.empty_like(logits)
    lib().orc_cross_entropy_rows_backward(p(logits), p(targets), p(out), targets.size,
                                          logits.shape[-1])
    return out


def rms(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x = _f32(x)
    out = np.empty(list(x.shape[:-1]) + [1], dtype=np.float32)
    lib().orc_rms(p(x), p(out), x.size // x.shape[-1], x.shape[-1], eps)
    return out


def rms_norm(x: np.ndarray, gain=None, eps: float = 1e-6) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    g = _f32(gain) if gain is not None else None
    lib().orc_rms_norm(p(x), p(g) if g is not None else None, p(y), None,
                       x.size // x.shape[-1], x.shape[-1], eps)
    return y


def rms_norm_backward(g: np.ndarray, x: np.ndarray, gain=None, eps: float = 1e-6):
    g, x = _f32(g), _f32(x)
    dx = np.empty_like(x)
    gn = _f32(gain) if gain is not None else None
    dgain = np.empty(x.shape[-1], dtype=np.float32) if gain is not None else None
    lib().orc_rms_norm_backward(p(g), p(x), p(gn) if gn is not None else None, p(dx),
                                p(dgain) if dgain is not None else None,
                                x.size // x.shape[-1], x.shape[-1], eps)
    return dx, dgain


def embedding_lookup(w: np.ndarray, ids: np.ndarray) -> np.ndarray:
    w, ids = _f32(w), _u32(ids)
    out = np.empty(list(ids.shape) + [w.shape[1]], dtype=np.float32)
    lib().orc_embedding_lookup(p(w), w.shape[1], p(ids), ids.size, p(out))
    return out


def scatter_add_rows(base: np.ndarray, ids: np.ndarray, values: np.ndarray) -> np.ndarray:
    out = _f32(base).copy()
    ids, values = _u32(ids), _f32(values)
    lib().orc_scatter_add_rows(p(values), p(ids), ids.size, out.shape[1], p(out))
    return out


def grad_norm_accumulate(grads, start: float = 0.0) -> float:
    s = np.array([start], dtype=np.float32)
    for g in grads:
        g = _f32(g)
        lib().orc_accumulate_gradient_squared_norm(p(g), g.size, p(s))
    return float(s[0])


def clip_gradient(g: np.ndarray, squared_norm: float, max_norm: float) -> np.ndarray:
    g = _f32(g)
    out = np.empty_like(g)
    s = np.array([squared_norm], dtype=np.float32)
    lib().orc_clip_gradient(p(g), p(s), max_norm, p(out), g.size)
    return out


def adamw(param, grad, m1, m2, beta1, beta2, decay, lr, eps, step):
    param, grad = _f32(param).copy(), _f32(grad)
    m1, m2 = _f32(m1).copy(), _f32(m2).copy()
    lib().orc_adamw(p(param), p(grad), p(param), p(m1), p(m2), beta1, beta2, decay, lr, eps,
                    step, param.size)
    return param, m1, m2


def attention_forward(q, k, v, causal=True):
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, T, D = q.shape
    o = np.empty_like(q)
    probs = np.empty((B, H, T, T), dtype=np.float32)
    lib().orc_attention_forward(p(q), p(k), p(v), p(o), p(probs), B, H, T, D, int(causal))
    return o, probs


def attention_backward(q, k, v, probs, dout):
    q, k, v, probs, dout = map(_f32, (q, k, v, probs, dout))
    B, H, T, D = q.shape
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    lib().orc_attention_backward(p(q), p(k), p(v), p(probs), p(dout), p(dq), p(dk), p(dv),
                                 B, H, T, D)
    return dq, dk, dv


# ---- GPT --------------------------------------------------------------------
def gpt_config(vocab, seq, dim, heads, layers, batch, ffn=None) -> GptConfig:
    return GptConfig(vocab, seq, dim, heads, layers, batch, ffn if ffn else 4 * dim)


def gpt_param_sizes(cfg: GptConfig) -> list[int]:
    n = lib().orc_gpt_param_count(ctypes.byref(cfg))
    return [int(lib().orc_gpt_param_size(ctypes.byref(cfg), i)) for i in range(n)]


def gpt_key_bias_indices(cfg: GptConfig) -> list[int]:
    """Indices of the K-projection biases. Their gradient is exactly zero:
    q.(k_j + b) = q.k_j + q.b shifts every score of a query row by the same
    constant and softmax is shift invariant, so both the oracle and the GPU
    hold only rounding noise there (and AdamW's first step turns that noise
    into +-lr)."""
    return [2 + 12 * l + 3 for l in range(cfg.layers)]


def gpt_train_step(cfg: GptConfig, params, m, v, step, tokens, targets, root_grad, lr, beta1,
                   beta2, eps, weight_decay, max_norm):
    params, m, v = _f32(params).copy(), _f32(m).copy(), _f32(v).copy()
    tokens, targets = _u32(tokens), _u32(targets)
    rows = cfg.batch * cfg.seq
    losses = np.empty(rows, dtype=np.float32)
    grads = np.empty_like(params)
    sq = np.zeros(1, dtype=np.float32)
    rc = lib().orc_gpt_train_step(ctypes.byref(cfg), p(params), p(m), p(v), step, p(tokens),
                                  p(targets), root_grad, lr, beta1, beta2, eps, weight_decay,
                                  max_norm, p(losses), p(grads), p(sq))
    assert rc == 0
    return dict(params=params, m=m, v=v, losses=losses, grads=grads, squared_norm=float(sq[0]))


def gpt_forward(cfg: GptConfig, params, tokens) -> np.ndarray:
    params, tokens = _f32(params), _u32(tokens)
    logits = np.empty((cfg.batch * cfg.seq, cfg.vocab), dtype=np.float32)
    assert lib().orc_gpt_forward(ctypes.byref(cfg), p(params), p(tokens), p(logits)) == 0
    return logits


# ---- reference CPU runtime (oracle/_ref) -------------------------------------
_REF: ctypes.CDLL | None = None


def ref_available() -> bool:
    return REF_LIB.exists()


def ref() -> ctypes.CDLL:
    global _REF
    if _REF is None:
        r = ctypes.CDLL(str(REF_LIB))
        V = c_void_p
        for name, args in {
            "ref_mult": [V, V, V, c_uint32, c_uint32, c_uint32],
            "ref_binary": [c_int, V, c_uint32, c_uint32, V, c_uint32, c_uint32, V],
            "ref_softmax": [V, V, c_uint32, c_uint32],
            "ref_transpose": [V, V, c_uint32, c_uint32],
            "ref_sum_to_shape": [V, c_uint32, c_uint32, V, c_uint32, c_uint32],
            "ref_sum": [V, c_uint32, c_uint32, V],
            "ref_unary": [c_int, V, V, c_uint32, c_uint32],
            "ref_argmax": [V, c_uint32, c_uint32, V],
        }.items():
            fn = getattr(r, name)
            fn.argtypes = args
            fn.restype = c_int
        _REF = r
    return _REF
