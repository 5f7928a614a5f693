"""ctypes bindings of the C-ABI in include/templit_hip.h (and of the GPT
program library).

Python is plumbing here: the tests and bench.py drive the native libraries
through these bindings, passing device pointers (from torch tensors) and
hipStream_t handles. Loading fails loudly when a library is missing -- there
is no fallback path.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float, c_int, c_int32, c_size_t, c_uint32, c_uint64, c_void_p
from pathlib import Path

PKG = Path(__file__).resolve().parent
HIP_LIB = PKG / "libtemplit_hip.so"
GPT_LIB = PKG / "libtemplit_gpt.so"

P = c_void_p
U32P = c_void_p  # device/host uint32 arrays are passed as raw addresses


class GemmDesc(ctypes.Structure):
    """Mirror of struct tlh_gemm_desc."""

    _fields_ = [
        ("a", c_void_p), ("b", c_void_p), ("c", c_void_p),
        ("bias", c_void_p), ("residual", c_void_p), ("aux", c_void_p),
        ("workspace", c_void_p),
        ("m", c_int32), ("n", c_int32), ("k", c_int32),
        ("lda", c_int32), ("ldb", c_int32), ("ldc", c_int32),
        ("trans_a", c_int32), ("trans_b", c_int32),
        ("beta", c_float),
        ("epilogue", c_int32),
        ("remap_t", c_int32), ("remap_h", c_int32), ("remap_d", c_int32),
        ("bias_grad", c_void_p),
        ("batch", c_int32),
        ("batch_stride_a", c_uint32), ("batch_stride_b", c_uint32),
        ("batch_stride_c", c_uint32), ("bias_batch_stride", c_uint32),
        ("sum_batches", c_int32),
        ("workspace_elems", c_size_t),
    ]


EPI_STORE, EPI_GELU, EPI_GELU_BWD = 0, 1, 2

# name -> argtypes (restype is always int = hipError_t, except tlh_error_string)
HIP_SIGNATURES: dict[str, list] = {
    "tlh_init": [c_int],
    "tlh_device_count": [POINTER(c_int)],
    "tlh_device_cu_count": [POINTER(c_int)],
    "tlh_device_synchronize": [],
    "tlh_stream_create": [POINTER(c_void_p)],
    "tlh_stream_destroy": [P],
    "tlh_stream_synchronize": [P],
    "tlh_malloc": [POINTER(c_void_p), c_size_t],
    "tlh_free": [P],
    "tlh_host_alloc": [POINTER(c_void_p), c_size_t],
    "tlh_host_free": [P],
    "tlh_memcpy_h2d": [P, P, c_size_t, P],
    "tlh_memcpy_d2h": [P, P, c_size_t, P],
    "tlh_memcpy_d2d": [P, P, c_size_t, P],
    "tlh_fill_f32": [P, c_float, c_size_t, P],
    "tlh_fill_u32": [P, c_uint32, c_size_t, P],
    "tlh_increment_u32": [P, c_size_t, c_uint32, P],
    "tlh_fill_normal": [P, c_size_t, c_uint64, c_float, c_float, P],
    "tlh_fill_uniform_u32": [P, c_size_t, c_uint64, c_uint32, P],
    "tlh_compare": [P, P, c_size_t, POINTER(c_int), P, P],
    "tlh_event_create": [POINTER(c_void_p)],
    "tlh_event_record": [P, P],
    "tlh_event_synchronize": [P],
    "tlh_event_elapsed_ms": [P, P, POINTER(c_float)],
    "tlh_event_destroy": [P],
    "tlh_stream_wait_event": [P, P],
    "tlh_graph_begin_capture": [P],
    "tlh_graph_end_capture": [P, POINTER(c_void_p)],
    "tlh_graph_launch": [P, P],
    "tlh_graph_destroy": [P],
    "tlh_graph_begin_capture_relaxed": [P],
    "tlh_graph_end_capture_graph": [P, POINTER(c_void_p)],
    "tlh_graph_instantiate": [P, POINTER(c_void_p)],
    "tlh_graph_exec_update": [P, P, POINTER(c_int)],
    "tlh_graph_free": [P],
    "tlh_stream_is_capturing": [P, POINTER(c_int)],
    "tlh_range_push": [ctypes.c_char_p],
    "tlh_range_pop": [],
    # elementwise
    "tlh_add": [P, P, P, c_uint32, U32P, U32P, U32P, P],
    "tlh_sub": [P, P, P, c_uint32, U32P, U32P, U32P, P],
    "tlh_hadamard": [P, P, P, c_uint32, U32P, U32P, U32P, P],
    "tlh_divide": [P, P, P, c_uint32, U32P, U32P, U32P, P],
    "tlh_add_scalar": [P, c_float, P, c_size_t, P],
    "tlh_divide_scalar": [P, c_float, P, c_size_t, P],
    "tlh_pow_scalar": [P, c_float, P, c_size_t, P],
    "tlh_sqrt": [P, P, c_size_t, P],
    "tlh_exp": [P, P, c_size_t, P],
    "tlh_sigmoid": [P, P, c_size_t, P],
    "tlh_gelu": [P, P, c_size_t, P],
    "tlh_gelu_derivative": [P, P, c_size_t, P],
    "tlh_copy": [P, P, c_size_t, P],
    "tlh_gelu_backward": [P, P, P, c_size_t, P],
    "tlh_transpose": [P, P, c_uint32, U32P, U32P, P],
    "tlh_transpose_multi": [P, P, P, c_uint32, c_uint32, P],
    # products
    "tlh_matmul": [P, P, P, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                   c_uint32, c_uint32, c_uint32, c_uint32, U32P, U32P, U32P, U32P, P],
    "tlh_matmul_workspace_size": [c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                                  c_uint32, c_uint32, c_uint32, c_uint32, U32P, U32P, U32P, U32P,
                                  POINTER(c_size_t)],
    "tlh_matmul_ws": [P, P, P, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                      c_uint32, c_uint32, c_uint32, c_uint32, U32P, U32P, U32P, U32P, P, c_size_t,
                      P],
    "tlh_matmul_bias_ws": [P, P, P, P, P, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                           c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, U32P, U32P, U32P,
                           U32P, P, c_size_t, P],
    "tlh_matmul_noalloc": [P, P, P, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                           c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, U32P, U32P, U32P,
                           U32P, P],
    "tlh_gemm": [POINTER(GemmDesc), P],
    "tlh_gemm_workspace_size": [POINTER(GemmDesc), POINTER(c_size_t)],
    "tlh_gemm_set_plan": [c_int, c_int, c_int, c_int],
    # reductions
    "tlh_sum": [P, c_size_t, P, P],
    "tlh_sum_to_shape": [P, P, c_uint32, U32P, U32P, P],
    "tlh_sum_to_shape_workspace": [c_uint32, U32P, U32P, P],
    "tlh_sum_to_shape_ws": [P, P, c_uint32, U32P, U32P, P, c_size_t, P],
    "tlh_max_to_shape": [P, P, c_uint32, U32P, U32P, P],
    "tlh_argmax": [P, c_size_t, P, P],
    "tlh_argmax_rows": [P, c_size_t, c_uint32, P, P],
    "tlh_sample_top_k": [P, c_uint32, c_uint32, c_uint32, c_uint32, c_float, c_uint64, c_uint64,
                         P, c_uint32, c_int, c_uint32, P, P, P],
    "tlh_accumulate_gradient_squared_norm": [P, c_size_t, P, P],
    "tlh_gradient_squared_norm_multi": [P, P, c_uint32, P, P, P],
    "tlh_column_sum": [P, c_size_t, c_uint32, P, c_float, P],
    # row ops
    "tlh_softmax": [P, P, c_size_t, c_uint32, P],
    "tlh_softmax_backward": [P, P, P, c_size_t, c_uint32, P],
    "tlh_cross_entropy_rows": [P, P, P, c_size_t, c_uint32, P],
    "tlh_cross_entropy_rows_backward": [P, P, P, c_size_t, c_uint32, P, P],
    "tlh_cross_entropy_rows_fused": [P, P, P, P, c_size_t, c_uint32, c_float, P],
    "tlh_rms": [P, P, c_size_t, c_uint32, c_float, P],
    "tlh_rms_norm": [P, P, P, P, c_size_t, c_uint32, c_float, P],
    "tlh_rms_norm_backward": [P, P, P, P, P, c_size_t, c_uint32, c_float, c_float, P],
    # embedding
    "tlh_embedding_lookup": [P, c_uint32, c_uint32, P, c_size_t, P, P],
    "tlh_embedding_add_positions": [P, c_uint32, P, P, c_uint32, c_uint32, c_uint32, P, P],
    "tlh_scatter_add_rows": [P, P, c_size_t, c_uint32, P, c_uint32, P],
    # attention
    "tlh_attention_forward": [P, P, P, P, P, c_uint32, c_uint32, c_uint32, c_uint32,
                              c_float, c_int, c_int, P],
    "tlh_attention_decode": [P, P, P, P, c_uint32, c_uint32, c_uint32, c_uint32, c_float, P],
    "tlh_attention_backward": [P, P, P, P, P, P, P, P, P, P, c_uint32, c_uint32, c_uint32,
                               c_uint32, c_float, c_int, c_int, c_int, P],
    # optimiser
    "tlh_clip_gradient": [P, P, c_float, P, c_size_t, P],
    "tlh_adamw": [P, P, P, P, P, P, P, P, P, c_float, c_uint32, c_size_t, P],
    "tlh_clip_multi": [P, P, P, c_uint32, P, c_float, P],
    "tlh_adamw_multi": [P, P, P, P, P, P, c_uint32, P, P, P, P, c_float, P, c_float, P],
}


class NativeError(RuntimeError):
    pass


_HIP: ctypes.CDLL | None = None


def load_hip(path: Path | None = None) -> ctypes.CDLL:
    """Loads libtemplit_hip.so and declares every C-ABI signature."""
    global _HIP
    if _HIP is not None and path is None:
        return _HIP
    lib_path = Path(path) if path else HIP_LIB
    if not lib_path.exists():
        raise NativeError(
            f"{lib_path} is missing: build it with `python -m templit_amd.build`")
    lib = ctypes.CDLL(str(lib_path))
    for name, argtypes in HIP_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = c_int
    lib.tlh_error_string.argtypes = [c_int]
    lib.tlh_error_string.restype = ctypes.c_char_p
    if path is None:
        _HIP = lib
    return lib


def check(code: int, what: str = "") -> None:
    if code != 0:
        msg = load_hip().tlh_error_string(code)
        raise NativeError(f"{what}: hip error {code} ({msg.decode() if msg else '?'})")


def u32_array(values) -> ctypes.Array:
    vals = list(values)
    return (c_uint32 * max(1, len(vals)))(*vals)


def addr(x) -> int:
    """Address of a ctypes array or 0 for None."""
    if x is None:
        return 0
    return ctypes.addressof(x)


# ---------------------------------------------------------------------------
# libtemplit_gpt.so (include/templit_gpt.h)
# ---------------------------------------------------------------------------
class GptConfig(ctypes.Structure):
    """Mirror of struct tlg_config."""

    _fields_ = [("vocab", c_uint32), ("seq", c_uint32), ("dim", c_uint32),
                ("heads", c_uint32), ("layers", c_uint32), ("batch", c_uint32),
                ("ffn", c_uint32)]


FP = POINTER(c_void_p)
GPT_SIGNATURES: dict[str, list] = {
    "tlg_create": [POINTER(GptConfig), P, POINTER(c_void_p)],
    "tlg_destroy": [P],
    "tlg_param_count": [P, POINTER(c_uint32)],
    "tlg_param_info": [P, c_uint32, POINTER(c_uint64), FP, FP, FP, FP],
    "tlg_total_params": [P, POINTER(c_uint64)],
    "tlg_set_params": [P, P],
    "tlg_get_params": [P, P],
    "tlg_get_grads": [P, P],
    "tlg_get_moments": [P, P, P],
    "tlg_get_steps": [P, P],
    "tlg_get_scalars": [P, P],
    "tlg_init_params": [P, c_uint64, c_float],
    "tlg_set_optimizer": [P, c_float, c_float, c_float, c_float, c_float],
    "tlg_set_lr": [P, c_float],
    "tlg_set_concurrency": [P, c_int],
    "tlg_get_concurrency": [P, POINTER(c_int)],
    "tlg_set_forward_copies": [P, c_int],
    "tlg_get_forward_copies": [P, POINTER(c_int)],
    "tlg_io": [P, FP, FP, FP, FP],
    "tlg_train_step": [P, c_float, c_float, c_int],
    "tlg_forward": [P],
    "tlg_generate_greedy": [P, P, c_uint32, c_uint32, c_uint32, c_int, P],
    "tlg_generate_sample": [P, P, c_uint32, c_uint32, c_uint32, c_uint32, c_float, c_uint32,
                            c_uint64, c_int, P, POINTER(c_uint32)],
    "tlg_last_squared_norm": [P, POINTER(c_float)],
    "tlg_profile_step": [P, c_float, c_float, POINTER(c_float), POINTER(ctypes.c_double),
                         POINTER(ctypes.c_double), POINTER(c_uint32), POINTER(c_float),
                         POINTER(c_float)],
    "tlg_time_gemms": [P, c_uint32, POINTER(c_float)],
    "tlg_capture_train_step": [P, c_float, c_float],
    "tlg_replay": [P],
    "tlg_save_archive": [P, ctypes.c_char_p, c_int],
    "tlg_load_archive": [P, ctypes.c_char_p, c_int],
    "tlg_archive_entry": [POINTER(GptConfig), c_uint32, POINTER(c_uint32), POINTER(c_uint32)],
    "tlg_set_batch": [P, P, P],
    "tlg_loader_open": [ctypes.c_char_p, ctypes.c_double, c_int, c_uint32, POINTER(c_void_p)],
    "tlg_loader_batch": [P, c_uint32, c_uint32, P, P],
    "tlg_loader_next": [P, P],
    "tlg_loader_close": [P],
}


class TokenLoader:
    """Batches of a raw uint32 token file, drawn like the reference's
    Loader over its Dataset split (host C++ in libtemplit_runtime.so)."""

    def __init__(self, path, training_fraction=0.95, validation=False, seed=1):
        self.lib = load_gpt()
        h = c_void_p()
        check(self.lib.tlg_loader_open(str(path).encode(), training_fraction, int(validation),
                                       seed, ctypes.byref(h)), "tlg_loader_open")
        self.handle = h.value

    def batch(self, batch, seq):
        import numpy as np

        x = np.empty(batch * seq, np.uint32)
        y = np.empty(batch * seq, np.uint32)
        check(self.lib.tlg_loader_batch(self.handle, batch, seq, x.ctypes.data, y.ctypes.data),
              "tlg_loader_batch")
        return x, y

    def next_into(self, program: "GptProgram"):
        check(self.lib.tlg_loader_next(self.handle, program.handle), "tlg_loader_next")

    def close(self):
        if self.handle:
            self.lib.tlg_loader_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def archive_entry(cfg: "GptConfig", index: int) -> tuple[int, tuple[int, int]]:
    """(canonical parameter index, [rows, cols]) of reference checkpoint entry
    `index` (host only)."""
    c = c_uint32()
    shape = (c_uint32 * 2)()
    check(load_gpt().tlg_archive_entry(ctypes.byref(cfg), index, ctypes.byref(c), shape),
          "tlg_archive_entry")
    return c.value, (shape[0], shape[1])

_GPT: ctypes.CDLL | None = None


def load_gpt() -> ctypes.CDLL:
    """Loads libtemplit_gpt.so (and through it libtemplit_hip.so)."""
    global _GPT
    if _GPT is not None:
        return _GPT
    load_hip()
    if not GPT_LIB.exists():
        raise NativeError(
            f"{GPT_LIB} is missing: build it with `python -m templit_amd.build`")
    lib = ctypes.CDLL(str(GPT_LIB))
    for name, argtypes in GPT_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = c_int
    _GPT = lib
    return lib


class GptProgram:
    """Thin owner of a tlg program handle (all work happens in native code)."""

    def __init__(self, vocab, seq, dim, heads, layers, batch, ffn=None, stream=None):
        import numpy as np  # local: numpy is only needed by this helper

        self._np = np
        self.lib = load_gpt()
        hip = load_hip()
        check(hip.tlh_init(0), "tlh_init")
        self.cfg = GptConfig(vocab, seq, dim, heads, layers, batch, ffn or 4 * dim)
        self.own_stream = stream is None
        if stream is None:
            s = c_void_p()
            check(hip.tlh_stream_create(ctypes.byref(s)), "tlh_stream_create")
            stream = s.value
        self.stream = stream
        h = c_void_p()
        check(self.lib.tlg_create(ctypes.byref(self.cfg), stream, ctypes.byref(h)), "tlg_create")
        self.handle = h.value
        tot = c_uint64()
        check(self.lib.tlg_total_params(self.handle, ctypes.byref(tot)), "tlg_total_params")
        self.total = tot.value
        ptrs = [c_void_p() for _ in range(4)]
        check(self.lib.tlg_io(self.handle, *[ctypes.byref(x) for x in ptrs]), "tlg_io")
        self.tokens_ptr, self.targets_ptr, self.losses_ptr, self.logits_ptr = (
            x.value for x in ptrs)
        self.rows = batch * seq

    def close(self):
        if self.handle:
            self.lib.tlg_destroy(self.handle)
            self.handle = None
        if self.own_stream and self.stream:
            load_hip().tlh_stream_destroy(self.stream)
            self.stream = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- host <-> device ----------------------------------------------------
    def set_params(self, flat):
        flat = self._np.ascontiguousarray(flat, dtype=self._np.float32)
        assert flat.size == self.total
        check(self.lib.tlg_set_params(self.handle, flat.ctypes.data), "tlg_set_params")

    def get_params(self):
        out = self._np.empty(self.total, self._np.float32)
        check(self.lib.tlg_get_params(self.handle, out.ctypes.data), "tlg_get_params")
        return out

    def get_grads(self):
        out = self._np.empty(self.total, self._np.float32)
        check(self.lib.tlg_get_grads(self.handle, out.ctypes.data), "tlg_get_grads")
        return out

    def get_moments(self):
        a = self._np.empty(self.total, self._np.float32)
        b = self._np.empty(self.total, self._np.float32)
        check(self.lib.tlg_get_moments(self.handle, a.ctypes.data, b.ctypes.data),
              "tlg_get_moments")
        return a, b

    def random_batch(self, seed):
        hip = load_hip()
        check(hip.tlh_fill_uniform_u32(self.tokens_ptr, self.rows, seed, self.cfg.vocab,
                                       self.stream), "tokens")
        check(hip.tlh_fill_uniform_u32(self.targets_ptr, self.rows, seed + 1, self.cfg.vocab,
                                       self.stream), "targets")

    def losses(self):
        hip = load_hip()
        out = self._np.empty(self.rows, self._np.float32)
        check(hip.tlh_memcpy_d2h(out.ctypes.data, self.losses_ptr, out.nbytes, self.stream), "d2h")
        check(hip.tlh_stream_synchronize(self.stream), "sync")
        return out

    def logits(self):
        hip = load_hip()
        out = self._np.empty((self.rows, self.cfg.vocab), self._np.float32)
        check(hip.tlh_memcpy_d2h(out.ctypes.data, self.logits_ptr, out.nbytes, self.stream), "d2h")
        check(hip.tlh_stream_synchronize(self.stream), "sync")
        return out

    def steps(self):
        n = c_uint32()
        check(self.lib.tlg_param_count(self.handle, ctypes.byref(n)), "count")
        out = self._np.empty(n.value, self._np.uint32)
        check(self.lib.tlg_get_steps(self.handle, out.ctypes.data), "steps")
        return out

    def scalars(self):
        out = self._np.empty(4, self._np.float32)
        check(self.lib.tlg_get_scalars(self.handle, out.ctypes.data), "scalars")
        return out

    def squared_norm(self):
        v = c_float()
        check(self.lib.tlg_last_squared_norm(self.handle, ctypes.byref(v)), "norm")
        return v.value

    # -- steps ---------------------------------------------------------------
    def init_params(self, seed, std):
        check(self.lib.tlg_init_params(self.handle, seed, std), "tlg_init_params")

    def set_optimizer(self, lr, beta1, beta2, eps, weight_decay):
        check(self.lib.tlg_set_optimizer(self.handle, lr, beta1, beta2, eps, weight_decay),
              "tlg_set_optimizer")

    def set_concurrency(self, mode):
        """-1 automatic (the default), 0 one stream, 1 weight gradients on a
        second stream; returns whether the step now uses two streams."""
        check(self.lib.tlg_set_concurrency(self.handle, int(mode)), "tlg_set_concurrency")
        out = c_int()
        check(self.lib.tlg_get_concurrency(self.handle, ctypes.byref(out)), "tlg_get_concurrency")
        return bool(out.value)

    def set_forward_copies(self, mode):
        """-1 automatic (the default), 0 forward products on the [in, out]
        weights, 1 on K-contiguous copies rebuilt at each forward; returns
        whether the forward now uses the copies."""
        check(self.lib.tlg_set_forward_copies(self.handle, int(mode)), "tlg_set_forward_copies")
        out = c_int()
        check(self.lib.tlg_get_forward_copies(self.handle, ctypes.byref(out)),
              "tlg_get_forward_copies")
        return bool(out.value)

    def train_step(self, root_grad, max_norm, update=True):
        check(self.lib.tlg_train_step(self.handle, root_grad, max_norm, int(update)), "train_step")

    def forward(self):
        check(self.lib.tlg_forward(self.handle), "forward")

    def generate_greedy(self, prompt, n_new, eos_token, prefix_only=False):
        """Greedy tokens after `prompt` (inference::autoregression, top_k 1).
        prefix_only: False / 0 recomputes the padded window per token, True / 1
        the valid prefix, 2 keeps a KV cache (tlg_generate_greedy)."""
        pr = self._np.ascontiguousarray(prompt, dtype=self._np.uint32)
        out = self._np.empty(n_new, self._np.uint32)
        check(self.lib.tlg_generate_greedy(self.handle, pr.ctypes.data, pr.size, n_new, eos_token,
                                           int(prefix_only), out.ctypes.data), "generate")
        return out

    def generate_sample(self, prompt, n_new, eos_token, top_k, temperature, minimum_length,
                        seed, prefix_only=0):
        """Top-k sampled generation (tlg_generate_sample): the tokens up to and
        including an emitted EOS, at most n_new."""
        pr = self._np.ascontiguousarray(prompt, dtype=self._np.uint32)
        out = self._np.empty(n_new, self._np.uint32)
        count = c_uint32()
        check(self.lib.tlg_generate_sample(self.handle, pr.ctypes.data, pr.size, n_new, eos_token,
                                           top_k, temperature, minimum_length, seed,
                                           int(prefix_only), out.ctypes.data,
                                           ctypes.byref(count)), "generate_sample")
        return out[:count.value]

    def capture(self, root_grad, max_norm):
        check(self.lib.tlg_capture_train_step(self.handle, root_grad, max_norm), "capture")

    def profile_step(self, root_grad, max_norm):
        gm, am, sm = c_float(), c_float(), c_float()
        fl, by, n = ctypes.c_double(), ctypes.c_double(), c_uint32()
        check(self.lib.tlg_profile_step(self.handle, root_grad, max_norm, ctypes.byref(gm),
                                        ctypes.byref(fl), ctypes.byref(by), ctypes.byref(n),
                                        ctypes.byref(am), ctypes.byref(sm)), "profile_step")
        return dict(gemm_ms=gm.value, gemm_flops=fl.value, gemm_bytes=by.value,
                    gemm_launches=n.value, attention_ms=am.value, step_ms=sm.value)

    def time_gemms(self, iters=10):
        """ms per step of the last profiled step's GEMMs, each re-launched
        `iters` times back to back (kernel time without the step's gaps)."""
        ms = c_float()
        check(self.lib.tlg_time_gemms(self.handle, iters, ctypes.byref(ms)), "time_gemms")
        return ms.value

    def replay(self):
        check(self.lib.tlg_replay(self.handle), "replay")

    def set_batch(self, tokens, targets):
        np = self._np
        t = np.ascontiguousarray(tokens, dtype=np.uint32).ravel()
        y = np.ascontiguousarray(targets, dtype=np.uint32).ravel()
        if t.size != self.rows or y.size != self.rows:
            raise ValueError("a batch is batch*seq tokens and targets")
        check(self.lib.tlg_set_batch(self.handle, t.ctypes.data, y.ctypes.data), "tlg_set_batch")

    def save_archive(self, path, optimiser=True):
        """Checkpoint in the reference's archive format (Compiled::save and,
        with `optimiser`, save_optimisers)."""
        check(self.lib.tlg_save_archive(self.handle, str(path).encode(), int(optimiser)),
              "tlg_save_archive")

    def load_archive(self, path, optimiser=True):
        check(self.lib.tlg_load_archive(self.handle, str(path).encode(), int(optimiser)),
              "tlg_load_archive")

    def synchronize(self):
        check(load_hip().tlh_stream_synchronize(self.stream), "sync")
