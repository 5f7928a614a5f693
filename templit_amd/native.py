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
    ]


EPI_STORE, EPI_GELU, EPI_GELU_BWD = 0, 1, 2

# name -> argtypes (restype is always int = hipError_t, except tlh_error_string)
HIP_SIGNATURES: dict[str, list] = {
    "tlh_init": [c_int],
    "tlh_device_count": [POINTER(c_int)],
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
    "tlh_compare": [P, P, c_size_t, POINTER(c_int), P, P],
    "tlh_event_create": [POINTER(c_void_p)],
    "tlh_event_record": [P, P],
    "tlh_event_synchronize": [P],
    "tlh_event_elapsed_ms": [P, P, POINTER(c_float)],
    "tlh_event_destroy": [P],
    "tlh_graph_begin_capture": [P],
    "tlh_graph_end_capture": [P, POINTER(c_void_p)],
    "tlh_graph_launch": [P, P],
    "tlh_graph_destroy": [P],
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
    # products
    "tlh_matmul": [P, P, P, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                   c_uint32, c_uint32, c_uint32, c_uint32, U32P, U32P, U32P, U32P, P],
    "tlh_gemm": [POINTER(GemmDesc), P],
    "tlh_gemm_workspace_size": [POINTER(GemmDesc), POINTER(c_size_t)],
    # reductions
    "tlh_sum": [P, c_size_t, P, P],
    "tlh_sum_to_shape": [P, P, c_uint32, U32P, U32P, P],
    "tlh_max_to_shape": [P, P, c_uint32, U32P, U32P, P],
    "tlh_argmax": [P, c_size_t, P, P],
    "tlh_argmax_rows": [P, c_size_t, c_uint32, P, P],
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
    "tlh_embedding_add_positions": [P, P, P, c_uint32, c_uint32, c_uint32, P, P],
    "tlh_scatter_add_rows": [P, P, c_size_t, c_uint32, P, P],
    # attention
    "tlh_attention_forward": [P, P, P, P, P, c_uint32, c_uint32, c_uint32, c_uint32,
                              c_float, c_int, c_int, P],
    "tlh_attention_backward": [P, P, P, P, P, P, P, P, P, P, c_uint32, c_uint32, c_uint32,
                               c_uint32, c_float, c_int, c_int, c_int, P],
    # optimiser
    "tlh_clip_gradient": [P, P, c_float, P, c_size_t, P],
    "tlh_adamw": [P, P, P, P, P, P, P, P, P, c_float, c_uint32, c_size_t, P],
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
