"""ctypes binding of libpagedattn.so (the C-ABI declared in include/pagedattn.h).

Loading fails loudly (ImportError) when the library has not been built: there
is no fallback implementation behind this package.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libpagedattn.so"

PA_MAX_DIMS = 4
PA_OK = 0
PA_ERR_INVALID_ARGUMENT = 1
PA_ERR_UNSUPPORTED = 2
PA_ERR_WORKSPACE = 3
PA_ERR_HIP = 4

DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_F64, DTYPE_I32, DTYPE_I64, DTYPE_FP8 = range(7)

# Every symbol include/pagedattn.h declares.
EXPORTS = (
    "pa_abi_version", "pa_last_error", "pa_last_launch", "paged_attention", "paged_attention_v2",
    "paged_attention_v3", "paged_attention_v3_scaled", "paged_attention_v3_workspace_size",
    "paged_attention_v3_noalloc",
    "pa_v3_partition", "pa_v3_reduce",
    "choose_num_splits", "choose_num_splits_for", "pa_plan_partitions",
    "paged_attention_prefill", "paged_attention_prefill_wmma", "paged_attention_prefill_wmma_scaled",
    "paged_attention_prefill_varlen", "paged_attention_prefill_varlen_scaled",
    "pa_write_kv", "pa_write_kv_scaled",
)


class PaTensor(C.Structure):
    """pa_tensor_t: device pointer, dtype, ndim, shape[4], stride[4] (elements)."""
    _fields_ = [
        ("data", C.c_void_p),
        ("dtype", C.c_int32),
        ("ndim", C.c_int32),
        ("shape", C.c_int64 * PA_MAX_DIMS),
        ("stride", C.c_int64 * PA_MAX_DIMS),
    ]

    @classmethod
    def make(cls, data: int, dtype: int, shape, stride) -> "PaTensor":
        t = cls()
        t.data = data
        t.dtype = dtype
        t.ndim = len(shape)
        for i, (n, s) in enumerate(zip(shape, stride)):
            t.shape[i] = int(n)
            t.stride[i] = int(s)
        return t


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
            "(there is no non-HIP fallback)")
    L = C.CDLL(str(LIB_PATH))
    T = C.POINTER(PaTensor)
    P, i64, sz = C.c_void_p, C.c_int64, C.c_size_t
    L.pa_abi_version.restype = C.c_int
    L.pa_abi_version.argtypes = []
    L.pa_last_error.restype = C.c_char_p
    L.pa_last_error.argtypes = []
    L.pa_last_launch.restype = C.c_char_p
    L.pa_last_launch.argtypes = []
    six = [T, T, T, T, T, T]
    for n in ("paged_attention", "paged_attention_v2", "paged_attention_prefill",
              "paged_attention_prefill_wmma"):
        f = getattr(L, n)
        f.restype = C.c_int
        f.argtypes = six + [C.c_double, P]
    for n in ("paged_attention_v3", "pa_v3_partition"):
        f = getattr(L, n)
        f.restype = C.c_int
        f.argtypes = six + [C.c_double, i64, P, sz, P]
    L.paged_attention_v3_scaled.restype = C.c_int
    L.paged_attention_v3_scaled.argtypes = six + [C.c_double, C.c_double, C.c_double, i64, P, sz, P]
    L.paged_attention_v3_noalloc.restype = C.c_int
    L.paged_attention_v3_noalloc.argtypes = six + [C.c_double, i64, P]
    L.pa_v3_reduce.restype = C.c_int
    L.pa_v3_reduce.argtypes = [T, T, T, T, T, i64, P, sz, P]
    L.paged_attention_v3_workspace_size.restype = sz
    L.paged_attention_v3_workspace_size.argtypes = [T, T, T, i64]
    L.choose_num_splits.restype = i64
    L.choose_num_splits.argtypes = [i64, i64, i64]
    L.choose_num_splits_for.restype = i64
    L.choose_num_splits_for.argtypes = [i64, i64, i64, i64]
    L.pa_plan_partitions.restype = C.c_int
    L.pa_plan_partitions.argtypes = [i64, i64, i64, i64, i64, i64, C.POINTER(i64), C.POINTER(i64)]
    L.paged_attention_prefill_wmma_scaled.restype = C.c_int
    L.paged_attention_prefill_wmma_scaled.argtypes = six + [C.c_double, C.c_double, C.c_double, P]
    L.paged_attention_prefill_varlen.restype = C.c_int
    L.paged_attention_prefill_varlen.argtypes = six + [T, i64, C.c_double, P]
    L.paged_attention_prefill_varlen_scaled.restype = C.c_int
    L.paged_attention_prefill_varlen_scaled.argtypes = six + [T, i64, C.c_double, C.c_double, C.c_double, P]
    L.pa_write_kv.restype = C.c_int
    L.pa_write_kv.argtypes = [T, T, T, T, T, P]
    L.pa_write_kv_scaled.restype = C.c_int
    L.pa_write_kv_scaled.argtypes = [T, T, T, T, T, C.c_double, C.c_double, P]
    _lib = L
    return L


def last_error() -> str:
    return lib().pa_last_error().decode()


def last_launch() -> str:
    """Kernel instances the last launching call on this thread dispatched."""
    return lib().pa_last_launch().decode()


def check(rc: int) -> None:
    """Raise RuntimeError for a failed call (the reference's TORCH_CHECK surfaces the same way)."""
    if rc != PA_OK:
        raise RuntimeError(last_error() or f"pagedattn error {rc}")
