"""ctypes/numpy front end of the C oracle (pa_oracle.c) and of oracle/_ref.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product never imports it.

Arrays are numpy.  K/V caches are [NB, BS, HKV, D] views (any strides, last
dim contiguous) of float32, float16, float64, or uint16 holding bfloat16 bits
(pass kv_dtype="bf16").  Block tables are int32 [B, MB] (row stride may
exceed MB), context lengths int32 [B].
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
SIMD_PATH = HERE / "liboracle_simd.so"
REF_PATH = HERE / "_ref" / "libgb10_ref.so"

DTYPE_CODE = {"f32": 0, "f16": 1, "bf16": 2, "f64": 3}
NP_OF = {"f32": np.float32, "f16": np.float16, "bf16": np.uint16, "f64": np.float64, "fp8": np.uint8}


class _KV(C.Structure):
    _fields_ = [
        ("k", C.c_void_p),
        ("v", C.c_void_p),
        ("dtype", C.c_int32),
        ("pad_", C.c_int32),
        ("num_blocks", C.c_int64),
        ("sb", C.c_int64),
        ("st", C.c_int64),
        ("sh", C.c_int64),
    ]


_lib = None
_ref = None


def lib():
    """The C oracle; raises if it has not been built (make -C oracle)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run __graft_entry__.build())")
        L = C.CDLL(str(LIB_PATH))
        P = C.c_void_p
        i32, i64, f32 = C.c_int32, C.c_int64, C.c_float
        L.oracle_f16_to_f32.restype = f32
        L.oracle_f16_to_f32.argtypes = [C.c_uint16]
        L.oracle_f32_to_f16.restype = C.c_uint16
        L.oracle_f32_to_f16.argtypes = [f32]
        for n in ("oracle_f16_decode", "oracle_f16_encode", "oracle_bf16_decode", "oracle_bf16_encode"):
            getattr(L, n).argtypes = [P, P, i64]
            getattr(L, n).restype = None
        L.oracle_partition_bounds.argtypes = [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]
        L.oracle_partition_bounds.restype = None
        L.oracle_choose_num_splits.argtypes = [i64, i64, i64, i64]
        L.oracle_choose_num_splits.restype = i64
        L.oracle_decode_min_bytes.argtypes = [P, C.c_int, C.c_int, C.c_int, C.c_int]
        L.oracle_decode_min_bytes.restype = C.c_double
        L.oracle_gather.argtypes = [P, P, C.POINTER(_KV), P, C.c_int, C.c_int, C.c_int, C.c_int]
        L.oracle_gather.restype = C.c_int
        dec = [P, P, C.POINTER(_KV), P, i64, P] + [C.c_int] * 6 + [f32]
        for n in ("oracle_decode", "oracle_decode_online"):
            getattr(L, n).argtypes = dec
            getattr(L, n).restype = None
        L.oracle_decode_partials.argtypes = [P, P, P, P, C.POINTER(_KV), P, i64, P] + [C.c_int] * 6 + [f32]
        L.oracle_decode_partials.restype = None
        L.oracle_merge.argtypes = [P, P, P, P, C.c_int, C.c_int, C.c_int, C.c_int]
        L.oracle_merge.restype = None
        L.oracle_prefill.argtypes = [P, P, C.POINTER(_KV), P, i64, P] + [C.c_int] * 7 + [f32]
        L.oracle_prefill.restype = None
        L.oracle_dot.argtypes = [P, P, i64]
        L.oracle_dot.restype = f32
        L.oracle_softmax_inplace.argtypes = [P, i64]
        L.oracle_softmax_inplace.restype = None
        _lib = L
    return _lib


def ref():
    """oracle/_ref (the reference's own scalar code), or None where it was not built."""
    global _ref
    if _ref is None and REF_PATH.exists():
        R = C.CDLL(str(REF_PATH))
        P = C.c_void_p
        R.ref_cpu_reference.argtypes = [P] * 6 + [C.c_int] * 7 + [C.c_float]
        R.ref_cpu_reference.restype = None
        R.ref_selftest_inputs.argtypes = [P] * 5
        R.ref_selftest_inputs.restype = None
        R.ref_dot_scalar.argtypes = [P, P, C.c_int64]
        R.ref_dot_scalar.restype = C.c_float
        R.ref_softmax_inplace.argtypes = [P, C.c_int64]
        R.ref_softmax_inplace.restype = None
        R.ref_attention_scores.argtypes = [P, P, P, C.c_int64, C.c_int64]
        R.ref_attention_scores.restype = None
        R.ref_scalar_smoke_inputs.argtypes = [P, P, C.c_int64, C.c_int64]
        R.ref_scalar_smoke_inputs.restype = None
        R.ref_call_create.argtypes = [P] * 5 + [C.c_int] * 7 + [C.c_float]
        R.ref_call_create.restype = P
        R.ref_call_run.argtypes = [P, P]
        R.ref_call_run.restype = None
        R.ref_call_free.argtypes = [P]
        R.ref_call_free.restype = None
        _ref = R
    return _ref


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


# ------------------------------------------------------------------ codecs --

def f16_encode(x) -> np.ndarray:
    """float32 -> float16 bits (uint16), round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f16_encode(_p(out), _p(x), x.size)
    return out


def f16_decode(bits) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().oracle_f16_decode(_p(out), _p(bits), bits.size)
    return out


def bf16_encode(x) -> np.ndarray:
    """float32 -> bfloat16 bits (uint16), round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_bf16_encode(_p(out), _p(x), x.size)
    return out


def bf16_decode(bits) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().oracle_bf16_decode(_p(out), _p(bits), bits.size)
    return out


def fp8_decode(bits) -> np.ndarray:
    """OCP FP8 E4M3 ("e4m3fn") bits (uint8) -> float32, from the format
    definition: sign, 4-bit exponent (bias 7), 3-bit mantissa; exponent 0 is
    subnormal (m/8 * 2^-6); S.1111.111 is NaN; there are no infinities."""
    b = np.asarray(bits, np.uint8).astype(np.int64)
    e, m = (b >> 3) & 15, b & 7
    mag = np.where(e == 0, m * 2.0 ** -9, (8 + m) * 2.0 ** (e - 10))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return np.where(b >> 7 == 1, -mag, mag).astype(np.float32)


_FP8_POS = None


def fp8_encode(x) -> np.ndarray:
    """float32 -> FP8 E4M3 bits, round to nearest (ties to the even code),
    saturating at +-448 (the largest finite value), as FP8 KV-cache
    quantisers do (torch's cast instead gives NaN past 464); NaN -> 0x7f."""
    global _FP8_POS
    if _FP8_POS is None:
        _FP8_POS = fp8_decode(np.arange(127, dtype=np.uint8)).astype(np.float64)  # codes 0..126, increasing
    x = np.asarray(x, np.float32).astype(np.float64)
    a = np.minimum(np.abs(x), 448.0)
    hi = np.clip(np.searchsorted(_FP8_POS, a, side="left"), 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    dlo, dhi = a - _FP8_POS[lo], _FP8_POS[hi] - a
    code = np.where(dlo < dhi, lo, np.where(dhi < dlo, hi, np.where(lo % 2 == 0, lo, hi)))
    code = np.where(a == _FP8_POS[hi], hi, code)
    out = (code | np.where(np.signbit(x), 128, 0)).astype(np.uint8)
    return np.where(np.isnan(x), np.uint8(0x7F), out)


def to_float(a: np.ndarray, dtype: str) -> np.ndarray:
    """Exact float32 values of an array stored as `dtype`."""
    if dtype == "fp8":
        return fp8_decode(a)
    if dtype == "bf16":
        return bf16_decode(a)
    if dtype == "f16":
        return f16_decode(np.asarray(a, np.float16).view(np.uint16))
    return np.asarray(a, np.float64 if dtype == "f64" else np.float32).astype(np.float32)


def quantize(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 data to storage `dtype` (numpy container per NP_OF)."""
    x = np.asarray(x, np.float32)
    if dtype == "fp8":
        return fp8_encode(x)
    if dtype == "bf16":
        return bf16_encode(x)
    if dtype == "f16":
        return f16_encode(x).view(np.float16)
    return x.astype(NP_OF[dtype])


# ------------------------------------------------------------- arithmetic --

def _kv(k: np.ndarray, v: np.ndarray, dtype: str) -> _KV:
    assert k.shape == v.shape and k.ndim == 4, (k.shape, v.shape)
    assert k.strides == v.strides, "oracle takes K and V with equal strides"
    es = k.itemsize
    assert k.dtype == NP_OF[dtype], (k.dtype, dtype)
    assert k.strides[3] == es, "last dim must be contiguous"
    return _KV(k.ctypes.data, v.ctypes.data, DTYPE_CODE[dtype], 0, k.shape[0],
               k.strides[0] // es, k.strides[1] // es, k.strides[2] // es)


def _tables(bt, ctx):
    bt = np.asarray(bt)
    assert bt.dtype == np.int32 and bt.ndim == 2 and bt.strides[1] == 4
    ctx = np.ascontiguousarray(ctx, dtype=np.int32)
    return bt, bt.strides[0] // 4, ctx


def decode(q, k, v, bt, ctx, scale, kv_dtype="f32", online=False) -> np.ndarray:
    """Paged decode; q [B,H,D] float32 -> out [B,H,D] float32.

    online=False follows cpu_reference (rocm/hip/paged_attn_v1_hip.cpp:104-141),
    online=True the v2 online-softmax loop (kernels/paged_attn_v2.cu:89-121)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, H, D = q.shape
    kv = _kv(k, v, kv_dtype)
    bt, bts, ctx = _tables(bt, ctx)
    HKV, BS, MB = k.shape[2], k.shape[1], bt.shape[1]
    assert k.shape[3] == D and H % HKV == 0
    out = np.empty((B, H, D), np.float32)
    fn = lib().oracle_decode_online if online else lib().oracle_decode
    fn(_p(out), _p(q), C.byref(kv), _p(bt), bts, _p(ctx), B, H, HKV, D, BS, MB, C.c_float(scale))
    return out


_simd = None


def decode_simd(q, k, v, bt, ctx, scale, kv_dtype="f32", threads=None) -> np.ndarray:
    """The SIMD/OpenMP CPU baseline (pa_oracle_simd.c): cpu_reference's algorithm,
    parallel over (b, h), AVX2-vectorised over D.  kv_dtype f32 / f16 / bf16."""
    global _simd
    if _simd is None:
        L = C.CDLL(str(SIMD_PATH))
        P, I, I64 = C.c_void_p, C.c_int, C.c_int64
        L.oracle_decode_simd.argtypes = [P, P, P, P, I, I64, I64, I64, P, I64, P] + [I] * 6 + [C.c_float, I]
        L.oracle_decode_simd.restype = I
        _simd = L
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, H, D = q.shape
    assert k.dtype == NP_OF[kv_dtype] and k.strides == v.strides and k.strides[3] == k.itemsize
    sb, st, sh = (x // k.itemsize for x in k.strides[:3])
    bt, bts, ctx = _tables(bt, ctx)
    out = np.empty((B, H, D), np.float32)
    threads = threads or os.cpu_count()
    rc = _simd.oracle_decode_simd(_p(out), _p(q), _p(k), _p(v), DTYPE_CODE[kv_dtype], sb, st, sh, _p(bt), bts,
                                  _p(ctx), B, H, k.shape[2], D, k.shape[1], bt.shape[1], C.c_float(scale),
                                  int(threads))
    assert rc == 0
    return out


def decode_partials(q, k, v, bt, ctx, scale, num_splits, kv_dtype="f32"):
    """v3 split pass (kernels/paged_attn_v3.cu:33-123): (acc [B,H,S,D], m [B,H,S], l [B,H,S]),
    m in natural-log units."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, H, D = q.shape
    S = int(num_splits)
    kv = _kv(k, v, kv_dtype)
    bt, bts, ctx = _tables(bt, ctx)
    acc = np.empty((B, H, S, D), np.float32)
    m = np.empty((B, H, S), np.float32)
    l = np.empty((B, H, S), np.float32)
    lib().oracle_decode_partials(_p(acc), _p(m), _p(l), _p(q), C.byref(kv), _p(bt), bts, _p(ctx),
                                 B, H, k.shape[2], D, k.shape[1], S, C.c_float(scale))
    return acc, m, l


def merge(acc, m, l) -> np.ndarray:
    """v3 merge pass (kernels/paged_attn_v3.cu:128-166)."""
    acc = np.ascontiguousarray(acc, np.float32)
    m = np.ascontiguousarray(m, np.float32)
    l = np.ascontiguousarray(l, np.float32)
    B, H, S, D = acc.shape
    out = np.empty((B, H, D), np.float32)
    lib().oracle_merge(_p(out), _p(acc), _p(m), _p(l), B, H, S, D)
    return out


def prefill(q, k, v, bt, ctx, scale, kv_dtype="f32") -> np.ndarray:
    """Causal chunked prefill (kernels/paged_attn_prefill.cu:33-118); q [B,S,H,D] float32."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, S, H, D = q.shape
    kv = _kv(k, v, kv_dtype)
    bt, bts, ctx = _tables(bt, ctx)
    out = np.empty((B, S, H, D), np.float32)
    lib().oracle_prefill(_p(out), _p(q), C.byref(kv), _p(bt), bts, _p(ctx), B, S, H, k.shape[2],
                         D, k.shape[1], bt.shape[1], C.c_float(scale))
    return out


def write_kv(k_cache, v_cache, key, value, slots, cache_dtype, src_dtype, k_scale=1.0, v_scale=1.0):
    """KV-cache write, in place on host caches [NB, BS, HKV, D] (storage per NP_OF):
    token t's rows key[t], value[t] ([T, HKV, D], stored as src_dtype) go to
    block slots[t] // BS, row slots[t] % BS, rounded to the cache type (round
    to nearest even; FP8 E4M3 saturating at +-448 as fp8_encode; the same
    16-bit type at scale 1 is copied bit for bit).  With scales the cache
    receives key / k_scale and value / v_scale, divided in float32.  A negative
    slot or one >= NB * BS is skipped.  This restates the serving engine's
    write_kv layout (token j of a sequence -> block_ids[j // BS], row j % BS;
    external to the reference, called at harness/repro_crash.py:52-58)."""
    NB, BS = k_cache.shape[:2]
    unit = np.float32(k_scale) == 1 and np.float32(v_scale) == 1
    for t, s in enumerate(np.asarray(slots).tolist()):
        if s < 0 or s >= NB * BS:
            continue
        b, o = divmod(int(s), BS)
        for cache, src, sc in ((k_cache, key, k_scale), (v_cache, value, v_scale)):
            if src_dtype == cache_dtype and unit:
                cache[b, o] = src[t]
            else:
                x = to_float(src[t], src_dtype)
                with np.errstate(invalid="ignore", over="ignore"):
                    if not unit:
                        x = (x / np.float32(sc)).astype(np.float32)
                    cache[b, o] = quantize(x, cache_dtype)


def gather(k, v, bt_row, n, kvh, kv_dtype="f32"):
    """K and V rows of tokens [0, n) of one sequence and KV head -> ([n,D], [n,D]) float32."""
    kv = _kv(k, v, kv_dtype)
    D, BS = k.shape[3], k.shape[1]
    row = np.ascontiguousarray(bt_row, dtype=np.int32)
    dk = np.empty((n, D), np.float32)
    dv = np.empty((n, D), np.float32)
    rc = lib().oracle_gather(_p(dk), _p(dv), C.byref(kv), _p(row), n, kvh, D, BS)
    if rc != 0:
        raise IndexError("block id outside [0, NB)")
    return dk, dv


def partition_bounds(ctx: int, num_splits: int, s: int):
    a, b = C.c_int(), C.c_int()
    lib().oracle_partition_bounds(ctx, num_splits, s, C.byref(a), C.byref(b))
    return a.value, b.value


def choose_num_splits(num_seqs, num_heads, max_context, sms) -> int:
    return int(lib().oracle_choose_num_splits(num_seqs, num_heads, max_context, sms))


def decode_min_bytes(ctx, HKV, D, kv_itemsize) -> float:
    ctx = np.ascontiguousarray(ctx, dtype=np.int32)
    return float(lib().oracle_decode_min_bytes(_p(ctx), ctx.size, HKV, D, kv_itemsize))


def dot(a, b) -> np.float32:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return np.float32(lib().oracle_dot(_p(a), _p(b), a.size))


def softmax(x) -> np.ndarray:
    x = np.array(x, np.float32, copy=True)
    lib().oracle_softmax_inplace(_p(x), x.size)
    return x


# ------------------------------------------------------------------ inputs --

def paged_inputs(B, H, HKV, D, BS, ctx_lens, *, seed, kv_dtype="f16", q_dtype="f32",
                 extra_blocks=0, mb=None):
    """Seeded N(0,1) paged-decode inputs with a random-permutation block table.

    Returns dict(q, q_f32, k, v, bt, ctx, NB): q stored in q_dtype (q_f32 its
    exact float32 values), k/v stored in kv_dtype, bt a permutation of all
    physical blocks, so every live page sits at a random place in the pool."""
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx_lens, np.int32).reshape(B)
    pages = [max(0, -(-int(c) // BS)) for c in ctx]
    MB = mb if mb is not None else max(1, max(pages))
    NB = sum(pages) + extra_blocks
    NB = max(NB, 1)
    perm = rng.permutation(NB).astype(np.int32)
    bt = np.zeros((B, MB), np.int32)
    pos = 0
    for b in range(B):
        bt[b, :pages[b]] = perm[pos:pos + pages[b]]
        pos += pages[b]
        if pages[b] < MB:
            bt[b, pages[b]:] = perm[rng.integers(0, NB, MB - pages[b])]
    q32 = rng.standard_normal((B, H, D), dtype=np.float32)
    k32 = rng.standard_normal((NB, BS, HKV, D), dtype=np.float32)
    v32 = rng.standard_normal((NB, BS, HKV, D), dtype=np.float32)
    q = quantize(q32, q_dtype)
    return dict(q=q, q_f32=to_float(q, q_dtype), k=quantize(k32, kv_dtype),
                v=quantize(v32, kv_dtype), bt=bt, ctx=ctx, NB=NB)
