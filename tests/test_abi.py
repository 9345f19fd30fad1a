"""CPU tests of the C-ABI library: it loads, exports every symbol include/pagedattn.h
declares, and rejects bad arguments on the host with the reference's messages
(kernels/paged_attn_v3.cu:199-216, kernels/paged_attn_wmma.cu:218-246) before any
HIP call.  No kernel is launched here: every call below fails validation or has
nothing to do."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "pagedattn.h"
FAKE = 0x7F0000000000  # never dereferenced: validation fails before any device access

F32, F16, BF16, F64, I32, I64 = range(6)


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w]+\s*\**\s+(\w+)\s*\(", text, flags=re.M)))


def test_library_loads_and_exports_header(pa):
    L = pa.lib()
    assert L.pa_abi_version() == 2
    declared = header_functions()
    assert declared == sorted(pa.EXPORTS)
    syms = subprocess.run(["nm", "-D", "--defined-only", str(pa.LIB_PATH)], capture_output=True,
                          text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in syms.splitlines() if " T " in ln}
    missing = [f for f in declared if f not in exported]
    assert not missing, missing


def T(pa, shape, dtype, data=FAKE, stride=None):
    if stride is None:
        stride, s = [], 1
        for n in reversed(shape):
            stride.insert(0, s)
            s *= n
    return pa.PaTensor.make(data, dtype, shape, stride)


def args(pa, B=2, H=4, HKV=2, D=64, NB=10, BS=16, MB=4, qdt=F32, kvdt=F16, odt=F32, prefill=False, S=3):
    qs = [B, S, H, D] if prefill else [B, H, D]
    return dict(out=T(pa, qs, odt), q=T(pa, qs, qdt), k=T(pa, [NB, BS, HKV, D], kvdt),
                v=T(pa, [NB, BS, HKV, D], kvdt), bt=T(pa, [B, MB], I32), ctx=T(pa, [B], I32))


def call(pa, fn, a, scale=0.1, extra=()):
    L = pa.lib()
    f = getattr(L, fn)
    rc = f(C.byref(a["out"]), C.byref(a["q"]), C.byref(a["k"]), C.byref(a["v"]), C.byref(a["bt"]),
           C.byref(a["ctx"]), scale, *extra)
    return rc, L.pa_last_error().decode()


ENTRY_EXTRA = {
    "paged_attention": (None,),
    "paged_attention_v2": (None,),
    "paged_attention_v3": (4, None, 0, None),
    "paged_attention_prefill": (None,),
    "paged_attention_prefill_wmma": (None,),
}


@pytest.mark.parametrize("fn", ["paged_attention", "paged_attention_v2", "paged_attention_v3"])
@pytest.mark.parametrize("case,code,msg", [
    (dict(H=6, HKV=4), 1, "n_head must be divisible by n_kv_head"),
    (dict(D=96), 2, "unsupported head_dim 96"),
    (dict(D=48), 2, "unsupported head_dim 48"),
    (dict(kvdt=I32), 1, "k_cache must be float32, float16, bfloat16, float64 or float8_e4m3fn"),
    (dict(qdt=F64), 1, "q must be float32, float16 or bfloat16"),
    (dict(odt=I64), 1, "out must be float32, float16 or bfloat16"),
    (dict(kvdt=F64, D=256), 2, "float64 KV caches support head_dim <= 128"),
])
def test_rejections(pa, fn, case, code, msg):
    a = args(pa, **case)
    rc, err = call(pa, fn, a, extra=ENTRY_EXTRA[fn])
    assert rc == code and msg in err, (rc, err)


def test_shape_rejections(pa):
    a = args(pa)
    a["q"] = T(pa, [2, 4, 64, 1], F32)
    assert call(pa, "paged_attention", a, extra=(None,)) == (1, "q must be [B, H, D]")
    a = args(pa)
    a["k"] = T(pa, [10, 16, 2 * 64], F16)
    assert call(pa, "paged_attention_v2", a, extra=(None,)) == (1, "k_cache must be [NB, BS, H, D]")
    a = args(pa)
    a["bt"] = T(pa, [2, 4], I64)
    assert call(pa, "paged_attention_v2", a, extra=(None,)) == (1, "block_tables must be int32")
    a = args(pa)
    a["ctx"] = T(pa, [3], I32)
    assert call(pa, "paged_attention_v2", a, extra=(None,)) == (1, "context_lens must have B entries")
    a = args(pa)
    a["v"] = T(pa, [10, 16, 2, 64], BF16)
    assert call(pa, "paged_attention_v2", a, extra=(None,))[0] == 1
    a = args(pa)
    a["out"] = T(pa, [2, 4, 32], F32)
    assert call(pa, "paged_attention_v2", a, extra=(None,)) == (1, "out must have the shape of q")
    a = args(pa)
    a["q"] = T(pa, [2, 4, 64], F32, stride=[1, 128, 2])
    assert call(pa, "paged_attention_v2", a, extra=(None,)) == (1, "q must be contiguous")
    a = args(pa)
    a["k"] = T(pa, [10, 16, 2, 64], F16, data=FAKE + 2)
    assert call(pa, "paged_attention_v2", a, extra=(None,)) == (2, "k_cache/v_cache must be 16-byte aligned")
    a = args(pa)
    a["k"] = T(pa, [10, 16, 2, 64], F16, stride=[2048, 128, 65, 1])
    assert call(pa, "paged_attention_v2", a, extra=(None,))[0] == 2
    a = args(pa)
    a["k"] = T(pa, [10, 16, 2, 64], F16, data=0)
    assert call(pa, "paged_attention_v2", a, extra=(None,)) == (1, "k_cache has a NULL data pointer")
    rc, err = call(pa, "paged_attention_v2", args(pa), scale=float("inf"), extra=(None,))
    assert rc == 1 and "scale" in err
    L = pa.lib()
    rc = L.paged_attention(None, None, None, None, None, None, 0.1, None)
    assert rc == 1 and pa.last_error() == "q is NULL"


def test_prefill_rejections(pa):
    a = args(pa, prefill=True, kvdt=F32)
    rc, err = call(pa, "paged_attention_prefill_wmma", a, extra=(None,))
    assert rc == 1 and "fp16, bf16 or float8_e4m3fn KV cache" in err
    a = args(pa, prefill=False)
    rc, err = call(pa, "paged_attention_prefill", a, extra=(None,))
    assert rc == 1 and err == "q must be [B, S, H, D]"
    a = args(pa, prefill=True, H=5, HKV=2)
    rc, err = call(pa, "paged_attention_prefill_wmma", a, extra=(None,))
    assert rc == 1 and err == "n_head must be divisible by n_kv_head"


def test_workspace_checks(pa):
    L = pa.lib()
    a = args(pa, B=3, H=4, D=64)
    need = L.paged_attention_v3_workspace_size(C.byref(a["q"]), C.byref(a["k"]), C.byref(a["bt"]), 5)
    rows = 3 * 4 * 5
    up = lambda x: (x + 255) // 256 * 256
    assert need == up(rows * 64 * 4) + 2 * up(rows * 4)
    assert L.paged_attention_v3_workspace_size(C.byref(a["q"]), C.byref(a["k"]), C.byref(a["bt"]), 1) == 0
    rc, err = call(pa, "paged_attention_v3", a, extra=(5, None, 0, None))
    assert rc == 3 and f"need {need} bytes" in err
    rc, err = call(pa, "paged_attention_v3", a, extra=(5, FAKE, need - 1, None))
    assert rc == 3
    rc, err = call(pa, "paged_attention_v3", a, extra=(5, FAKE + 8, need, None))
    assert rc == 3 and "256-byte aligned" in err


def test_empty_batch_is_a_no_op(pa):
    for fn in ("paged_attention", "paged_attention_v2"):
        a = args(pa, B=0)
        assert call(pa, fn, a, extra=(None,)) == (0, call(pa, fn, a, extra=(None,))[1])
    a = args(pa, B=0, prefill=True)
    for fn in ("paged_attention_prefill", "paged_attention_prefill_wmma"):
        assert call(pa, fn, a, extra=(None,))[0] == 0


def test_choose_num_splits_for_matches_reference_formula(pa):
    rng = np.random.default_rng(0)
    for _ in range(2000):
        B, H = int(rng.integers(0, 300)), int(rng.integers(1, 64))
        ctx, cus = int(rng.integers(0, 200000)), int(rng.integers(1, 400))
        assert pa.choose_num_splits_for(B, H, ctx, cus) == oracle.choose_num_splits(B, H, ctx, cus)
    # GB10 values printed by the reference (48 SMs, H=12)
    for B, ctx, S in [(2, 64, 16), (1, 512, 32), (1, 2048, 64), (4, 512, 16), (4, 2048, 64),
                      (16, 512, 16), (16, 2048, 64), (64, 512, 16), (128, 512, 16)]:
        assert pa.choose_num_splits_for(B, 12, ctx, 48) == S


def test_plan_partitions(pa):
    # BASELINE config 2 on 256 CUs: 768 (sequence, KV head) units already fill the GPU.
    assert pa.plan_partitions(64, 12, 12, 64, 2048, 256) == (2048, 1)
    # config 3: 32 x 8 units, contexts up to 32768 -> split, partitions bounded.
    ptok, n = pa.plan_partitions(32, 32, 8, 128, 32768, 256)
    assert n > 1 and ptok * n >= 32768 and ptok % 128 == 0 and ptok <= 2048
    # ... at the longest partition, 2048 tokens (groups of 4 and of 8 alike).
    assert (ptok, n) == (2048, 16)
    assert pa.plan_partitions(32, 64, 8, 128, 8192, 256) == (2048, 4)
    # tiny problem: no split
    assert pa.plan_partitions(1, 1, 1, 64, 100, 256) == (100, 1)
    # tiny grids (a few short sequences, far from filling 256 CUs): 64- or 128-token partitions
    # instead of 256, so that more work-groups stream at once (B=4 ctx=2048: 16 x 128)
    assert pa.plan_partitions(4, 12, 12, 64, 2048, 256) == (128, 16)
    assert pa.plan_partitions(1, 12, 12, 64, 1024, 256) == (64, 16)
    assert pa.plan_partitions(8, 12, 12, 64, 1536, 256)[1] > 1
    assert pa.plan_partitions(16, 12, 12, 64, 2048, 256) == (512, 4)
    # ... but a split must pay for its reduce launch: short contexts, or grids whose
    # unsplit streams are short for their width, run direct (one launch)
    assert pa.plan_partitions(1, 12, 12, 64, 512, 256) == (512, 1)
    assert pa.plan_partitions(32, 12, 12, 64, 768, 256) == (768, 1)
    assert pa.plan_partitions(16, 12, 12, 64, 1536, 256) == (1536, 1)
    assert pa.plan_partitions(32, 12, 12, 64, 1024, 256) == (1024, 1)
    assert pa.plan_partitions(32, 12, 12, 64, 2048, 256) == (2048, 1)
    # (head_dim counts: 128-element rows are twice the bytes per token)
    assert pa.plan_partitions(1, 12, 12, 128, 512, 256)[1] > 1
    for B in (1, 2, 7, 64, 300):
        for ctx in (1, 31, 256, 4096, 100000):
            ptok, n = pa.plan_partitions(B, 32, 8, 128, ctx, 256)
            assert n >= 1 and ptok * n >= ctx and (n == 1 or ptok % 128 == 0 or ptok == 64)
            assert n == 1 or (n - 1) * ptok < ctx
    rc = pa.lib().pa_plan_partitions(1, 6, 4, 64, 10, 256, C.byref(C.c_int64()), C.byref(C.c_int64()))
    assert rc == 1


def test_import_without_library_fails_loudly(tmp_path):
    """The package has no fallback: without libpagedattn.so, lib() raises."""
    import importlib.util
    import shutil
    import sys
    pkg = ROOT / "gb10-attn_amd"
    dst = tmp_path / "pkgcopy"
    dst.mkdir()
    for f in ("__init__.py", "_lib.py", "ops.py"):
        shutil.copy(pkg / f, dst / f)
    spec = importlib.util.spec_from_file_location("pkgcopy", dst / "__init__.py",
                                                  submodule_search_locations=[str(dst)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["pkgcopy"] = mod
    try:
        spec.loader.exec_module(mod)
        with pytest.raises(ImportError):
            mod.lib()
    finally:
        sys.modules.pop("pkgcopy", None)
        for k in [k for k in sys.modules if k.startswith("pkgcopy.")]:
            sys.modules.pop(k)


def write_args(pa, T_=5, HKV=2, D=64, NB=10, BS=16, cdt=F16, sdt=F32, slot=I64):
    return dict(kc=T(pa, [NB, BS, HKV, D], cdt), vc=T(pa, [NB, BS, HKV, D], cdt), key=T(pa, [T_, HKV, D], sdt),
                val=T(pa, [T_, HKV, D], sdt), slots=T(pa, [T_], slot))


def write_call(pa, a):
    L = pa.lib()
    rc = L.pa_write_kv(C.byref(a["kc"]), C.byref(a["vc"]), C.byref(a["key"]), C.byref(a["val"]),
                       C.byref(a["slots"]), None)
    return rc, L.pa_last_error().decode()


@pytest.mark.parametrize("case,code,msg", [
    (dict(cdt=F64), 1, "k_cache must be float16, bfloat16, float32 or float8_e4m3fn"),
    (dict(sdt=I32), 1, "key must be float16, bfloat16 or float32"),
    (dict(slot=F32), 1, "slot_mapping must be int32 or int64"),
    (dict(D=60), 2, "head_dim must be a positive multiple of 8"),
])
def test_write_kv_rejections(pa, case, code, msg):
    rc, err = write_call(pa, write_args(pa, **case))
    assert rc == code and msg in err, (rc, err)


def test_write_kv_shape_rejections(pa):
    a = write_args(pa)
    a["key"] = T(pa, [5, 3, 64], F32)
    a["val"] = T(pa, [5, 3, 64], F32)
    rc, err = write_call(pa, a)
    assert rc == 1 and "key must be [T, 2, 64]" in err
    a = write_args(pa)
    a["slots"] = T(pa, [4], I64)
    rc, err = write_call(pa, a)
    assert rc == 1 and "slot_mapping must have T entries" in err
    a = write_args(pa)
    a["val"] = T(pa, [5, 2, 64], F16)
    rc, err = write_call(pa, a)
    assert rc == 1 and "value must have the dtype of key" in err
    a = write_args(pa)
    a["key"] = T(pa, [5, 2, 64], F32, data=FAKE + 4)
    rc, err = write_call(pa, a)
    assert rc == 2 and "key/value must be 16-byte aligned" in err
    a = write_args(pa)
    a["key"] = T(pa, [5, 2, 64], F16, stride=[130, 65, 1])
    a["val"] = T(pa, [5, 2, 64], F16)
    a["key"].dtype = F16
    rc, err = write_call(pa, write_args(pa, sdt=F16) | {"key": a["key"]})
    assert rc == 2 and "multiples of 16 bytes" in err


@pytest.mark.parametrize("ks,vs", [(0.0, 1.0), (1.0, float("inf")), (float("nan"), 1.0), (1e-50, 1.0),
                                   (1e39, 1.0), (1.0, -1e39)])
def test_write_kv_scaled_rejects_bad_scales(pa, ks, vs):
    """Scales must be finite and nonzero as float32 (1e-50 rounds to 0, 1e39 to inf); refused
    before any HIP call."""
    a = write_args(pa, cdt=6)
    L = pa.lib()
    rc = L.pa_write_kv_scaled(C.byref(a["kc"]), C.byref(a["vc"]), C.byref(a["key"]), C.byref(a["val"]),
                              C.byref(a["slots"]), ks, vs, None)
    err = L.pa_last_error().decode()
    assert rc == 1 and "k_scale and v_scale must be finite and nonzero" in err, (rc, err)


def test_write_kv_zero_tokens_is_a_no_op(pa):
    rc, err = write_call(pa, write_args(pa, T_=0))
    assert rc == 0, err


def test_torch_ops_load_with_reference_signatures(pa):
    """torch.ops.gb10_attn carries the reference's kernels/*.h signatures (loads without a GPU)."""
    ops = pa.torch_ops()
    want = {
        "paged_attention": "(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, Tensor context_lens, float scale) -> Tensor",
        "paged_attention_v3": "(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, Tensor context_lens, float scale, int num_splits) -> Tensor",
        "choose_num_splits": "(int num_seqs, int num_heads, int max_context) -> int",
        "paged_attention_prefill_wmma": "(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, Tensor context_lens, float scale) -> Tensor",
    }
    for name, sig in want.items():
        schema = str(getattr(ops, name).default._schema)
        assert schema == f"gb10_attn::{name}{sig}", schema
    import torch
    with pytest.raises(RuntimeError, match="q must be on CUDA"):
        ops.paged_attention(torch.zeros(1, 4, 64), torch.zeros(1, 16, 4, 64), torch.zeros(1, 16, 4, 64),
                            torch.zeros(1, 1, dtype=torch.int32), torch.ones(1, dtype=torch.int32), 0.1)


@pytest.mark.parametrize("fn,extra", [
    ("paged_attention_v3_scaled", lambda ks, vs: (ks, vs, 4, None, 0, None)),
    ("paged_attention_prefill_wmma_scaled", lambda ks, vs: (ks, vs, None)),
])
@pytest.mark.parametrize("scale,ks,vs,msg", [
    (0.1, 1e39, 1.0, "k_scale and v_scale must be finite"),
    (0.1, 1.0, -1e39, "k_scale and v_scale must be finite"),
    (0.1, float("nan"), 1.0, "k_scale and v_scale must be finite"),
    (1e30, 1e10, 1.0, "must be finite"),   # each finite, the folded softmax scale is not (as float32)
])
def test_scaled_entries_reject_scales_past_float32(pa, fn, extra, scale, ks, vs, msg):
    """The kernels take the scales as float32: a finite double that overflows it is refused."""
    a = args(pa, prefill="prefill" in fn, qdt=F16, odt=F16)
    if "prefill" in fn:
        a["q"] = T(pa, [2, 3, 4, 64], F16)
    rc, err = call(pa, fn, a, scale=scale, extra=extra(ks, vs))
    assert rc == 1 and msg in err, (rc, err)


@pytest.mark.parametrize("fn", ["paged_attention", "paged_attention_v3", "paged_attention_prefill_wmma"])
def test_scale_past_float32_rejected(pa, fn):
    """scale * log2(e) must be finite as float32 (the kernels' softmax scale)."""
    a = args(pa, prefill="prefill" in fn, qdt=F16, odt=F16, kvdt=F16)
    rc, err = call(pa, fn, a, scale=3e38, extra=ENTRY_EXTRA[fn])
    assert rc == 1 and "scale must be finite" in err, (rc, err)
