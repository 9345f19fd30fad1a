"""torch-facing mirror of the reference launchers (kernels/*.h), served by libpagedattn.so.

Each function keeps the reference's name, argument order and meaning
(q, k_cache, v_cache, block_tables, context_lens, scale[, num_splits]) and
its error behaviour (a failed check raises RuntimeError, as TORCH_CHECK
does).  As in the reference, the output is a new fp32 tensor by default;
`out_dtype=` selects fp16/bf16 output.  Work is enqueued on torch's current
stream of q's device; nothing synchronises.

Differences from the reference, all in the direction of accepting more:
K/V may be fp16, bf16, fp32, fp64 or float8_e4m3fn (with k_scale/v_scale on
v3) for every decode entry point and bf16 for
the matrix-core prefill; q may be fp32, fp16 or bf16; K/V may be strided
views (e.g. one layer of a larger pool) without a copy.  Rows of a sequence
with context_lens <= 0 are zeros; context_lens beyond the block table or
out-of-range block ids give NaN rows (the reference reads out of bounds).

PyTorch only supplies device memory and streams here; all arithmetic runs in
the HIP kernels behind include/pagedattn.h.
"""
from __future__ import annotations

import ctypes as C

import torch

from ._lib import (DTYPE_BF16, DTYPE_F16, DTYPE_F32, DTYPE_F64, DTYPE_FP8, DTYPE_I32, DTYPE_I64,
                   PaTensor, check, last_error, lib)

_DT = {
    torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16,
    torch.float64: DTYPE_F64, torch.int32: DTYPE_I32, torch.int64: DTYPE_I64,
    torch.float8_e4m3fn: DTYPE_FP8,
}


def view(t: torch.Tensor) -> PaTensor:
    """pa_tensor_t describing a torch tensor (no copy)."""
    if t.dtype not in _DT:
        raise RuntimeError(f"unsupported dtype {t.dtype}")
    return PaTensor.make(t.data_ptr(), _DT[t.dtype], t.shape, t.stride())


def _kv_ok(t: torch.Tensor) -> bool:
    es = t.element_size()
    if t.dim() != 4 or t.stride(3) != 1 or t.data_ptr() % 16:
        return False
    return all((t.stride(i) * es) % 16 == 0 or t.shape[i] == 1 for i in range(3))


def _prep(q, k_cache, v_cache, block_tables, context_lens, qdim, what):
    if not q.is_cuda:
        raise RuntimeError("q must be on CUDA")
    if not (k_cache.is_cuda and v_cache.is_cuda):
        raise RuntimeError("kv cache must be on CUDA")
    if q.dim() != qdim:
        raise RuntimeError(f"q must be {what}")
    if k_cache.dim() != 4:
        raise RuntimeError("k_cache must be [NB, BS, H, D]")
    q = q.contiguous()
    # Strided K/V views are read in place; anything the kernels cannot
    # address directly is made contiguous, as the reference does for all inputs.
    if not _kv_ok(k_cache):
        k_cache = k_cache.contiguous()
    if not _kv_ok(v_cache):
        v_cache = v_cache.contiguous()
    block_tables = block_tables.to(torch.int32).contiguous()
    context_lens = context_lens.to(torch.int32).contiguous()
    return q, k_cache, v_cache, block_tables, context_lens


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _out(q, out_dtype, out):
    if out is not None:
        return out
    return torch.empty(q.shape, dtype=out_dtype, device=q.device)


def _call_simple(fn, q, k_cache, v_cache, block_tables, context_lens, scale, out_dtype, out,
                 qdim, what):
    q, k_cache, v_cache, block_tables, context_lens = _prep(
        q, k_cache, v_cache, block_tables, context_lens, qdim, what)
    o = _out(q, out_dtype, out)
    with torch.cuda.device(q.device):
        check(fn(C.byref(view(o)), C.byref(view(q)), C.byref(view(k_cache)), C.byref(view(v_cache)),
                 C.byref(view(block_tables)), C.byref(view(context_lens)), float(scale),
                 _stream(q.device)))
    return o


def paged_attention(q, k_cache, v_cache, block_tables, context_lens, scale, *,
                    out_dtype=torch.float32, out=None):
    """kernels/paged_attn_v1.h:13-15 -- decode, q [B,H,D] -> out [B,H,D]."""
    return _call_simple(lib().paged_attention, q, k_cache, v_cache, block_tables, context_lens,
                        scale, out_dtype, out, 3, "[B, H, D]")


def paged_attention_v2(q, k_cache, v_cache, block_tables, context_lens, scale, *,
                       out_dtype=torch.float32, out=None):
    """kernels/paged_attn_v2.h:13-15 -- online-softmax decode."""
    return _call_simple(lib().paged_attention_v2, q, k_cache, v_cache, block_tables, context_lens,
                        scale, out_dtype, out, 3, "[B, H, D]")


def paged_attention_prefill(q, k_cache, v_cache, block_tables, context_lens, scale, *,
                            out_dtype=torch.float32, out=None):
    """kernels/paged_attn_prefill.h:13-15 -- causal chunked prefill, fp32 arithmetic."""
    return _call_simple(lib().paged_attention_prefill, q, k_cache, v_cache, block_tables,
                        context_lens, scale, out_dtype, out, 4, "[B, S, H, D]")


def paged_attention_prefill_wmma(q, k_cache, v_cache, block_tables, context_lens, scale, *,
                                 out_dtype=torch.float32, out=None, k_scale=1.0, v_scale=1.0):
    """kernels/paged_attn_wmma.h:13-15 -- causal chunked prefill on MFMA (fp16/bf16/FP8 KV).
    k_scale / v_scale dequantise a scaled cache (paged_attention_prefill_wmma_scaled)."""
    if k_scale == 1.0 and v_scale == 1.0:
        return _call_simple(lib().paged_attention_prefill_wmma, q, k_cache, v_cache, block_tables,
                            context_lens, scale, out_dtype, out, 4, "[B, S, H, D]")
    q, k_cache, v_cache, block_tables, context_lens = _prep(
        q, k_cache, v_cache, block_tables, context_lens, 4, "[B, S, H, D]")
    o = _out(q, out_dtype, out)
    with torch.cuda.device(q.device):
        check(lib().paged_attention_prefill_wmma_scaled(
            C.byref(view(o)), C.byref(view(q)), C.byref(view(k_cache)), C.byref(view(v_cache)),
            C.byref(view(block_tables)), C.byref(view(context_lens)), float(scale), float(k_scale),
            float(v_scale), _stream(q.device)))
    return o


def paged_attention_prefill_varlen(q, k_cache, v_cache, block_tables, context_lens, cu_seqlens_q,
                                   max_q_len, scale, *, out_dtype=torch.float32, out=None, k_scale=1.0,
                                   v_scale=1.0):
    """Mixed decode + prefill batch on the MFMA path: q/out packed [T, H, D],
    sequence b's q_len_b = cu_seqlens_q[b+1] - cu_seqlens_q[b] new tokens at
    rows cu_seqlens_q[b] .., positions context_lens[b] - q_len_b + r (causal).
    k_scale / v_scale dequantise a scaled cache (paged_attention_prefill_varlen_scaled)."""
    q, k_cache, v_cache, block_tables, context_lens = _prep(
        q, k_cache, v_cache, block_tables, context_lens, 3, "[T, H, D]")
    cu = cu_seqlens_q.to(q.device, torch.int32).contiguous()
    o = _out(q, out_dtype, out)
    with torch.cuda.device(q.device):
        check(lib().paged_attention_prefill_varlen_scaled(
            C.byref(view(o)), C.byref(view(q)), C.byref(view(k_cache)), C.byref(view(v_cache)),
            C.byref(view(block_tables)), C.byref(view(context_lens)), C.byref(view(cu)), int(max_q_len),
            float(scale), float(k_scale), float(v_scale), _stream(q.device)))
    return o


def workspace_size(q, k_cache, block_tables, num_splits) -> int:
    """Bytes of scratch paged_attention_v3 needs (0 when no split is planned)."""
    with torch.cuda.device(q.device):
        n = lib().paged_attention_v3_workspace_size(C.byref(view(q)), C.byref(view(k_cache)),
                                                   C.byref(view(block_tables)), int(num_splits))
    if n == C.c_size_t(-1).value:
        raise RuntimeError(last_error())
    return int(n)


def paged_attention_v3(q, k_cache, v_cache, block_tables, context_lens, scale, num_splits, *,
                       out_dtype=torch.float32, out=None, workspace=None, k_scale=1.0, v_scale=1.0):
    """kernels/paged_attn_v3.h:13-16 -- context-split decode + separate LSE reduce.

    num_splits > 0 cuts each sequence exactly as the reference does;
    num_splits <= 0 lets the library plan the split from the CU count.
    k_scale / v_scale dequantise a scaled cache (e.g. torch.float8_e4m3fn):
    attention runs on k_cache * k_scale and v_cache * v_scale."""
    q, k_cache, v_cache, block_tables, context_lens = _prep(
        q, k_cache, v_cache, block_tables, context_lens, 3, "[B, H, D]")
    o = _out(q, out_dtype, out)
    need = workspace_size(q, k_cache, block_tables, num_splits)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        if k_scale == 1.0 and v_scale == 1.0:
            check(lib().paged_attention_v3(
                C.byref(view(o)), C.byref(view(q)), C.byref(view(k_cache)), C.byref(view(v_cache)),
                C.byref(view(block_tables)), C.byref(view(context_lens)), float(scale),
                int(num_splits), workspace.data_ptr(), workspace.numel(), _stream(q.device)))
        else:
            check(lib().paged_attention_v3_scaled(
                C.byref(view(o)), C.byref(view(q)), C.byref(view(k_cache)), C.byref(view(v_cache)),
                C.byref(view(block_tables)), C.byref(view(context_lens)), float(scale), float(k_scale),
                float(v_scale), int(num_splits), workspace.data_ptr(), workspace.numel(), _stream(q.device)))
    return o


def choose_num_splits(num_seqs: int, num_heads: int, max_context: int) -> int:
    """kernels/paged_attn_v3.h:17 -- the reference split heuristic on this device's CU count."""
    n = lib().choose_num_splits(int(num_seqs), int(num_heads), int(max_context))
    if n < 0:
        raise RuntimeError(last_error())
    return int(n)


def choose_num_splits_for(num_seqs, num_heads, max_context, num_compute_units) -> int:
    return int(lib().choose_num_splits_for(int(num_seqs), int(num_heads), int(max_context),
                                           int(num_compute_units)))


def plan_partitions(num_seqs, num_heads, num_kv_heads, head_dim, max_context, num_compute_units):
    """(partition_tokens, num_partitions) the library uses when num_splits <= 0."""
    a, b = C.c_int64(), C.c_int64()
    check(lib().pa_plan_partitions(int(num_seqs), int(num_heads), int(num_kv_heads), int(head_dim),
                                   int(max_context), int(num_compute_units), C.byref(a), C.byref(b)))
    return int(a.value), int(b.value)


def write_kv(k_cache, v_cache, key, value, slot_mapping, k_scale=1.0, v_scale=1.0):
    """KV-cache write: key/value [T, HKV, D] (fp32/fp16/bf16, any token/head
    strides) into k_cache/v_cache [NB, BS, HKV, D] at slot_mapping[t]
    (block slot // BS, row slot % BS; negative slots skipped), converted to the
    cache dtype with round-to-nearest-even.  With scales the cache receives
    key / k_scale and value / v_scale (pa_write_kv_scaled); an FP8 E4M3 cache
    saturates at +-448.  In place; returns nothing."""
    for t, n in ((k_cache, "k_cache"), (v_cache, "v_cache"), (key, "key"), (value, "value")):
        if not t.is_cuda:
            raise RuntimeError(f"{n} must be on CUDA")
    if key.dim() != 3 or value.dim() != 3:
        raise RuntimeError("key/value must be [T, HKV, D]")
    if not _kv_ok(k_cache) or not _kv_ok(v_cache):
        raise RuntimeError("k_cache/v_cache must be 16-byte aligned [NB, BS, HKV, D] views with a contiguous last dim")
    if key.stride(2) != 1 or key.data_ptr() % 16:
        key = key.contiguous()
    if value.stride(2) != 1 or value.data_ptr() % 16:
        value = value.contiguous()
    if slot_mapping.dtype not in (torch.int32, torch.int64):
        slot_mapping = slot_mapping.to(torch.int64)
    slot_mapping = slot_mapping.to(key.device).contiguous()
    with torch.cuda.device(key.device):
        check(lib().pa_write_kv_scaled(C.byref(view(k_cache)), C.byref(view(v_cache)), C.byref(view(key)),
                                       C.byref(view(value)), C.byref(view(slot_mapping)), float(k_scale),
                                       float(v_scale), _stream(key.device)))


def write_kv_blocks(kv_pool, block_ids, start, k, v, k_scale=1.0, v_scale=1.0):
    """The serving engine's write_kv(block_ids, start, k, v): one sequence's
    K/V for all layers, k/v [n_layer, n_head, ctx, head_dim] (host numpy or
    torch), into kv_pool [n_layer, 2, NB, BS, HKV, D] at token positions
    start .. start + ctx - 1 of the sequence whose pages are block_ids.  Each
    layer is one pa_write_kv_scaled call on the [ctx, HKV, D] view of k[layer]."""
    L, _, NB, BS, HKV, D = kv_pool.shape
    k = torch.as_tensor(k).to(kv_pool.device)
    v = torch.as_tensor(v).to(kv_pool.device)
    ctx = k.shape[2]
    pos = torch.arange(start, start + ctx, device=kv_pool.device)
    blocks = torch.as_tensor(block_ids, dtype=torch.int64, device=kv_pool.device)
    if (start + ctx + BS - 1) // BS > blocks.numel():
        raise RuntimeError("block_ids do not cover the written positions")
    slots = blocks[pos // BS] * BS + pos % BS
    for layer in range(L):
        write_kv(kv_pool[layer, 0], kv_pool[layer, 1], k[layer].permute(1, 0, 2), v[layer].permute(1, 0, 2), slots,
                 k_scale, v_scale)


def torch_ops():
    """The same launchers as PyTorch operators, torch.ops.gb10_attn.* (built from
    csrc/torch_ext.cpp into libpagedattn_torch.so): the reference's exact
    torch::Tensor signatures for callers that bind them from C++ or TorchScript,
    with no Python/ctypes work per call.  Raises ImportError when not built."""
    from ._lib import LIB_PATH
    path = LIB_PATH.with_name("libpagedattn_torch.so")
    if not path.exists():
        raise ImportError(f"{path} is missing: build it with __graft_entry__.build()")
    if not hasattr(torch.ops, "gb10_attn") or not hasattr(torch.ops.gb10_attn, "paged_attention_v3"):
        torch.ops.load_library(str(path))
    return torch.ops.gb10_attn

