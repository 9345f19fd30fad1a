"""Host <-> device plumbing shared by the GPU tests (numpy fixtures -> torch tensors)."""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

import oracle

TORCH_OF = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16,
            "f64": torch.float64}

# North-star tolerance for fp16/bf16 data: |got - want| <= ATOL + RTOL * |want|.
ATOL, RTOL = 2e-3, 1e-2
# fp32 data through fp32 arithmetic.
ATOL32, RTOL32 = 1e-4, 1e-4


def to_dev(a: np.ndarray, tag: str, dev) -> torch.Tensor:
    """numpy array stored as `tag` (bf16 = uint16 bits) -> device tensor of that dtype."""
    t = torch.from_numpy(np.ascontiguousarray(a))
    if tag == "bf16":
        t = t.view(torch.bfloat16)
    return t.to(dev)


def to_host(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def close(got, want, atol=ATOL, rtol=RTOL):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, (got.shape, want.shape)
    bad = ~(np.abs(got - want) <= atol + rtol * np.abs(want))
    bad &= ~(np.isnan(got) & np.isnan(want))
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(
            f"{int(bad.sum())} of {bad.size} outside tol (atol={atol}, rtol={rtol}); first at "
            f"{tuple(i)}: got {got[tuple(i)]} want {want[tuple(i)]}; "
            f"max_abs={np.nanmax(np.abs(got - want)):.3e}")


def oracle_decode_rows(q, k, v, bt, ctx, scale, kv, rows_per_call=8):
    """oracle.decode over the rows of q (axis 0) in parallel threads (the C oracle
    runs without the interpreter lock), for full-size checks."""
    n = q.shape[0]
    chunks = [slice(i, min(n, i + rows_per_call)) for i in range(0, n, rows_per_call)]
    workers = max(1, min(16, os.cpu_count() or 1))
    with ThreadPoolExecutor(workers) as ex:
        parts = list(ex.map(lambda s: oracle.decode(q[s], k, v, bt[s], ctx[s], scale, kv), chunks))
    return np.concatenate(parts, axis=0)


def decode_case(B, H, HKV, D, BS, ctx, *, seed, kv="f16", q="f32", extra_blocks=0, mb=None):
    inp = oracle.paged_inputs(B, H, HKV, D, BS, ctx, seed=seed, kv_dtype=kv, q_dtype=q,
                              extra_blocks=extra_blocks, mb=mb)
    inp["kv"] = kv
    inp["qt"] = q
    return inp


def dev_inputs(inp, dev):
    return (to_dev(inp["q"], inp["qt"], dev), to_dev(inp["k"], inp["kv"], dev),
            to_dev(inp["v"], inp["kv"], dev), torch.from_numpy(inp["bt"]).to(dev),
            torch.from_numpy(inp["ctx"]).to(dev))
