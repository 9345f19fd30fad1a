"""Writes the golden fixtures of tests/golden/ from the reference's own code.

Run in the build container, where /root/reference exists and oracle/_ref
(the reference's cpu_reference and arm scalar primitives, compiled from the
reference sources by oracle/Makefile) is built:

    python tests/golden/make_golden.py

Fixtures (data only: inputs and expected outputs):
  hip_selftest.npz   -- the HIP self-test of rocm/hip/paged_attn_v1_hip.cpp:151-198:
                        inputs from its std::mt19937(7) stream, output of its cpu_reference.
  config1.npz        -- BASELINE config 1 (GPT-2 decode, fp16): numpy seed + input
                        hashes + output of the reference cpu_reference on those inputs.
  gqa_bf16.npz       -- GQA (H=32, HKV=8, D=128) bf16 ragged decode, same recipe.
  scalar_smoke.npz   -- arm_cpu scalar_smoke inputs (mt19937(2026), tokens=64, dim=128)
                        with the reference's dot_scalar scores and softmax_inplace output.
Values quoted from the reference's result files (choose_num_splits, traffic)
live in reference_values.json, written by hand with file:line sources.
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
import oracle  # noqa: E402
from oracle.pa_oracle import _p  # noqa: E402


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def ref_decode(q32, k32, v32, bt, ctx, scale):
    R = oracle.ref()
    B, H, D = q32.shape
    NB, BS, HKV, _ = k32.shape
    MB = bt.shape[1]
    out = np.zeros(B * H * D, np.float32)
    R.ref_cpu_reference(_p(out), _p(np.ascontiguousarray(k32)), _p(np.ascontiguousarray(v32)),
                        _p(np.ascontiguousarray(q32)), _p(np.ascontiguousarray(bt)),
                        _p(np.ascontiguousarray(ctx)), B, H, HKV, D, BS, MB, NB, np.float32(scale))
    return out.reshape(B, H, D)


def seeded_case(path, B, H, HKV, D, BS, ctx, seed, kv, q, scale):
    inp = oracle.paged_inputs(B, H, HKV, D, BS, ctx, seed=seed, kv_dtype=kv, q_dtype=q)
    k32 = oracle.to_float(inp["k"], kv)
    v32 = oracle.to_float(inp["v"], kv)
    out = ref_decode(inp["q_f32"], k32, v32, inp["bt"], inp["ctx"], scale)
    np.savez_compressed(path, seed=seed, B=B, H=H, HKV=HKV, D=D, BS=BS, ctx=inp["ctx"],
                        kv=kv, q=q, scale=np.float32(scale),
                        input_sha256=sha(inp["q"], inp["k"], inp["v"], inp["bt"]), out=out)


def main() -> None:
    R = oracle.ref()
    if R is None:
        raise SystemExit("oracle/_ref is not built (needs the reference checkout)")

    # HIP self-test (rocm/hip/paged_attn_v1_hip.cpp:151-162).
    B, H, HKV, D, BS, MB, NB = 2, 4, 2, 32, 16, 4, 8
    q = np.zeros(B * H * D, np.float32)
    k = np.zeros(NB * BS * HKV * D, np.float32)
    v = np.zeros_like(k)
    bt = np.zeros(B * MB, np.int32)
    ctx = np.zeros(B, np.int32)
    R.ref_selftest_inputs(_p(q), _p(k), _p(v), _p(bt), _p(ctx))
    scale = np.float32(1.0) / np.sqrt(np.float32(D))
    q, k, v, bt = q.reshape(B, H, D), k.reshape(NB, BS, HKV, D), v.reshape(NB, BS, HKV, D), bt.reshape(B, MB)
    out = ref_decode(q, k, v, bt, ctx, scale)
    np.savez_compressed(HERE / "hip_selftest.npz", q=q, k=k, v=v, bt=bt, ctx=ctx,
                        scale=np.float32(scale), out=out)

    # BASELINE config 1 and a GQA bf16 ragged case.
    seeded_case(HERE / "config1.npz", 4, 12, 12, 64, 16, [512] * 4, 11, "f16", "f16", 1.0 / 8.0)
    seeded_case(HERE / "gqa_bf16.npz", 4, 32, 8, 128, 16, [1, 100, 1024, 777], 31, "bf16", "bf16",
                1.0 / np.sqrt(128.0))

    # arm scalar_smoke (arm_cpu/src/bench.cpp:60-86, arm_cpu/CMakeLists.txt:45-47).
    tokens, dim = 64, 128
    query = np.zeros(dim, np.float32)
    keys = np.zeros(tokens * dim, np.float32)
    R.ref_scalar_smoke_inputs(_p(query), _p(keys), tokens, dim)
    scores = np.zeros(tokens, np.float32)
    R.ref_attention_scores(_p(query), _p(keys), _p(scores), tokens, dim)
    probs = scores.copy()
    R.ref_softmax_inplace(_p(probs), tokens)
    np.savez_compressed(HERE / "scalar_smoke.npz", query=query, keys=keys.reshape(tokens, dim),
                        scores=scores, softmax=probs)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
