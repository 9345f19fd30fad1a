"""Seeded random sweep of the decode and prefill entry points against the CPU
oracle: each case draws its geometry (batch, query and KV heads, head_dim,
block size, ragged contexts including empty and single-token ones), cache and
q dtypes (fp16, bf16, fp32, FP8 E4M3 with per-tensor scales), entry point and
split count, so that combinations the targeted tests do not enumerate still
meet the north-star tolerance (fp32 caches: 1e-4).  Cases are small enough
for the oracle to finish in milliseconds; the case parameters are printed
before each GPU call."""
import numpy as np
import pytest
import torch

import oracle
from _helpers import ATOL32, RTOL32, close, to_dev, to_host

pytestmark = pytest.mark.gpu

KV_TYPES = ["f16", "bf16", "f32", "fp8"]
Q_TYPES = {"f16": ["f16", "f32"], "bf16": ["bf16", "f32"], "f32": ["f32"], "fp8": ["f16", "bf16", "f32"]}
TORCH_OF = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def draw(seed):
    rng = np.random.default_rng(1000 + seed)
    kv = KV_TYPES[seed % len(KV_TYPES)]
    D = int(rng.choice([32, 64, 128, 256] if kv != "fp8" else [64, 128, 256]))
    HKV = int(rng.choice([1, 2, 3, 4]))
    G = int(rng.choice([1, 2, 4, 5, 8]))
    BS = int(rng.choice([16, 32, 8, 5]))
    B = int(rng.integers(1, 6))
    ctx = rng.integers(0, 900, B)
    ctx[rng.integers(0, B)] = int(rng.choice([1, 16, 17, 2049]))
    qt = str(rng.choice(Q_TYPES[kv]))
    ks, vs = (float(rng.choice([1.0, 0.05, 0.5])), float(rng.choice([1.0, 0.04]))) if kv == "fp8" else (1.0, 1.0)
    return rng, dict(kv=kv, D=D, HKV=HKV, G=G, BS=BS, B=B, ctx=ctx.astype(np.int32), qt=qt, ks=ks, vs=vs)


def pool(c, seed, H):
    """Host K/V in the cache's storage and as the oracle reads them (fp32 values for FP8)."""
    src = "f32" if c["kv"] == "fp8" else c["kv"]
    inp = oracle.paged_inputs(c["B"], H, c["HKV"], c["D"], c["BS"], c["ctx"], seed=seed, kv_dtype=src, q_dtype=c["qt"])
    if c["kv"] != "fp8":
        return inp, inp["k"], inp["v"], c["kv"]
    k8 = oracle.fp8_encode(inp["k"] / np.float32(c["ks"]))
    v8 = oracle.fp8_encode(inp["v"] / np.float32(c["vs"]))
    inp["k8"], inp["v8"] = k8, v8
    return inp, oracle.fp8_decode(k8) * np.float32(c["ks"]), oracle.fp8_decode(v8) * np.float32(c["vs"]), "f32"


def dev_kv(inp, c, dev):
    if c["kv"] == "fp8":
        f8 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).view(torch.float8_e4m3fn).to(dev)  # noqa: E731
        return f8(inp["k8"]), f8(inp["v8"])
    return to_dev(inp["k"], c["kv"], dev), to_dev(inp["v"], c["kv"], dev)


@pytest.mark.parametrize("seed", range(48))
def test_random_decode(pa, dev, seed):
    rng, c = draw(seed)
    H = c["HKV"] * c["G"]
    entry = str(rng.choice(["v1", "v2", "v3auto", "v3split"]))
    ns = int(rng.choice([2, 3, 8, 64])) if entry == "v3split" else 0
    ot = TORCH_OF[str(rng.choice(["f32", "f16", "bf16"]))]
    print(f"decode case seed={seed} {c} entry={entry} splits={ns} out={ot}", flush=True)
    inp, kref, vref, kvname = pool(c, seed, H)
    k, v = dev_kv(inp, c, dev)
    q = to_dev(inp["q"], c["qt"], dev)
    bt, ctx = torch.from_numpy(inp["bt"]).to(dev), torch.from_numpy(inp["ctx"]).to(dev)
    scale = float(rng.choice([1.0 / np.sqrt(c["D"]), 0.3, -0.2]))
    scaled = c["ks"] != 1.0 or c["vs"] != 1.0
    if entry in ("v1", "v2") and not scaled:
        got = (pa.paged_attention if entry == "v1" else pa.paged_attention_v2)(q, k, v, bt, ctx, scale, out_dtype=ot)
    else:
        got = pa.paged_attention_v3(q, k, v, bt, ctx, scale, ns, out_dtype=ot, k_scale=c["ks"], v_scale=c["vs"])
    want = oracle.decode(inp["q_f32"], kref, vref, inp["bt"], inp["ctx"], scale, kvname)
    tol = dict(atol=ATOL32, rtol=RTOL32) if c["kv"] == "f32" and c["qt"] == "f32" and ot == torch.float32 else {}
    if ot != torch.float32:  # the output's own rounding
        want = oracle.to_float(oracle.quantize(want, "f16" if ot == torch.float16 else "bf16"),
                               "f16" if ot == torch.float16 else "bf16")
    close(to_host(got), want, **tol)


@pytest.mark.parametrize("seed", range(32))
def test_random_prefill(pa, dev, seed):
    rng, c = draw(seed + 500)
    if c["kv"] == "f32":  # the matrix-core path takes 16-bit and FP8 caches
        c["kv"], c["qt"] = "bf16", "bf16"
    # Smaller than the decode cases: the oracle's prefill is scalar C.
    c["B"] = min(c["B"], 3)
    c["ctx"] = np.minimum(c["ctx"][:c["B"]], 1200)
    c["HKV"], c["G"] = min(c["HKV"], 2), min(c["G"], 2)
    H = c["HKV"] * c["G"]
    S = int(rng.integers(1, 200))
    ctx = np.maximum(c["ctx"], 0)
    print(f"prefill case seed={seed} {c} S={S}", flush=True)
    inp, kref, vref, kvname = pool(c, seed, H)
    qh = oracle.quantize(rng.standard_normal((c["B"], S, H, c["D"]), dtype=np.float32), c["qt"])
    q32 = oracle.to_float(qh, c["qt"])
    k, v = dev_kv(inp, c, dev)
    bt, ctxd = torch.from_numpy(inp["bt"]).to(dev), torch.from_numpy(ctx.astype(np.int32)).to(dev)
    scale = float(rng.choice([1.0 / np.sqrt(c["D"]), 0.2]))
    got = pa.paged_attention_prefill_wmma(to_dev(qh, c["qt"], dev), k, v, bt, ctxd, scale,
                                          k_scale=c["ks"], v_scale=c["vs"])
    want = oracle.prefill(q32, kref, vref, inp["bt"], ctx.astype(np.int32), scale, kvname)
    close(to_host(got), want)
