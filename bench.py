#!/usr/bin/env python3
"""Benchmark of the paged-attention hot path on one MI355X.

Headline (the JSON line's `value`): BASELINE config 2 -- GPT-2 geometry paged
decode through paged_attention_v3 (H=12, D=64, BS=16, B=64, ctx=2048, fp16),
with several disjoint KV pools rotated per step so the working set is well
above the 256 MB Infinity Cache and every K/V byte comes from HBM.

A step is one paged_attention_v3 call (partition kernel, plus the reduce
kernel when the plan splits) on one pool, inputs resident in HBM.  `value` is
algorithmic bytes per step (K and V of every live token once, plus q, out,
block tables and context lengths) / measured time per step (median of
three timed loops, each bracketed by HIP events on the launch stream).  The
dominant kernel's average duration (`roofline.achieved`): when the step is
that one kernel, the same loops; when the plan splits, HIP events on the
launch stream around each partition launch, in loops alternating with the
step loops.

Also measured (the "also" list): config 3 (GQA bf16 ragged decode), config 5
(77 GB pool, 64-bit offsets), configs 2 and 3 over FP8 E4M3 caches, a GQA
group of 8 heads (matrix-core decode kernel), configs 4a/4b (MFMA causal
prefill, TFLOP/s), the KV-cache write of the 4a/4b prompts into their pools
(GB/s), a mixed decode + prefill batch, and the per-call host cost.

cpu_baseline: the reference's own scalar cpu_reference
(rocm/hip/paged_attn_v1_hip.cpp:104-141, built into oracle/_ref), one thread,
on a bounded sample of config 2's sequences, timed on this host; the GPU
result for the sample is checked against it.  cpu_extra: our SIMD/OpenMP
port of it and torch's CPU SDPA on the gathered layout, 16 threads.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--workload decode_c2]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
import __graft_entry__  # noqa: E402

PEAK_HBM_GBS = 8000.0           # MI355X HBM3E, published
PEAK_MFMA_TFLOPS = 2500.0       # MI355X dense fp16/bf16 MFMA, published
METRIC = "decode achieved HBM GB/s (% of 8 TB/s) cold-pool; prefill TFLOP/s (% MFMA peak)"
PROFILES = ROOT / "profiles"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ decode --

class DecodeWorkload:
    """Paged decode with `pools` disjoint K/V pools, each holding every page of the batch."""

    def __init__(self, pa, *, B, H, HKV, D, BS, ctx, dtype, pools, seed, name, q_dtype=None,
                 out_dtype=None, pool_tensor=None, kv_scale=None):
        self.pa, self.name = pa, name
        self.kv_scale = kv_scale  # quantised (FP8) cache: it holds N(0,1) / kv_scale
        self.B, self.H, self.HKV, self.D, self.BS = B, H, HKV, D, BS
        self.dtype = dtype
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.ctx_host = np.asarray(ctx, np.int32)
        pages = [-(-int(c) // BS) for c in self.ctx_host]
        self.MB = max(pages)
        nb = sum(pages)
        self.k, self.v, self.bt = [], [], []
        rng = np.random.default_rng(seed)
        for p in range(pools):
            if pool_tensor is not None:
                k, v = pool_tensor(p)
            else:
                inv = 1.0 / kv_scale if kv_scale else 1.0
                k = (torch.randn((nb, BS, HKV, D), generator=g, device=dev, dtype=torch.float32) * inv).to(dtype)
                v = (torch.randn((nb, BS, HKV, D), generator=g, device=dev, dtype=torch.float32) * inv).to(dtype)
            nbp = k.shape[0]
            perm = rng.permutation(nbp)[:nb].astype(np.int32)
            bt = np.zeros((B, self.MB), np.int32)
            pos = 0
            for b in range(B):
                bt[b, :pages[b]] = perm[pos:pos + pages[b]]
                pos += pages[b]
            self.k.append(k)
            self.v.append(v)
            self.bt.append(torch.from_numpy(bt).to(dev))
            self.bt_host = bt if p == 0 else self.bt_host
        qd = q_dtype or (torch.float16 if kv_scale else dtype)
        self.q = torch.randn((B, H, D), generator=g, device=dev, dtype=torch.float32).to(qd)
        self.out = torch.empty((B, H, D), device=dev, dtype=out_dtype or (torch.float16 if kv_scale else dtype))
        self.ctx = torch.from_numpy(self.ctx_host).to(dev)
        self.scale = 1.0 / float(np.sqrt(D))
        self.pools = pools
        self.L = pa.lib()
        ws = pa.workspace_size(self.q, self.k[0], self.bt[0], 0)
        self.ws = torch.empty(max(ws, 256), dtype=torch.uint8, device=dev)
        self.ws_bytes = ws
        self.split = ws > 0
        V = pa.view
        self._keep = []
        self.args = []
        for p in range(pools):
            views = [V(self.out), V(self.q), V(self.k[p]), V(self.v[p]), V(self.bt[p]), V(self.ctx)]
            self._keep.append(views)
            self.args.append([C.byref(x) for x in views])
        self.kv_bytes = 2.0 * float(self.ctx_host.clip(min=0).sum()) * HKV * D * self.k[0].element_size()
        self.bytes = (self.kv_bytes + self.q.numel() * self.q.element_size()
                      + self.out.numel() * self.out.element_size() + B * self.MB * 4 + B * 4)

    def footprint_gb(self):
        return sum(t.numel() * t.element_size() for t in self.k + self.v) / 1e9

    def launch(self, i, stream, ev_mid=None):
        a = self.args[i % self.pools]
        ws = self.ws.data_ptr()
        if self.kv_scale:  # one call (partition and reduce): the timed kernel includes the reduce
            rc = self.L.paged_attention_v3_scaled(*a, self.scale, self.kv_scale, self.kv_scale, 0, ws,
                                                  self.ws_bytes, stream)
            if rc == 0 and ev_mid is not None:
                ev_mid.record()
        elif not self.split:
            rc = self.L.paged_attention_v3(*a, self.scale, 0, ws, self.ws_bytes, stream)
        else:
            rc = self.L.pa_v3_partition(*a, self.scale, 0, ws, self.ws_bytes, stream)
            if rc == 0 and ev_mid is not None:
                ev_mid.record()
            if rc == 0:
                rc = self.L.pa_v3_reduce(a[0], a[1], a[2], a[4], a[5], 0, ws, self.ws_bytes, stream)
        if rc != 0:
            raise RuntimeError(self.pa.last_error())


# ----------------------------------------------------------------- prefill --

class PrefillWorkload:
    """Causal paged prefill: K/V of S prompt tokens written into a paged pool, then attended."""

    def __init__(self, pa, *, B, S, H, HKV, D, BS, dtype, seed, name):
        self.pa, self.name = pa, name
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        pages = -(-S // BS)
        nb = B * pages
        rng = np.random.default_rng(seed)
        perm = rng.permutation(nb).astype(np.int32).reshape(B, pages)
        self.q = torch.randn((B, S, H, D), generator=g, device=dev, dtype=torch.float32).to(dtype)
        k_new = torch.randn((B, S, HKV, D), generator=g, device=dev, dtype=torch.float32).to(dtype)
        v_new = torch.randn((B, S, HKV, D), generator=g, device=dev, dtype=torch.float32).to(dtype)
        # Write the prompt's K/V into the paged pool with pa_write_kv (untimed setup).
        self.k = torch.zeros((nb, BS, HKV, D), device=dev, dtype=dtype)
        self.v = torch.zeros_like(self.k)
        tok = torch.arange(S, device=dev)
        bt = torch.from_numpy(perm).to(dev)
        slots = (bt[:, tok // BS].long() * BS + tok % BS).reshape(-1)
        pa.write_kv(self.k, self.v, k_new.reshape(B * S, HKV, D), v_new.reshape(B * S, HKV, D), slots)
        self.bt = bt
        self.ctx = torch.full((B,), S, dtype=torch.int32, device=dev)
        self.out = torch.empty((B, S, H, D), device=dev, dtype=dtype)
        self.scale = 1.0 / float(np.sqrt(D))
        self.flops = 4.0 * D * H * B * S * (S + 1) / 2.0  # causal pairs, QK^T and PV
        self.dtype = dtype
        V = pa.view
        self._views = [V(self.out), V(self.q), V(self.k), V(self.v), V(self.bt), V(self.ctx)]
        self.args = [C.byref(x) for x in self._views]
        self.L = pa.lib()

    def launch(self, i, stream, ev_mid=None):
        rc = self.L.paged_attention_prefill_wmma(*self.args, self.scale, stream)
        if rc != 0:
            raise RuntimeError(self.pa.last_error())


# ------------------------------------------------------------------ timing --

class WriteWorkload:
    """KV-cache write: a prompt's K/V ([B*S, HKV, D]) into its paged pool at the
    block table's slots (pa_write_kv), rotated over `copies` disjoint
    (source, pool) pairs so each step reads and writes HBM, not cache."""

    def __init__(self, pa, *, B, S, HKV, D, BS, dtype, seed, name, copies=8):
        self.pa, self.name, self.dtype = pa, name, dtype
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        rng = np.random.default_rng(seed)
        pages = -(-S // BS)
        nb, T = B * pages, B * S
        tok = np.arange(S)
        V = pa.view
        self._keep, self.args = [], []
        for _ in range(copies):
            perm = rng.permutation(nb).reshape(B, pages)
            slots = torch.from_numpy((perm[:, tok // BS] * BS + tok % BS).reshape(-1)).to(dev)
            key = torch.randn((T, HKV, D), generator=g, device=dev, dtype=torch.float32).to(dtype)
            val = torch.randn((T, HKV, D), generator=g, device=dev, dtype=torch.float32).to(dtype)
            kc = torch.zeros((nb, BS, HKV, D), device=dev, dtype=dtype)
            vc = torch.zeros_like(kc)
            views = [V(kc), V(vc), V(key), V(val), V(slots)]
            self._keep.append((slots, key, val, kc, vc, views))
            self.args.append([C.byref(x) for x in views])
        es = torch.tensor([], dtype=dtype).element_size()
        self.bytes = 2.0 * T * HKV * D * 2 * es + T * 8  # K and V read + written, slot mapping
        self.L = pa.lib()

    def launch(self, i, stream, ev_mid=None):
        rc = self.L.pa_write_kv(*self.args[i % len(self.args)], stream)
        if rc != 0:
            raise RuntimeError(self.pa.last_error())


# The prompt K/V of configs 4a and 4b written into their paged pools.
WRITE_CFG = {
    "write_kv_c4a": dict(B=8, S=1024, HKV=12, D=64, dtype=torch.float16, seed=14),
    "write_kv_c4b": dict(B=2, S=4096, HKV=32, D=128, dtype=torch.bfloat16, seed=16),
}


def write_record(work, steps, warmup):
    ms, kms, _ = timed(work, steps, warmup)
    gbs = work.bytes / (kms * 1e-3) / 1e9
    return {
        "workload": work.name, "value": round(gbs, 1), "unit": "GB/s",
        "frac_of_hbm_peak": round(gbs / PEAK_HBM_GBS, 4), "ms_per_step": round(ms, 5),
        "kernel_ms": round(kms, 5), "bytes_per_step": work.bytes, "dtype": str(work.dtype).replace("torch.", ""),
    }


class MixedWorkload:
    """Mixed decode + prefill batch (GPT-2 geometry, fp16): `nd` sequences decoding
    one token at context 2048 and `npf` sequences prefilling a `chunk`-token
    chunk at context 2048, in one pool.  launch(): one varlen MFMA call;
    launch_split(): a v3 decode of the decoders plus a uniform MFMA prefill of
    the chunks (two launches)."""

    def __init__(self, pa, nd=64, npf=4, chunk=256, ctx=2048, H=12, D=64, BS=16, seed=21):
        self.pa, self.name = pa, "mixed_c2"
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        rng = np.random.default_rng(seed)
        B, pages = nd + npf, ctx // BS
        self.k = torch.randn((B * pages, BS, H, D), generator=g, device=dev).half()
        self.v = torch.randn((B * pages, BS, H, D), generator=g, device=dev).half()
        self.bt = torch.from_numpy(rng.permutation(B * pages).astype(np.int32).reshape(B, pages)).to(dev)
        self.ctx = torch.full((B,), ctx, dtype=torch.int32, device=dev)
        qlens = [1] * nd + [chunk] * npf
        self.q = torch.randn((sum(qlens), H, D), generator=g, device=dev).half()
        self.cu = torch.tensor(np.concatenate([[0], np.cumsum(qlens)]), dtype=torch.int32, device=dev)
        self.max_q = chunk
        self.scale = 1.0 / float(np.sqrt(D))
        self.q_dec = self.q[:nd].contiguous()
        self.q_pf = self.q[nd:].reshape(npf, chunk, H, D).contiguous()
        self.out = torch.empty_like(self.q)
        self.out_dec = torch.empty_like(self.q_dec)
        self.out_pf = torch.empty_like(self.q_pf)
        self.nd, self.npf, self.chunk = nd, npf, chunk
        self.tokens = sum(qlens)
        self.kv_bytes = 2.0 * B * ctx * H * D * 2
        self.flops = 4.0 * D * H * (nd * ctx + npf * sum(ctx - chunk + r + 1 for r in range(chunk)))

    def launch(self, i, stream, ev_mid=None):
        self.pa.paged_attention_prefill_varlen(self.q, self.k, self.v, self.bt, self.ctx, self.cu, self.max_q,
                                               self.scale, out=self.out)

    def launch_split(self, i, stream, ev_mid=None):
        nd = self.nd
        self.pa.paged_attention_v3(self.q_dec, self.k, self.v, self.bt[:nd], self.ctx[:nd], self.scale, 0,
                                   out=self.out_dec)
        self.pa.paged_attention_prefill_wmma(self.q_pf, self.k, self.v, self.bt[nd:], self.ctx[nd:], self.scale,
                                             out=self.out_pf)


def mixed_record(pa, steps, warmup):
    w = MixedWorkload(pa)
    ms, _, _ = timed(w, steps, warmup)

    class Split:
        launch = w.launch_split
    ms_split, _, _ = timed(Split(), steps, warmup)
    return {"workload": w.name, "unit": "ms per step",
            "case": f"{w.nd} decode rows + {w.npf} x {w.chunk}-token prefill chunks, ctx 2048, H=12 D=64 fp16",
            "varlen_ms": round(ms, 5), "split_ms": round(ms_split, 5),
            "varlen_tokens_per_s": round(w.tokens / (ms * 1e-3), 1),
            "varlen_kv_GBs": round(w.kv_bytes / (ms * 1e-3) / 1e9, 1),
            "flops_per_step": w.flops}


def call_overhead(pa, calls=3000):
    """Wall time per call of a tiny v3 decode (B=1, H=12, ctx=64: microseconds of
    GPU work) through each binding, so host cost dominates: the C-ABI with
    prebuilt descriptors (ctypes), the Python mirror (ops.paged_attention_v3),
    the torch operator (torch.ops.gb10_attn), and a HIP graph replay of it."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    q = torch.randn((1, 12, 64), generator=g, device=dev).half()
    k = torch.randn((4, 16, 12, 64), generator=g, device=dev).half()
    v = torch.randn((4, 16, 12, 64), generator=g, device=dev).half()
    bt = torch.arange(4, dtype=torch.int32, device=dev)[None]
    ctx = torch.full((1,), 64, dtype=torch.int32, device=dev)
    out = torch.empty((1, 12, 64), device=dev)
    V = pa.view
    views = [V(out), V(q), V(k), V(v), V(bt), V(ctx)]
    args = [C.byref(x) for x in views]
    L = pa.lib()
    sp = torch.cuda.current_stream().cuda_stream
    ops = pa.torch_ops()

    def per_call(fn):
        for _ in range(50):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(calls):
            fn()
        torch.cuda.synchronize()
        return round((time.perf_counter() - t0) / calls * 1e6, 2)

    res = {"c_abi_ctypes_us": per_call(lambda: L.paged_attention_v3(*args, 0.125, 0, None, 0, sp)),
           "python_mirror_us": per_call(lambda: pa.paged_attention_v3(q, k, v, bt, ctx, 0.125, 0)),
           "torch_op_us": per_call(lambda: ops.paged_attention_v3(q, k, v, bt, ctx, 0.125, 0))}
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.paged_attention_v3(q, k, v, bt, ctx, 0.125, 0)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(graph):
        ops.paged_attention_v3(q, k, v, bt, ctx, 0.125, 0)
    res["graph_replay_us"] = per_call(graph.replay)
    return {"workload": "call_overhead", "unit": "us per call", "case": "v3 decode B=1 H=12 D=64 ctx=64 fp16",
            **res}


REPEATS = 3
# The reference's published figure for config 2 (v3 split decode, B=64,
# ctx=2048), measured on NVIDIA GB10: 231.3 GB/s = 84.7 % of its 273 GB/s.
REF_GB10_C2_GBS = 231.3


def timed(work, steps, warmup):
    """(ms per step, mean dominant-kernel ms, per-repeat step ms).

    REPEATS rounds after `warmup` launches; each round is a step loop
    (`steps` back-to-back launches bracketed by a synchronize and one pair of
    HIP events on the launch stream) followed by a kernel loop (`steps`
    launches with an event pair on the launch stream around each partition
    launch; events between launches add a small gap, so they stay out of
    the step loops).  ms per step is the median over the step loops.  The
    dominant kernel's time: when a step is that one kernel, the step loops
    already measure it (events over the timed region / launches; a pair
    around every launch would add ~2 us to a 66 us kernel); otherwise the
    mean over every bracketed launch.  Step and kernel loops alternate so
    both sample the same span: this device runs the first work of a process
    a few percent faster than what follows."""
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    for i in range(warmup):
        work.launch(i, sp)
    torch.cuda.synchronize()
    split = getattr(work, "split", False)
    reps, kern = [], []
    n = warmup
    for r in range(REPEATS):
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for i in range(steps):
            work.launch(n + i, sp)
        t1.record(stream)
        torch.cuda.synchronize()
        reps.append(t0.elapsed_time(t1) / steps)
        n += steps
        starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
        mids = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
        for i in range(steps):
            starts[i].record(stream)
            work.launch(n + i, sp, mids[i] if split else None)
            ends[i].record(stream)
        torch.cuda.synchronize()
        kern += [starts[i].elapsed_time(mids[i] if split else ends[i]) for i in range(steps)]
        n += steps
    ms = float(np.median(reps))
    return ms, (float(np.mean(kern)) if split else ms), [round(x, 5) for x in reps]


def traffic_from_profiles(kernel_key):
    """HBM bytes per launch from the committed rocprofv3 counter summary, if present."""
    f = PROFILES / "traffic.json"
    if not f.exists():
        return None
    try:
        d = json.loads(f.read_text())
        return d.get(kernel_key, {}).get("bytes_per_launch")
    except (ValueError, OSError):
        return None


# ------------------------------------------------------------- cpu baseline --

def cpu_baseline(work, seconds):
    """The reference's scalar cpu_reference (oracle/_ref), one thread, on a sample of the
    workload's sequences (all heads, full context), timed on this host.  Also checks the
    GPU output of those sequences against it."""
    import oracle
    from oracle.pa_oracle import _p
    R = oracle.ref()
    kind = "reference" if R is not None else "port"
    nsamp = 2
    bt = work.bt_host[:nsamp]
    used = np.unique(bt[bt >= 0])
    remap = np.full(work.k[0].shape[0], -1, np.int64)
    remap[used] = np.arange(used.size)
    k = work.k[0][torch.from_numpy(used).to(work.k[0].device)].float().cpu().numpy()
    v = work.v[0][torch.from_numpy(used).to(work.v[0].device)].float().cpu().numpy()
    bts = np.ascontiguousarray(remap[bt].astype(np.int32))
    ctx = np.ascontiguousarray(work.ctx_host[:nsamp])
    q = np.ascontiguousarray(work.q[:nsamp].float().cpu().numpy())
    B, H, D = q.shape
    NB, BS, HKV, _ = k.shape
    out = np.zeros((B, H, D), np.float32)
    if R is not None:
        h = R.ref_call_create(_p(k), _p(v), _p(q), _p(bts), _p(ctx), B, H, HKV, D, BS, bts.shape[1],
                              NB, C.c_float(work.scale))
        run = lambda: R.ref_call_run(h, _p(out))
    else:
        def run():
            out[...] = oracle.decode(q, k, v, bts, ctx, work.scale, "f32")
    run()  # warm-up and correctness sample
    torch.cuda.synchronize()
    work.launch(0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    gpu = work.out[:nsamp].float().cpu().numpy()
    err = float(np.abs(gpu - out).max())
    ok = bool(np.allclose(gpu, out, atol=2e-3, rtol=1e-2))
    n, t0 = 0, time.perf_counter()
    while True:
        run()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 10000:
            break
    if R is not None:
        R.ref_call_free(h)
    sample_bytes = 2.0 * float(ctx.sum()) * HKV * D * work.k[0].element_size()
    return {
        "value": round(sample_bytes * n / el / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind,
        "sample": (f"{nsamp} of {work.B} sequences (all {work.H} heads, ctx {int(ctx[0])}), "
                   f"{n} calls in {el:.1f} s; KV widened to fp32 for the reference's float API, "
                   f"bytes counted at the GPU's {work.dtype} size"),
        "check_vs_gpu": {"max_abs": err, "within_tol": ok},
    }


def simd_cpu(work, threads, seconds=2.0):
    """Our SIMD/OpenMP port of cpu_reference (oracle/pa_oracle_simd.c, AVX2 + F16C),
    parallel over (sequence, head) on `threads` host cores (BASELINE CPU path 2)."""
    import oracle
    nsamp = min(16, work.B)
    bt = work.bt_host[:nsamp]
    used = np.unique(bt[bt >= 0])
    remap = np.full(work.k[0].shape[0], -1, np.int64)
    remap[used] = np.arange(used.size)
    idx = torch.from_numpy(used).to(work.k[0].device)
    tag = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}[work.k[0].dtype]
    as_np = (lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16)) if tag == "bf16" else (lambda t: t.cpu().numpy())
    k = np.ascontiguousarray(as_np(work.k[0][idx]))
    v = np.ascontiguousarray(as_np(work.v[0][idx]))
    bts = np.ascontiguousarray(remap[bt].astype(np.int32))
    ctx = np.ascontiguousarray(work.ctx_host[:nsamp])
    q = np.ascontiguousarray(work.q[:nsamp].float().cpu().numpy())
    run = lambda: oracle.decode_simd(q, k, v, bts, ctx, work.scale, tag, threads=threads)
    run()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        run()
        n += 1
    el = time.perf_counter() - t0
    sample_bytes = 2.0 * float(ctx.sum()) * work.HKV * work.D * work.k[0].element_size()
    return {"value": round(sample_bytes * n / el / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port_simd_openmp",
            "sample": f"{nsamp} sequences (all heads), {n} calls in {el:.1f} s; the same sample each call "
                      f"(host-cache resident)"}


def host_info():
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu": model, "nproc": os.cpu_count(), "threads_used": 16}


def torch_sdpa_cpu(work, threads):
    """PyTorch SDPA on the gathered paged layout, on the host CPU (BASELINE CPU path 3)."""
    torch.set_num_threads(threads)
    nsamp = 2
    idx = torch.from_numpy(work.bt_host[:nsamp].reshape(-1).astype(np.int64)).to(work.k[0].device)
    k = work.k[0][idx].float().cpu().reshape(nsamp, -1, work.HKV, work.D)[:, :int(work.ctx_host[0])]
    v = work.v[0][idx].float().cpu().reshape(nsamp, -1, work.HKV, work.D)[:, :int(work.ctx_host[0])]
    q = work.q[:nsamp].float().cpu()[:, :, None, :]
    kt = k.permute(0, 2, 1, 3).repeat_interleave(work.H // work.HKV, 1).contiguous()
    vt = v.permute(0, 2, 1, 3).repeat_interleave(work.H // work.HKV, 1).contiguous()
    torch.nn.functional.scaled_dot_product_attention(q, kt, vt, scale=work.scale)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 2.0:
        torch.nn.functional.scaled_dot_product_attention(q, kt, vt, scale=work.scale)
        n += 1
    el = time.perf_counter() - t0
    sample_bytes = 2.0 * nsamp * float(work.ctx_host[0]) * work.HKV * work.D * work.k[0].element_size()
    return {"value": round(sample_bytes * n / el / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "torch_sdpa_gathered",
            "sample": f"{nsamp} sequences gathered to fp32, {n} calls; the same sample each call (host-cache resident)"}


# --------------------------------------------------------------- workloads --

def make_c2(pa, pools):
    return DecodeWorkload(pa, B=64, H=12, HKV=12, D=64, BS=16, ctx=[2048] * 64, dtype=torch.float16,
                          pools=pools, seed=2, name="decode_c2")


def make_c2_fp8(pa, pools):
    """Config 2's geometry over an FP8 E4M3 cache (per-tensor scale 1/16)."""
    return DecodeWorkload(pa, B=64, H=12, HKV=12, D=64, BS=16, ctx=[2048] * 64, dtype=torch.float8_e4m3fn,
                          pools=pools, seed=2, name="decode_c2_fp8", kv_scale=1.0 / 16)


def make_c3(pa, pools):
    ctx = np.random.default_rng(3).integers(1024, 32769, 32)
    return DecodeWorkload(pa, B=32, H=32, HKV=8, D=128, BS=16, ctx=ctx, dtype=torch.bfloat16,
                          pools=pools, seed=3, name="decode_c3")


def make_c3_fp8(pa, pools):
    """Config 3 over an FP8 E4M3 cache (bf16 q; per-tensor scale 1/16)."""
    ctx = np.random.default_rng(3).integers(1024, 32769, 32)
    return DecodeWorkload(pa, B=32, H=32, HKV=8, D=128, BS=16, ctx=ctx, dtype=torch.float8_e4m3fn,
                          pools=pools, seed=3, name="decode_c3_fp8", kv_scale=1.0 / 16, q_dtype=torch.bfloat16,
                          out_dtype=torch.bfloat16)


def make_gqa8(pa, pools):
    """GQA group of 8 (Llama-3-70B-like heads: HQ=64, HKV=8, D=128), bf16, ctx 8192: the matrix-core decode path."""
    return DecodeWorkload(pa, B=32, H=64, HKV=8, D=128, BS=16, ctx=[8192] * 32, dtype=torch.bfloat16,
                          pools=pools, seed=8, name="decode_gqa8")


def make_c5(pa):
    """[12 layers, 2, 131072 blocks, 16, 12, 64] fp16 pool (77.3 GB), decode on layer 11."""
    dev = torch.device("cuda:0")
    nb = 131072
    pool = torch.empty((12, 2, nb, 16, 12, 64), dtype=torch.float16, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    flat = pool.view(-1)
    step = 1 << 30
    for off in range(0, flat.numel(), step):
        n = min(step, flat.numel() - off)
        flat[off:off + n] = torch.randn(n, generator=g, device=dev, dtype=torch.float16)
    w = DecodeWorkload(pa, B=256, H=12, HKV=12, D=64, BS=16, ctx=[8192] * 256, dtype=torch.float16,
                       pools=1, seed=5, name="decode_c5", pool_tensor=lambda p: (pool[11, 0], pool[11, 1]))
    w.pool = pool
    w.k_offset_elems = pool[11, 0].storage_offset()
    return w


def decode_record(work, steps, warmup):
    ms, kms, reps = timed(work, steps, warmup)
    gbs = work.bytes / (ms * 1e-3) / 1e9
    return ms, kms, {
        "workload": work.name, "value": round(gbs, 1), "unit": "GB/s",
        "frac_of_8TBs": round(gbs / PEAK_HBM_GBS, 4), "ms_per_step": round(ms, 5), "repeats_ms": reps,
        "kernel_ms": round(kms, 5), "tokens_per_s": round(work.B / (ms * 1e-3), 1),
        "bytes_per_step": int(work.bytes), "split": work.split,
        "pools": work.pools, "footprint_GB": round(work.footprint_gb(), 2),
    }


_GEMM_REF = {}


def library_gemm_tflops(dtype, n=8192, reps=10):
    """Dense n x n x n product of N(0,1) operands through torch.matmul (the
    ROCm GEMM library) on this device: what its matrix cores sustain on
    random data in this run, for reading the prefill fraction against.
    Sustained MFMA throughput depends on the operand values (random operands
    draw more power than constant ones and the clock drops), so the published
    dense peak is not reachable with real data."""
    if dtype in _GEMM_REF:
        return _GEMM_REF[dtype]
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    a = torch.randn((n, n), generator=g, device="cuda", dtype=torch.float32).to(dtype)
    b = torch.randn((n, n), generator=g, device="cuda", dtype=torch.float32).to(dtype)
    for _ in range(3):
        c = torch.matmul(a, b)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        c = torch.matmul(a, b)
    t1.record()
    torch.cuda.synchronize()
    tf = 2.0 * n ** 3 * reps / (t0.elapsed_time(t1) * 1e-3) / 1e12
    del a, b, c
    _GEMM_REF[dtype] = round(tf, 1)
    return _GEMM_REF[dtype]


def prefill_record(work, steps, warmup):
    ms, kms, _ = timed(work, steps, warmup)
    tf = work.flops / (kms * 1e-3) / 1e12
    gemm = library_gemm_tflops(work.dtype)
    return {
        "workload": work.name, "value": round(tf, 1), "unit": "TFLOP/s",
        "frac_of_mfma_peak": round(tf / PEAK_MFMA_TFLOPS, 4),
        "library_gemm_tflops": gemm, "frac_of_library_gemm": round(tf / gemm, 4),
        "ms_per_step": round(ms, 5),
        "kernel_ms": round(kms, 5), "flops_per_step": work.flops,
        "prompt_tokens_per_s": round(work.q.shape[0] * work.q.shape[1] / (ms * 1e-3), 1),
        "dtype": str(work.dtype).replace("torch.", ""),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--pools", type=int, default=6, help="rotated KV pools (config 2)")
    ap.add_argument("--workload", default="decode_c2",
                    choices=["decode_c2", "decode_c3", "decode_c5", "decode_c2_fp8", "decode_c3_fp8", "decode_gqa8",
                             "prefill_c4a", "prefill_c4b",
                             "write_kv_c4a", "write_kv_c4b", "call_overhead", "mixed_c2", "copy_calib"],
                    help="with --only: run just this workload's kernel loop (for profiling)")
    ap.add_argument("--only", action="store_true", help="time only --workload, print its record")
    ap.add_argument("--no-also", action="store_true", help="skip the secondary configs")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (decode would shard "
              "by sequence or KV head with no exchange, prefill by head or sequence).", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    pa = __graft_entry__.load_package()

    if args.only:
        w = args.workload
        if w == "copy_calib":
            # A plain device copy of known size, to scale the FETCH_SIZE / WRITE_SIZE counters.
            n = 1 << 30
            src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda")
            dst = torch.empty_like(src)
            for _ in range(args.warmup + args.steps):
                dst.copy_(src)
            torch.cuda.synchronize()
            print(json.dumps({"workload": "copy_calib", "bytes_read_per_copy": n,
                              "bytes_written_per_copy": n, "copies": args.warmup + args.steps}), flush=True)
            return
        if w.startswith("prefill"):
            work = (PrefillWorkload(pa, B=8, S=1024, H=12, HKV=12, D=64, BS=16, dtype=torch.float16, seed=4,
                                    name="prefill_c4a") if w == "prefill_c4a" else
                    PrefillWorkload(pa, B=2, S=4096, H=32, HKV=32, D=128, BS=16, dtype=torch.bfloat16,
                                    seed=6, name="prefill_c4b"))
            print(json.dumps(prefill_record(work, args.steps, args.warmup)), flush=True)
        elif w == "mixed_c2":
            print(json.dumps(mixed_record(pa, args.steps, args.warmup)), flush=True)
        elif w == "call_overhead":
            print(json.dumps(call_overhead(pa)), flush=True)
        elif w.startswith("write_kv"):
            work = WriteWorkload(pa, BS=16, name=w, **WRITE_CFG[w])
            print(json.dumps(write_record(work, args.steps, args.warmup)), flush=True)
        else:
            work = {"decode_c2": lambda: make_c2(pa, args.pools), "decode_c3": lambda: make_c3(pa, 2),
                    "decode_c2_fp8": lambda: make_c2_fp8(pa, args.pools),
                    "decode_c3_fp8": lambda: make_c3_fp8(pa, 2),
                    "decode_gqa8": lambda: make_gqa8(pa, 2),
                    "decode_c5": lambda: make_c5(pa)}[w]()
            print(json.dumps(decode_record(work, args.steps, args.warmup)[2]), flush=True)
        return

    # Nothing is handed back to the driver (no torch.cuda.empty_cache) until the process
    # ends: every workload fits in HBM together (about 90 GB), and freeing a multi-GB pool
    # mid-process left every later kernel 3-5 % slower on this device, allocations made
    # before the free included.  A serving process allocates its pool once.
    # ---- headline: config 2 ----
    log("bench: config 2 (GPT-2 decode, B=64 ctx=2048 fp16, rotated pools)")
    work = make_c2(pa, args.pools)
    ms, kms, rec = decode_record(work, args.steps, args.warmup)
    achieved = work.bytes / (kms * 1e-3) / 1e9
    log(f"bench: {rec['value']} GB/s per step, kernel {kms * 1e3:.1f} us")

    line = {
        "metric": METRIC, "value": rec["value"], "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "timing": f"median of {REPEATS} repeats of {args.steps} steps", "repeats_ms": rec["repeats_ms"],
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": round(rec["value"] / REF_GB10_C2_GBS, 2),
        "baseline": {"value": REF_GB10_C2_GBS, "unit": "GB/s", "frac_of_its_peak": 0.847,
                     "what": "reference v3 split decode, B=64 ctx=2048 fp16 (this config), on NVIDIA GB10 "
                             "(273 GB/s LPDDR5X): different hardware, compare frac_of_peak",
                     "source": "docs/REPORT.md:124"},
        "dtype": "f16",
        "data": "synthetic N(0,1), seeded; random-permutation block tables",
        "config": {"workload": "decode_c2", "batch": 64, "context_len": 2048, "heads": 12,
                   "kv_heads": 12, "head_dim": 64, "block_size": 16, "kv_dtype": "f16",
                   "q_dtype": "f16", "out_dtype": "f16", "entry": "paged_attention_v3(num_splits=0)",
                   "pools": work.pools, "working_set_GB": rec["footprint_GB"],
                   "split": work.split},
        "frac_of_peak": rec["frac_of_8TBs"],
        "tokens_per_s": rec["tokens_per_s"],
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": traffic_from_profiles("decode_c2"),
                     "kernel": "pa::decode_kernel<KvF16, 64, 1, 1, 1>",
                     "kernel_ms": round(kms, 5), "bytes_per_launch": int(work.bytes)},
    }
    log("bench: cpu baseline (reference cpu_reference, 1 thread)")
    line["cpu_baseline"] = cpu_baseline(work, args.cpu_seconds)
    line["cpu_extra"] = [simd_cpu(work, 16), torch_sdpa_cpu(work, 16)]
    line["host"] = host_info()
    del work

    also = []
    if not args.no_also:
        for make in (lambda: make_c3(pa, 2), lambda: make_c5(pa), lambda: make_c2_fp8(pa, args.pools),
                     lambda: make_c3_fp8(pa, 2), lambda: make_gqa8(pa, 2)):
            w = make()
            log(f"bench: {w.name}")
            also.append(decode_record(w, max(20, args.steps // 4), 5)[2])
            if w.name == "decode_c5":
                also[-1]["k_base_offset_elements"] = int(w.k_offset_elems)
            del w
        for name, kw in (("prefill_c4a", dict(B=8, S=1024, H=12, HKV=12, D=64, dtype=torch.float16, seed=4)),
                         ("prefill_c4b", dict(B=2, S=4096, H=32, HKV=32, D=128, dtype=torch.bfloat16, seed=6))):
            log(f"bench: {name}")
            w = PrefillWorkload(pa, BS=16, name=name, **kw)
            also.append(prefill_record(w, max(20, args.steps // 4), 5))
            del w
        for name, kw in WRITE_CFG.items():
            log(f"bench: {name}")
            w = WriteWorkload(pa, BS=16, name=name, **kw)
            also.append(write_record(w, max(20, args.steps // 4), 5))
            del w
        log("bench: mixed decode + prefill batch")
        also.append(mixed_record(pa, max(20, args.steps // 4), 5))
        log("bench: per-call host overhead")
        also.append(call_overhead(pa))
    line["also"] = also
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
