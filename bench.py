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
                 out_dtype=None, pool_tensor=None, kv_scale=None, num_splits=0):
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
            perm = self._tables(rng, nbp, nb, B, pages, p)
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
        self.num_splits = num_splits
        ws = pa.workspace_size(self.q, self.k[0], self.bt[0], num_splits)
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

    def _tables(self, rng, nbp, nb, B, pages, p):
        """Physical blocks of pool p's pages: a random choice of nb of its nbp blocks."""
        return rng.permutation(nbp)[:nb].astype(np.int32)

    def footprint_gb(self):
        return sum(t.numel() * t.element_size() for t in self.k + self.v) / 1e9

    def launch(self, i, stream, ev_mid=None):
        a = self.args[i % self.pools]
        ws, ns = self.ws.data_ptr(), self.num_splits
        if self.kv_scale:  # one call (partition and reduce): the timed kernel includes the reduce
            rc = self.L.paged_attention_v3_scaled(*a, self.scale, self.kv_scale, self.kv_scale, ns, ws,
                                                  self.ws_bytes, stream)
            if rc == 0 and ev_mid is not None:
                ev_mid.record()
        elif not self.split:
            rc = self.L.paged_attention_v3(*a, self.scale, ns, ws, self.ws_bytes, stream)
        else:
            rc = self.L.pa_v3_partition(*a, self.scale, ns, ws, self.ws_bytes, stream)
            if rc == 0 and ev_mid is not None:
                ev_mid.record()
            if rc == 0:
                rc = self.L.pa_v3_reduce(a[0], a[1], a[2], a[4], a[5], ns, ws, self.ws_bytes, stream)
        if rc != 0:
            raise RuntimeError(self.pa.last_error())


class ScatteredWorkload(DecodeWorkload):
    """GPT-2 decode (H=12, D=64, BS=16, fp16) at batch B and context ctx over ONE
    shared pool cut into disjoint block-table sets used in rotation, one per
    step, each set's pages a random draw from the whole pool: the layout of a
    serving cache whose free list has been shuffled by many requests."""

    def __init__(self, pa, pool, *, B, ctx, seed, name, max_sets=4096):
        k, v = pool
        BS = k.shape[1]
        per_call = B * (-(-ctx // BS))
        sets = max(1, min(k.shape[0] // per_call, max_sets))
        self._sets, self._per_call, self._pool_blocks = sets, per_call, k.shape[0]
        super().__init__(pa, B=B, H=12, HKV=12, D=64, BS=BS, ctx=[ctx] * B, dtype=torch.float16, pools=sets,
                         seed=seed, name=name, pool_tensor=lambda p: (k, v))

    def _tables(self, rng, nbp, nb, B, pages, p):
        if p == 0:
            self._perm = rng.permutation(nbp).astype(np.int32)
        return self._perm[p * nb:(p + 1) * nb]

    def footprint_gb(self):
        """Bytes of the distinct pages the rotation reads (K and V)."""
        return self._sets * self._per_call * 2 * self.BS * self.HKV * self.D * 2 / 1e9

    def pool_gb(self):
        return self._pool_blocks * 2 * self.BS * self.HKV * self.D * 2 / 1e9


class SweepWorkload(ScatteredWorkload):
    """The small-batch / short-context cold sweep of the reference
    (harness/gb10_burst.sh:103-116) through paged_attention_v3 with the
    library's plan: one shared pool of at least 4x the 256 MB Infinity Cache,
    cut into disjoint block-table sets used in rotation (the reference's
    --cold-pools)."""

    def __init__(self, pa, pool, *, B, ctx, seed):
        super().__init__(pa, pool, B=B, ctx=ctx, seed=seed, name=f"sweep_b{B}_c{ctx}")


# ----------------------------------------------------------------- prefill --

class PrefillWorkload:
    """Causal paged prefill: the K/V of a ctx-token prompt written into a paged
    pool, then the last S positions attended (ctx = S: a whole prompt; ctx > S:
    a trailing chunk, kernels/paged_attn_prefill.cu:62-64)."""

    def __init__(self, pa, *, B, S, H, HKV, D, BS, dtype, seed, name, ctx=None, cache_dtype=None, kv_scale=None):
        self.pa, self.name = pa, name
        self.kv_scale = kv_scale  # scaled (FP8) pool: it holds K / kv_scale and V / kv_scale
        ctx = ctx or S
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        pages = -(-ctx // BS)
        nb = B * pages
        rng = np.random.default_rng(seed)
        perm = rng.permutation(nb).astype(np.int32).reshape(B, pages)
        self.q = torch.randn((B, S, H, D), generator=g, device=dev, dtype=torch.float32).to(dtype)
        k_new = torch.randn((B, ctx, HKV, D), generator=g, device=dev, dtype=torch.float32).to(dtype)
        v_new = torch.randn((B, ctx, HKV, D), generator=g, device=dev, dtype=torch.float32).to(dtype)
        # Write the prompt's K/V into the paged pool with pa_write_kv (untimed setup).
        if cache_dtype == torch.float8_e4m3fn:
            self.k = torch.zeros((nb, BS, HKV, D), device=dev, dtype=torch.uint8).view(cache_dtype)
        else:
            self.k = torch.zeros((nb, BS, HKV, D), device=dev, dtype=dtype)
        self.v = torch.zeros_like(self.k)
        tok = torch.arange(ctx, device=dev)
        bt = torch.from_numpy(perm).to(dev)
        slots = (bt[:, tok // BS].long() * BS + tok % BS).reshape(-1)
        ks = kv_scale or 1.0
        pa.write_kv(self.k, self.v, k_new.reshape(B * ctx, HKV, D), v_new.reshape(B * ctx, HKV, D), slots,
                    k_scale=ks, v_scale=ks)
        self.bt = bt
        self.ctx = torch.full((B,), ctx, dtype=torch.int32, device=dev)
        self.out = torch.empty((B, S, H, D), device=dev, dtype=dtype)
        self.scale = 1.0 / float(np.sqrt(D))
        # Causal pairs, QK^T and PV: row r sees ctx - S + r + 1 keys.
        self.flops = 4.0 * D * H * B * (S * (ctx - S) + S * (S + 1) / 2.0)
        self.dtype = dtype
        V = pa.view
        self._views = [V(self.out), V(self.q), V(self.k), V(self.v), V(self.bt), V(self.ctx)]
        self.args = [C.byref(x) for x in self._views]
        self.L = pa.lib()

    def launch(self, i, stream, ev_mid=None):
        if self.kv_scale:
            rc = self.L.paged_attention_prefill_wmma_scaled(*self.args, self.scale, self.kv_scale, self.kv_scale,
                                                             stream)
        else:
            rc = self.L.paged_attention_prefill_wmma(*self.args, self.scale, stream)
        if rc != 0:
            raise RuntimeError(self.pa.last_error())


# -------------------------------------------------------- correctness gate --
# Every workload is checked against the CPU oracle on a sample of its own
# inputs before it is timed (the reference publishes no number for a path that
# fails its check, docs/REPORT.md:41-43); a failing workload is reported as
# FAILED with no value.

ATOL, RTOL = 2e-3, 1e-2  # north-star tolerance for 16-bit data: |got - want| <= ATOL + RTOL |want|


def _compare(got, want, what):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    err = np.abs(got - want)
    bad = ~(err <= ATOL + RTOL * np.abs(want))
    bad &= ~(np.isnan(got) & np.isnan(want))
    return {"what": what, "max_abs": float(np.nanmax(err)) if err.size else 0.0,
            "outside_tol": int(bad.sum()), "ok": bool(not bad.any())}


def _gather_pages(k, v, bt, ctx, BS, scale=None):
    """Host fp32 copies of the pages the rows of bt read, and bt remapped to them."""
    ctx = np.asarray(ctx, np.int64)
    used = np.unique(np.concatenate([bt[i, :max(0, -(-int(c) // BS))] for i, c in enumerate(ctx)]))
    remap = np.zeros(int(k.shape[0]), np.int64)
    remap[used] = np.arange(used.size)
    idx = torch.from_numpy(used).to(k.device)
    kh, vh = k[idx].float(), v[idx].float()
    if scale:
        kh, vh = kh * scale, vh * scale
    return kh.cpu().numpy(), vh.cpu().numpy(), np.ascontiguousarray(remap[bt].astype(np.int32))


def check_decode(work, nseq=2, entry="v3"):
    """One call on pool 0 (v3: the plan the timed loop runs; v1 / v2: the
    reference's other decode entry points); the sampled sequences (the longest
    and shortest, else the first and last) against the oracle's cpu_reference
    restatement.  Also returns the dispatched kernels."""
    import oracle
    ctx = work.ctx_host
    seqs = sorted({int(np.argmax(ctx)), int(np.argmin(ctx))} if ctx.min() != ctx.max() else {0, work.B - 1})[:nseq]
    work.out.fill_(float("nan"))
    a = work.args[0]
    sp = torch.cuda.current_stream().cuda_stream
    if entry == "v3":
        rc = work.L.paged_attention_v3_scaled(*a, work.scale, work.kv_scale or 1.0, work.kv_scale or 1.0,
                                              work.num_splits, work.ws.data_ptr(), work.ws_bytes, sp)
    else:
        rc = getattr(work.L, "paged_attention" if entry == "v1" else "paged_attention_v2")(*a, work.scale, sp)
    if rc != 0:
        raise RuntimeError(work.pa.last_error())
    kernels = work.pa.last_launch()
    torch.cuda.synchronize()
    got = work.out[seqs].float().cpu().numpy()
    k, v, bts = _gather_pages(work.k[0], work.v[0], work.bt_host[seqs], ctx[seqs], work.BS, work.kv_scale)
    want = oracle.decode(work.q[seqs].float().cpu().numpy(), k, v, bts, ctx[seqs], work.scale, "f32")
    return _compare(got, want, f"sequences {seqs}, all {work.H} heads, vs oracle.decode"), kernels


def check_prefill(work, rows=(0, 1, 63, 64, 127, 128, 129, 511, -2, -1)):
    """One call; sampled query rows of the first and last sequence against the
    oracle's decode of each row's visible prefix (position ctx - S + r)."""
    import oracle
    work.out.fill_(float("nan"))
    work.launch(0, torch.cuda.current_stream().cuda_stream)
    kernels = work.pa.last_launch()
    torch.cuda.synchronize()
    B, S = work.q.shape[0], work.q.shape[1]
    ctx = work.ctx.cpu().numpy()
    bt = work.bt.cpu().numpy()
    rs = sorted({r % S for r in rows})
    bs = [b for b in (0, B - 1) for _ in rs]
    rr = [r for _ in (0, B - 1) for r in rs]
    pos = np.asarray([int(ctx[b]) - S + r for b, r in zip(bs, rr)], np.int32)
    k, v, bts = _gather_pages(work.k, work.v, bt[bs], pos + 1, work.k.shape[1], work.kv_scale)
    want = oracle.decode(work.q.float().cpu().numpy()[bs, rr], k, v, bts, pos + 1, work.scale, "f32")
    got = work.out.float().cpu().numpy()[bs, rr]
    return _compare(got, want, f"{len(rr)} query rows of sequences 0 and {B - 1} vs oracle.decode of their prefix"), kernels


def check_write(work):
    """One write (copy 0); sampled tokens' K and V rows read back from their
    slots must equal the source rows bit for bit (same dtype: a copy)."""
    slots, key, val, kc, vc, _ = work._keep[0]
    kc.zero_()
    vc.zero_()
    work.launch(0, torch.cuda.current_stream().cuda_stream)
    kernels = work.pa.last_launch()
    torch.cuda.synchronize()
    T = key.shape[0]
    t = torch.tensor(sorted({0, 1, T // 3, T // 2, T - 2, T - 1}), device=key.device)
    sl = slots[t].long()
    blk, row = sl // work.BS, sl % work.BS
    if work.cache_dtype == work.dtype and work.kv_scale == 1.0:
        ok = bool(torch.equal(kc[blk, row], key[t]) and torch.equal(vc[blk, row], val[t]))
        what = f"{t.numel()} tokens' K/V rows at their slots vs the source rows, bit for bit"
    else:  # torch's own cast of source / scale (no value here reaches the FP8 saturation range)
        sc = torch.tensor(work.kv_scale, dtype=torch.float32, device=key.device)
        wk = (key[t].float() / sc).to(work.cache_dtype)
        wv = (val[t].float() / sc).to(work.cache_dtype)
        as_bits = (lambda x: x.view(torch.uint8)) if work.cache_dtype == torch.float8_e4m3fn else (lambda x: x)
        ok = bool(torch.equal(as_bits(kc[blk, row]), as_bits(wk)) and torch.equal(as_bits(vc[blk, row]), as_bits(wv)))
        what = f"{t.numel()} tokens' K/V rows at their slots vs torch's cast of source / scale, bit for bit"
    return {"what": what, "ok": ok}, kernels


def check_mixed(w):
    """The varlen call; the first and last decode rows and sampled rows of the
    first and last prefill chunk against the oracle's decode of their prefix."""
    import oracle
    w.out.fill_(float("nan"))
    w.launch(0, None)
    kernels = w.pa.last_launch()
    torch.cuda.synchronize()
    ctx = w.ctx.cpu().numpy()
    cu = w.cu.cpu().numpy()
    bt = w.bt.cpu().numpy()
    seqs, rows = [], []
    for b in (0, w.nd - 1):
        seqs.append(b)
        rows.append(0)
    for b in (w.nd, w.nd + w.npf - 1):
        for r in (0, 1, w.chunk // 2, w.chunk - 1):
            seqs.append(b)
            rows.append(r)
    qlen = np.diff(cu)
    pos = np.asarray([int(ctx[b]) - int(qlen[b]) + r for b, r in zip(seqs, rows)], np.int32)
    trow = [int(cu[b]) + r for b, r in zip(seqs, rows)]
    k, v, bts = _gather_pages(w.k, w.v, bt[seqs], pos + 1, w.k.shape[1])
    want = oracle.decode(w.q.float().cpu().numpy()[trow], k, v, bts, pos + 1, w.scale, "f32")
    got = w.out.float().cpu().numpy()[trow]
    return _compare(got, want, f"{len(trow)} rows (decode rows and prefill-chunk rows) vs oracle.decode"), kernels


def failed_record(name, check, kernels=None):
    log(f"bench: {name} FAILED its correctness check: {check}")
    return {"workload": name, "status": "FAILED", "check": check, "kernels": kernels}


# ------------------------------------------------------------------ timing --

class WriteWorkload:
    """KV-cache write: a prompt's K/V ([B*S, HKV, D]) into its paged pool at the
    block table's slots (pa_write_kv), rotated over `copies` disjoint
    (source, pool) pairs so each step reads and writes HBM, not cache."""

    def __init__(self, pa, *, B, S, HKV, D, BS, dtype, seed, name, copies=8, cache_dtype=None, kv_scale=1.0):
        self.pa, self.name, self.dtype, self.BS = pa, name, dtype, BS
        self.cache_dtype = cache_dtype or dtype
        self.kv_scale = kv_scale  # the cache holds key / kv_scale and value / kv_scale
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
            kc = torch.zeros((nb, BS, HKV, D), device=dev, dtype=torch.uint8).view(self.cache_dtype) \
                if self.cache_dtype == torch.float8_e4m3fn else torch.zeros((nb, BS, HKV, D), device=dev, dtype=dtype)
            vc = torch.zeros_like(kc)
            views = [V(kc), V(vc), V(key), V(val), V(slots)]
            self._keep.append((slots, key, val, kc, vc, views))
            self.args.append([C.byref(x) for x in views])
        es = torch.tensor([], dtype=dtype).element_size()
        ces = torch.tensor([], dtype=self.cache_dtype).element_size()
        self.bytes = 2.0 * T * HKV * D * (es + ces) + T * 8  # K and V read + written, slot mapping
        self.L = pa.lib()

    def launch(self, i, stream, ev_mid=None):
        rc = self.L.pa_write_kv_scaled(*self.args[i % len(self.args)], self.kv_scale, self.kv_scale, stream)
        if rc != 0:
            raise RuntimeError(self.pa.last_error())


# Configs 4a and 4b (whole prompts, S = ctx) and the reference's own prefill
# shape: a 512-token chunk at context 2048, B = 4, GPT-2 heads, fp16
# (results/c001-20260901-223111/bench_prefill.txt:40-42).
PREFILL_CFG = {
    "prefill_c4a": dict(B=8, S=1024, H=12, HKV=12, D=64, dtype=torch.float16, seed=4),
    "prefill_c4b": dict(B=2, S=4096, H=32, HKV=32, D=128, dtype=torch.bfloat16, seed=6),
    "prefill_ref_chunk": dict(B=4, S=512, ctx=2048, H=12, HKV=12, D=64, dtype=torch.float16, seed=7),
    # Config 4b's geometry over an FP8 E4M3 pool (per-tensor scale 1/16, bf16 q): tiles converted to fp16.
    "prefill_c4b_fp8": dict(B=2, S=4096, H=32, HKV=32, D=128, dtype=torch.bfloat16, seed=6,
                            cache_dtype=torch.float8_e4m3fn, kv_scale=1.0 / 16),
}

# The prompt K/V of configs 4a and 4b written into their paged pools.
WRITE_CFG = {
    "write_kv_c4a": dict(B=8, S=1024, HKV=12, D=64, dtype=torch.float16, seed=14),
    "write_kv_c4b": dict(B=2, S=4096, HKV=32, D=128, dtype=torch.bfloat16, seed=16),
    # Config 4b's bf16 prompt quantised into an FP8 E4M3 pool (per-tensor scale 1/16).
    "write_kv_c4b_fp8": dict(B=2, S=4096, HKV=32, D=128, dtype=torch.bfloat16, seed=16,
                             cache_dtype=torch.float8_e4m3fn, kv_scale=1.0 / 16),
}


def copy_reference_ms(nbytes, steps, copies=8):
    """ms per launch of torch's own contiguous device copy moving the same
    bytes (nbytes / 2 read, nbytes / 2 written), rotated over `copies`
    buffer pairs like the write workloads: the device's rate for a plain copy
    launch of this size, measured in the same process."""
    dev = torch.device("cuda:0")
    n = int(nbytes // 4)  # 16-bit elements per side
    srcs = [torch.ones(n, device=dev, dtype=torch.float16) for _ in range(copies)]
    dsts = [torch.empty_like(x) for x in srcs]
    stream = torch.cuda.current_stream()
    for i in range(20):
        dsts[i % copies].copy_(srcs[i % copies])
    torch.cuda.synchronize()
    reps = []
    for _ in range(REPEATS):
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for i in range(steps):
            dsts[i % copies].copy_(srcs[i % copies])
        t1.record(stream)
        torch.cuda.synchronize()
        reps.append(t0.elapsed_time(t1) / steps)
    return float(np.median(reps))


def write_record(work, steps, warmup):
    chk, kernels = check_write(work)
    if not chk["ok"]:
        return failed_record(work.name, chk, kernels)
    ms, kms, _ = timed(work, steps, warmup)
    gbs = work.bytes / (kms * 1e-3) / 1e9
    cms = copy_reference_ms(work.bytes, steps)
    return {
        "workload": work.name, "value": round(gbs, 1), "unit": "GB/s",
        "frac_of_hbm_peak": round(gbs / PEAK_HBM_GBS, 4), "ms_per_step": round(ms, 5),
        "kernel_ms": round(kms, 5), "bytes_per_step": work.bytes, "dtype": str(work.dtype).replace("torch.", ""),
        "cache_dtype": str(work.cache_dtype).replace("torch.", ""),
        "plain_copy_same_bytes": {"ms": round(cms, 5), "GBs": round(work.bytes / (cms * 1e-3) / 1e9, 1),
                                  "what": "torch copy_ of one contiguous buffer, same bytes moved, 8 rotated pairs"},
        "kernels": kernels, "check": chk,
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
    chk, kernels = check_mixed(w)
    if not chk["ok"]:
        return failed_record(w.name, chk, kernels)
    ms, _, _ = timed(w, steps, warmup)

    class Split:
        launch = w.launch_split
    ms_split, _, _ = timed(Split(), steps, warmup)
    return {"workload": w.name, "unit": "ms per step",
            "case": f"{w.nd} decode rows + {w.npf} x {w.chunk}-token prefill chunks, ctx 2048, H=12 D=64 fp16",
            "varlen_ms": round(ms, 5), "split_ms": round(ms_split, 5),
            "varlen_tokens_per_s": round(w.tokens / (ms * 1e-3), 1),
            "varlen_kv_GBs": round(w.kv_bytes / (ms * 1e-3) / 1e9, 1),
            "flops_per_step": w.flops, "kernels": kernels, "check": chk}


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
    # What a replay costs the runtime by itself: a graph of one trivial torch
    # kernel, and the decode call's cost when 20 of them share one replay.
    x = torch.zeros(1, device=dev)
    tg = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        x.add_(1)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(tg):
        x.add_(1)
    res["graph_replay_trivial_kernel_us"] = per_call(tg.replay)
    g20 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g20):
        for _ in range(20):
            ops.paged_attention_v3(q, k, v, bt, ctx, 0.125, 0)
    res["graph_of_20_calls_us_per_call"] = round(per_call(g20.replay) / 20, 2)
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
    reps, kern, tail = [], [], []
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
        if split:
            tail += [mids[i].elapsed_time(ends[i]) for i in range(steps)]
        n += steps
    ms = float(np.median(reps))
    # Split steps: the mean time from the partition kernel's end to the step's
    # end (the reduce launch, plus the gap an event pair adds).
    work.reduce_ms = float(np.mean(tail)) if split else None
    return ms, (float(np.mean(kern)) if split else ms), [round(x, 5) for x in reps]


def traffic_from_profiles(workload, kernel, algorithmic_bytes):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary (profiles/traffic.json), with the reason when there is none: the
    entry must name the kernel this run dispatched and the same algorithmic
    bytes, else it describes another build or plan and is not used."""
    f = PROFILES / "traffic.json"
    if not f.exists():
        return None, "no profiles/traffic.json"
    try:
        d = json.loads(f.read_text()).get(workload)
    except (ValueError, OSError) as e:
        return None, f"profiles/traffic.json unreadable: {e}"
    if not d:
        return None, f"no counter entry for {workload}"
    if d.get("kernel") != kernel:
        return None, f"stale: the counters were taken on {d.get('kernel')}, this run dispatched {kernel}"
    if abs(d.get("algorithmic_bytes", 0) - algorithmic_bytes) > 0.001 * algorithmic_bytes:
        return None, "stale: the counters were taken on another workload size"
    return d.get("bytes_per_launch"), "rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated (profiles/traffic.json)"


# ------------------------------------------------------------- cpu baseline --

def _llc_bytes():
    """Total last-level cache of this host (sum over distinct L3 instances), or None."""
    seen, total = set(), 0
    base = Path("/sys/devices/system/cpu")
    try:
        for c in base.glob("cpu[0-9]*/cache/index3"):
            key = (c / "shared_cpu_list").read_text().strip()
            if key in seen:
                continue
            seen.add(key)
            sz = (c / "size").read_text().strip()
            total += int(sz[:-1]) * (1024 if sz.endswith("K") else 1024 * 1024) if sz[-1] in "KM" else int(sz)
    except (OSError, ValueError):
        return None
    return total or None


def cpu_baseline(work, seconds):
    """The reference's scalar cpu_reference (oracle/_ref), one thread, on ALL of
    the workload's sequences (config 2: 64 x 12 heads x 2048 tokens, 805 MB of
    fp32 K/V, far above the host's last-level cache, so it streams from DRAM as
    the GPU's cold pools do), timed on this host.  Also checks every GPU output
    row against it."""
    import oracle
    from oracle.pa_oracle import _p
    R = oracle.ref()
    kind = "reference" if R is not None else "port"
    B, H, D = work.q.shape
    k, v, bts = _gather_pages(work.k[0], work.v[0], work.bt_host, work.ctx_host, work.BS)
    ctx = np.ascontiguousarray(work.ctx_host)
    q = np.ascontiguousarray(work.q.float().cpu().numpy())
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
    gpu = work.out.float().cpu().numpy()
    chk = _compare(gpu, out, "every GPU output row vs the reference's cpu_reference")
    n, t0 = 0, time.perf_counter()
    while True:
        run()
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 3) or n >= 10000:
            break
    if R is not None:
        R.ref_call_free(h)
    sample_bytes = 2.0 * float(ctx.sum()) * HKV * D * work.k[0].element_size()
    return {
        "value": round(sample_bytes * n / el / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind,
        "sample": (f"all {B} sequences (all {H} heads, ctx {int(ctx[0])}): {k.nbytes * 2 / 1e6:.0f} MB of fp32 K/V "
                   f"per call (KV widened to fp32 for the reference's float API; bytes counted at the GPU's "
                   f"{work.dtype} size), {n} calls in {el:.1f} s"),
        "check_vs_gpu": {"max_abs": chk["max_abs"], "within_tol": chk["ok"]},
    }


def simd_cpu(work, threads, seconds=3.0):
    """Our SIMD/OpenMP port of cpu_reference (oracle/pa_oracle_simd.c, AVX2 + F16C),
    parallel over (sequence, head) on `threads` host cores (BASELINE CPU path 2),
    on all of the workload's sequences in their storage type (config 2: 403 MB of
    fp16 K/V per call, above the host's last-level cache)."""
    import oracle
    bt = work.bt_host
    used = np.unique(bt[bt >= 0])
    remap = np.full(work.k[0].shape[0], -1, np.int64)
    remap[used] = np.arange(used.size)
    idx = torch.from_numpy(used).to(work.k[0].device)
    tag = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}[work.k[0].dtype]
    as_np = (lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16)) if tag == "bf16" else (lambda t: t.cpu().numpy())
    k = np.ascontiguousarray(as_np(work.k[0][idx]))
    v = np.ascontiguousarray(as_np(work.v[0][idx]))
    bts = np.ascontiguousarray(remap[bt].astype(np.int32))
    ctx = np.ascontiguousarray(work.ctx_host)
    q = np.ascontiguousarray(work.q.float().cpu().numpy())
    run = lambda: oracle.decode_simd(q, k, v, bts, ctx, work.scale, tag, threads=threads)
    run()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds or n < 3:
        run()
        n += 1
    el = time.perf_counter() - t0
    sample_bytes = 2.0 * float(ctx.sum()) * work.HKV * work.D * work.k[0].element_size()
    return {"value": round(sample_bytes * n / el / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port_simd_openmp",
            "sample": f"all {work.B} sequences (all heads): {k.nbytes * 2 / 1e6:.0f} MB of {tag} K/V per call, "
                      f"{n} calls in {el:.1f} s"}


def host_info():
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    llc = _llc_bytes()
    return {"cpu": model, "nproc": os.cpu_count(), "threads_used": 16,
            "llc_MB_total": round(llc / 2**20, 1) if llc else None,
            "note": "CPU samples stream their whole K/V set each call; every set exceeds the last-level cache"}


def torch_sdpa_cpu(work, threads, seconds=3.0):
    """PyTorch SDPA on the gathered paged layout, on the host CPU (BASELINE CPU
    path 3), all of the workload's sequences (config 2: 805 MB of fp32 K/V per
    call, above the host's last-level cache)."""
    torch.set_num_threads(threads)
    ctx = int(work.ctx_host[0])
    idx = torch.from_numpy(work.bt_host.reshape(-1).astype(np.int64)).to(work.k[0].device)
    Bn = work.B
    k = work.k[0][idx].float().cpu().reshape(Bn, -1, work.HKV, work.D)[:, :ctx]
    v = work.v[0][idx].float().cpu().reshape(Bn, -1, work.HKV, work.D)[:, :ctx]
    q = work.q.float().cpu()[:, :, None, :]
    kt = k.permute(0, 2, 1, 3).repeat_interleave(work.H // work.HKV, 1).contiguous()
    vt = v.permute(0, 2, 1, 3).repeat_interleave(work.H // work.HKV, 1).contiguous()
    del k, v
    torch.nn.functional.scaled_dot_product_attention(q, kt, vt, scale=work.scale)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds or n < 3:
        torch.nn.functional.scaled_dot_product_attention(q, kt, vt, scale=work.scale)
        n += 1
    el = time.perf_counter() - t0
    sample_bytes = 2.0 * Bn * float(ctx) * work.HKV * work.D * work.k[0].element_size()
    return {"value": round(sample_bytes * n / el / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "torch_sdpa_gathered",
            "sample": f"all {Bn} sequences gathered to fp32 ({(kt.nbytes + vt.nbytes) / 1e6:.0f} MB of K/V per "
                      f"call), {n} calls in {el:.1f} s; bytes counted at the GPU's {work.dtype} size"}


# --------------------------------------------------------------- workloads --

def make_c2(pa, pools):
    return DecodeWorkload(pa, B=64, H=12, HKV=12, D=64, BS=16, ctx=[2048] * 64, dtype=torch.float16,
                          pools=pools, seed=2, name="decode_c2")


def make_c2_scattered(pa, sets):
    """Config 2 over one pool of `sets` x the batch's 8192 pages (at least 4x:
    2.4 GB of K and V at 6 sets), each step's block tables a disjoint random
    draw from the whole pool: the same bytes per step and the same number of
    rotated sets as the headline, whose pools each hold exactly one batch."""
    sets = max(4, sets)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(22)
    nb = sets * 64 * (2048 // 16)
    k = torch.randn((nb, 16, 12, 64), generator=g, device=dev, dtype=torch.float32).half()
    v = torch.randn((nb, 16, 12, 64), generator=g, device=dev, dtype=torch.float32).half()
    return ScatteredWorkload(pa, (k, v), B=64, ctx=2048, seed=2, name="decode_c2_scattered")


def make_c2_fp32io(pa, pools):
    """Config 2 with the reference's operator dtypes: fp32 q and fp32 out over
    the fp16 cache (kernels/paged_attn_v3.cu:40,130,220-221)."""
    return DecodeWorkload(pa, B=64, H=12, HKV=12, D=64, BS=16, ctx=[2048] * 64, dtype=torch.float16,
                          pools=pools, seed=2, name="decode_c2_fp32io", q_dtype=torch.float32,
                          out_dtype=torch.float32)


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
    """(ms, kernel ms, record), or (None, None, FAILED record) when the check fails."""
    chk, kernels = check_decode(work)
    if not chk["ok"]:
        return None, None, failed_record(work.name, chk, kernels)
    ms, kms, reps = timed(work, steps, warmup)
    gbs = work.bytes / (ms * 1e-3) / 1e9
    return ms, kms, {
        "workload": work.name, "value": round(gbs, 1), "unit": "GB/s",
        "frac_of_8TBs": round(gbs / PEAK_HBM_GBS, 4), "ms_per_step": round(ms, 5), "repeats_ms": reps,
        "kernel_ms": round(kms, 5), "tokens_per_s": round(work.B / (ms * 1e-3), 1),
        "bytes_per_step": int(work.bytes), "split": work.split,
        "pools": work.pools, "footprint_GB": round(work.footprint_gb(), 2),
        "kernels": kernels, "check": chk,
    }


# The reference's v3 per-call times at the sweep's points, NVIDIA GB10
# (results/c000-20260901-225701-verify/{cold,hot}_b{B}_c{ctx}.txt:19; the
# "hot" points' working sets already exceed GB10's 24 MiB L2; b64_c2048 from
# docs/REPORT.md:124, 402.65 MB / 231.3 GB/s; b64_c4096 from docs/REPORT.md:125,
# 805.3 MB / 227.6 GB/s).
SWEEP_REF_US = {(1, 512): (21.7, "cold_b1_c512.txt:19"), (1, 2048): (34.4, "cold_b1_c2048.txt:19"),
                (4, 512): (30.5, "cold_b4_c512.txt:19"), (4, 2048): (120.5, "cold_b4_c2048.txt:19"),
                (16, 512): (116.7, "cold_b16_c512.txt:19"), (16, 2048): (464.2, "hot_b16_c2048.txt:19"),
                (64, 512): (471.5, "hot_b64_c512.txt:19"), (64, 2048): (1740.8, "docs/REPORT.md:124"),
                (128, 512): (907.8, "hot_b128_c512.txt:19"),
                (64, 4096): (3538.2, "docs/REPORT.md:125")}


def graph_us_per_call(work, calls):
    """GPU time per call with host launch cost removed: `calls` consecutive
    steps (rotating block-table sets) captured in one HIP graph, replayed."""
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(calls):
            work.launch(i, s.cuda_stream)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(g):
        st = torch.cuda.current_stream().cuda_stream
        for i in range(calls):
            work.launch(i, st)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 10
    t0.record()
    for _ in range(reps):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) * 1e3 / (reps * calls)


def _time_calls(fn, steps, warmup=5):
    """Median over REPEATS of the mean time (ms) of `steps` back-to-back fn(i)
    (i indexes the rotating block-table sets), HIP events on the launch stream."""
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    reps, n = [], warmup
    for _ in range(REPEATS):
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for i in range(steps):
            fn(n + i)
        t1.record(stream)
        torch.cuda.synchronize()
        reps.append(t0.elapsed_time(t1) / steps)
        n += steps
    return float(np.median(reps))


def sweep_legs(w, steps):
    """The paths the reference prints beside v3 at each sweep point
    (results/c000-20260901-225701-verify/cold_b16_c512.txt:15-19), timed on
    the same rotating block-table sets, each behind its correctness check:
    v1 and v2 (paged_attention, paged_attention_v2: one partition per
    (sequence, head unit)), and on the GPU through torch the pages gathered
    into a dense [B, H, ctx, D] layout then attended densely (fp32 scores,
    softmax, weighted sum) or by torch's fused SDPA (flash / memory-efficient
    backends only; fp16 operands made contiguous)."""
    import oracle
    legs = {}
    sp = torch.cuda.current_stream().cuda_stream
    for name, entry in (("v1", "paged_attention"), ("v2", "paged_attention_v2")):
        chk, kern = check_decode(w, entry=name)
        leg = {"check_ok": chk["ok"], "max_abs": chk["max_abs"], "kernels": kern}
        if chk["ok"]:
            f = getattr(w.L, entry)

            def call(i, f=f):
                if f(*w.args[i % w.pools], w.scale, sp) != 0:
                    raise RuntimeError(w.pa.last_error())
            us = _time_calls(call, steps) * 1e3
            leg.update(us_per_call=round(us, 2), GBs=round(w.bytes / (us * 1e-6) / 1e9, 1))
        legs[name] = leg
    B, H, D, BS = w.B, w.H, w.D, w.BS
    ctx = int(w.ctx_host[0])
    pages = -(-ctx // BS)
    q16 = w.q.view(B, H, 1, D)
    from torch.nn.attention import SDPBackend, sdpa_kernel

    def gathered(i):
        idx = w.bt[i % w.pools][:, :pages].reshape(-1).long()
        kg = w.k[0].index_select(0, idx).view(B, pages * BS, H, D)[:, :ctx]
        vg = w.v[0].index_select(0, idx).view(B, pages * BS, H, D)[:, :ctx]
        return kg, vg

    def dense(i):
        kg, vg = gathered(i)
        kt = kg.permute(0, 2, 3, 1).float().contiguous()  # [B, H, D, ctx]
        vt = vg.permute(0, 2, 1, 3).float().contiguous()  # [B, H, ctx, D]
        p = torch.softmax(torch.matmul(q16.float(), kt) * w.scale, dim=-1)
        return torch.matmul(p, vt).view(B, H, D)

    def sdpa(i):
        kg, vg = gathered(i)
        kt = kg.permute(0, 2, 1, 3).contiguous()
        vt = vg.permute(0, 2, 1, 3).contiguous()
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return torch.nn.functional.scaled_dot_product_attention(q16, kt, vt, scale=w.scale).view(B, H, D)

    ctxh = w.ctx_host
    seqs = sorted({0, B - 1})
    k, v, bts = _gather_pages(w.k[0], w.v[0], w.bt_host[seqs], ctxh[seqs], BS)
    want = oracle.decode(w.q[seqs].float().cpu().numpy(), k, v, bts, ctxh[seqs], w.scale, "f32")
    for name, fn in (("gather_dense_torch", dense), ("gather_sdpa_torch", sdpa)):
        try:
            got = fn(0)
        except RuntimeError as e:  # no fused SDPA backend for this shape / device
            legs[name] = {"unavailable": str(e).splitlines()[0][:160]}
            continue
        torch.cuda.synchronize()
        chk = _compare(got[seqs].float().cpu().numpy(), want, f"sequences {seqs} vs oracle.decode")
        leg = {"check_ok": chk["ok"], "max_abs": chk["max_abs"]}
        if chk["ok"]:
            us = _time_calls(fn, max(5, steps // 4), 2) * 1e3
            leg.update(us_per_call=round(us, 2), GBs=round(w.bytes / (us * 1e-6) / 1e9, 1))
        legs[name] = leg
    return legs


SWEEP_POINTS = [(B, c) for B in (1, 4, 16, 64, 128) for c in (512, 2048)] + [(64, 4096)]


def sweep_records(pa, steps):
    """The reference's small-batch cold sweep, B in {1,4,16,64,128} x ctx in
    {512,2048}, and its 805 MB point B=64 ctx=4096 (docs/REPORT.md:125); v3
    timed as whole calls and in a graph, v1 / v2 / torch paths beside it."""
    dev = torch.device("cuda:0")
    BS, H, D = 16, 12, 64
    blk_bytes = BS * H * D * 2
    nb = max(int(1.2e9 // (2 * blk_bytes)), 2 * 128 * 2048 // BS)  # >= 4x the Infinity Cache; 2 sets of the largest
    g = torch.Generator(device=dev)
    g.manual_seed(71)
    k = torch.randn((nb, BS, H, D), generator=g, device=dev, dtype=torch.float32).half()
    v = torch.randn((nb, BS, H, D), generator=g, device=dev, dtype=torch.float32).half()
    out = []
    for B, ctx in SWEEP_POINTS:
        w = SweepWorkload(pa, (k, v), B=B, ctx=ctx, seed=B * 10000 + ctx)
        log(f"bench: sweep B={B} ctx={ctx} ({w._sets} block-table sets, {w.footprint_gb():.2f} GB)")
        chk, kernels = check_decode(w)
        if not chk["ok"]:
            out.append(failed_record(w.name, chk, kernels))
            continue
        w.split = False  # time whole calls (partition + reduce)
        ms, _, _ = timed(w, max(steps, 50), 10)
        # The graph's calls cover >= 1.1 GB of distinct pages, so its replays stay cold too.
        gus = graph_us_per_call(w, min(w._sets, max(4, -(-int(1.1e9) // int(w.bytes))), 1024))
        ref_us, ref_src = SWEEP_REF_US.get((B, ctx), (None, None))
        us = ms * 1e3
        rec = {"workload": w.name, "batch": B, "context_len": ctx, "us_per_call": round(us, 2),
               "GBs": round(w.bytes / (us * 1e-6) / 1e9, 1),
               "frac_of_8TBs": round(w.bytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
               "us_per_call_graph": round(gus, 2),
               "GBs_graph": round(w.bytes / (gus * 1e-6) / 1e9, 1),
               "frac_of_8TBs_graph": round(w.bytes / (gus * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
               "bytes_per_call": int(w.bytes), "split": w.ws_bytes > 0, "kernels": kernels,
               "block_table_sets": w._sets, "footprint_GB": round(w.footprint_gb(), 2), "check": chk}
        if ref_us:
            rec["reference_gb10_us"] = ref_us
            rec["reference_source"] = "results/c000-20260901-225701-verify/" + ref_src \
                if ref_src.endswith(":19") else ref_src
        log(f"bench: sweep B={B} ctx={ctx}: v1, v2, torch gather paths")
        rec["beside_v3"] = sweep_legs(w, max(20, steps // 2))
        out.append(rec)
        del w
    return out


def c2_split_records(pa, pools, steps):
    """Config 2 through an explicit split: the reference's own count
    (choose_num_splits on its 48-SM GB10: 64) and the fastest of a few
    explicit counts, each timed as the API call the reference makes
    (paged_attention_v3 with num_splits: partition + reduce, or the fused
    one-launch form where the plan allows it).  The reference's count is
    also timed as two launches (pa_v3_partition, then pa_v3_reduce) with the
    partition kernel and the reduce timed apart."""
    recs = []
    for ns in (64, 2, 4, 8, 16):
        w = DecodeWorkload(pa, B=64, H=12, HKV=12, D=64, BS=16, ctx=[2048] * 64, dtype=torch.float16,
                           pools=pools, seed=2, name=f"decode_c2_split{ns}", num_splits=ns)
        log(f"bench: {w.name}")
        w.split = False  # one call, as the reference's v3 entry point
        ms, kms, rec = decode_record(w, max(20, steps), 5)
        if ms is not None:
            rec["num_splits"] = ns
            rec["fused"] = "reduce_kernel" not in rec["kernels"]
            if ns == 64:
                w.split = True
                ms2, kms2, rec2 = decode_record(w, max(20, steps), 5)
                if ms2 is not None:
                    rec["two_launch"] = {"value": rec2["value"], "unit": "GB/s", "ms_per_step": rec2["ms_per_step"],
                                         "partition_kernel_ms": round(kms2, 5), "reduce_ms": round(w.reduce_ms, 5),
                                         "partition_kernel_GBs": round(w.bytes / (kms2 * 1e-3) / 1e9, 1)}
        recs.append(rec)
        del w
    ok = [r for r in recs[1:] if r.get("value")]
    best = max(ok, key=lambda r: r["value"]) if ok else None
    return [recs[0]] + ([dict(best, workload="decode_c2_split_best")] if best else [])


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
    chk, kernels = check_prefill(work)
    if not chk["ok"]:
        return failed_record(work.name, chk, kernels)
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
        "kv_dtype": str(work.k.dtype).replace("torch.", ""), "kernels": kernels, "check": chk,
    }


def summarize(line):
    """Every workload of the line in a few numbers: [value, unit, fraction of
    its roofline, ms per step] (decode: of 8 TB/s; prefill: of the 2.5 PFLOP/s
    dense peak); sweep points add the v1 / v2 / torch gather-dense / torch
    SDPA GB/s measured beside v3 (null when unavailable or failed)."""
    out = {line["config"]["workload"]: [line["value"], line["unit"], line["roofline"]["frac"], line["ms_per_step"]]}
    for r in line.get("also", []):
        name = r.get("workload")
        if not name or r.get("status") == "FAILED":
            if name:
                out[name] = "FAILED"
            continue
        if name.startswith("sweep_"):
            legs = r.get("beside_v3", {})
            out[name] = [r["GBs"], "GB/s", r["frac_of_8TBs"], round(r["us_per_call"] / 1e3, 5),
                         {k: legs.get(k, {}).get("GBs") for k in ("v1", "v2", "gather_dense_torch",
                                                                  "gather_sdpa_torch")}]
        elif "value" in r and "unit" in r:
            frac = r.get("frac_of_8TBs", r.get("frac_of_hbm_peak", r.get("frac_of_mfma_peak")))
            out[name] = [r["value"], r["unit"], frac, r.get("ms_per_step")]
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--pools", type=int, default=6, help="rotated KV pools (config 2)")
    ap.add_argument("--workload", default="decode_c2",
                    choices=["decode_c2", "decode_c2_fp32io", "decode_c3", "decode_c5", "decode_c2_fp8", "decode_c3_fp8", "decode_gqa8",
                             "decode_c2_split", "decode_c2_scattered", "sweep", "prefill_c4a", "prefill_c4b", "prefill_ref_chunk", "prefill_c4b_fp8",
                             "write_kv_c4a", "write_kv_c4b", "write_kv_c4b_fp8", "call_overhead", "mixed_c2", "copy_calib"],
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
            work = PrefillWorkload(pa, BS=16, name=w, **PREFILL_CFG[w])
            print(json.dumps(prefill_record(work, args.steps, args.warmup)), flush=True)
        elif w == "sweep":
            for rec in sweep_records(pa, args.steps):
                print(json.dumps(rec), flush=True)
        elif w == "decode_c2_split":
            for rec in c2_split_records(pa, args.pools, args.steps):
                print(json.dumps(rec), flush=True)
        elif w == "mixed_c2":
            print(json.dumps(mixed_record(pa, args.steps, args.warmup)), flush=True)
        elif w == "call_overhead":
            print(json.dumps(call_overhead(pa)), flush=True)
        elif w.startswith("write_kv"):
            work = WriteWorkload(pa, BS=16, name=w, **WRITE_CFG[w])
            print(json.dumps(write_record(work, args.steps, args.warmup)), flush=True)
        else:
            work = {"decode_c2": lambda: make_c2(pa, args.pools), "decode_c3": lambda: make_c3(pa, 2),
                    "decode_c2_fp32io": lambda: make_c2_fp32io(pa, args.pools),
                    "decode_c2_scattered": lambda: make_c2_scattered(pa, args.pools),
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
    base = {
        "metric": METRIC, "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "higher_is_better": True, "scaling": "weak", "dtype": "f16",
        "data": "synthetic N(0,1), seeded; random-permutation block tables",
        "config": {"workload": "decode_c2", "batch": 64, "context_len": 2048, "heads": 12,
                   "kv_heads": 12, "head_dim": 64, "block_size": 16, "kv_dtype": "f16",
                   "q_dtype": "f16", "out_dtype": "f16", "entry": "paged_attention_v3(num_splits=0)",
                   "pools": work.pools, "working_set_GB": round(work.footprint_gb(), 2),
                   "split": work.split},
    }
    if ms is None:  # failed its correctness check: no number is published
        print(json.dumps({**base, "value": None, "vs_baseline": None, "status": "FAILED", "check": rec["check"]}),
              flush=True)
        sys.exit(1)
    achieved = work.bytes / (kms * 1e-3) / 1e9
    log(f"bench: {rec['value']} GB/s per step, kernel {kms * 1e3:.1f} us")
    kernel = rec["kernels"].split("; ")[0]
    traffic, traffic_src = traffic_from_profiles("decode_c2", kernel, work.bytes)
    line = {
        **base, "value": rec["value"], "ms_per_step": round(ms, 5),
        "timing": f"median of {REPEATS} repeats of {args.steps} steps", "repeats_ms": rec["repeats_ms"],
        "vs_baseline": round(rec["value"] / REF_GB10_C2_GBS, 2),
        "baseline": {"value": REF_GB10_C2_GBS, "unit": "GB/s", "frac_of_its_peak": 0.847,
                     "what": "reference v3 split decode, B=64 ctx=2048 fp16 (this config), on NVIDIA GB10 "
                             "(273 GB/s LPDDR5X): different hardware, compare frac_of_peak",
                     "source": "docs/REPORT.md:124"},
        "frac_of_peak": rec["frac_of_8TBs"],
        "tokens_per_s": rec["tokens_per_s"],
        "check": rec["check"],
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": traffic, "traffic_source": traffic_src,
                     "kernel": kernel, "kernels_per_step": rec["kernels"],
                     "kernel_ms": round(kms, 5), "bytes_per_launch": int(work.bytes)},
    }
    log("bench: cpu baseline (reference cpu_reference, 1 thread)")
    line["cpu_baseline"] = cpu_baseline(work, args.cpu_seconds)
    line["cpu_extra"] = [simd_cpu(work, 16), torch_sdpa_cpu(work, 16)]
    line["host"] = host_info()
    del work

    also = []
    if not args.no_also:
        log("bench: config 2 through the explicit split + LSE reduce")
        also += c2_split_records(pa, args.pools, max(20, args.steps // 4))
        for make in (lambda: make_c2_scattered(pa, args.pools), lambda: make_c2_fp32io(pa, args.pools),
                     lambda: make_c3(pa, 2), lambda: make_c5(pa),
                     lambda: make_c2_fp8(pa, args.pools),
                     lambda: make_c3_fp8(pa, 2), lambda: make_gqa8(pa, 2)):
            w = make()
            log(f"bench: {w.name}")
            rec = decode_record(w, max(20, args.steps // 4), 5)[2]
            if rec.get("value") is not None:
                rec["traffic"], rec["traffic_source"] = traffic_from_profiles(
                    w.name, rec["kernels"].split("; ")[0], w.bytes)
            if w.name == "decode_c5":
                rec["k_base_offset_elements"] = int(w.k_offset_elems)
            if isinstance(w, ScatteredWorkload):
                rec["pool_GB"] = round(w.pool_gb(), 2)
            also.append(rec)
            del w
        for name, kw in PREFILL_CFG.items():
            log(f"bench: {name}")
            w = PrefillWorkload(pa, BS=16, name=name, **kw)
            rec = prefill_record(w, max(20, args.steps // 4), 5)
            if name == "prefill_ref_chunk":
                rec["reference_gb10_us"] = 6956.9
                rec["reference_source"] = "results/c001-20260901-223111/bench_prefill.txt:42 (WMMA kernel)"
            also.append(rec)
            del w
        for name, kw in WRITE_CFG.items():
            log(f"bench: {name}")
            w = WriteWorkload(pa, BS=16, name=name, **kw)
            also.append(write_record(w, max(20, args.steps // 4), 5))
            del w
        log("bench: mixed decode + prefill batch")
        also.append(mixed_record(pa, max(20, args.steps // 4), 5))
        log("bench: small-batch cold sweep")
        also += sweep_records(pa, max(50, args.steps // 4))
        log("bench: per-call host overhead")
        also.append(call_overhead(pa))
    line["also"] = also
    line["summary"] = summarize(line)  # last key: survives a truncated tail of this line
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
