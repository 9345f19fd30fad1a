"""paged_attention_v3_noalloc through the C-ABI: the same results as
paged_attention_v3 with a caller workspace, bit for bit (same plan, same
kernels), on two calls in a row whose second input is smaller, and a clear
PA_ERR_WORKSPACE (with the output untouched) when a split needs more than the
fixed scratch; and the entry recorded into a HIP graph and replayed on
changed inputs."""
import ctypes as C

import numpy as np
import pytest
import torch

from _helpers import close, decode_case, dev_inputs, to_host

import oracle

pytestmark = pytest.mark.gpu


def _noalloc(pa, out, q, k, v, bt, ctx, scale, num_splits):
    V = pa.view
    views = [V(out), V(q), V(k), V(v), V(bt), V(ctx)]
    sp = torch.cuda.current_stream(q.device).cuda_stream
    return pa.lib().paged_attention_v3_noalloc(*[C.byref(x) for x in views], float(scale), int(num_splits), sp)


def _with_workspace(pa, out, q, k, v, bt, ctx, scale, num_splits):
    return pa.paged_attention_v3(q, k, v, bt, ctx, scale, num_splits, out=out)


def test_noalloc_matches_workspace_entry_twice(pa, dev):
    cases = [
        # GQA-4 bf16, ragged contexts long enough for the auto plan to split.
        (dict(B=8, H=32, HKV=8, D=128, BS=16, ctx=[1000, 9000, 1, 4097, 0, 3000, 8191, 77], seed=31,
              kv="bf16", q="bf16"), 0, torch.bfloat16),
        # The smaller second call: MHA fp16, the reference partition with 7 splits.
        (dict(B=3, H=12, HKV=12, D=64, BS=16, ctx=[300, 17, 96], seed=32, kv="f16", q="f16"), 7,
         torch.float16),
    ]
    for spec, ns, odt in cases:
        spec = dict(spec)
        B, H, HKV, D, BS, ctx = (spec.pop(x) for x in ("B", "H", "HKV", "D", "BS", "ctx"))
        inp = decode_case(B, H, HKV, D, BS, ctx, **spec)
        q, k, v, bt, ctxd = dev_inputs(inp, dev)
        scale = 1.0 / np.sqrt(D)
        assert pa.workspace_size(q, k, bt, ns) > 0, "the case must exercise the split scratch"
        print(f"noalloc case B={B} H={H} HKV={HKV} D={D} splits={ns}", flush=True)
        got = torch.full(q.shape, float("nan"), dtype=odt, device=dev)
        rc = _noalloc(pa, got, q, k, v, bt, ctxd, scale, ns)
        assert rc == 0, pa.last_error()
        ref = torch.empty(q.shape, dtype=odt, device=dev)
        _with_workspace(pa, ref, q, k, v, bt, ctxd, scale, ns)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        want = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], scale, inp["kv"])
        close(to_host(got), want)


def test_noalloc_rejects_oversized_split(pa, dev):
    """A split whose partials exceed the fixed scratch is refused before any device work."""
    B, H, D = 256, 64, 256
    q = torch.zeros((B, H, D), dtype=torch.float16, device=dev)
    k = torch.zeros((1, 16, H, D), dtype=torch.float16, device=dev)
    bt = torch.zeros((B, 1), dtype=torch.int32, device=dev)
    ctx = torch.full((B,), 16, dtype=torch.int32, device=dev)
    need = pa.workspace_size(q, k, bt, 64)
    assert need > (64 << 20)
    out = torch.full((B, H, D), 7.0, dtype=torch.float16, device=dev)
    rc = _noalloc(pa, out, q, k, k, bt, ctx, 0.1, 64)
    assert rc == 3, rc  # PA_ERR_WORKSPACE
    assert "paged_attention_v3_noalloc" in pa.last_error() and str(need) in pa.last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


def test_noalloc_graph_capture_and_replay(pa, dev):
    """paged_attention_v3_noalloc recorded into a HIP graph (after one eager
    call on the capture stream, which does the per-device set-up: scratch
    address, CU count), replayed three times after q and context_lens change
    in place, with eager work and synchronisation between replays: every
    replay equals eager paged_attention_v3 with a workspace, bit for bit."""
    inp = decode_case(6, 32, 8, 128, 16, [900, 4000, 17, 2500, 1, 3100], seed=41, kv="bf16", q="bf16")
    q, k, v, bt, ctx = dev_inputs(inp, dev)
    scale = 1.0 / np.sqrt(128)
    assert pa.workspace_size(q, k, bt, 0) > 0, "the auto plan must split (the scratch is in use)"
    out = torch.empty_like(q)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        assert _noalloc(pa, out, q, k, v, bt, ctx, scale, 0) == 0, pa.last_error()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = _noalloc(pa, out, q, k, v, bt, ctx, scale, 0)
    assert rc == 0, pa.last_error()
    gen = torch.Generator(device=dev)
    gen.manual_seed(42)
    maxctx = bt.shape[1] * k.shape[1]
    for i in range(3):
        print(f"noalloc graph replay {i}", flush=True)
        q.copy_(torch.randn(q.shape, generator=gen, device=dev).to(q.dtype))
        ctx.copy_(torch.randint(0, maxctx + 1, ctx.shape, generator=gen, device=dev).to(ctx.dtype))
        ref = torch.empty_like(out)
        _with_workspace(pa, ref, q, k, v, bt, ctx, scale, 0)
        out.fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), i


def test_noalloc_fused_explicit_split_and_graph(pa, dev):
    """The reference's split count over an MHA grid that fills the GPU runs
    fused (one launch, the partials kept in registers, the fixed scratch not
    written): the allocation-free entry equals the workspace entry bit for
    bit, eagerly and recorded into a HIP graph replayed on changed q and
    context lengths."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    H, D, BS, MB, ns = 8, 64, 16, 64, 64
    B = -(-cus // H)
    rng = np.random.default_rng(5)
    ctxs = rng.integers(1, MB * BS + 1, size=B).tolist()
    inp = decode_case(B, H, H, D, BS, ctxs, seed=51, kv="f16", q="f16", mb=MB)
    q, k, v, bt, ctx = dev_inputs(inp, dev)
    scale = 1.0 / np.sqrt(D)
    out = torch.empty_like(q)
    ref = torch.empty_like(q)
    print(f"noalloc fused case B={B} H={H} D={D} splits={ns}", flush=True)
    assert _noalloc(pa, out, q, k, v, bt, ctx, scale, ns) == 0, pa.last_error()
    assert pa.last_launch() == "pa::decode_kernel<pa::KvF16, 64, 1, 1, 1>", pa.last_launch()
    _with_workspace(pa, ref, q, k, v, bt, ctx, scale, ns)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    close(to_host(out), oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], scale, "f16"))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = _noalloc(pa, out, q, k, v, bt, ctx, scale, ns)
    assert rc == 0, pa.last_error()
    gen = torch.Generator(device=dev)
    gen.manual_seed(52)
    for i in range(3):
        print(f"noalloc fused graph replay {i}", flush=True)
        q.copy_(torch.randn(q.shape, generator=gen, device=dev).to(q.dtype))
        ctx.copy_(torch.randint(0, MB * BS + 1, ctx.shape, generator=gen, device=dev).to(ctx.dtype))
        _with_workspace(pa, ref, q, k, v, bt, ctx, scale, ns)
        out.fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), i
