"""GPU parity of the torch.ops.gb10_attn operators (csrc/torch_ext.cpp): each
returns the oracle's result within tolerance and the same bits as the ctypes
mirror (the same kernels run), raises the reference's messages, and a
captured HIP graph of the v3 operator replays to the eager result."""
import numpy as np
import pytest
import torch

import oracle
from _helpers import close, decode_case, dev_inputs, to_host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["paged_attention", "paged_attention_v2", "paged_attention_v3"])
def test_decode_ops(pa, dev, name):
    ops = pa.torch_ops()
    inp = decode_case(3, 8, 2, 64, 16, [100, 37, 513], seed=31, kv="f16", q="f32")
    q, k, v, bt, ctx = dev_inputs(inp, dev)
    extra = (0,) if name == "paged_attention_v3" else ()
    got = getattr(ops, name)(q, k, v, bt, ctx, 0.125, *extra)
    assert got.dtype == torch.float32 and got.shape == q.shape
    mirror = getattr(pa, name)(q, k, v, bt, ctx, 0.125, *extra)
    assert torch.equal(got, mirror)
    close(to_host(got), oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.125, "f16"))


def test_v3_explicit_splits_and_chooser(pa, dev):
    ops = pa.torch_ops()
    inp = decode_case(2, 4, 4, 128, 16, [300, 64], seed=32, kv="bf16", q="bf16")
    q, k, v, bt, ctx = dev_inputs(inp, dev)
    want = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.1, "bf16")
    for s in (1, 3, 7):
        close(to_host(ops.paged_attention_v3(q, k, v, bt, ctx, 0.1, s)), want)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    for B, H, mc in ((64, 12, 2048), (1, 32, 32768), (4, 12, 512)):
        assert ops.choose_num_splits(B, H, mc) == oracle.choose_num_splits(B, H, mc, cus)


@pytest.mark.parametrize("name", ["paged_attention_prefill", "paged_attention_prefill_wmma"])
def test_prefill_ops(pa, dev, name):
    ops = pa.torch_ops()
    B, S, H, HKV, D, BS = 2, 70, 4, 2, 64, 16
    inp = oracle.paged_inputs(B, 1, HKV, D, BS, [70, 120], seed=33, kv_dtype="f16")
    q32 = np.random.default_rng(34).standard_normal((B, S, H, D), dtype=np.float32)
    qd = torch.from_numpy(q32).to(dev)
    _, k, v, bt, ctx = dev_inputs(dict(inp, qt="f32", kv="f16"), dev)
    got = getattr(ops, name)(qd, k, v, bt, ctx, 0.125)
    assert torch.equal(got, getattr(pa, name)(qd, k, v, bt, ctx, 0.125))
    close(to_host(got), oracle.prefill(q32, inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.125, "f16"))


def test_write_kv_op(pa, dev):
    ops = pa.torch_ops()
    g = torch.Generator().manual_seed(35)
    key = torch.randn(50, 2, 64, generator=g)
    val = torch.randn(50, 2, 64, generator=g)
    slots = torch.randperm(8 * 16, generator=g)[:50]
    slots[5] = -1
    kc = torch.zeros(8, 16, 2, 64, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    ops.write_kv(kc, vc, key.to(dev), val.to(dev), slots.to(dev))
    wk = np.zeros((8, 16, 2, 64), np.float16)
    wv = np.zeros_like(wk)
    oracle.write_kv(wk, wv, key.numpy(), val.numpy(), slots.numpy(), "f16", "f32")
    assert np.array_equal(kc.cpu().numpy(), wk) and np.array_equal(vc.cpu().numpy(), wv)


def test_write_kv_scaled_op(pa, dev):
    """torch.ops.gb10_attn.write_kv_scaled into an FP8 cache equals the oracle's scaled write."""
    ops = pa.torch_ops()
    g = torch.Generator().manual_seed(37)
    key = torch.randn(40, 2, 64, generator=g) * 5
    val = torch.randn(40, 2, 64, generator=g) * 5
    slots = torch.randperm(6 * 16, generator=g)[:40]
    kc = torch.zeros(6, 16, 2, 64, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    vc = torch.zeros_like(kc)
    ops.write_kv_scaled(kc, vc, key.to(dev), val.to(dev), slots.to(dev), 0.25, 0.02)
    wk = np.zeros((6, 16, 2, 64), np.uint8)
    wv = np.zeros_like(wk)
    oracle.write_kv(wk, wv, key.numpy(), val.numpy(), slots.numpy(), "fp8", "f32", k_scale=0.25, v_scale=0.02)
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), wk)
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), wv)


def test_prefill_wmma_scaled_op(pa, dev):
    """torch.ops.gb10_attn.paged_attention_prefill_wmma_scaled over an FP8 pool equals the Python mirror."""
    ops = pa.torch_ops()
    inp = decode_case(2, 4, 2, 64, 16, [70, 130], seed=41, kv="f32")
    k8 = torch.from_numpy(oracle.fp8_encode(inp["k"] / np.float32(0.05))).view(torch.float8_e4m3fn).to(dev)
    v8 = torch.from_numpy(oracle.fp8_encode(inp["v"] / np.float32(0.03))).view(torch.float8_e4m3fn).to(dev)
    q = torch.randn(2, 40, 4, 64, generator=torch.Generator().manual_seed(41)).to(dev)
    bt, ctx = torch.from_numpy(inp["bt"]).to(dev), torch.from_numpy(inp["ctx"]).to(dev)
    got = ops.paged_attention_prefill_wmma_scaled(q, k8, v8, bt, ctx, 0.125, 0.05, 0.03)
    want = pa.paged_attention_prefill_wmma(q, k8, v8, bt, ctx, 0.125, k_scale=0.05, v_scale=0.03)
    assert got.dtype == torch.float32 and torch.equal(got, want)


def test_reference_error_messages(pa, dev):
    ops = pa.torch_ops()
    inp = decode_case(1, 8, 4, 64, 16, [20], seed=36)
    q, k, v, bt, ctx = dev_inputs(inp, dev)
    with pytest.raises(RuntimeError, match="n_head must be divisible by n_kv_head"):
        ops.paged_attention_v3(q[:, :6].contiguous(), k, v, bt, ctx, 0.1, 0)
    inp = decode_case(1, 4, 4, 64, 16, [20], seed=36, kv="f32")
    q, k, v, bt, ctx = dev_inputs(inp, dev)
    with pytest.raises(RuntimeError, match="the MFMA path needs an fp16, bf16 or float8_e4m3fn KV cache"):
        ops.paged_attention_prefill_wmma(q[:, None], k, v, bt, ctx, 0.1)


def test_v3_op_graph_replay(pa, dev):
    """Captured once, replayed three times with eager work and synchronisation
    in between; every replay equals the eager result."""
    ops = pa.torch_ops()
    inp = decode_case(4, 8, 8, 64, 16, [700, 30, 1500, 256], seed=37, kv="f16", q="f16")
    q, k, v, bt, ctx = dev_inputs(inp, dev)
    eager = ops.paged_attention_v3(q, k, v, bt, ctx, 0.125, 0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.paged_attention_v3(q, k, v, bt, ctx, 0.125, 0)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.paged_attention_v3(q, k, v, bt, ctx, 0.125, 0)
    for i in range(3):
        out.fill_(float(i + 7))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
