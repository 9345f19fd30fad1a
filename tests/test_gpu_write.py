"""GPU parity of pa_write_kv (the KV-cache write) against the CPU oracle's
restatement, bit for bit: every source/cache type pair, int32/int64 slot
mappings with padding slots, the engine's head-major [n_head, ctx, D] layer
slices as strided sources, a pool layer past 2^31 elements, and a
write -> attend round trip through the decode and prefill kernels."""
import numpy as np
import pytest
import torch

import oracle
from _helpers import close, to_dev, to_host

pytestmark = pytest.mark.gpu

TAGS = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


def host_bits(t: torch.Tensor) -> np.ndarray:
    """Device tensor -> numpy array in the oracle's storage convention (bf16 as uint16 bits)."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("cache_dt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("src_dt", [torch.float32, torch.float16, torch.bfloat16])
def test_write_kv_bit_exact(pa, dev, src_dt, cache_dt, slot_dtype):
    g = torch.Generator().manual_seed(3)
    NB, BS, HKV, D, T = 37, 16, 4, 64, 301
    key = (torch.randn(T, HKV, D, generator=g) * 4).to(src_dt)
    val = (torch.randn(T, HKV, D, generator=g) * 4).to(src_dt)
    slots = torch.randperm(NB * BS, generator=g)[:T]
    slots[::17] = -1  # padding tokens
    kc = torch.randn(NB, BS, HKV, D, generator=g).to(cache_dt)
    vc = torch.randn(NB, BS, HKV, D, generator=g).to(cache_dt)
    want_k, want_v = host_bits(kc).copy(), host_bits(vc).copy()
    oracle.write_kv(want_k, want_v, host_bits(key), host_bits(val), slots.numpy(), TAGS[cache_dt], TAGS[src_dt])
    kd, vd = kc.to(dev), vc.to(dev)
    pa.write_kv(kd, vd, key.to(dev), val.to(dev), slots.to(slot_dtype).to(dev))
    assert np.array_equal(host_bits(kd), want_k)
    assert np.array_equal(host_bits(vd), want_v)


def test_write_kv_engine_layout_and_pool_views(pa, dev):
    """write_kv_blocks: one sequence's [n_layer, n_head, ctx, D] fp32 K/V into a
    [L, 2, NB, BS, HKV, D] fp16 pool at its block ids from a start position."""
    L, NB, BS, HKV, D, ctx, start = 3, 40, 16, 4, 32, 75, 21
    rng = np.random.default_rng(8)
    k = rng.standard_normal((L, HKV, ctx, D)).astype(np.float32)
    v = rng.standard_normal((L, HKV, ctx, D)).astype(np.float32)
    block_ids = rng.permutation(NB)[:(start + ctx + BS - 1) // BS]
    pool = torch.zeros(L, 2, NB, BS, HKV, D, dtype=torch.float16, device=dev)
    pa.write_kv_blocks(pool, block_ids, start, k, v)
    want = np.zeros((L, 2, NB, BS, HKV, D), np.float16)
    pos = np.arange(start, start + ctx)
    slots = block_ids[pos // BS] * BS + pos % BS
    for layer in range(L):
        oracle.write_kv(want[layer, 0], want[layer, 1], k[layer].transpose(1, 0, 2),
                        v[layer].transpose(1, 0, 2), slots, "f16", "f32")
    assert np.array_equal(pool.cpu().numpy(), want)


def test_write_kv_past_2_31_elements(pa, dev):
    """Layer 1 of the pool starts past 2^31 elements: 64-bit slot offsets."""
    NB, BS, HKV, D = 65600, 16, 8, 128
    pool = torch.zeros(2, 2, NB, BS, HKV, D, dtype=torch.bfloat16, device=dev)
    assert pool[1, 0].storage_offset() > 2 ** 31
    T = 40
    key = torch.randn(T, HKV, D, device=dev).to(torch.bfloat16)
    val = torch.randn(T, HKV, D, device=dev).to(torch.bfloat16)
    slots = torch.arange(NB * BS - T, NB * BS, device=dev)
    pa.write_kv(pool[1, 0], pool[1, 1], key, val, slots)
    assert torch.equal(pool[1, 0].reshape(-1, HKV, D)[-T:], key)
    assert torch.equal(pool[1, 1].reshape(-1, HKV, D)[-T:], val)
    assert not pool[0].any() and not pool[1, 0].reshape(-1, HKV, D)[:-T].any()
    del pool
    torch.cuda.empty_cache()


@pytest.mark.parametrize("kv", ["f16", "bf16"])
def test_write_then_attend(pa, dev, kv):
    """A prompt's K/V written into an empty paged pool, then attended causally
    (MFMA prefill) and by a decode step, equals the oracle on the oracle's
    write of the same data."""
    B, S, H, HKV, D, BS = 2, 96, 4, 2, 64, 16
    rng = np.random.default_rng(12)
    MB = S // BS
    NB = B * MB + 3
    bt = rng.permutation(NB)[:B * MB].reshape(B, MB).astype(np.int32)
    k_new = rng.standard_normal((B * S, HKV, D)).astype(np.float32)
    v_new = rng.standard_normal((B * S, HKV, D)).astype(np.float32)
    slots = np.concatenate([bt[b][np.arange(S) // BS] * BS + np.arange(S) % BS for b in range(B)])
    kd = torch.zeros(NB, BS, HKV, D, dtype=torch.float16 if kv == "f16" else torch.bfloat16, device=dev)
    vd = torch.zeros_like(kd)
    pa.write_kv(kd, vd, torch.from_numpy(k_new).to(dev), torch.from_numpy(v_new).to(dev),
                torch.from_numpy(slots).to(dev))
    kh = np.zeros((NB, BS, HKV, D), oracle.NP_OF[kv])
    vh = np.zeros_like(kh)
    oracle.write_kv(kh, vh, k_new, v_new, slots, kv, "f32")
    assert np.array_equal(host_bits(kd), kh) and np.array_equal(host_bits(vd), vh)
    ctx = np.full(B, S, np.int32)
    q = rng.standard_normal((B, S, H, D)).astype(np.float32)
    got = to_host(pa.paged_attention_prefill_wmma(torch.from_numpy(q).to(dev), kd, vd, torch.from_numpy(bt).to(dev),
                                                  torch.from_numpy(ctx).to(dev), 0.125))
    close(got, oracle.prefill(q, kh, vh, bt, ctx, 0.125, kv))
    qd = q[:, -1]
    got = to_host(pa.paged_attention_v3(torch.from_numpy(qd).to(dev), kd, vd, torch.from_numpy(bt).to(dev),
                                        torch.from_numpy(ctx).to(dev), 0.125, 0))
    close(got, oracle.decode(qd, kh, vh, bt, ctx, 0.125, kv))
