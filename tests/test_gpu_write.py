"""GPU parity of pa_write_kv / pa_write_kv_scaled (the KV-cache write) against
the CPU oracle's restatement, bit for bit: every source/cache type pair (FP8
E4M3 caches over every fp16 bit pattern and the saturation edges), per-tensor
scales, int32/int64 slot mappings with padding slots, the engine's head-major
[n_head, ctx, D] layer slices as strided sources, a pool layer past 2^31
elements, and write -> attend round trips through the decode and prefill
kernels (FP8 through the scaled decode)."""
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


def _fp8_host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.uint8).numpy()


@pytest.mark.parametrize("cache", ["fp8", "f32"])
@pytest.mark.parametrize("scale", [1.0, 0.37, 3.7e-3, 12.5])
@pytest.mark.parametrize("src_dt", [torch.float16, torch.float32])
def test_write_kv_fp8_every_code_path(pa, dev, src_dt, scale, cache):
    """FP8 E4M3 (and, for the division alone, fp32) caches, bit for bit
    against the oracle: every fp16 bit pattern (all FP8 halfway points, the
    subnormal steps, NaN, infinities), and for fp32 sources values past 448 /
    464 / 480, fp32 subnormals, -0; unscaled and divided by a scale."""
    vals = np.arange(1 << 16, dtype=np.uint16).view(np.float16).astype(np.float32)
    if src_dt == torch.float32:
        extra = np.float32([447.9, 448, 455.9, 464, 464.1, 479.9, 480, 1e30, -1e30, 1e-40, -1e-40, -0.0,
                            2.0 ** -10, 3 * 2.0 ** -10, 5 * 2.0 ** -11, np.nan, -np.inf])
        rng = np.random.default_rng(9)
        vals = np.concatenate([vals, extra, (rng.standard_normal(4096) * 50).astype(np.float32)])
    HKV, D, BS = 1, 64, 16
    T = -(-vals.size // D)
    vals = np.concatenate([vals, np.zeros(T * D - vals.size, np.float32)]).reshape(T, HKV, D)
    NB = -(-T // BS) + 1
    key = torch.from_numpy(vals).to(src_dt)
    val = -key
    slots = torch.arange(T, dtype=torch.int64)
    if cache == "fp8":
        kc = torch.zeros(NB, BS, HKV, D, dtype=torch.uint8).view(torch.float8_e4m3fn).to(dev)
        bits = _fp8_host
    else:
        kc = torch.zeros(NB, BS, HKV, D, dtype=torch.float32, device=dev)
        bits = lambda t: t.detach().cpu().numpy().view(np.uint32)  # noqa: E731
    vc = torch.zeros_like(kc)
    tag = TAGS[src_dt]
    want_k = np.zeros((NB, BS, HKV, D), oracle.NP_OF[cache])
    want_v = np.zeros_like(want_k)
    oracle.write_kv(want_k, want_v, host_bits(key), host_bits(val), slots.numpy(), cache, tag,
                    k_scale=scale, v_scale=scale)
    pa.write_kv(kc, vc, key.to(dev), val.to(dev), slots.to(dev), k_scale=scale, v_scale=scale)
    if cache == "f32":  # NaN payloads aside, the quotients bit for bit
        want_k, want_v = want_k.view(np.uint32), want_v.view(np.uint32)
        nan_k, nan_v = np.isnan(want_k.view(np.float32)), np.isnan(want_v.view(np.float32))
        assert np.array_equal(np.isnan(bits(kc).view(np.float32)), nan_k)
        assert np.array_equal(bits(kc)[~nan_k], want_k[~nan_k]) and np.array_equal(bits(vc)[~nan_v], want_v[~nan_v])
    else:
        assert np.array_equal(bits(kc), want_k)
        assert np.array_equal(bits(vc), want_v)


@pytest.mark.parametrize("cache_dt", [torch.float8_e4m3fn, torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("src_dt", [torch.float32, torch.float16, torch.bfloat16])
def test_write_kv_scaled_bit_exact(pa, dev, src_dt, cache_dt):
    """pa_write_kv_scaled: the cache holds key / k_scale and value / v_scale
    (float32 division, then the cache type's rounding) for every source and
    cache type, padding slots skipped, int32 slots."""
    g = torch.Generator().manual_seed(21)
    NB, BS, HKV, D, T = 29, 16, 2, 128, 211
    key = (torch.randn(T, HKV, D, generator=g) * 6).to(src_dt)
    val = (torch.randn(T, HKV, D, generator=g) * 6).to(src_dt)
    slots = torch.randperm(NB * BS, generator=g)[:T].to(torch.int32)
    slots[::13] = -1
    ks, vs = 0.05, 3.7
    fp8 = cache_dt == torch.float8_e4m3fn
    ctag = "fp8" if fp8 else TAGS[cache_dt]
    kc = torch.zeros(NB, BS, HKV, D, dtype=torch.uint8).view(torch.float8_e4m3fn) if fp8 \
        else torch.randn(NB, BS, HKV, D, generator=g).to(cache_dt)
    vc = kc.clone()
    bits = _fp8_host if fp8 else host_bits
    want_k, want_v = bits(kc).copy(), bits(vc).copy()
    oracle.write_kv(want_k, want_v, host_bits(key), host_bits(val), slots.numpy(), ctag, TAGS[src_dt],
                    k_scale=ks, v_scale=vs)
    kd, vd = kc.to(dev), vc.to(dev)
    pa.write_kv(kd, vd, key.to(dev), val.to(dev), slots.to(dev), k_scale=ks, v_scale=vs)
    assert np.array_equal(bits(kd), want_k)
    assert np.array_equal(bits(vd), want_v)


def test_fp8_write_then_decode(pa, dev):
    """bf16 K/V quantised into an FP8 pool with per-tensor scales, then decoded
    through the scaled v3 entry point with the same scales: equal to the oracle
    on the dequantised cache."""
    B, H, HKV, D, BS = 4, 16, 4, 128, 16
    ctx = np.int32([1000, 77, 513, 2048])
    rng = np.random.default_rng(14)
    MB = int(-(-ctx.max() // BS))
    NB = B * MB + 2
    bt = rng.permutation(NB)[:B * MB].reshape(B, MB).astype(np.int32)
    slots = np.concatenate([bt[b][np.arange(c) // BS] * BS + np.arange(c) % BS for b, c in enumerate(ctx)])
    T = slots.size
    key = torch.from_numpy(rng.standard_normal((T, HKV, D)).astype(np.float32)).to(torch.bfloat16)
    val = torch.from_numpy(rng.standard_normal((T, HKV, D)).astype(np.float32)).to(torch.bfloat16)
    ks, vs = 1.0 / 32, 1.0 / 48
    kc = torch.zeros(NB, BS, HKV, D, dtype=torch.uint8).view(torch.float8_e4m3fn).to(dev)
    vc = torch.zeros_like(kc)
    pa.write_kv(kc, vc, key.to(dev), val.to(dev), torch.from_numpy(slots).to(dev), k_scale=ks, v_scale=vs)
    kh, vh = np.zeros((NB, BS, HKV, D), np.uint8), np.zeros((NB, BS, HKV, D), np.uint8)
    oracle.write_kv(kh, vh, host_bits(key), host_bits(val), slots, "fp8", "bf16", k_scale=ks, v_scale=vs)
    assert np.array_equal(_fp8_host(kc), kh) and np.array_equal(_fp8_host(vc), vh)
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    scale = 1.0 / np.sqrt(D)
    want = oracle.decode(q, oracle.fp8_decode(kh) * np.float32(ks), oracle.fp8_decode(vh) * np.float32(vs),
                         bt, ctx, scale, "f32")
    got = to_host(pa.paged_attention_v3(torch.from_numpy(q).to(dev), kc, vc, torch.from_numpy(bt).to(dev),
                                        torch.from_numpy(ctx).to(dev), scale, 0, k_scale=ks, v_scale=vs))
    close(got, want)
