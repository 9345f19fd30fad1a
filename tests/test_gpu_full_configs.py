"""GPU parity at the BASELINE configurations' full sizes.

The other GPU tests compare every entry point with the CPU oracle at small
and medium shapes.  These run the five BASELINE workloads at their real sizes
and check what the oracle can afford there:

  * config 2 (B=64, ctx 2048, fp16): every output row against the oracle,
    for the library's split plan and for the reference's split count; block
    permutation invariance bit for bit;
  * config 3 (B=32, 32 query / 8 KV heads, D=128, bf16, ragged contexts in
    [1024, 32768]): every sequence against the oracle; block permutation
    invariance bit for bit;
  * config 3 over an FP8 E4M3 pool written by the scaled KV write: every
    sequence against the oracle on the dequantised pool;
  * configs 4a / 4b (causal prefill): query rows against the oracle's decode
    of the row's prefix (a prefill row is the decode of its prefix, which
    tests/test_oracle.py pins) -- every row of 4a, and at 4b every 16th row
    plus the rows on each side of every 128-row work-group boundary; 4b's
    geometry also over a scaled FP8 E4M3 pool (bf16 q);
  * config 5 (layer 11 of a [12, 2, 131072, 16, 12, 64] fp16 pool, 77 GB,
    K base 35.4 G elements in): the layer read in place against a copy of
    it, bit for bit, and sampled sequences against the oracle;
  * in-kernel offsets past 2^31 elements: a block-major pool
    [NB, L, 2, BS, HKV, D] whose block stride times the block ids in the
    tables exceeds 2^31, against the oracle and a compact copy.

Inputs are drawn on the device from seeded generators; host copies feed the
oracle.  Tolerance: max-abs 2e-3 / rel 1e-2 (fp16/bf16 data).
"""
import numpy as np
import pytest
import torch

import oracle
from _helpers import close, oracle_decode_rows, to_host

pytestmark = pytest.mark.gpu


def host_kv(t: torch.Tensor) -> np.ndarray:
    """Device K/V (fp16 or bf16) -> the oracle's storage container (float16 / uint16 bits)."""
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def kv_tag(dtype) -> str:
    return "bf16" if dtype == torch.bfloat16 else "f16"


def randn(shape, g, dev, dtype):
    return torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(dtype)


def ragged_tables(ctx, BS, seed):
    """Block tables over a shared pool: every live page a distinct random block."""
    pages = [-(-int(c) // BS) for c in ctx]
    nb, MB = sum(pages), max(pages)
    perm = np.random.default_rng(seed).permutation(nb).astype(np.int32)
    bt = np.zeros((len(ctx), MB), np.int32)
    pos = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[pos:pos + n]
        pos += n
    return bt, nb


def permuted(k, v, bt, seed):
    """The same pages at other physical blocks: block i moves to sigma[i], tables follow."""
    nb = k.shape[0]
    sigma = torch.from_numpy(np.random.default_rng(seed).permutation(nb)).to(k.device)
    k2, v2 = torch.empty_like(k), torch.empty_like(v)
    k2[sigma] = k
    v2[sigma] = v
    return k2, v2, sigma[bt.long()].to(torch.int32)


def test_config2_full(pa, dev):
    B, H, D, BS, ctx = 64, 12, 64, 16, 2048
    g = torch.Generator(device=dev)
    g.manual_seed(21)
    bt_np, nb = ragged_tables([ctx] * B, BS, 22)
    k = randn((nb, BS, H, D), g, dev, torch.float16)
    v = randn((nb, BS, H, D), g, dev, torch.float16)
    q = randn((B, H, D), g, dev, torch.float16)
    bt = torch.from_numpy(bt_np).to(dev)
    cl = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    scale = 1.0 / np.sqrt(D)
    want = oracle.decode(q.float().cpu().numpy(), host_kv(k), host_kv(v), bt_np, cl.cpu().numpy(), scale, "f16")
    # The library's plan (one partition per sequence here) and the reference's
    # count (choose_num_splits -> 64 partitions of 32 tokens, plus the reduce).
    for ns in (0, 64):
        got = pa.paged_attention_v3(q, k, v, bt, cl, scale, ns, out_dtype=torch.float32)
        close(to_host(got), want)
        # Both run as one launch of one head per work-group (768 work-groups on
        # 256 CUs): the plan unsplit, the reference's count fused.
        assert pa.last_launch() == "pa::decode_kernel<pa::KvF16, 64, 1, 1, 1>", (ns, pa.last_launch())
    got = pa.paged_attention_v3(q, k, v, bt, cl, scale, 0, out_dtype=torch.float16)
    k2, v2, bt2 = permuted(k, v, bt, 23)
    got2 = pa.paged_attention_v3(q, k2, v2, bt2, cl, scale, 0, out_dtype=torch.float16)
    assert torch.equal(got, got2), "block permutation changed the output"


def test_config3_full(pa, dev):
    B, H, HKV, D, BS = 32, 32, 8, 128, 16
    ctx = np.random.default_rng(3).integers(1024, 32769, B).astype(np.int32)
    g = torch.Generator(device=dev)
    g.manual_seed(31)
    bt_np, nb = ragged_tables(ctx, BS, 32)
    k = randn((nb, BS, HKV, D), g, dev, torch.bfloat16)
    v = randn((nb, BS, HKV, D), g, dev, torch.bfloat16)
    q = randn((B, H, D), g, dev, torch.bfloat16)
    bt = torch.from_numpy(bt_np).to(dev)
    cl = torch.from_numpy(ctx).to(dev)
    scale = 1.0 / np.sqrt(D)
    got = pa.paged_attention_v3(q, k, v, bt, cl, scale, 0, out_dtype=torch.float32)
    want = oracle_decode_rows(q.float().cpu().numpy(), host_kv(k), host_kv(v), bt_np, ctx, scale, "bf16", 1)
    close(to_host(got), want)
    got16 = pa.paged_attention_v3(q, k, v, bt, cl, scale, 0, out_dtype=torch.bfloat16)
    k2, v2, bt2 = permuted(k, v, bt, 33)
    got2 = pa.paged_attention_v3(q, k2, v2, bt2, cl, scale, 0, out_dtype=torch.bfloat16)
    assert torch.equal(got16, got2), "block permutation changed the output"


def test_config3_fp8_full(pa, dev):
    """Config 3 over an FP8 E4M3 pool: bf16 K/V quantised by pa_write_kv_scaled
    (scale 1/16), decoded by the scaled v3 path; every sequence against the
    oracle on the dequantised pool."""
    B, H, HKV, D, BS = 32, 32, 8, 128, 16
    ks = vs = 1.0 / 16
    ctx = np.random.default_rng(3).integers(1024, 32769, B).astype(np.int32)
    g = torch.Generator(device=dev)
    g.manual_seed(34)
    bt_np, nb = ragged_tables(ctx, BS, 35)
    k8 = torch.zeros((nb, BS, HKV, D), dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    v8 = torch.zeros_like(k8)
    for part in torch.arange(nb, device=dev).chunk(8):  # the pool written in slices (bounded source size)
        n = part.numel()
        slots = (part[:, None] * BS + torch.arange(BS, device=dev)).reshape(-1)
        pa.write_kv(k8, v8, randn((n * BS, HKV, D), g, dev, torch.bfloat16),
                    randn((n * BS, HKV, D), g, dev, torch.bfloat16), slots, k_scale=ks, v_scale=vs)
    q = randn((B, H, D), g, dev, torch.bfloat16)
    bt = torch.from_numpy(bt_np).to(dev)
    cl = torch.from_numpy(ctx).to(dev)
    scale = 1.0 / np.sqrt(D)
    got = pa.paged_attention_v3(q, k8, v8, bt, cl, scale, 0, out_dtype=torch.float32, k_scale=ks, v_scale=vs)
    kf = oracle.fp8_decode(k8.view(torch.uint8).cpu().numpy()) * np.float32(ks)
    vf = oracle.fp8_decode(v8.view(torch.uint8).cpu().numpy()) * np.float32(vs)
    want = oracle_decode_rows(q.float().cpu().numpy(), kf, vf, bt_np, ctx, scale, "f32", 1)
    close(to_host(got), want)


PREFILL = {  # name: (B, S, H, D, dtype, rows checked)
    "4a": (8, 1024, 12, 64, torch.float16, list(range(1024))),
    "4b": (2, 4096, 32, 128, torch.bfloat16,
           sorted(set(range(0, 4096, 16)) | {r + d for r in range(128, 4096, 128) for d in (-1, 0)} | {1, 4095})),
}


@pytest.mark.parametrize("name", sorted(PREFILL))
def test_prefill_config_full(pa, dev, name):
    B, S, H, D, dt, rows = PREFILL[name]
    BS = 16
    g = torch.Generator(device=dev)
    g.manual_seed(41 if name == "4a" else 42)
    bt_np, nb = ragged_tables([S] * B, BS, 43)
    k = randn((nb, BS, H, D), g, dev, dt)
    v = randn((nb, BS, H, D), g, dev, dt)
    q = randn((B, S, H, D), g, dev, dt)
    bt = torch.from_numpy(bt_np).to(dev)
    cl = torch.full((B,), S, dtype=torch.int32, device=dev)
    scale = 1.0 / np.sqrt(D)
    got = to_host(pa.paged_attention_prefill_wmma(q, k, v, bt, cl, scale, out_dtype=torch.float32))
    assert np.isfinite(got).all()
    # Query row r of sequence b (position r, S == ctx) is the decode of keys [0, r].
    bs = [b for b in range(B) for _ in rows]
    rs = [r for _ in range(B) for r in rows]
    qd = q.float().cpu().numpy()[bs, rs]                    # [N, H, D]
    want = oracle_decode_rows(qd, host_kv(k), host_kv(v), bt_np[bs], np.asarray(rs, np.int32) + 1, scale, kv_tag(dt))
    close(got[bs, rs], want)


def test_prefill_config4b_fp8_full(pa, dev):
    """Config 4b's geometry over an FP8 E4M3 pool (bf16 q, k and v scales
    1/16) on the 8-wave kernel, the codes staged in registers: the rows of the
    4b check against the oracle on the dequantised pool."""
    B, S, H, D, _, rows = PREFILL["4b"]
    BS, ks, vs = 16, 1.0 / 16, 1.0 / 16
    g = torch.Generator(device=dev)
    g.manual_seed(44)
    bt_np, nb = ragged_tables([S] * B, BS, 45)
    k8 = (randn((nb, BS, H, D), g, dev, torch.float32) / ks).to(torch.float8_e4m3fn)
    v8 = (randn((nb, BS, H, D), g, dev, torch.float32) / vs).to(torch.float8_e4m3fn)
    q = randn((B, S, H, D), g, dev, torch.bfloat16)
    bt = torch.from_numpy(bt_np).to(dev)
    cl = torch.full((B,), S, dtype=torch.int32, device=dev)
    scale = 1.0 / np.sqrt(D)
    got = to_host(pa.paged_attention_prefill_wmma(q, k8, v8, bt, cl, scale, k_scale=ks, v_scale=vs,
                                                  out_dtype=torch.float32))
    assert pa.last_launch().startswith("pa::prefill_pp_kernel<pa::KvFP8QkBf16, 128>"), pa.last_launch()
    assert np.isfinite(got).all()
    kf = oracle.fp8_decode(k8.view(torch.uint8).cpu().numpy()) * np.float32(ks)
    vf = oracle.fp8_decode(v8.view(torch.uint8).cpu().numpy()) * np.float32(vs)
    bs = [b for b in range(B) for _ in rows]
    rs = [r for _ in range(B) for r in rows]
    qd = q.float().cpu().numpy()[bs, rs]
    want = oracle_decode_rows(qd, kf, vf, bt_np[bs], np.asarray(rs, np.int32) + 1, scale, "f32")
    close(got[bs, rs], want)


def _config5(pa, dev, L, NB, BS, H, D, B, ctx):
    pool = torch.empty((L, 2, NB, BS, H, D), dtype=torch.float16, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(51)
    for kv in (0, 1):  # only layer 11 is read: fill it, in 1 GB pieces
        flat = pool[11, kv].view(-1)
        step = 1 << 28
        for off in range(0, flat.numel(), step):
            n = min(step, flat.numel() - off)
            flat[off:off + n] = torch.randn(n, generator=g, device=dev, dtype=torch.float32).half()
    k, v = pool[11, 0], pool[11, 1]
    assert k.storage_offset() == 11 * 2 * NB * BS * H * D > 2 ** 31
    bt_np, nb = ragged_tables([ctx] * B, BS, 52)
    assert nb == NB  # the tables cover every block of the layer
    q = randn((B, H, D), g, dev, torch.float16)
    bt = torch.from_numpy(bt_np).to(dev)
    cl = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    scale = 1.0 / np.sqrt(D)
    got = pa.paged_attention_v3(q, k, v, bt, cl, scale, 0, out_dtype=torch.float32)
    # The layer read in place (35.4 G elements into the pool) against a
    # separate copy of it: identical bits.
    got_c = pa.paged_attention_v3(q, k.clone(), v.clone(), bt, cl, scale, 0, out_dtype=torch.float32)
    assert torch.equal(got, got_c), "layer 11 read in place differs from a copy of it"
    # Sampled sequences against the oracle: their pages gathered to a compact host pool.
    sel = [0, 127, 255]
    pages = torch.from_numpy(bt_np[sel].reshape(-1).astype(np.int64)).to(dev)
    kc, vc = host_kv(k[pages]), host_kv(v[pages])
    btc = np.arange(len(sel) * bt_np.shape[1], dtype=np.int32).reshape(len(sel), -1)
    want = oracle.decode(q[sel].float().cpu().numpy(), kc, vc, btc, np.full(len(sel), ctx, np.int32), scale, "f16")
    close(to_host(got)[sel], want)


def test_config5_full_pool(pa, dev):
    L, NB, BS, H, D, B, ctx = 12, 131072, 16, 12, 64, 256, 8192
    need = L * 2 * NB * BS * H * D * 2
    free, _ = torch.cuda.mem_get_info(dev)
    if free < need + (16 << 30):
        pytest.skip(f"needs {need / 1e9:.0f} GB of free device memory, {free / 1e9:.0f} GB free")
    try:
        _config5(pa, dev, L, NB, BS, H, D, B, ctx)
    finally:
        torch.cuda.empty_cache()  # the pool's 77 GB go back before the next test


def test_block_major_pool_offsets_past_2_31(pa, dev):
    """Block ids times the block stride pass 2^31 elements inside the kernels:
    a [NB, L, 2, BS, HKV, D] pool (block stride L*2*BS*HKV*D = 131072
    elements), layer 63, tables that use blocks 16400 .. 19999 only."""
    NB, L, BS, HKV, D, H = 20000, 64, 16, 1, 64, 4
    pool = torch.empty((NB, L, 2, BS, HKV, D), dtype=torch.float16, device=dev)
    ctx = np.array([1500, 777, 3600], np.int32)
    pages = [-(-int(c) // BS) for c in ctx]
    rng = np.random.default_rng(61)
    ids = rng.permutation(np.arange(16400, NB))[:sum(pages)].astype(np.int32)
    bt_np = np.zeros((len(ctx), max(pages)), np.int32)
    pos = 0
    for b, n in enumerate(pages):
        bt_np[b, :n] = ids[pos:pos + n]
        pos += n
    assert int(ids.max()) * L * 2 * BS * HKV * D > 2 ** 31
    g = torch.Generator(device=dev)
    g.manual_seed(62)
    used = torch.from_numpy(ids.astype(np.int64)).to(dev)
    k, v = pool[:, L - 1, 0], pool[:, L - 1, 1]            # strided views, no copy
    k[used] = randn((len(ids), BS, HKV, D), g, dev, torch.float16)
    v[used] = randn((len(ids), BS, HKV, D), g, dev, torch.float16)
    q = randn((len(ctx), H, D), g, dev, torch.float16)
    bt = torch.from_numpy(bt_np).to(dev)
    cl = torch.from_numpy(ctx).to(dev)
    scale = 0.125
    # Compact copy of the used pages, tables renumbered in order.
    kc, vc = k[used].contiguous(), v[used].contiguous()
    remap = np.zeros(NB, np.int32)
    remap[ids] = np.arange(len(ids), dtype=np.int32)
    btc_np = np.where(np.arange(bt_np.shape[1])[None, :] < np.asarray(pages)[:, None], remap[bt_np], 0).astype(np.int32)
    btc = torch.from_numpy(btc_np).to(dev)
    want = oracle.decode(q.float().cpu().numpy(), host_kv(kc), host_kv(vc), btc_np, ctx, scale, "f16")
    for ns in (0, 1, 7):
        got = pa.paged_attention_v3(q, k, v, bt, cl, scale, ns, out_dtype=torch.float32)
        close(to_host(got), want)
        got_c = pa.paged_attention_v3(q, kc, vc, btc, cl, scale, ns, out_dtype=torch.float32)
        assert torch.equal(got, got_c), f"num_splits={ns}: strided pool differs from the compact copy"
    got = to_host(pa.paged_attention(q, k, v, bt, cl, scale))
    close(got, want)
    # Chunked prefill of each context's trailing 64 tokens on the same pool.
    qp = randn((len(ctx), 64, H, D), g, dev, torch.float16)
    gp = pa.paged_attention_prefill_wmma(qp, k, v, bt, cl, scale, out_dtype=torch.float32)
    gpc = pa.paged_attention_prefill_wmma(qp, kc, vc, btc, cl, scale, out_dtype=torch.float32)
    assert torch.equal(gp, gpc), "prefill: strided pool differs from the compact copy"
    wantp = oracle.prefill(qp.float().cpu().numpy(), host_kv(kc), host_kv(vc), btc_np, ctx, scale, "f16")
    close(to_host(gp), wantp)
    del pool, k, v
    torch.cuda.empty_cache()
