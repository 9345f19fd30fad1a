"""GPU parity of the prefill entry points against the CPU oracle.

paged_attention_prefill (fp32 arithmetic) and paged_attention_prefill_wmma
(MFMA, Q and P rounded to the 16-bit KV type) are both checked against the
oracle's restatement of kernels/paged_attn_prefill.cu:33-118 on the same
host buffers, for S == ctx (plain causal), S < ctx (chunked prefill: the
chunk is the trailing S tokens) and S > ctx (padded rows, q_pos < 0 -> 0).
"""
import numpy as np
import pytest
import torch

import oracle
from _helpers import ATOL32, RTOL32, close, to_dev, to_host

pytestmark = pytest.mark.gpu


def prefill_case(B, S, H, HKV, D, BS, ctx, *, seed, kv="f16", qt="f32"):
    inp = oracle.paged_inputs(B, 1, HKV, D, BS, ctx, seed=seed, kv_dtype=kv)
    rng = np.random.default_rng(seed + 1000)
    q32 = rng.standard_normal((B, S, H, D), dtype=np.float32)
    q = oracle.quantize(q32, qt)
    inp.update(q=q, q_f32=oracle.to_float(q, qt), kv=kv, qt=qt)
    return inp


def dev_args(inp, dev):
    return (to_dev(inp["q"], inp["qt"], dev), to_dev(inp["k"], inp["kv"], dev),
            to_dev(inp["v"], inp["kv"], dev), torch.from_numpy(inp["bt"]).to(dev),
            torch.from_numpy(inp["ctx"]).to(dev))


def want_of(inp, scale):
    return oracle.prefill(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], scale, inp["kv"])


SHAPES = [  # (B, S, ctx list)
    (2, 64, [64, 64]),        # causal, one tile
    (1, 200, [200]),          # causal, ragged last tile
    (3, 50, [50, 120, 300]),  # chunked prefill: trailing 50 tokens
    (2, 40, [25, 0]),         # padded rows (q_pos < 0) and an empty sequence
]


@pytest.mark.parametrize("kv", ["f16", "bf16"])
@pytest.mark.parametrize("D", [32, 64, 128, 256])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"B{s[0]}S{s[1]}")
def test_mfma_prefill(pa, dev, kv, D, shape):
    B, S, ctx = shape
    inp = prefill_case(B, S, 4, 2, D, 16, ctx, seed=D + S, kv=kv)
    scale = 1.0 / np.sqrt(D)
    got = pa.paged_attention_prefill_wmma(*dev_args(inp, dev), scale)
    close(to_host(got), want_of(inp, scale))


@pytest.mark.parametrize("BS", [8, 16, 32, 7])
def test_mfma_prefill_block_sizes(pa, dev, BS):
    inp = prefill_case(2, 100, 6, 3, 64, BS, [100, 180], seed=BS, kv="f16")
    got = pa.paged_attention_prefill_wmma(*dev_args(inp, dev), 0.125)
    close(to_host(got), want_of(inp, 0.125))


@pytest.mark.parametrize("qt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("ot", [torch.float32, torch.float16, torch.bfloat16])
def test_mfma_prefill_dtypes(pa, dev, qt, ot):
    inp = prefill_case(2, 70, 4, 4, 64, 16, [70, 90], seed=7, kv="bf16", qt=qt)
    got = pa.paged_attention_prefill_wmma(*dev_args(inp, dev), 0.125, out_dtype=ot)
    assert got.dtype == ot
    close(to_host(got), want_of(inp, 0.125))


@pytest.mark.parametrize("ot", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shift", [0, 1, 2, 4])
def test_mfma_prefill_output_alignment(pa, dev, ot, shift):
    """The epilogue writes 4 consecutive dims per store (8 bytes for 16-bit
    out, 16 for fp32) when the output base allows it and single elements
    otherwise: outputs at element offsets 0, 1, 2 and 4 into a larger buffer
    cover both paths for every output dtype, D = 64 and 128."""
    for D in (64, 128):
        inp = prefill_case(2, 70, 4, 2, D, 16, [70, 130], seed=31 + shift + D, kv="f16", qt="f16")
        q = to_dev(inp["q"], "f16", dev)
        buf = torch.full((q.numel() + shift,), float("nan"), dtype=ot, device=dev)
        out = buf[shift:].view(q.shape)
        pa.paged_attention_prefill_wmma(q, *dev_args(inp, dev)[1:], 0.1, out=out)
        close(to_host(out), want_of(inp, 0.1))


def test_mfma_prefill_config4a_shape(pa, dev):
    """BASELINE config 4a geometry (H=12, D=64, fp16, BS=16, S=ctx=1024), batch 2."""
    inp = prefill_case(2, 1024, 12, 12, 64, 16, [1024, 1024], seed=44, kv="f16", qt="f16")
    got = pa.paged_attention_prefill_wmma(*dev_args(inp, dev), 0.125)
    close(to_host(got), want_of(inp, 0.125))


def test_mfma_prefill_vs_torch_sdpa(pa, dev):
    """ctx == S: plain causal attention, pinned to torch's CPU SDPA (is_causal) on the gathered cache."""
    B, S, H, D, BS = 2, 96, 4, 64, 16
    inp = prefill_case(B, S, H, H, D, BS, [S, S], seed=5, kv="f16", qt="f16")
    got = to_host(pa.paged_attention_prefill_wmma(*dev_args(inp, dev), 0.125))
    for b in range(B):
        k = np.stack([oracle.gather(inp["k"], inp["v"], inp["bt"][b], S, h, "f16")[0] for h in range(H)])
        v = np.stack([oracle.gather(inp["k"], inp["v"], inp["bt"][b], S, h, "f16")[1] for h in range(H)])
        qb = torch.from_numpy(inp["q_f32"][b].transpose(1, 0, 2).copy()).double()
        ref = torch.nn.functional.scaled_dot_product_attention(
            qb, torch.from_numpy(k).double(), torch.from_numpy(v).double(), is_causal=True,
            scale=0.125)
        close(got[b], ref.numpy().transpose(1, 0, 2))


@pytest.mark.parametrize("kv", ["f32", "f16", "bf16", "f64"])
def test_fp32_prefill(pa, dev, kv):
    """paged_attention_prefill keeps fp32 arithmetic: fp32 tolerance on fp32 data."""
    inp = prefill_case(3, 33, 8, 2, 64, 16, [33, 100, 20], seed=3, kv=kv)
    got = pa.paged_attention_prefill(*dev_args(inp, dev), 0.2)
    tol = dict(atol=ATOL32, rtol=RTOL32) if kv in ("f32", "f64") else {}
    close(to_host(got), want_of(inp, 0.2), **tol)


@pytest.mark.parametrize("D", [32, 128, 256])
def test_fp32_prefill_dims(pa, dev, D):
    inp = prefill_case(2, 17, 4, 4, D, 8, [17, 40], seed=D, kv="f16")
    got = pa.paged_attention_prefill(*dev_args(inp, dev), 0.1)
    close(to_host(got), want_of(inp, 0.1))


def test_prefill_bad_block_and_long_context(pa, dev):
    """A row is NaN iff its sequence's context exceeds the table or a page the
    row attends has an invalid block id; other rows are unaffected."""
    inp = prefill_case(3, 40, 4, 4, 64, 16, [40, 40, 40], seed=9, kv="f16")
    bt = inp["bt"].copy()
    bt[1, 1] = 10 ** 6          # keys 16..31 of sequence 1: rows 16.. are poisoned
    ctx = inp["ctx"].copy()
    ctx[2] = bt.shape[1] * 16 + 1
    q, k, v, _, _ = dev_args(inp, dev)
    want = oracle.prefill(inp["q_f32"], inp["k"], inp["v"], bt, ctx, 0.1, "f16")
    assert np.all(np.isnan(want[1, 16:])) and not np.isnan(want[1, :16]).any()
    for fn in (pa.paged_attention_prefill, pa.paged_attention_prefill_wmma):
        got = to_host(fn(q, k, v, torch.from_numpy(bt).to(dev), torch.from_numpy(ctx).to(dev), 0.1))
        assert np.array_equal(np.isnan(got), np.isnan(want))
        close(got, want)


@pytest.mark.parametrize("D", [64, 128])
def test_mfma_prefill_bf16_values_beyond_fp16(pa, dev, D):
    """bf16 V values that fp16 cannot hold (|v| >= 65520) on a few keys, one of
    them on the diagonal tile: rows that see them and rows that do not must
    both match the oracle (the kernel redoes such work-groups with V in bf16)."""
    S, BS = 200, 16
    inp = prefill_case(2, S, 4, 2, D, BS, [S, S + 37], seed=D + 1, kv="bf16", qt="bf16")
    v = inp["v"].copy()
    for b, key, val in ((0, 100, 1.0e6), (0, 3, -7.0e4), (1, 150, 3.0e5)):
        blk, row = inp["bt"][b, key // BS], key % BS
        v[blk, row] = oracle.quantize(np.full(v.shape[2:], val, np.float32), "bf16")
    inp["v"] = v
    got = pa.paged_attention_prefill_wmma(*dev_args(inp, dev), 1.0 / np.sqrt(D))
    want = want_of(inp, 1.0 / np.sqrt(D))
    assert np.isfinite(want).all() and np.abs(want).max() > 1e3
    close(to_host(got), want)


@pytest.mark.parametrize("kv,D", [("f16", 64), ("f16", 128), ("bf16", 64)])
def test_mfma_prefill_score_jumps(pa, dev, kv, D):
    """Scores that jump far above every earlier key's: the chunk's first page
    of K rows scaled by 1/40, a middle page's by 40 (scores spread over ~40 in
    natural units), so the running maximum moves by far more than the lazy
    rescale's 2^8 on a late tile; the rows that see the large keys and those
    that do not must both match the oracle."""
    S, BS = 300, 16
    inp = prefill_case(2, S, 4, 2, D, BS, [S, S + 50], seed=D + 5, kv=kv, qt=kv)
    k = oracle.to_float(inp["k"], kv).copy()
    for b in range(2):
        off = inp["ctx"][b] - S
        for key, f in [(off + j, 1.0 / 40) for j in range(BS)] + [(off + 150 + j, 40.0) for j in range(BS)]:
            k[inp["bt"][b, key // BS], key % BS] *= f
    inp["k"] = oracle.quantize(k, kv)
    scale = 1.0 / np.sqrt(D)
    got = pa.paged_attention_prefill_wmma(*dev_args(inp, dev), scale)
    close(to_host(got), want_of(inp, scale))


@pytest.mark.parametrize("scale", [-0.15, 0.0])
@pytest.mark.parametrize("kv,qt", [("f16", "f16"), ("bf16", "bf16"), ("f16", "f32")])
def test_mfma_prefill_scale_sign(pa, dev, scale, kv, qt):
    """A negative scale (the running max must follow the scaled scores) and a
    zero scale (uniform weights over the visible keys)."""
    inp = prefill_case(2, 90, 4, 4, 64, 16, [90, 130], seed=11, kv=kv, qt=qt)
    got = pa.paged_attention_prefill_wmma(*dev_args(inp, dev), scale)
    close(to_host(got), want_of(inp, scale))


def varlen_case(qlens, ctxs, H, HKV, D, BS, seed, kv, qt="f32"):
    B = len(qlens)
    inp = oracle.paged_inputs(B, 1, HKV, D, BS, ctxs, seed=seed, kv_dtype=kv)
    T = int(sum(qlens))
    rng = np.random.default_rng(seed + 7)
    q = oracle.quantize(rng.standard_normal((T, H, D), dtype=np.float32), qt)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    return inp, q, oracle.to_float(q, qt), cu


@pytest.mark.parametrize("kv,D", [("f16", 64), ("bf16", 128), ("f16", 256)])
def test_varlen_mixed_decode_and_prefill(pa, dev, kv, D):
    """Sequences bringing 1 (decode), 0, 37, 130 and 300 new tokens against
    contexts of equal or larger length (chunked): each sequence's rows equal
    the oracle's prefill of that sequence alone; decode rows (served by the
    decode kernel in the same call) equal decode."""
    qlens = [1, 37, 0, 130, 1, 300]
    ctxs = [700, 37, 20, 1000, 1, 333]
    H, HKV, BS = 4, 2, 16
    inp, q, q32, cu = varlen_case(qlens, ctxs, H, HKV, D, BS, seed=D, kv=kv, qt=kv)
    got = to_host(pa.paged_attention_prefill_varlen(
        to_dev(q, kv, dev), to_dev(inp["k"], kv, dev), to_dev(inp["v"], kv, dev),
        torch.from_numpy(inp["bt"]).to(dev), torch.from_numpy(inp["ctx"]).to(dev),
        torch.from_numpy(cu).to(dev), max(qlens), 1.0 / np.sqrt(D)))
    # The one-row sequences went to the decode kernel, the others to the prefill kernel.
    launched = pa.last_launch()
    assert "decode_kernel" in launched and "prefill_mfma_kernel" in launched, launched
    for b, n in enumerate(qlens):
        if n == 0:
            continue
        rows = slice(cu[b], cu[b + 1])
        want = oracle.prefill(q32[rows][None], inp["k"], inp["v"], inp["bt"][b:b + 1], inp["ctx"][b:b + 1],
                              1.0 / np.sqrt(D), kv)[0]
        close(got[rows], want)
        if n == 1:
            close(got[rows], oracle.decode(q32[rows], inp["k"], inp["v"], inp["bt"][b:b + 1],
                                           inp["ctx"][b:b + 1], 1.0 / np.sqrt(D), kv))


@pytest.mark.parametrize("B", [130, 300])
def test_varlen_many_sequences(pa, dev, B):
    """Many sequences of assorted lengths (0, 1, 2, 63, 64, 65, 129, 200 rows)
    in one varlen call: up to 256 sequences the prefill grid holds only the
    query blocks that have rows (numbered across chunks of 64 sequences),
    beyond that every block of every sequence; every row against the oracle."""
    rng = np.random.default_rng(B)
    qlens = rng.choice([0, 1, 2, 63, 64, 65, 129, 200], size=B).tolist()
    qlens[-1] = 200
    ctxs = [int(n + rng.integers(0, 100)) for n in qlens]
    inp, q, q32, cu = varlen_case(qlens, ctxs, 2, 2, 64, 16, seed=B, kv="f16", qt="f16")
    T = int(cu[-1])
    out = torch.full((max(T, 1), 2, 64), 7.0, device=dev)
    pa.paged_attention_prefill_varlen(to_dev(q, "f16", dev), to_dev(inp["k"], "f16", dev),
                                      to_dev(inp["v"], "f16", dev), torch.from_numpy(inp["bt"]).to(dev),
                                      torch.from_numpy(inp["ctx"]).to(dev), torch.from_numpy(cu).to(dev),
                                      max(qlens), 0.125, out=out)
    got = to_host(out)
    for b, n in enumerate(qlens):
        if n == 0:
            continue
        rows = slice(cu[b], cu[b + 1])
        want = oracle.prefill(q32[rows][None], inp["k"], inp["v"], inp["bt"][b:b + 1], inp["ctx"][b:b + 1],
                              0.125, "f16")[0]
        close(got[rows], want)


@pytest.mark.parametrize("kv", ["f16", "bf16"])
def test_varlen_on_the_8_wave_kernel(pa, dev, kv):
    """A varlen batch whose rows fill the GPU twice over in 256-row blocks
    (H x ceil(T / 256) >= 2 x CUs) runs on the 8-wave kernel: decode rows
    (served by the decode kernel), an empty sequence, chunks of 1, 255, 256,
    257 and 700 rows against longer contexts; every row against the oracle."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    qlens = [1, 255, 0, 256, 1, 257, 700, 2]
    ctxs = [900, 300, 50, 256, 17, 400, 1000, 2]
    T = sum(qlens)
    H = 8 * -(-2 * cus // (8 * -(-T // 256)))  # H x ceil(T / 256) >= 2 x CUs
    HKV = H // 4
    D = 64
    inp, q, q32, cu = varlen_case(qlens, ctxs, H, HKV, D, 16, seed=H + (kv == "bf16"), kv=kv, qt=kv)
    got = to_host(pa.paged_attention_prefill_varlen(
        to_dev(q, kv, dev), to_dev(inp["k"], kv, dev), to_dev(inp["v"], kv, dev),
        torch.from_numpy(inp["bt"]).to(dev), torch.from_numpy(inp["ctx"]).to(dev),
        torch.from_numpy(cu).to(dev), max(qlens), 0.125))
    launched = pa.last_launch()
    assert "prefill_pp_kernel" in launched and "decode_kernel" in launched, launched
    for b, n in enumerate(qlens):
        if n == 0:
            continue
        rows = slice(cu[b], cu[b + 1])
        want = oracle.prefill(q32[rows][None], inp["k"], inp["v"], inp["bt"][b:b + 1], inp["ctx"][b:b + 1],
                              0.125, kv)[0]
        close(got[rows], want)


@pytest.mark.parametrize("qt", ["f16", "bf16"])
def test_varlen_fp8_on_the_8_wave_kernel(pa, dev, qt):
    """The same varlen batch over a scaled FP8 E4M3 pool (q fp16 or bf16):
    the chunks run on the 8-wave kernel with the codes staged in registers,
    the decode rows on the FP8 decode kernel; every row against the oracle on
    the dequantised cache."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    qlens = [1, 255, 0, 256, 1, 257, 700, 2]
    ctxs = [900, 300, 50, 256, 17, 400, 1000, 2]
    T = sum(qlens)
    H = 8 * -(-2 * cus // (8 * -(-T // 256)))  # H x ceil(T / 256) >= 2 x CUs
    HKV, D, ks, vs = H // 4, 64, 0.04, 0.03
    inp, q, q32, cu = varlen_case(qlens, ctxs, H, HKV, D, 16, seed=H + 5, kv="f32", qt=qt)
    k8, v8 = oracle.fp8_encode(inp["k"] / np.float32(ks)), oracle.fp8_encode(inp["v"] / np.float32(vs))
    kf, vf = oracle.fp8_decode(k8) * np.float32(ks), oracle.fp8_decode(v8) * np.float32(vs)
    got = to_host(pa.paged_attention_prefill_varlen(
        to_dev(q, qt, dev), _fp8(k8, dev), _fp8(v8, dev), torch.from_numpy(inp["bt"]).to(dev),
        torch.from_numpy(inp["ctx"]).to(dev), torch.from_numpy(cu).to(dev), max(qlens), 0.125,
        k_scale=ks, v_scale=vs))
    launched = pa.last_launch()
    assert "prefill_pp_kernel<pa::KvFP8" in launched and "decode_kernel" in launched, launched
    for b, n in enumerate(qlens):
        if n == 0:
            continue
        rows = slice(cu[b], cu[b + 1])
        want = oracle.prefill(q32[rows][None], kf, vf, inp["bt"][b:b + 1], inp["ctx"][b:b + 1], 0.125, "f32")[0]
        close(got[rows], want)


@pytest.mark.parametrize("scale", [-0.15, 0.0])
@pytest.mark.parametrize("kv", ["f16", "bf16", "fp8"])
def test_mfma_prefill_pingpong_scale_sign(pa, dev, scale, kv):
    """A negative scale (its sign is folded into q exactly; the running max
    follows the scaled scores) and a zero scale (uniform weights over the
    visible keys) on the 8-wave kernel, over fp16, bf16 and FP8 (bf16 q)
    pools: the first and last KV heads' query heads against the oracle."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    H = 4 * (-(-cus // 16))  # 4 sequences x 2 blocks of 256 rows x H heads >= 2 x CUs
    S, BS, G, D = 260, 16, 4, 64
    ctx = [600, 120, 260, 400]
    groups = [0, H // G - 1]
    heads = np.r_[0:G, H - G:H]
    if kv == "fp8":
        inp, k8, v8, kf, vf = fp8_prefill_case(4, S, H, H // G, D, BS, ctx, seed=91, qt="bf16", k_scale=0.05,
                                               v_scale=0.02)
        q, k, v = to_dev(inp["q"], "bf16", dev), _fp8(k8, dev), _fp8(v8, dev)
        kw = dict(k_scale=0.05, v_scale=0.02)
        kref, vref, tag = kf, vf, "f32"
    else:
        inp = prefill_case(4, S, H, H // G, D, BS, ctx, seed=92, kv=kv, qt=kv)
        q, k, v = to_dev(inp["q"], kv, dev), to_dev(inp["k"], kv, dev), to_dev(inp["v"], kv, dev)
        kw = {}
        kref, vref, tag = inp["k"], inp["v"], kv
    got = pa.paged_attention_prefill_wmma(q, k, v, torch.from_numpy(inp["bt"]).to(dev),
                                          torch.from_numpy(inp["ctx"]).to(dev), scale, **kw)
    assert pa.last_launch().startswith("pa::prefill_pp_kernel<"), pa.last_launch()
    want = np.concatenate([oracle.prefill(inp["q_f32"][:, :, g * G:(g + 1) * G], kref[:, :, g:g + 1],
                                          vref[:, :, g:g + 1], inp["bt"], inp["ctx"], scale, tag) for g in groups],
                          axis=2)
    close(to_host(got)[:, :, heads], want)


@pytest.mark.parametrize("ot", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shift", [0, 1])
def test_mfma_prefill_pingpong_output(pa, dev, ot, shift):
    """The 8-wave kernel's epilogue: fp32, fp16 and bf16 outputs, at an
    aligned base (4 dims per store) and one element off (per-element
    stores), against the oracle on the first and last KV heads' query heads."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    H = 4 * (-(-cus // 16))  # 4 sequences x 2 blocks of 256 rows x H heads >= 2 x CUs
    S, BS, G, D = 260, 16, 4, 64
    inp = prefill_case(4, S, H, H // G, D, BS, [600, 120, 260, 400], seed=93 + shift, kv="bf16", qt="bf16")
    q = to_dev(inp["q"], "bf16", dev)
    buf = torch.full((q.numel() + shift,), float("nan"), dtype=ot, device=dev)
    out = buf[shift:].view(q.shape)
    pa.paged_attention_prefill_wmma(q, *dev_args(inp, dev)[1:], 0.125, out=out)
    assert pa.last_launch().startswith("pa::prefill_pp_kernel<"), pa.last_launch()
    groups = [0, H // G - 1]
    heads = np.r_[0:G, H - G:H]
    close(to_host(out)[:, :, heads], _want_head_groups(inp, 0.125, groups))


def test_mfma_prefill_pingpong_edge_contexts(pa, dev):
    """Edge rows on the 8-wave kernel: an empty sequence (every row padded:
    zeros), a context longer than the block table holds (rows at q_pos >= 0
    NaN, padded rows zeros), a 5-token context under a 260-row prompt, and a
    plain one; every row of the first and last KV heads' query heads against
    the oracle, NaN positions exactly."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    H = 4 * (-(-cus // 16))  # 4 sequences x 2 blocks of 256 rows x H heads >= 2 x CUs
    S, BS, G, D = 260, 16, 4, 64
    inp = prefill_case(4, S, H, H // G, D, BS, [0, 300, 5, 260], seed=94, kv="f16", qt="f16")
    ctx = inp["ctx"].copy()
    ctx[1] = inp["bt"].shape[1] * BS + 1  # beyond the table
    q, k, v, bt, _ = dev_args(inp, dev)
    got = to_host(pa.paged_attention_prefill_wmma(q, k, v, bt, torch.from_numpy(ctx).to(dev), 0.125))
    assert pa.last_launch().startswith("pa::prefill_pp_kernel<"), pa.last_launch()
    heads = np.r_[0:G, H - G:H]
    groups = [0, H // G - 1]
    want = np.concatenate([oracle.prefill(inp["q_f32"][:, :, g * G:(g + 1) * G], inp["k"][:, :, g:g + 1],
                                          inp["v"][:, :, g:g + 1], inp["bt"], ctx, 0.125, "f16") for g in groups],
                          axis=2)
    got = got[:, :, heads]
    assert np.all(want[0] == 0.0) and np.isnan(want[1]).any() and not np.isnan(want[2:]).any()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    close(got, want)


def test_varlen_malformed_ranges_and_max_q_len(pa, dev):
    """A decreasing range and a range past T are skipped, rows past max_q_len
    are not written (sentinel kept), and the other sequences are unaffected."""
    qlens = [5, 40, 10]
    ctxs = [50, 40, 70]
    inp, q, q32, cu = varlen_case(qlens, ctxs, 4, 4, 64, 16, seed=3, kv="f16")
    args = (torch.from_numpy(q).to(dev), to_dev(inp["k"], "f16", dev), to_dev(inp["v"], "f16", dev),
            torch.from_numpy(inp["bt"]).to(dev), torch.from_numpy(inp["ctx"]).to(dev))
    T = int(cu[-1])
    for cu_bad, max_q, good in (([0, 5, 3, 56], 40, [0]),          # sequence 1 decreasing, 2 past T (55)
                                ([0, 5, 45, 55], 32, [0, 2])):     # sequence 1 longer than max_q_len
        out = torch.full((T, 4, 64), 7.0, device=dev)
        pa.paged_attention_prefill_varlen(*args, torch.tensor(cu_bad, dtype=torch.int32, device=dev), max_q,
                                          0.125, out=out)
        got = to_host(out)
        for b in good:
            rows = slice(cu[b], cu[b + 1])
            want = oracle.prefill(q32[rows][None], inp["k"], inp["v"], inp["bt"][b:b + 1],
                                  inp["ctx"][b:b + 1], 0.125, "f16")[0]
            close(got[rows], want)
        if max_q == 40:
            assert np.all(got[5:] == 7.0)
        else:  # the 32 served rows of sequence 1 keep their positions ctx - 40 + r
            assert np.all(got[5 + 32:45] == 7.0)
            want = oracle.prefill(q32[5:45][None], inp["k"], inp["v"], inp["bt"][1:2], inp["ctx"][1:2],
                                  0.125, "f16")[0]
            close(got[5:5 + 32], want[:32])


@pytest.mark.parametrize("kv,D,H,HKV", [("f16", 64, 8, 2), ("bf16", 128, 8, 2), ("bf16", 128, 16, 2)])
def test_varlen_all_single_rows(pa, dev, kv, D, H, HKV):
    """A batch of decode steps (max_q_len = 1), served by the decode kernel in
    the varlen call: sequences of one row match the oracle's decode, one with
    an empty context is zeros, and a sequence without rows writes nothing.
    GQA groups of 4 and of 8 (the latter on the vector-ALU decode kernel: the
    matrix-core decode does not serve varlen calls)."""
    qlens = [1, 1, 0, 1, 1]
    ctxs = [300, 17, 40, 1, 900]
    BS = 16
    inp, q, q32, cu = varlen_case(qlens, ctxs, H, HKV, D, BS, seed=D + 2, kv=kv, qt=kv)
    ctx = inp["ctx"].copy()
    ctx[3] = 0
    T = int(cu[-1])
    out = torch.full((T, H, D), 7.0, device=dev)
    pa.paged_attention_prefill_varlen(to_dev(q, kv, dev), to_dev(inp["k"], kv, dev), to_dev(inp["v"], kv, dev),
                                      torch.from_numpy(inp["bt"]).to(dev), torch.from_numpy(ctx).to(dev),
                                      torch.from_numpy(cu).to(dev), 1, 1.0 / np.sqrt(D), out=out)
    launched = pa.last_launch()
    assert "decode_kernel" in launched and "decode_mfma_kernel" not in launched, launched
    assert f"{D}, {H // HKV}, 1, " in launched, launched  # one KV head's group per work-group
    got = to_host(out)
    for b in (0, 1, 4):
        rows = slice(cu[b], cu[b + 1])
        close(got[rows], oracle.decode(q32[rows], inp["k"], inp["v"], inp["bt"][b:b + 1], ctx[b:b + 1],
                                       1.0 / np.sqrt(D), kv))
    assert np.all(got[cu[3]:cu[4]] == 0.0)


def test_varlen_single_rows_packed_gqa4(pa, dev):
    """Enough one-row sequences of a GQA-4 bf16 model that the decode launch of
    the varlen call packs two KV heads per work-group (groups of four, quad-
    shared); every row against the oracle's decode."""
    B, H, HKV, D, BS = 200, 32, 8, 128, 16
    rng = np.random.default_rng(50)
    ctxs = [int(c) for c in rng.integers(1, 300, B)]
    qlens = [1] * B
    inp, q, q32, cu = varlen_case(qlens, ctxs, H, HKV, D, BS, seed=50, kv="bf16", qt="bf16")
    got = to_host(pa.paged_attention_prefill_varlen(
        to_dev(q, "bf16", dev), to_dev(inp["k"], "bf16", dev), to_dev(inp["v"], "bf16", dev),
        torch.from_numpy(inp["bt"]).to(dev), torch.from_numpy(inp["ctx"]).to(dev),
        torch.from_numpy(cu).to(dev), 1, 1.0 / np.sqrt(D)))
    launched = pa.last_launch()
    assert "decode_kernel<pa::KvBF16, 128, 4, 2, " in launched, launched
    close(got, oracle.decode(q32, inp["k"], inp["v"], inp["bt"], inp["ctx"], 1.0 / np.sqrt(D), "bf16"))


@pytest.mark.parametrize("kv,qt", [("f16", "f16"), ("bf16", "bf16"), ("f16", "f32"), ("bf16", "f32")])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_mfma_prefill_plain_and_key_split_modes(pa, dev, kv, qt, D):
    """The MFMA prefill serves a grid of fewer work-groups than CUs in its
    key-split mode (64 query rows per work-group, each tile's two 32-key
    halves on different waves, merged through LDS) and larger grids in the
    plain mode (128 rows, whole tiles).  The same causal + chunked shapes in
    both modes (a few heads; many heads), against the oracle; the dispatched
    kernel names the mode."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    h_plain = 2 * (-(-cus // 8))  # 2 sequences x 2 blocks of 128 rows x h_plain heads >= CUs
    for H, split in ((4, True), (h_plain, False)):
        inp = prefill_case(2, 200, H, 2, D, 16, [200, 500], seed=D + H, kv=kv, qt=qt)
        got = pa.paged_attention_prefill_wmma(*dev_args(inp, dev), 1.0 / np.sqrt(D))
        kern = pa.last_launch()
        assert kern.endswith(", true>" if split else ", false>"), kern
        close(to_host(got), want_of(inp, 1.0 / np.sqrt(D)))


def _want_head_groups(inp, scale, groups, bt=None):
    """The oracle for the query heads of the given KV-head groups only (a
    KV head's G query heads are contiguous), as [B, S, len(groups) * G, D]."""
    H, HKV = inp["q_f32"].shape[2], inp["k"].shape[2]
    G = H // HKV
    parts = [oracle.prefill(inp["q_f32"][:, :, g * G:(g + 1) * G], inp["k"][:, :, g:g + 1], inp["v"][:, :, g:g + 1],
                            inp["bt"] if bt is None else bt, inp["ctx"], scale, inp["kv"]) for g in groups]
    return np.concatenate(parts, axis=2)


@pytest.mark.parametrize("kv", ["f16", "bf16"])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_mfma_prefill_pingpong(pa, dev, kv, D):
    """Grids of at least two work-groups per CU with q in the KV type run the
    8-wave kernel (256 query rows per work-group).  Chunked (S < ctx), plain
    and padded (S > ctx) rows over GQA-4 heads, checked on the first and last
    KV heads' query heads; then the same inputs with a page of invalid block
    id (exactly the rows that attend it are NaN) and, for bf16, V values fp16
    cannot hold on a few keys (the work-group reruns with V in bf16)."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    H = 4 * (-(-cus // 16))  # 4 sequences x 2 blocks of 256 rows x H heads >= 2 x CUs
    S, BS = 260, 16
    inp = prefill_case(4, S, H, H // 4, D, BS, [600, 120, 260, 400], seed=D + 40, kv=kv, qt=kv)
    scale = 1.0 / np.sqrt(D)
    groups = [0, H // 4 - 1]
    heads = np.r_[0:4, H - 4:H]
    print(f"pingpong kv={kv} D={D} H={H}", flush=True)
    got = pa.paged_attention_prefill_wmma(*dev_args(inp, dev), scale)
    assert pa.last_launch().startswith("pa::prefill_pp_kernel<"), pa.last_launch()
    close(to_host(got)[:, :, heads], _want_head_groups(inp, scale, groups))

    bt = inp["bt"].copy()
    bt[0, 30] = 10 ** 6  # keys 480..495 of sequence 0: rows at positions >= 480 are NaN
    if kv == "bf16":
        v = inp["v"].copy()
        for b, key, val in ((0, 100, 1.0e6), (0, 550, -7.0e4), (3, 50, 3.0e5)):
            v[inp["bt"][b, key // BS], key % BS] = oracle.quantize(np.full(v.shape[2:], val, np.float32), "bf16")
        inp["v"] = v
    q, k, vd, _, ctx = dev_args(inp, dev)
    got = to_host(pa.paged_attention_prefill_wmma(q, k, vd, torch.from_numpy(bt).to(dev), ctx, scale))[:, :, heads]
    want = _want_head_groups(inp, scale, groups, bt)
    assert np.isnan(want[0]).any() and not np.isnan(want[1:]).any()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    close(got, want)


def fp8_prefill_case(B, S, H, HKV, D, BS, ctx, *, seed, qt, k_scale, v_scale, poison=False):
    """FP8 E4M3 pool holding K / k_scale and V / v_scale, plus the oracle's
    inputs: the dequantised values (code * scale) as fp32.  poison: NaN codes
    (0x7f) in every page slot past a sequence's context and in a spare block
    that no page references."""
    inp = prefill_case(B, S, H, HKV, D, BS, ctx, seed=seed, kv="f32", qt=qt)
    k8 = oracle.fp8_encode(inp["k"] / np.float32(k_scale))
    v8 = oracle.fp8_encode(inp["v"] / np.float32(v_scale))
    if poison:
        k8, v8 = np.concatenate([k8, np.full_like(k8[:1], 0x7F)]), np.concatenate([v8, np.full_like(v8[:1], 0xFF)])
        for b, c in enumerate(inp["ctx"]):
            if c > 0 and c % BS:
                blk = inp["bt"][b, (int(c) - 1) // BS]
                k8[blk, int(c) % BS:] = 0x7F
                v8[blk, int(c) % BS:] = 0xFF
    kf = oracle.fp8_decode(k8) * np.float32(k_scale)
    vf = oracle.fp8_decode(v8) * np.float32(v_scale)
    return inp, k8, v8, kf, vf


def _fp8(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).view(torch.float8_e4m3fn).to(dev)


@pytest.mark.parametrize("qt", ["f16", "bf16"])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("BS", [16, 5])
def test_mfma_prefill_pingpong_fp8(pa, dev, qt, D, BS):
    """FP8 E4M3 pools on the 8-wave kernel (q in fp16 or bf16, grids of at
    least two work-groups per CU): the K and V codes are staged in registers
    and written to LDS as exact 16-bit tiles.  Chunked, plain and padded rows
    over GQA-4 heads with per-tensor scales and NaN codes in every slot no row
    attends, on pages of 16 and of 5 tokens, checked on the first and last KV
    heads' query heads; then a page of invalid block id (exactly the rows
    that attend it are NaN)."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    H = 4 * (-(-cus // 16))  # 4 sequences x 2 blocks of 256 rows x H heads >= 2 x CUs
    S, G = 260, 4
    ks, vs = 0.05, 0.02
    inp, k8, v8, kf, vf = fp8_prefill_case(4, S, H, H // G, D, BS, [600, 120, 260, 400], seed=D + 7, qt=qt,
                                           k_scale=ks, v_scale=vs, poison=True)
    scale = 1.0 / np.sqrt(D)
    groups = [0, H // G - 1]
    heads = np.r_[0:G, H - G:H]
    print(f"pingpong fp8 q={qt} D={D} BS={BS} H={H}", flush=True)
    q, k, v = to_dev(inp["q"], qt, dev), _fp8(k8, dev), _fp8(v8, dev)
    ctx = torch.from_numpy(inp["ctx"]).to(dev)

    def want(bt):
        return np.concatenate([oracle.prefill(inp["q_f32"][:, :, g * G:(g + 1) * G], kf[:, :, g:g + 1],
                                              vf[:, :, g:g + 1], bt, inp["ctx"], scale, "f32") for g in groups], axis=2)

    got = pa.paged_attention_prefill_wmma(q, k, v, torch.from_numpy(inp["bt"]).to(dev), ctx, scale,
                                          k_scale=ks, v_scale=vs)
    assert pa.last_launch().startswith("pa::prefill_pp_kernel<pa::KvFP8"), pa.last_launch()
    got = to_host(got)[:, :, heads]
    assert np.isfinite(got).all()
    close(got, want(inp["bt"]))

    bt = inp["bt"].copy()
    bt[0, 480 // BS] = 10 ** 6  # the page of key 480 of sequence 0: rows at positions >= its first key are NaN
    got = to_host(pa.paged_attention_prefill_wmma(q, k, v, torch.from_numpy(bt).to(dev), ctx, scale,
                                                  k_scale=ks, v_scale=vs))[:, :, heads]
    w = want(bt)
    assert np.isnan(w[0]).any() and not np.isnan(w[1:]).any()
    assert np.array_equal(np.isnan(got), np.isnan(w))
    close(got, w)


@pytest.mark.parametrize("qt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("D", [32, 64, 128, 256])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"B{s[0]}S{s[1]}")
def test_mfma_prefill_fp8(pa, dev, qt, D, shape):
    """FP8 E4M3 caches on the matrix-core prefill (codes converted exactly to
    fp16 tiles), unscaled through paged_attention_prefill_wmma and with
    per-tensor scales through paged_attention_prefill_wmma_scaled, against the
    oracle on the dequantised cache; q in fp16 (as the tiles) or split hi + lo."""
    B, S, ctx = shape
    scale = 1.0 / np.sqrt(D)
    for ks, vs in ((1.0, 1.0), (0.05, 0.02)):
        inp, k8, v8, kf, vf = fp8_prefill_case(B, S, 4, 2, D, 16, ctx, seed=D + S + 3, qt=qt, k_scale=ks, v_scale=vs)
        args = (to_dev(inp["q"], qt, dev), _fp8(k8, dev), _fp8(v8, dev), torch.from_numpy(inp["bt"]).to(dev),
                torch.from_numpy(inp["ctx"]).to(dev))
        got = pa.paged_attention_prefill_wmma(*args, scale, k_scale=ks, v_scale=vs)
        assert "prefill_mfma_kernel<pa::KvFP8" in pa.last_launch(), pa.last_launch()
        close(to_host(got), oracle.prefill(inp["q_f32"], kf, vf, inp["bt"], inp["ctx"], scale, "f32"))


@pytest.mark.parametrize("D,S,ctx,H", [(64, 1024, 1024, 32), (128, 512, 2048, 8)])
def test_mfma_prefill_fp8_longer_and_poisoned(pa, dev, D, S, ctx, H):
    """Longer prompts (a plain grid of 512 work-groups and a key-split one)
    over a scaled FP8 pool whose unattended slots hold NaN codes: every row
    equals the oracle."""
    B = 2
    inp, k8, v8, kf, vf = fp8_prefill_case(B, S, H, 2, D, 16, [ctx - 5, ctx], seed=D, qt="bf16",
                                           k_scale=1 / 32, v_scale=1 / 24, poison=True)
    assert not np.isfinite(kf).all()
    args = (to_dev(inp["q"], "bf16", dev), _fp8(k8, dev), _fp8(v8, dev), torch.from_numpy(inp["bt"]).to(dev),
            torch.from_numpy(inp["ctx"]).to(dev))
    scale = 1.0 / np.sqrt(D)
    got = to_host(pa.paged_attention_prefill_wmma(*args, scale, k_scale=1 / 32, v_scale=1 / 24))
    assert ("true>" in pa.last_launch()) == (H == 8), pa.last_launch()  # key-split mode for the small grid
    assert np.isfinite(got).all()
    close(got, oracle.prefill(inp["q_f32"], kf, vf, inp["bt"], inp["ctx"], scale, "f32"))


@pytest.mark.parametrize("ks,vs,qt", [(1.0, 1.0, "f16"), (0.04, 0.03, "bf16")])
def test_varlen_fp8(pa, dev, ks, vs, qt):
    """Mixed decode + prefill batch over an FP8 pool, unscaled and through
    paged_attention_prefill_varlen_scaled: decode rows on the decode kernel,
    chunks on the FP8 matrix-core prefill."""
    qlens = [1, 37, 130, 1]
    ctxs = [700, 37, 1000, 40]
    H, HKV, D, BS = 4, 2, 128, 16
    inp, q, q32, cu = varlen_case(qlens, ctxs, H, HKV, D, BS, seed=17, kv="f32", qt=qt)
    k8, v8 = oracle.fp8_encode(inp["k"] / np.float32(ks)), oracle.fp8_encode(inp["v"] / np.float32(vs))
    kf, vf = oracle.fp8_decode(k8) * np.float32(ks), oracle.fp8_decode(v8) * np.float32(vs)
    got = to_host(pa.paged_attention_prefill_varlen(
        to_dev(q, qt, dev), _fp8(k8, dev), _fp8(v8, dev), torch.from_numpy(inp["bt"]).to(dev),
        torch.from_numpy(inp["ctx"]).to(dev), torch.from_numpy(cu).to(dev), max(qlens), 1.0 / np.sqrt(D),
        k_scale=ks, v_scale=vs))
    launched = pa.last_launch()
    assert "decode_kernel" in launched and "prefill_mfma_kernel<pa::KvFP8" in launched, launched
    for b in range(len(qlens)):
        rows = slice(cu[b], cu[b + 1])
        want = oracle.prefill(q32[rows][None], kf, vf, inp["bt"][b:b + 1], inp["ctx"][b:b + 1], 1.0 / np.sqrt(D),
                              "f32")[0]
        close(got[rows], want)
