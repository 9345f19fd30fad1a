"""Pins the CPU oracle (oracle/pa_oracle.c) before it is trusted as the checker.

What pins each oracle function:
  f16 / bf16 codecs   exhaustive over all 65536 bit patterns against numpy's float16
                      and torch's bfloat16 conversions (library routines).
  decode              bit-exact against the reference's own cpu_reference
                      (rocm/hip/paged_attn_v1_hip.cpp:104-141, built into oracle/_ref)
                      on random configs and the committed golden fixtures; float64
                      brute force; torch CPU SDPA on the gathered cache; closed forms
                      (one token, constant keys, zero scale); GQA == MHA on replicated
                      KV heads; block-permutation invariance.
  decode_online       float64 brute force; within 1e-6 of decode.
  partials / merge    merge(partials(S)) == decode for S in {1,2,7,64}; each partition's
                      (m, l, acc) against float64 brute force over exactly its tokens
                      (m = the maximum scaled score); empty splits are exactly
                      (m=-3e38, l=0); an all-empty merge is NaN as in
                      kernels/paged_attn_v3.cu:162.
  partition_bounds    tiling invariants over a grid of (ctx, S) plus known answers.
  choose_num_splits   the 9 split counts printed in the reference's results
                      (SMs = 48, H = 12).
  decode_min_bytes    the "minimum traffic per call" figures printed in the results.
  prefill             float64 brute force (with the chunk offset), torch SDPA with
                      is_causal when S == ctx, and row s == decode_online with
                      ctx = q_pos + 1.
  dot / softmax       bit-exact against arm_cpu/src/scalar.cpp (oracle/_ref) and the
                      scalar_smoke fixture.
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
needs_ref = pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref not built (no reference checkout)")


def gathered(inp, kv, b, n):
    """K, V of sequence b as [HKV, n, D] float64 (via the oracle's gather)."""
    HKV = inp["k"].shape[2]
    ks, vs = [], []
    for h in range(HKV):
        k, v = oracle.gather(inp["k"], inp["v"], inp["bt"][b], n, h, kv)
        ks.append(k)
        vs.append(v)
    return np.stack(ks).astype(np.float64), np.stack(vs).astype(np.float64)


def brute_decode(inp, kv, scale):
    q = inp["q_f32"].astype(np.float64)
    B, H, D = q.shape
    HKV = inp["k"].shape[2]
    out = np.zeros((B, H, D))
    for b in range(B):
        n = int(inp["ctx"][b])
        if n <= 0:
            continue
        K, V = gathered(inp, kv, b, n)
        for h in range(H):
            s = K[h // (H // HKV)] @ q[b, h] * scale
            p = np.exp(s - s.max())
            out[b, h] = p @ V[h // (H // HKV)] / p.sum()
    return out


# ------------------------------------------------------------------ codecs --

def test_f16_decode_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    got = oracle.f16_decode(bits)
    want = bits.view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))


def test_f16_encode_matches_numpy_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 10.0 ** rng.integers(-8, 6, 200000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf, 2 ** -24,
                  2 ** -25, 2 ** -25 * 1.0000001, 3 * 2 ** -26, 2 ** -14, 2 ** -14 - 2 ** -25],
                 np.float32),
        oracle.f16_decode(np.arange(0, 65536, dtype=np.uint16)),  # every representable value
    ])
    x = x.astype(np.float32)
    x = x[~np.isnan(x)]
    # halfway points between adjacent float16 values (ties to even)
    h = np.arange(0, 0x7bff, dtype=np.uint16).view(np.float16).astype(np.float64)
    mid = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    x = np.concatenate([x, mid, -mid])
    got = oracle.f16_encode(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_bf16_codecs_match_torch():
    bits = np.arange(65536, dtype=np.uint16)
    got = oracle.bf16_decode(bits)
    want = torch.from_numpy(bits.astype(np.int32).astype(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(300000) * 10.0 ** rng.integers(-30, 30, 300000)).astype(np.float32)
    mids = (oracle.bf16_decode(np.arange(0, 0x7f7f, dtype=np.uint16)).astype(np.float64)
            + oracle.bf16_decode(np.arange(1, 0x7f80, dtype=np.uint16)).astype(np.float64)) / 2
    x = np.concatenate([x, mids.astype(np.float32), np.array([np.inf, -np.inf, 0.0, -0.0], np.float32)])
    got = oracle.bf16_encode(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- decode --

CONFIGS = [  # (B, H, HKV, D, BS, ctx)
    (2, 4, 2, 32, 16, [48, 48]),
    (3, 12, 12, 64, 16, [1, 17, 300]),
    (2, 8, 2, 128, 8, [63, 129]),
    (4, 6, 3, 64, 5, [5, 6, 99, 1]),
    (1, 32, 8, 128, 16, [1000]),
]


@needs_ref
@pytest.mark.parametrize("cfg", CONFIGS)
def test_decode_bit_exact_vs_reference_cpu_reference(cfg):
    B, H, HKV, D, BS, ctx = cfg
    inp = oracle.paged_inputs(B, H, HKV, D, BS, ctx, seed=D + B, kv_dtype="f32")
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    ours = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], scale, "f32")
    from oracle.pa_oracle import _p
    ref = np.zeros(B * H * D, np.float32)
    NB = inp["k"].shape[0]
    oracle.ref().ref_cpu_reference(_p(ref), _p(inp["k"]), _p(inp["v"]), _p(inp["q_f32"]),
                                   _p(np.ascontiguousarray(inp["bt"])), _p(inp["ctx"]),
                                   B, H, HKV, D, BS, inp["bt"].shape[1], NB, np.float32(scale))
    assert np.array_equal(ours.ravel().view(np.uint32), ref.view(np.uint32))


def test_golden_hip_selftest():
    g = np.load(GOLDEN / "hip_selftest.npz")
    out = oracle.decode(g["q"], g["k"], g["v"], g["bt"], g["ctx"], float(g["scale"]), "f32")
    assert np.array_equal(out, g["out"])
    # the reference's own self-test threshold (rocm/hip/paged_attn_v1_hip.cpp:198)
    assert np.abs(out - g["out"]).max() < 3e-4


@pytest.mark.parametrize("name", ["config1", "gqa_bf16"])
def test_golden_seeded_cases(name):
    g = np.load(GOLDEN / f"{name}.npz")
    kv, qt = str(g["kv"]), str(g["q"])
    inp = oracle.paged_inputs(int(g["B"]), int(g["H"]), int(g["HKV"]), int(g["D"]), int(g["BS"]),
                              g["ctx"], seed=int(g["seed"]), kv_dtype=kv, q_dtype=qt)
    h = hashlib.sha256()
    for a in (inp["q"], inp["k"], inp["v"], inp["bt"]):
        h.update(np.ascontiguousarray(a).tobytes())
    assert h.hexdigest() == str(g["input_sha256"]), "input generator drifted"
    out = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], float(g["scale"]), kv)
    assert np.array_equal(out, g["out"])


@pytest.mark.parametrize("cfg", CONFIGS)
@pytest.mark.parametrize("kv", ["f32", "f16", "bf16", "f64"])
def test_decode_vs_float64_brute_force(cfg, kv):
    B, H, HKV, D, BS, ctx = cfg
    inp = oracle.paged_inputs(B, H, HKV, D, BS, ctx, seed=7, kv_dtype=kv)
    want = brute_decode(inp, kv, 0.2)
    for online in (False, True):
        got = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.2, kv, online=online)
        np.testing.assert_allclose(got, want, atol=2e-5, rtol=1e-5)


def test_decode_vs_torch_sdpa():
    B, H, HKV, D, BS = 3, 8, 2, 64, 16
    inp = oracle.paged_inputs(B, H, HKV, D, BS, [33, 200, 512], seed=3, kv_dtype="f16")
    got = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.125, "f16")
    for b in range(B):
        n = int(inp["ctx"][b])
        K, V = gathered(inp, "f16", b, n)
        K = torch.from_numpy(np.repeat(K, H // HKV, 0))
        V = torch.from_numpy(np.repeat(V, H // HKV, 0))
        q = torch.from_numpy(inp["q_f32"][b].astype(np.float64))[:, None, :]
        ref = torch.nn.functional.scaled_dot_product_attention(q, K, V, scale=0.125)[:, 0, :]
        np.testing.assert_allclose(got[b], ref.numpy(), atol=1e-5, rtol=1e-5)


def test_closed_forms():
    B, H, D, BS = 2, 3, 32, 4
    inp = oracle.paged_inputs(B, H, H, D, BS, [1, 37], seed=5, kv_dtype="f32")
    out = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.3, "f32")
    # ctx = 1: softmax of one score is exactly 1, out = v_0.
    blk = inp["bt"][0, 0]
    assert np.array_equal(out[0], inp["v"][blk, 0])
    # scale = 0 (and constant K): uniform weights -> mean of V.
    for k in (inp["k"], np.ones_like(inp["k"])):
        o0 = oracle.decode(inp["q_f32"], k, inp["v"], inp["bt"], inp["ctx"],
                           0.0 if k is inp["k"] else 0.7, "f32")
        _, V = gathered(inp, "f32", 1, 37)
        np.testing.assert_allclose(o0[1], V.mean(axis=1), atol=1e-6)


def test_gqa_equals_mha_with_replicated_heads():
    B, H, HKV, D, BS = 2, 8, 2, 64, 16
    inp = oracle.paged_inputs(B, H, HKV, D, BS, [70, 150], seed=9, kv_dtype="bf16")
    gqa = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.1, "bf16")
    rep = lambda a: np.ascontiguousarray(np.repeat(a, H // HKV, axis=2))  # head h -> h // G
    mha = oracle.decode(inp["q_f32"], rep(inp["k"]), rep(inp["v"]), inp["bt"], inp["ctx"], 0.1, "bf16")
    assert np.array_equal(gqa, mha)
    # The wrong map (h -> h % HKV) is distinguishable, so this pin catches it.
    wrong = lambda a: np.ascontiguousarray(np.tile(a, (1, 1, H // HKV, 1)))
    bad = oracle.decode(inp["q_f32"], wrong(inp["k"]), wrong(inp["v"]), inp["bt"], inp["ctx"], 0.1, "bf16")
    assert not np.allclose(bad, gqa, atol=1e-3)


def test_block_permutation_invariance():
    inp = oracle.paged_inputs(3, 4, 4, 64, 16, [100, 3, 250], seed=2, kv_dtype="f16", extra_blocks=5)
    perm = np.random.default_rng(0).permutation(inp["NB"])
    k2 = np.empty_like(inp["k"]); k2[perm] = inp["k"]
    v2 = np.empty_like(inp["v"]); v2[perm] = inp["v"]
    a = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.1, "f16")
    b = oracle.decode(inp["q_f32"], k2, v2, perm[inp["bt"]].astype(np.int32), inp["ctx"], 0.1, "f16")
    assert np.array_equal(a, b)


def test_edge_conventions():
    inp = oracle.paged_inputs(3, 2, 2, 32, 16, [0, 20, 20], seed=1, kv_dtype="f32", mb=2)
    ctx = inp["ctx"].copy(); ctx[2] = 33  # beyond MB*BS
    bt = inp["bt"].copy(); bt[1, 1] = 99  # invalid block on a live page
    out = oracle.decode(inp["q_f32"], inp["k"], inp["v"], bt, ctx, 0.1, "f32")
    assert np.all(out[0] == 0) and np.all(np.isnan(out[1])) and np.all(np.isnan(out[2]))


# ------------------------------------------------------------ split / merge --

@pytest.mark.parametrize("S", [1, 2, 7, 64])
def test_merge_of_partials_equals_decode(S):
    inp = oracle.paged_inputs(4, 6, 2, 64, 16, [1, 31, 500, 2048], seed=S, kv_dtype="f16")
    acc, m, l = oracle.decode_partials(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.125, S, "f16")
    out = oracle.merge(acc, m, l)
    want = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.125, "f16")
    np.testing.assert_allclose(out, want, atol=2e-6, rtol=1e-5)
    # empty splits are exactly (m = -3e38, l = 0, acc = 0)
    for b, n in enumerate(inp["ctx"]):
        for s in range(S):
            st, en = oracle.partition_bounds(int(n), S, s)
            if en <= st:
                assert np.all(m[b, :, s] == np.float32(-3e38)) and np.all(l[b, :, s] == 0)
                assert np.all(acc[b, :, s] == 0)


@pytest.mark.parametrize("S", [2, 7, 64])
def test_partials_vs_float64_brute_force(S):
    """Each non-empty partition's state, directly: m is the maximum of the
    scaled scores over exactly the partition's tokens, l = sum exp(s - m),
    acc = sum exp(s - m) v (kernels/paged_attn_v3.cu:86-122), in float64."""
    inp = oracle.paged_inputs(3, 4, 2, 32, 16, [1, 77, 300], seed=10 + S, kv_dtype="f16")
    scale = 0.2
    acc, m, l = oracle.decode_partials(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], scale, S, "f16")
    q = inp["q_f32"].astype(np.float64)
    G = 4 // 2
    for b, n in enumerate(inp["ctx"]):
        K, V = gathered(inp, "f16", b, int(n))
        for h in range(4):
            sc = K[h // G] @ q[b, h] * scale
            for s in range(S):
                st, en = oracle.partition_bounds(int(n), S, s)
                if en <= st:
                    continue
                mm = sc[st:en].max()
                w = np.exp(sc[st:en] - mm)
                np.testing.assert_allclose(m[b, h, s], mm, rtol=1e-6, atol=1e-6)
                np.testing.assert_allclose(l[b, h, s], w.sum(), rtol=1e-5)
                np.testing.assert_allclose(acc[b, h, s], w @ V[h // G][st:en], rtol=1e-4, atol=1e-5)


def test_all_empty_merge_is_nan_like_reference():
    acc = np.zeros((1, 1, 4, 32), np.float32)
    m = np.full((1, 1, 4), -3e38, np.float32)
    l = np.zeros((1, 1, 4), np.float32)
    assert np.all(np.isnan(oracle.merge(acc, m, l)))


def test_partition_bounds_tiling():
    for ctx in list(range(0, 70)) + [511, 512, 513, 2048, 32768]:
        for S in (1, 2, 3, 7, 16, 63, 64):
            chunk = -(-ctx // S) if ctx > 0 else 0
            cover = []
            for s in range(S):
                st, en = oracle.partition_bounds(ctx, S, s)
                assert st == s * chunk
                if en > st:
                    cover.extend(range(st, en))
                    assert en - st == chunk or en == ctx
            assert cover == list(range(ctx)), (ctx, S)
    # "target a chain length (~32 tokens per split)": 2048 tokens over 64 splits
    assert oracle.partition_bounds(2048, 64, 5) == (160, 192)
    assert oracle.partition_bounds(50, 16, 15) == (60, 50)  # empty tail split


def test_choose_num_splits_reference_values():
    vals = json.loads((GOLDEN / "reference_values.json").read_text())["choose_num_splits"]
    for row in vals["cases"]:
        got = oracle.choose_num_splits(row["batch"], vals["num_heads"], row["context"], vals["sms"])
        assert got == row["splits"], row


def test_min_traffic_reference_values():
    vals = json.loads((GOLDEN / "reference_values.json").read_text())["min_traffic_mb"]
    for row in vals["cases"]:
        ctx = np.full(row["batch"], row["context"], np.int32)
        mb = oracle.decode_min_bytes(ctx, vals["num_kv_heads"], vals["head_dim"], vals["kv_itemsize"]) / 1e6
        assert round(mb, 1) == row["mb"], row


# ---------------------------------------------------------------- prefill --

def brute_prefill(q, inp, kv, scale):
    B, S, H, D = q.shape
    HKV = inp["k"].shape[2]
    out = np.zeros((B, S, H, D))
    for b in range(B):
        ctx = int(inp["ctx"][b])
        if ctx <= 0:
            continue
        K, V = gathered(inp, kv, b, ctx)
        for s in range(S):
            qp = ctx - S + s
            if qp < 0:
                continue
            for h in range(H):
                sc = K[h // (H // HKV), :qp + 1] @ q[b, s, h].astype(np.float64) * scale
                p = np.exp(sc - sc.max())
                out[b, s, h] = p @ V[h // (H // HKV), :qp + 1] / p.sum()
    return out


@pytest.mark.parametrize("S,ctx", [(16, [16, 16]), (20, [50, 20]), (30, [10, 0])])
def test_prefill_vs_brute_force(S, ctx):
    B, H, HKV, D, BS = len(ctx), 4, 2, 32, 8
    inp = oracle.paged_inputs(B, H, HKV, D, BS, ctx, seed=S, kv_dtype="bf16")
    q = np.random.default_rng(S).standard_normal((B, S, H, D), dtype=np.float32)
    got = oracle.prefill(q, inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.2, "bf16")
    np.testing.assert_allclose(got, brute_prefill(q, inp, "bf16", 0.2), atol=2e-5, rtol=1e-5)


def test_prefill_vs_torch_sdpa_causal():
    B, S, H, D, BS = 2, 40, 3, 64, 16
    inp = oracle.paged_inputs(B, H, H, D, BS, [S, S], seed=4, kv_dtype="f16")
    q = np.random.default_rng(0).standard_normal((B, S, H, D), dtype=np.float32)
    got = oracle.prefill(q, inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.125, "f16")
    for b in range(B):
        K, V = gathered(inp, "f16", b, S)
        ref = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(q[b].transpose(1, 0, 2).astype(np.float64)), torch.from_numpy(K),
            torch.from_numpy(V), is_causal=True, scale=0.125)
        np.testing.assert_allclose(got[b], ref.numpy().transpose(1, 0, 2), atol=1e-5, rtol=1e-5)


def test_prefill_row_is_decode_of_its_prefix():
    B, S, H, D, BS = 2, 12, 2, 32, 4
    inp = oracle.paged_inputs(B, H, H, D, BS, [30, 12], seed=6, kv_dtype="f32")
    q = np.random.default_rng(1).standard_normal((B, S, H, D), dtype=np.float32)
    got = oracle.prefill(q, inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.3, "f32")
    for b in range(B):
        for s in range(S):
            qp = int(inp["ctx"][b]) - S + s
            d = oracle.decode(q[b:b + 1, s], inp["k"], inp["v"], inp["bt"][b:b + 1],
                              np.array([qp + 1], np.int32), 0.3, "f32", online=True)
            assert np.array_equal(got[b, s], d[0])


# ------------------------------------------------------- scalar primitives --

def test_dot_softmax_vs_arm_scalar_fixture():
    g = np.load(GOLDEN / "scalar_smoke.npz")
    scores = np.array([oracle.dot(g["query"], g["keys"][t]) for t in range(g["keys"].shape[0])], np.float32)
    assert np.array_equal(scores, g["scores"])
    assert np.array_equal(oracle.softmax(scores), g["softmax"])


@needs_ref
def test_dot_softmax_bit_exact_vs_arm_scalar():
    from oracle.pa_oracle import _p
    rng = np.random.default_rng(3)
    for n in (1, 7, 64, 128, 1000):
        a = rng.standard_normal(n, dtype=np.float32)
        b = rng.standard_normal(n, dtype=np.float32)
        assert oracle.dot(a, b) == np.float32(oracle.ref().ref_dot_scalar(_p(a), _p(b), n))
        x = rng.standard_normal(n, dtype=np.float32) * 5
        r = x.copy()
        oracle.ref().ref_softmax_inplace(_p(r), n)
        assert np.array_equal(oracle.softmax(x), r)


@pytest.mark.parametrize("kv", ["f32", "f16", "bf16"])
def test_simd_baseline_matches_scalar_oracle(kv):
    """The SIMD/OpenMP CPU baseline computes cpu_reference's result (summation order
    differs: fp32 rounding only), including GQA and an empty context."""
    inp = oracle.paged_inputs(3, 8, 2, 64, 16, [70, 0, 33], seed=21, kv_dtype=kv)
    want = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.125, kv)
    got = oracle.decode_simd(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.125, kv, threads=4)
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-5)
    assert not got[1].any()


def test_write_kv_oracle_pins():
    """The write restatement against library routines: f32 -> f16 is numpy's
    float16 cast, f32 -> bf16 is torch's bfloat16 cast (both round to nearest
    even), same-type writes copy bits; written rows read back through the
    block-table gather at the engine's slot layout; padding slots write nothing."""
    rng = np.random.default_rng(5)
    NB, BS, HKV, D, T = 6, 4, 2, 16, 9
    key = (rng.standard_normal((T, HKV, D)) * 3).astype(np.float32)
    val = (rng.standard_normal((T, HKV, D)) * 3).astype(np.float32)
    blocks = np.array([4, 1, 5], np.int64)
    slots = blocks[np.arange(T) // BS] * BS + np.arange(T) % BS
    slots[3] = -1
    for cd in ("f16", "bf16"):
        kc = np.zeros((NB, BS, HKV, D), oracle.NP_OF[cd])
        vc = np.zeros_like(kc)
        oracle.write_kv(kc, vc, key, val, slots, cd, "f32")
        if cd == "f16":
            want_k = key.astype(np.float16)
        else:
            want_k = torch.from_numpy(key).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        for t, s in enumerate(slots):
            if s < 0:
                assert not kc[blocks[t // BS], t % BS].any()
                continue
            assert np.array_equal(kc[s // BS, s % BS], want_k[t])
        bt = np.zeros((1, 3), np.int32)
        bt[0] = blocks
        gk, gv = oracle.gather(kc, vc, bt[0], T, 1, cd)
        live = slots >= 0
        np.testing.assert_array_equal(gk[live], oracle.to_float(want_k[:, 1], cd)[live])
    kc = np.zeros((NB, BS, HKV, D), np.uint16)
    vc = np.zeros_like(kc)
    bits = rng.integers(0, 1 << 16, (T, HKV, D)).astype(np.uint16)
    oracle.write_kv(kc, vc, bits, bits, slots, "bf16", "bf16")
    assert np.array_equal(kc[slots[0] // BS, slots[0] % BS], bits[0])


def test_fp8_codec_matches_torch():
    """fp8_decode over all 256 E4M3 codes equals torch.float8_e4m3fn's widening
    (an independent implementation), NaN included; fp8_encode equals torch's
    round-to-nearest-even narrowing on random data and every halfway point."""
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = oracle.fp8_decode(codes)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(got)], ref[~np.isnan(ref)])
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s for s in (1e-3, 0.1, 1.0, 30.0, 200.0)])
    finite = np.sort(np.unique(ref[np.isfinite(ref) & (ref >= 0)]))
    mids = ((finite[1:].astype(np.float64) + finite[:-1]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids, finite, -finite])
    x = x[np.abs(x) <= 464.0]  # past 464 torch gives NaN; the encoder saturates (checked below)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(oracle.fp8_encode(x), want)
    assert list(oracle.fp8_encode(np.float32([470, 1e6, -500, np.nan]))) == [0x7E, 0x7E, 0xFE, 0x7F]
    specials = np.float32([-0.0, 0.0, -np.inf, np.inf, 448, 464, 1e-30, -1e-30, 2.0 ** -10, 3 * 2.0 ** -10])
    assert list(oracle.fp8_encode(specials)) == [0x80, 0x00, 0xFE, 0x7E, 0x7E, 0x7E, 0x00, 0x80, 0x00, 0x02]


@pytest.mark.parametrize("cache", ["fp8", "f16", "bf16"])
def test_write_kv_scaled_matches_torch(cache):
    """oracle.write_kv with per-tensor scales stores (x / scale) rounded to the
    cache type, as torch computes it independently (float32 division, then the
    cast), for values inside the FP8 range."""
    rng = np.random.default_rng(4)
    NB, BS, HKV, D, T = 6, 4, 2, 8, 20
    key = (rng.standard_normal((T, HKV, D)) * 3).astype(np.float32)
    val = (rng.standard_normal((T, HKV, D)) * 3).astype(np.float32)
    slots = rng.permutation(NB * BS)[:T]
    kc = np.zeros((NB, BS, HKV, D), oracle.NP_OF[cache])
    vc = np.zeros_like(kc)
    oracle.write_kv(kc, vc, key, val, slots, cache, "f32", k_scale=0.05, v_scale=3.7)
    tdt = {"fp8": torch.float8_e4m3fn, "f16": torch.float16, "bf16": torch.bfloat16}[cache]
    for c, x, sc in ((kc, key, 0.05), (vc, val, 3.7)):
        want = (torch.from_numpy(x) / torch.tensor(sc, dtype=torch.float32)).to(tdt)
        got = torch.from_numpy(c.reshape(NB * BS, HKV, D)[slots]).view(tdt) if cache != "f16" else \
            torch.from_numpy(c.reshape(NB * BS, HKV, D)[slots])
        assert torch.equal(got.view(torch.uint8) if cache == "fp8" else got, want.view(torch.uint8) if cache == "fp8" else want)
