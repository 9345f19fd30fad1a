"""GPU parity of the fused explicit split: a paged_attention_v3 call with an
explicit num_splits of short partitions, one query head per work-group's head
chunk, and a grid of one work-group per (sequence, head) that fills the GPU
runs as ONE kernel launch.  Each work-group serves every partition of its
sequence and head in rounds of one partition per token slot (4 waves x TPI
slots, TPI = token rows per load instruction), computes each partition's
partials as the split pass does (kernels/paged_attn_v3.cu:33-123) and merges
them into the output by the reduce's log-sum-exp rule
(kernels/paged_attn_v3.cu:128-166) in registers: the partials are never
written (the workspace is the split's scratch; the reference allocates its
partials inside the call and never returns them, paged_attn_v3.cu:221-224).
The two-launch path's partials keep their own bit-exact partition test.

Checked against the oracle: the output, equal scores
(K = 0), a bad block id poisoning only its row, the workspace left
untouched, and the two-launch path (pa_v3_partition + pa_v3_reduce) on the
same inputs.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle
from _helpers import ATOL32, RTOL32, close, decode_case, dev_inputs, to_host

pytestmark = pytest.mark.gpu

WAVES = 4          # waves per work-group
MAX_ROUNDS = 8     # most rounds per work-group
BT_CHUNK = 256     # block-table entries one work-group stages
WAVE_PART_TOKENS = 256  # longest explicit partition of the short-split modes


def expect_fused(pa, B, H, D, kv_bytes, MB, BS, S, dev):
    """The host plan's fuse rule restated for these grids (one work-group per
    (row, head) at the narrowest packing, just filling the GPU): explicit
    short partitions, at least one per token slot, rounds and pages within
    bounds."""
    maxctx = MB * BS
    chunk = -(-maxctx // S)
    hp = 2 if D * kv_bytes < 128 and H % 2 == 0 else 1
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    if S < 2 or chunk > WAVE_PART_TOKENS or B * (H // hp) < cus:
        return False
    vec = 8 if kv_bytes == 1 else 16 // kv_bytes
    tpi = max(1, 64 // (D * hp // vec))
    slots = WAVES * tpi
    R = -(-S // slots)
    pages = -(-(R * slots * chunk) // BS) + 1
    return S >= slots and R <= MAX_ROUNDS and pages <= BT_CHUNK


def two_launch(pa, out, q, k, v, bt, ctx, scale, S, ws):
    V = pa.view
    st = torch.cuda.current_stream().cuda_stream
    pa.check(pa.lib().pa_v3_partition(C.byref(V(out)), C.byref(V(q)), C.byref(V(k)), C.byref(V(v)),
                                      C.byref(V(bt)), C.byref(V(ctx)), scale, S, ws.data_ptr(), ws.numel(), st))
    pa.check(pa.lib().pa_v3_reduce(C.byref(V(out)), C.byref(V(q)), C.byref(V(k)), C.byref(V(bt)),
                                   C.byref(V(ctx)), S, ws.data_ptr(), ws.numel(), st))


def grid_rows(dev, H, lo=1):
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    return -(-cus * lo // H)


CASES = [  # kv, D, BS, MB, S
    ("f16", 64, 16, 64, 64),    # config 2's shape of split: 2 rounds of 32 16-token partitions
    ("f16", 64, 16, 64, 40),    # ragged rounds: the second has 8 partitions
    ("bf16", 128, 16, 32, 24),  # 16 slots: 2 rounds, 22-token partitions
    ("f32", 64, 8, 64, 48),     # 3 rounds of 11-token partitions
    ("f16", 256, 32, 16, 64),   # 8 slots: 8 rounds
    ("f16", 32, 16, 32, 64),    # two heads packed per work-group (64-byte rows)
    ("bf16", 64, 1, 64, 64),    # one token per page and per partition
    ("f16", 64, 5, 50, 33),     # page size not a multiple of the token slots
]


@pytest.mark.parametrize("kv,D,BS,MB,S", CASES)
def test_fused_split_matches_oracle(pa, dev, kv, D, BS, MB, S):
    """Ragged contexts (empty, one token, the whole table, beyond the table,
    random) through the one-launch fused split, against the oracle and the
    two-launch split on the same inputs."""
    H = 8
    kvb = {"f16": 2, "bf16": 2, "f32": 4}[kv]
    lo = 2 if D * kvb < 128 else 1
    B = grid_rows(dev, H, lo)
    maxctx = MB * BS
    rng = np.random.default_rng(D * 131 + S)
    ctx = rng.integers(1, maxctx + 1, size=B).astype(np.int32)
    ctx[:4] = [0, 1, maxctx, maxctx - 1]
    inp = decode_case(B, H, H, D, BS, ctx.tolist(), seed=70 + S, kv=kv, q=kv, mb=MB)
    q, k, v, bt, _ = dev_inputs(inp, dev)
    ctx_run = inp["ctx"].copy()
    ctx_run[4] = maxctx + 1  # beyond the table: NaN row
    cd = torch.from_numpy(ctx_run).to(dev)
    assert expect_fused(pa, B, H, D, kvb, MB, BS, S, dev)
    got = to_host(pa.paged_attention_v3(q, k, v, bt, cd, 0.125, S))
    launched = pa.last_launch()
    assert "reduce_kernel" not in launched and launched.count("decode_kernel") == 1, launched
    assert np.all(got[0] == 0.0)
    assert np.all(np.isnan(got[4]))
    want = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], ctx_run, 0.125, kv)
    tol = dict(atol=ATOL32, rtol=RTOL32) if kv == "f32" else {}
    live = np.ones(B, bool)
    live[[0, 4]] = False
    close(got[live], want[live], **tol)
    # The two-launch split over the same partitions.
    ws = torch.zeros(pa.workspace_size(q, k, bt, S), dtype=torch.uint8, device=dev)
    out2 = torch.empty((B, H, D), dtype=torch.float32, device=dev)
    two_launch(pa, out2, q, k, v, bt, cd, 0.125, S, ws)
    torch.cuda.synchronize()
    close(got[live], to_host(out2)[live], **tol)


@pytest.mark.parametrize("S", [16, 33, 64])
def test_fused_split_equal_scores(pa, dev, S):
    """With K = 0 every score is 0, every partition's maximum the same: the
    output is the plain mean of V over each row's context, whatever its
    partitions (empty ones included: ctx 1, 2, 7 leave most of the 16-64
    partitions empty).  The workspace (filled with 0xFF) is left untouched."""
    H, D, BS, MB = 8, 64, 16, 64
    B = grid_rows(dev, H)
    maxctx = MB * BS
    rng = np.random.default_rng(S)
    ctx = rng.integers(1, maxctx + 1, size=B).astype(np.int32)
    ctx[:5] = [1, 2, 7, S + 1, maxctx]
    inp = decode_case(B, H, H, D, BS, ctx.tolist(), seed=5, kv="f32", q="f32", mb=MB)
    q, _, v, bt, cd = dev_inputs(inp, dev)
    k = torch.zeros_like(v)
    need = pa.workspace_size(q, k, bt, S)
    ws = torch.full((need,), 0xFF, dtype=torch.uint8, device=dev)
    got = to_host(pa.paged_attention_v3(q, k, v, bt, cd, 1.0, S, workspace=ws))
    assert "reduce_kernel" not in pa.last_launch(), pa.last_launch()
    assert bool((ws == 0xFF).all())
    want = oracle.decode(inp["q_f32"], np.zeros_like(inp["k"]), inp["v"], inp["bt"], inp["ctx"], 1.0, "f32")
    close(got, want, atol=ATOL32, rtol=RTOL32)


def test_fused_split_bad_block_id(pa, dev):
    """A block id outside the pool in one sequence's table: that row is NaN
    (every head) and every other row matches the oracle."""
    H, D, BS, MB, S = 8, 64, 16, 64, 64
    B = grid_rows(dev, H)
    maxctx = MB * BS
    inp = decode_case(B, H, H, D, BS, [maxctx] * B, seed=9, kv="f16", q="f16", mb=MB)
    q, k, v, _, cd = dev_inputs(inp, dev)
    bt_h = inp["bt"].copy()
    nb = inp["k"].shape[0]
    bt_h[3, 10] = nb + 5  # page 10 = tokens 160..175: partition 10 of 16-token partitions
    bt = torch.from_numpy(bt_h).to(dev)
    got = to_host(pa.paged_attention_v3(q, k, v, bt, cd, 0.125, S))
    assert "reduce_kernel" not in pa.last_launch(), pa.last_launch()
    assert np.all(np.isnan(got[3]))
    keep = np.arange(B) != 3
    want = oracle.decode(inp["q_f32"][keep], inp["k"], inp["v"], inp["bt"][keep], inp["ctx"][keep], 0.125, "f16")
    close(got[keep], want)


@pytest.mark.parametrize("D", [64, 128])
def test_fused_split_fp8_scaled(pa, dev, D):
    """An FP8 E4M3 cache with per-tensor scales (k_scale folded into the
    softmax scale, v_scale applied to the merged output) through the fused
    split, against the oracle on the dequantised cache and against a split
    that runs as two launches."""
    from test_gpu_decode import fp8_case, fp8_dev
    H, BS, MB = 8, 16, 32
    kvb = 1
    lo = 2 if D * kvb < 128 else 1
    B = grid_rows(dev, H, lo)
    maxctx = MB * BS
    rng = np.random.default_rng(D)
    ctx = rng.integers(1, maxctx + 1, size=B).astype(np.int32)
    ctx[:3] = [1, maxctx, 2]
    inp, k8, v8, kf, vf = fp8_case(B, H, H, D, BS, ctx.tolist(), seed=D + 3, k_scale=0.05, v_scale=0.02)
    bt = torch.from_numpy(inp["bt"]).to(dev)
    cd = torch.from_numpy(inp["ctx"]).to(dev)
    q = torch.from_numpy(inp["q_f32"]).to(dev).half()
    k, v = fp8_dev(k8, dev), fp8_dev(v8, dev)
    S = 64
    assert expect_fused(pa, B, H, D, kvb, MB, BS, S, dev)
    got = to_host(pa.paged_attention_v3(q, k, v, bt, cd, 0.1, S, k_scale=0.05, v_scale=0.02))
    assert "reduce_kernel" not in pa.last_launch(), pa.last_launch()
    q32 = oracle.to_float(oracle.quantize(inp["q_f32"], "f16"), "f16")
    close(got, oracle.decode(q32, kf, vf, inp["bt"], inp["ctx"], 0.1, "f32"))
    # Beside it, a split of five partitions (too few for the token slots: two launches).
    got5 = to_host(pa.paged_attention_v3(q, k, v, bt, cd, 0.1, 5, k_scale=0.05, v_scale=0.02))
    assert "reduce_kernel" in pa.last_launch(), pa.last_launch()
    close(got, got5)


def test_small_grid_keeps_two_launches(pa, dev):
    """A grid of one work-group per (row, head) that would not fill the GPU
    keeps the partition kernel and the reduce (both launched by one call)."""
    H, D, BS, MB, S = 8, 64, 16, 64, 64
    B = 2
    inp = decode_case(B, H, H, D, BS, [MB * BS, 300], seed=11, kv="f16", q="f16", mb=MB)
    q, k, v, bt, cd = dev_inputs(inp, dev)
    got = to_host(pa.paged_attention_v3(q, k, v, bt, cd, 0.125, S))
    assert "reduce_kernel" in pa.last_launch(), pa.last_launch()
    close(got, oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.125, "f16"))
