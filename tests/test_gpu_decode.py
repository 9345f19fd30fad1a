"""GPU parity of the decode entry points (paged_attention, _v2, _v3) against the CPU oracle.

Inputs are seeded on the host; the oracle and the HIP kernels read the same
buffers.  Bar: max-abs 2e-3 / rel 1e-2 for fp16/bf16 data (north star),
1e-4 for fp32 data; block-table gather and partition indexing bit-exact.
"""
import numpy as np
import pytest
import torch

import oracle
from _helpers import ATOL32, RTOL32, close, decode_case, dev_inputs, to_dev, to_host

pytestmark = pytest.mark.gpu

ENTRIES = ["v1", "v2", "v3auto", "v3s1", "v3s2", "v3s7", "v3s64"]


def run(pa, entry, q, k, v, bt, ctx, scale, **kw):
    if entry == "v1":
        return pa.paged_attention(q, k, v, bt, ctx, scale, **kw)
    if entry == "v2":
        return pa.paged_attention_v2(q, k, v, bt, ctx, scale, **kw)
    ns = 0 if entry == "v3auto" else int(entry[3:])
    return pa.paged_attention_v3(q, k, v, bt, ctx, scale, ns, **kw)


def want_of(inp, scale):
    return oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], scale, inp["kv"])


@pytest.mark.parametrize("entry", ENTRIES)
def test_config1_gpt2_fp16(pa, dev, entry):
    """H=12, D=64, BS=16, B=4, ctx=512, fp16 Q/K/V, fp16 out,
    128 physical blocks, block table a seeded permutation."""
    inp = decode_case(4, 12, 12, 64, 16, [512] * 4, seed=11, kv="f16", q="f16")
    assert inp["NB"] == 128
    scale = 1.0 / np.sqrt(64)
    got = run(pa, entry, *dev_inputs(inp, dev), scale, out_dtype=torch.float16)
    close(to_host(got), want_of(inp, scale))


@pytest.mark.parametrize("entry", ENTRIES)
def test_hip_selftest_shape_fp32(pa, dev, entry):
    """rocm/hip/paged_attn_v1_hip.cpp:151-162 shape (B=2 H=4 HKV=2 D=32 BS=16 MB=4
    NB=8 ctx=48, U(-0.25,0.25)) against the committed golden output of the
    reference's own cpu_reference."""
    g = np.load(oracle.HERE.parent / "tests" / "golden" / "hip_selftest.npz")
    q = torch.from_numpy(g["q"]).to(dev)
    k = torch.from_numpy(g["k"]).to(dev)
    v = torch.from_numpy(g["v"]).to(dev)
    bt = torch.from_numpy(g["bt"]).to(dev)
    ctx = torch.from_numpy(g["ctx"]).to(dev)
    got = run(pa, entry, q, k, v, bt, ctx, float(g["scale"]))
    close(to_host(got), g["out"], atol=3e-6, rtol=1e-5)


@pytest.mark.parametrize("kv", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("D", [32, 64, 128, 256])
@pytest.mark.parametrize("G", [1, 4])
def test_dtype_dim_gqa_matrix(pa, dev, kv, D, G):
    HKV = 2
    ctx = [1, 15, 16, 17, 333, 1000]
    inp = decode_case(len(ctx), HKV * G, HKV, D, 16, ctx, seed=D * 10 + G, kv=kv)
    scale = 1.0 / np.sqrt(D)
    want = want_of(inp, scale)
    tol = dict(atol=ATOL32, rtol=RTOL32) if kv == "f32" else {}
    for entry in ("v2", "v3auto", "v3s7"):
        got = run(pa, entry, *dev_inputs(inp, dev), scale)
        close(to_host(got), want, **tol)


@pytest.mark.parametrize("D", [32, 64, 128])
def test_fp64_cache(pa, dev, D):
    inp = decode_case(3, 8, 4, D, 16, [5, 64, 200], seed=3, kv="f64")
    scale = 0.3
    got = run(pa, "v3s2", *dev_inputs(inp, dev), scale)
    close(to_host(got), want_of(inp, scale), atol=ATOL32, rtol=RTOL32)


@pytest.mark.parametrize("G", [1, 2, 3, 4, 5, 6, 8, 12, 16, 32])
def test_gqa_groups(pa, dev, G):
    HKV = 2 if G <= 8 else 1
    inp = decode_case(3, HKV * G, HKV, 128, 16, [77, 513, 2000], seed=G, kv="bf16", q="bf16")
    scale = 1.0 / np.sqrt(128)
    want = want_of(inp, scale)
    for entry in ("v1", "v3auto", "v3s3"):
        got = run(pa, entry, *dev_inputs(inp, dev), scale, out_dtype=torch.bfloat16)
        close(to_host(got), want)


@pytest.mark.parametrize("BS", [1, 5, 8, 32, 64])
def test_block_sizes(pa, dev, BS):
    ctx = [1, BS, BS + 1, 3 * BS + 2, 300]
    inp = decode_case(len(ctx), 4, 4, 64, BS, ctx, seed=BS, kv="f16")
    scale = 0.125
    want = want_of(inp, scale)
    for entry in ENTRIES:
        close(to_host(run(pa, entry, *dev_inputs(inp, dev), scale)), want)


@pytest.mark.parametrize("qt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("ot", [torch.float32, torch.float16, torch.bfloat16])
def test_q_and_out_dtypes(pa, dev, qt, ot):
    inp = decode_case(2, 8, 2, 64, 16, [100, 257], seed=5, kv="f16", q=qt)
    got = run(pa, "v3s4", *dev_inputs(inp, dev), 0.125, out_dtype=ot)
    assert got.dtype == ot
    close(to_host(got), want_of(inp, 0.125))


@pytest.mark.parametrize("entry", ENTRIES)
def test_edge_contexts(pa, dev, entry):
    """ctx 0 -> zero rows; ctx beyond MB*BS -> NaN rows; both without any read past the table."""
    inp = decode_case(4, 4, 4, 64, 16, [0, 40, 33, 7], seed=9, kv="f16", mb=3)
    ctx = inp["ctx"].copy()
    ctx[2] = 49  # > MB*BS = 48
    q, k, v, bt, _ = dev_inputs(inp, dev)
    got = to_host(run(pa, entry, q, k, v, bt, torch.from_numpy(ctx).to(dev), 0.125))
    assert np.all(got[0] == 0.0)
    assert np.all(np.isnan(got[2]))
    want = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], ctx, 0.125, "f16")
    close(got[[1, 3]], want[[1, 3]])


@pytest.mark.parametrize("entry", ENTRIES)
def test_bad_block_id_poisons_row(pa, dev, entry):
    inp = decode_case(3, 4, 2, 64, 16, [40, 40, 40], seed=4, kv="f16")
    bt = inp["bt"].copy()
    bt[1, 1] = inp["NB"] + 5  # outside [0, NB)
    bt[2, 2] = -1
    q, k, v, _, ctx = dev_inputs(inp, dev)
    got = to_host(run(pa, entry, q, k, v, torch.from_numpy(bt).to(dev), ctx, 0.125))
    assert np.all(np.isnan(got[1])) and np.all(np.isnan(got[2]))
    want = want_of(inp, 0.125)
    close(got[0], want[0])


def test_gather_bit_exact_planted_keys(pa, dev):
    """Each (b, h) gets one dominant key (score ~ +1e4 above the rest), so
    softmax is exactly one-hot and out must equal that token's V row bit for
    bit: proves the block-table gather of every planted position."""
    B, H, D, BS = 4, 4, 64, 16
    ctx = [123, 256, 31, 400]
    rng = np.random.default_rng(0)
    inp = decode_case(B, H, H, D, BS, ctx, seed=21, kv="f32", q="f32")
    k = np.zeros_like(inp["k"])
    q = np.zeros((B, H, D), np.float32)
    for trial in range(3):
        pos = np.zeros((B, H), np.int64)
        for b in range(B):
            for h in range(H):
                j = int(rng.integers(0, ctx[b]))
                pos[b, h] = j
                blk, off = inp["bt"][b, j // BS], j % BS
                k[blk, off, h, :] = 0.0
                k[blk, off, h, h] = 100.0
                q[b, h, :] = 0.0
                q[b, h, h] = 1000.0
        qd = torch.from_numpy(q).to(dev)
        kd = torch.from_numpy(k).to(dev)
        vd = torch.from_numpy(inp["v"]).to(dev)
        bt = torch.from_numpy(inp["bt"]).to(dev)
        cd = torch.from_numpy(inp["ctx"]).to(dev)
        for entry in ENTRIES:
            got = to_host(run(pa, entry, qd, kd, vd, bt, cd, 1.0))
            for b in range(B):
                for h in range(H):
                    j = pos[b, h]
                    row = inp["v"][inp["bt"][b, j // BS], j % BS, h, :]
                    assert np.array_equal(got[b, h], row), (entry, b, h, j)
        for b in range(B):
            for h in range(H):
                j = pos[b, h]
                k[inp["bt"][b, j // BS], j % BS, h, :] = 0.0


def test_block_permutation_invariance_bit_exact(pa, dev):
    """Moving physical blocks and rewriting the table identically must not change a bit."""
    inp = decode_case(3, 8, 2, 128, 16, [300, 64, 511], seed=8, kv="bf16", extra_blocks=7)
    perm = np.random.default_rng(1).permutation(inp["NB"])
    k2 = np.empty_like(inp["k"])
    v2 = np.empty_like(inp["v"])
    k2[perm] = inp["k"]
    v2[perm] = inp["v"]
    bt2 = perm[inp["bt"]].astype(np.int32)
    q, k, v, bt, ctx = dev_inputs(inp, dev)
    for entry in ENTRIES:
        a = to_host(run(pa, entry, q, k, v, bt, ctx, 0.1))
        b = to_host(run(pa, entry, q, to_dev(k2, "bf16", dev), to_dev(v2, "bf16", dev),
                        torch.from_numpy(bt2).to(dev), ctx, 0.1))
        assert np.array_equal(a, b), entry


def test_repeat_calls_bit_identical(pa, dev):
    inp = decode_case(5, 12, 12, 64, 16, [2048, 1, 700, 1500, 64], seed=2, kv="f16")
    args = dev_inputs(inp, dev)
    for entry in ("v2", "v3auto", "v3s64"):
        a = to_host(run(pa, entry, *args, 0.125))
        for _ in range(3):
            assert np.array_equal(a, to_host(run(pa, entry, *args, 0.125)))


def test_strided_layer_view_of_pool(pa, dev):
    """K/V passed as one layer of a [L, 2, NB, BS, HKV, D] pool (no copy)."""
    L, NB, BS, HKV, D = 3, 40, 16, 4, 64
    rng = np.random.default_rng(6)
    pool = rng.standard_normal((L, 2, NB, BS, HKV, D), dtype=np.float32).astype(np.float16)
    inp = decode_case(2, 8, HKV, D, BS, [200, 311], seed=6, kv="f16", extra_blocks=NB - 33)
    assert inp["NB"] == NB
    layer = 2
    pd = torch.from_numpy(pool).to(dev)
    q, _, _, bt, ctx = dev_inputs(inp, dev)
    kd, vd = pd[layer, 0], pd[layer, 1]
    want = oracle.decode(inp["q_f32"], pool[layer, 0], pool[layer, 1], inp["bt"], inp["ctx"], 0.125, "f16")
    for entry in ENTRIES:
        close(to_host(run(pa, entry, q, kd, vd, bt, ctx, 0.125)), want)
    # Block-major pool [NB, L, 2, BS, HKV, D]: block stride L*2*BS*HKV*D elements.
    pool2 = np.ascontiguousarray(np.transpose(pool, (2, 0, 1, 3, 4, 5)))
    p2 = torch.from_numpy(pool2).to(dev)
    for entry in ENTRIES:
        close(to_host(run(pa, entry, q, p2[:, layer, 0], p2[:, layer, 1], bt, ctx, 0.125)), want)


def test_partition_bounds_bit_exact(pa, dev):
    """With K = 0 every score is 0, so each partition's l is exactly its token
    count: the kernel's partitions must be [s*chunk, min((s+1)*chunk, ctx)),
    chunk = ceil(ctx/S) (kernels/paged_attn_v3.cu:65-68), empty ones m=-3e38, l=0."""
    import ctypes as C
    ctx = [1, 2, 7, 33, 64, 65, 100, 1000]
    B, H, D = len(ctx), 2, 64
    inp = decode_case(B, H, H, D, 16, ctx, seed=1, kv="f32")
    k0 = np.zeros_like(inp["k"])
    q, _, v, bt, cd = dev_inputs(inp, dev)
    k = torch.from_numpy(k0).to(dev)
    out = torch.empty((B, H, D), dtype=torch.float32, device=dev)
    for S in (1, 2, 3, 7, 64):
        ws_bytes = pa.workspace_size(q, k, bt, S)
        ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        V = pa.view
        pa.check(pa.lib().pa_v3_partition(C.byref(V(out)), C.byref(V(q)), C.byref(V(k)), C.byref(V(v)),
                                          C.byref(V(bt)), C.byref(V(cd)), 1.0, S, ws.data_ptr(),
                                          ws.numel(), torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        if S == 1:
            continue  # one split is served directly, no workspace
        rows = B * H * S
        up = lambda x: (x + 255) // 256 * 256
        wsh = ws.cpu().numpy()
        m = wsh[up(rows * D * 4): up(rows * D * 4) + rows * 4].view(np.float32).reshape(B, H, S)
        l = wsh[up(rows * D * 4) + up(rows * 4): up(rows * D * 4) + up(rows * 4) + rows * 4].view(
            np.float32).reshape(B, H, S)
        for b in range(B):
            for s in range(S):
                st, en = oracle.partition_bounds(ctx[b], S, s)
                n = max(0, en - st)
                assert np.all(l[b, :, s] == n), (S, b, s, l[b, :, s], n)
                if n == 0:
                    assert np.all(m[b, :, s] == np.float32(-3.0e38))
                else:
                    assert np.all(m[b, :, s] == 0.0)


def test_partials_match_oracle_split(pa, dev):
    """The split pass's partials, in natural-log units, match the reference's
    split semantics (kernels/paged_attn_v3.cu:33-123) from the oracle."""
    import ctypes as C
    ctx = [50, 300, 17]
    B, H, HKV, D, S = 3, 4, 2, 64, 5
    inp = decode_case(B, H, HKV, D, 16, ctx, seed=12, kv="f16")
    q, k, v, bt, cd = dev_inputs(inp, dev)
    out = torch.empty((B, H, D), dtype=torch.float32, device=dev)
    ws_bytes = pa.workspace_size(q, k, bt, S)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    V = pa.view
    pa.check(pa.lib().pa_v3_partition(C.byref(V(out)), C.byref(V(q)), C.byref(V(k)), C.byref(V(v)),
                                      C.byref(V(bt)), C.byref(V(cd)), 0.125, S, ws.data_ptr(),
                                      ws.numel(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    rows = B * H * S
    up = lambda x: (x + 255) // 256 * 256
    w = ws.cpu().numpy()
    acc = w[:rows * D * 4].view(np.float32).reshape(B, H, S, D)
    m = w[up(rows * D * 4): up(rows * D * 4) + rows * 4].view(np.float32).reshape(B, H, S)
    l = w[up(rows * D * 4) + up(rows * 4):][:rows * 4].view(np.float32).reshape(B, H, S)
    pacc, pm, pl = oracle.decode_partials(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"],
                                          0.125, S, "f16")
    live = pl > 0
    assert np.array_equal(live, l > 0)
    m_nat = m * np.float32(np.log(2.0))
    close(m_nat[live], pm[live], atol=1e-5, rtol=1e-5)
    # Kernel partials are relative to its own max: acc_ref = acc_kernel * e^(m_kernel - m_ref).
    f = np.exp(m_nat - pm)
    close((l * f)[live], pl[live], atol=1e-4, rtol=1e-4)
    close((acc * f[..., None])[live], pacc[live], atol=1e-3, rtol=1e-3)


def fp8_case(B, H, HKV, D, BS, ctx, *, seed, k_scale, v_scale):
    """FP8 E4M3 caches holding K / k_scale and V / v_scale, and the oracle's
    inputs: the dequantised values (fp8_decode(code) * scale) as fp32."""
    inp = decode_case(B, H, HKV, D, BS, ctx, seed=seed, kv="f32", q="f32")
    k8 = oracle.fp8_encode(inp["k"] / np.float32(k_scale))
    v8 = oracle.fp8_encode(inp["v"] / np.float32(v_scale))
    kf = oracle.fp8_decode(k8) * np.float32(k_scale)
    vf = oracle.fp8_decode(v8) * np.float32(v_scale)
    return inp, k8, v8, kf, vf


def fp8_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).view(torch.float8_e4m3fn).to(dev)


@pytest.mark.parametrize("D", [32, 64, 128, 256])
@pytest.mark.parametrize("H,HKV", [(4, 4), (8, 2), (16, 2)])
def test_fp8_decode_v3_scaled(pa, dev, D, H, HKV):
    inp, k8, v8, kf, vf = fp8_case(3, H, HKV, D, 16, [300, 17, 1100], seed=D + H, k_scale=0.05, v_scale=0.02)
    q = torch.from_numpy(inp["q_f32"]).to(dev)
    bt, ctx = torch.from_numpy(inp["bt"]).to(dev), torch.from_numpy(inp["ctx"]).to(dev)
    want = oracle.decode(inp["q_f32"], kf, vf, inp["bt"], inp["ctx"], 0.1, "f32")
    for splits in (0, 1, 5):
        got = pa.paged_attention_v3(q, fp8_dev(k8, dev), fp8_dev(v8, dev), bt, ctx, 0.1, splits,
                                    k_scale=0.05, v_scale=0.02)
        close(to_host(got), want)
    got = pa.torch_ops().paged_attention_v3_scaled(q, fp8_dev(k8, dev), fp8_dev(v8, dev), bt, ctx, 0.1, 0,
                                                   0.05, 0.02)
    close(to_host(got), want)


def test_fp8_unscaled_entry_points(pa, dev):
    """v1, v2, the fp32 prefill and the MFMA prefill read an FP8 cache as is (scale 1)."""
    inp, k8, v8, kf, vf = fp8_case(2, 8, 4, 64, 16, [90, 200], seed=5, k_scale=1.0, v_scale=1.0)
    q = torch.from_numpy(inp["q_f32"]).to(dev)
    args = (fp8_dev(k8, dev), fp8_dev(v8, dev), torch.from_numpy(inp["bt"]).to(dev),
            torch.from_numpy(inp["ctx"]).to(dev))
    want = oracle.decode(inp["q_f32"], kf, vf, inp["bt"], inp["ctx"], 0.125, "f32")
    close(to_host(pa.paged_attention(q, *args, 0.125)), want)
    close(to_host(pa.paged_attention_v2(q, *args, 0.125)), want)
    got = to_host(pa.paged_attention_prefill(q[:, None], *args, 0.125))[:, 0]
    close(got, want)
    close(to_host(pa.paged_attention_prefill_wmma(q[:, None], *args, 0.125))[:, 0], want)


def test_fp8_every_code_through_the_kernel(pa, dev):
    """V rows cycle through all 254 finite E4M3 codes, K is constant (uniform
    weights): the output is the mean of the decoded codes the row sees, so a
    wrong hardware widening of any code shows."""
    NB, BS, HKV, D = 16, 16, 1, 64
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], np.uint8)
    v8 = np.resize(codes, NB * BS * HKV * D).reshape(NB, BS, HKV, D)
    k8 = np.full_like(v8, 0x38)  # 1.0
    bt = np.arange(NB, dtype=np.int32)[None]
    ctx = np.array([NB * BS], np.int32)
    q = np.ones((1, 1, D), np.float32)
    want = oracle.decode(q, oracle.fp8_decode(k8), oracle.fp8_decode(v8), bt, ctx, 0.01, "f32")
    got = pa.paged_attention_v3(torch.from_numpy(q).to(dev), fp8_dev(k8, dev), fp8_dev(v8, dev),
                                torch.from_numpy(bt).to(dev), torch.from_numpy(ctx).to(dev), 0.01, 3)
    close(to_host(got), want, atol=1e-4, rtol=1e-5)


@pytest.mark.parametrize("kv,qt", [("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32"), ("f16", "f16")])
@pytest.mark.parametrize("D", [32, 64, 128, 256])
@pytest.mark.parametrize("G,BS", [(4, 16), (8, 32), (16, 16)])
def test_gqa_matrix_core_path(pa, dev, kv, qt, D, G, BS):
    """GQA groups of >= 8 heads with 16-aligned pages run on the MFMA decode
    kernel (groups of 4 on the VALU kernel): ragged contexts (partial last tiles), a context long enough for the
    planner to split it (partials + reduce), v1 (one partition), and rows poisoned
    by an invalid block id or a context past the table."""
    HKV = 2
    inp = decode_case(4, HKV * G, HKV, D, BS, [37, 3000, 1, 701], seed=D + G, kv=kv, q=qt, extra_blocks=2)
    q, k, v, bt, ctx = dev_inputs(inp, dev)
    want = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], inp["ctx"], 0.09, kv)
    close(to_host(pa.paged_attention_v3(q, k, v, bt, ctx, 0.09, 0)), want)
    close(to_host(pa.paged_attention(q, k, v, bt, ctx, 0.09)), want)
    bt2 = inp["bt"].copy()
    bt2[3, 5] = -7
    ctx2 = inp["ctx"].copy()
    ctx2[2] = bt2.shape[1] * BS + 1
    want2 = oracle.decode(inp["q_f32"], inp["k"], inp["v"], bt2, ctx2, 0.09, kv)
    got2 = to_host(pa.paged_attention_v3(q, k, v, torch.from_numpy(bt2).to(dev), torch.from_numpy(ctx2).to(dev),
                                         0.09, 0))
    assert np.array_equal(np.isnan(got2), np.isnan(want2)) and np.isnan(want2[2]).all() and np.isnan(want2[3]).all()
    close(got2, want2)


@pytest.mark.parametrize("kind", ["fp8_d64", "fp8_d32", "f16_d32", "bf16_d32"])
@pytest.mark.parametrize("HKV", [2, 6, 3])
@pytest.mark.parametrize("BS", [16, 5])
def test_head_pairing(pa, dev, kind, HKV, BS):
    """MHA whose head rows are under 128 bytes: with an even head count and
    contiguous heads two KV heads share a work-group (whole-line reads); odd
    counts and strided head views take the one-head kernel.  All entry points,
    ragged and empty contexts, split plans, the fast (BS % rows-per-load == 0)
    and general gathers, rows poisoned by a bad block id or a context past the
    table, and FP8 scales."""
    D = 64 if kind == "fp8_d64" else 32
    ctx = [0, 1, 37, 700, 2500]
    seed = D + HKV * 7 + BS
    if kind.startswith("fp8"):
        inp, k8, v8, kf, vf = fp8_case(len(ctx), HKV, HKV, D, BS, ctx, seed=seed, k_scale=1.0, v_scale=1.0)
        q = torch.from_numpy(inp["q_f32"]).to(dev)
        k, v = fp8_dev(k8, dev), fp8_dev(v8, dev)
        kref, vref, kvname = kf, vf, "f32"
    else:
        inp = decode_case(len(ctx), HKV, HKV, D, BS, ctx, seed=seed, kv=kind[:-4])
        q, k, v, _, _ = dev_inputs(inp, dev)
        kref, vref, kvname = inp["k"], inp["v"], inp["kv"]
    bt, ctxd = torch.from_numpy(inp["bt"]).to(dev), torch.from_numpy(inp["ctx"]).to(dev)
    want = oracle.decode(inp["q_f32"], kref, vref, inp["bt"], inp["ctx"], 0.15, kvname)
    for entry in ("v1", "v2", "v3auto", "v3s1", "v3s3", "v3s64"):
        got = to_host(run(pa, entry, q, k, v, bt, ctxd, 0.15))
        assert np.all(got[0] == 0.0)
        close(got, want)
    # Heads strided by 2 * D (every other head of a wider pool): not paired.
    k2 = torch.zeros((k.shape[0], BS, 2 * HKV, D), dtype=k.dtype, device=dev)
    v2 = torch.zeros_like(k2)
    k2[:, :, ::2] = k
    v2[:, :, ::2] = v
    close(to_host(run(pa, "v3auto", q, k2[:, :, ::2], v2[:, :, ::2], bt, ctxd, 0.15)), want)
    # Poisoned rows.
    bt2 = inp["bt"].copy()
    bt2[4, 3] = -3
    ctx2 = inp["ctx"].copy()
    ctx2[2] = bt2.shape[1] * BS + 1
    want2 = oracle.decode(inp["q_f32"], kref, vref, bt2, ctx2, 0.15, kvname)
    got2 = to_host(pa.paged_attention_v3(q, k, v, torch.from_numpy(bt2).to(dev), torch.from_numpy(ctx2).to(dev),
                                         0.15, 0))
    assert np.isnan(got2[2]).all() and np.isnan(got2[4]).all()
    assert np.array_equal(np.isnan(got2), np.isnan(want2))
    close(got2, want2)
    if kind.startswith("fp8"):  # per-tensor scales through the scaled entry
        inp, k8, v8, kf, vf = fp8_case(len(ctx), HKV, HKV, D, BS, ctx, seed=seed, k_scale=0.05, v_scale=0.03)
        want = oracle.decode(inp["q_f32"], kf, vf, inp["bt"], inp["ctx"], 0.15, "f32")
        got = pa.paged_attention_v3(torch.from_numpy(inp["q_f32"]).to(dev), fp8_dev(k8, dev), fp8_dev(v8, dev),
                                    bt, ctxd, 0.15, 0, k_scale=0.05, v_scale=0.03)
        close(to_host(got), want)


@pytest.mark.parametrize("kind,D,HKV", [("f16", 64, 12), ("f16", 64, 6), ("bf16", 128, 4), ("fp8", 128, 8),
                                        ("f32", 32, 4), ("bf16", 32, 8)])
@pytest.mark.parametrize("BS", [16, 5])
def test_head_packing_wide_rows(pa, dev, kind, D, HKV, BS):
    """Head packing up to 512-byte rows.  The planner packs four heads (128-byte
    rows: fp16 D=64 with 12 heads, FP8 D=128, fp32 D=32; 64-byte bf16 D=32
    rows) or two (256-byte rows, or a head count not divisible by four) when
    the packed work-groups still fill the GPU -- here the explicit 256-way
    split (whose reduce also walks more than 64 partitions per row); v1, the
    3-way split and the auto plan of this small batch keep the narrow packing.
    Ragged and empty contexts, both gathers (BS=5 is the general one), a
    strided V (the kernel then serves one head per work-group under the same
    plan), and rows poisoned by a bad block id or a context past the table."""
    ctx = [0, 1, 37, 700, 9000]
    seed = 3 * D + HKV + BS
    if kind == "fp8":
        inp, k8, v8, kf, vf = fp8_case(len(ctx), HKV, HKV, D, BS, ctx, seed=seed, k_scale=1.0, v_scale=1.0)
        q = torch.from_numpy(inp["q_f32"]).to(dev)
        k, v = fp8_dev(k8, dev), fp8_dev(v8, dev)
        kref, vref, kvname = kf, vf, "f32"
    else:
        inp = decode_case(len(ctx), HKV, HKV, D, BS, ctx, seed=seed, kv=kind)
        q, k, v, _, _ = dev_inputs(inp, dev)
        kref, vref, kvname = inp["k"], inp["v"], inp["kv"]
    bt, ctxd = torch.from_numpy(inp["bt"]).to(dev), torch.from_numpy(inp["ctx"]).to(dev)
    want = oracle.decode(inp["q_f32"], kref, vref, inp["bt"], inp["ctx"], 0.11, kvname)
    for entry in ("v1", "v3auto", "v3s3", "v3s256"):
        got = to_host(run(pa, entry, q, k, v, bt, ctxd, 0.11))
        assert np.all(got[0] == 0.0)
        close(got, want)
    # V with heads strided by 2 * D: packing is off for this call's kernel.
    v2 = torch.zeros((v.shape[0], BS, 2 * HKV, D), dtype=v.dtype, device=dev)
    v2[:, :, ::2] = v
    close(to_host(run(pa, "v3auto", q, k, v2[:, :, ::2], bt, ctxd, 0.11)), want)
    # Poisoned rows.
    bt2 = inp["bt"].copy()
    bt2[4, 300] = -3
    ctx2 = inp["ctx"].copy()
    ctx2[2] = bt2.shape[1] * BS + 1
    want2 = oracle.decode(inp["q_f32"], kref, vref, bt2, ctx2, 0.11, kvname)
    for entry in ("v3auto", "v3s256"):
        got2 = to_host(run(pa, entry, q, k, v, torch.from_numpy(bt2).to(dev), torch.from_numpy(ctx2).to(dev), 0.11))
        assert np.isnan(got2[2]).all() and np.isnan(got2[4]).all()
        assert np.array_equal(np.isnan(got2), np.isnan(want2))
        close(got2, want2)


@pytest.mark.parametrize("kv", ["f16", "bf16", "fp8"])
@pytest.mark.parametrize("H,HKV", [(2, 2), (8, 2)])
def test_long_sequence_many_partitions(pa, dev, kv, H, HKV):
    """One 32768-token sequence: the auto plan has too few (sequence, head)
    units to fill the GPU and cuts the context into 128 partitions of 256
    tokens (more than one 64-lane window of the reduce kernel, fixed-length
    mode), with two heads packed per work-group for MHA and the lazy softmax
    rescale for the GQA group; a second sequence of 300 tokens rides along."""
    ctx = [32768, 300]
    D = 64
    if kv == "fp8":
        inp, k8, v8, kf, vf = fp8_case(len(ctx), H, HKV, D, 16, ctx, seed=40 + H, k_scale=1.0, v_scale=1.0)
        q = torch.from_numpy(inp["q_f32"]).to(dev).half()
        k, v = fp8_dev(k8, dev), fp8_dev(v8, dev)
        want = oracle.decode(oracle.to_float(oracle.quantize(inp["q_f32"], "f16"), "f16"), kf, vf, inp["bt"],
                             inp["ctx"], 0.125, "f32")
    else:
        inp = decode_case(len(ctx), H, HKV, D, 16, ctx, seed=40 + H, kv=kv, q=kv)
        q, k, v, _, _ = dev_inputs(inp, dev)
        want = want_of(inp, 0.125)
    bt, ctxd = torch.from_numpy(inp["bt"]).to(dev), torch.from_numpy(inp["ctx"]).to(dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    ptok, nparts = pa.plan_partitions(len(ctx), H, HKV, D, 32768, cus)
    assert nparts > 64 and ptok * nparts >= 32768
    close(to_host(pa.paged_attention_v3(q, k, v, bt, ctxd, 0.125, 0)), want)


@pytest.mark.parametrize("qt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("G", [1, 4, 8])
def test_q_alignment(pa, dev, qt, G):
    """q read at every base alignment: element offsets 0, 1, 2 and 4 into a
    larger buffer give 16-, 2/4-, 4/8- and 8/16-byte aligned rows, covering
    the vector and per-element load paths of the VALU and matrix-core kernels."""
    H, D = 2 * G, 64
    inp = decode_case(3, H, 2, D, 16, [300, 17, 96], seed=70 + G, kv="bf16", q=qt)
    _, k, v, bt, ctx = dev_inputs(inp, dev)
    want = want_of(inp, 0.125)
    qd = to_dev(inp["q"], qt, dev)
    for off in (0, 1, 2, 4):
        buf = torch.zeros(qd.numel() + off, dtype=qd.dtype, device=dev)
        buf[off:] = qd.reshape(-1)
        q = buf[off:].view(qd.shape)
        for entry in ("v1", "v3auto", "v3s7"):
            close(to_host(run(pa, entry, q, k, v, bt, ctx, 0.125)), want)


# Non-finite codes planted in pool slots no sequence attends: (NaN, +Inf) per KV
# type as stored (fp16 0x7E00 / 0x7C00, bf16 0x7FC0 / 0x7F80, FP8 E4M3 0x7F / 0xFF,
# which has no infinity, and fp32 NaN / Inf).
_POISON = {"f16": (0x7E00, 0x7C00), "bf16": (0x7FC0, 0x7F80), "fp8": (0x7F, 0xFF),
           "f32": (0x7FC00000, 0x7F800000)}


def _poison_unattended(k, v, bt, ctx, BS, kind):
    """Copies of k / v (stored arrays) and bt where every slot no live token
    reads holds NaN or Inf: the rows past the context end in each sequence's
    last page, and the whole of block 0, which is made unreferenced by
    swapping it with a block no live page uses (the caller adds a spare)."""
    k, v, bt = k.copy(), v.copy(), bt.copy()
    nb = k.shape[0]
    live = set()
    for b, c in enumerate(ctx):
        live.update(int(x) for x in bt[b, :max(0, -(-int(c) // BS))])
    spare = next(i for i in range(nb) if i not in live)
    for a in (k, v):
        a[[0, spare]] = a[[spare, 0]]
    bt = np.where(bt == 0, spare, np.where(bt == spare, 0, bt)).astype(np.int32)
    bits = {1: np.uint8, 2: np.uint16, 4: np.uint32}[k.itemsize]
    nan, inf = (bits(x) for x in _POISON[kind])
    for a in (k, v):
        raw = a.view(bits)
        raw[0] = nan
        raw[0, 1::3] = inf
        for b, c in enumerate(ctx):
            if c > 0 and c % BS:
                blk = bt[b, (int(c) - 1) // BS]
                raw[blk, int(c) % BS:] = nan
                raw[blk, int(c) % BS + 1::2] = inf
    return k, v, bt


@pytest.mark.parametrize("kind,H,HKV,D,BS", [
    ("f16", 12, 12, 64, 16),   # MHA: one head per work-group (small batch), four packed (256-way split)
    ("f16", 4, 4, 32, 16),     # MHA 64-byte rows: two heads per work-group
    ("f16", 8, 2, 128, 16),    # GQA-4: quad-shared softmax, packed P.V over fp16 pairs
    ("bf16", 8, 2, 128, 16),   # GQA-4 over bf16 (fp32 P.V)
    ("fp8", 8, 2, 128, 16),    # GQA-4 over FP8
    ("fp8", 4, 4, 64, 16),     # FP8 MHA, two heads per work-group
    ("f32", 8, 4, 64, 16),     # fp32 cache, GQA-2
    ("bf16", 16, 2, 128, 16),  # GQA-8: matrix-core decode kernel
    ("f16", 8, 2, 64, 5),      # general gather (BS not a multiple of the rows per load)
])
def test_unattended_slots_hold_nan(pa, dev, kind, H, HKV, D, BS):
    """Slots that no live token reads may hold any bits (freed pages, an FP8
    pool from torch.empty): NaN and Inf planted in the tail of every last page
    and in an unreferenced block 0 must not reach any output.  Every decode
    entry point (v1, v2, v3 with the auto plan and explicit splits), the fp32
    prefill path and, for 16-bit caches, the MFMA prefill."""
    ctx = [1, 17, 300, 1000, 2049, 37]
    seed = D + H + BS
    scale = 0.11
    if kind == "fp8":
        inp, k8, v8, _, _ = fp8_case(len(ctx), H, HKV, D, BS, ctx, seed=seed, k_scale=1.0, v_scale=1.0)
        # fp8_case has no spare block: append one that no page references.
        k8, v8 = np.concatenate([k8, k8[:1]]), np.concatenate([v8, v8[:1]])
        k, v, bt = _poison_unattended(k8, v8, inp["bt"], inp["ctx"], BS, kind)
        kref, vref, kvname = oracle.fp8_decode(k), oracle.fp8_decode(v), "f32"
        kd, vd = fp8_dev(k, dev), fp8_dev(v, dev)
        q = torch.from_numpy(inp["q_f32"]).to(dev)
    else:
        inp = decode_case(len(ctx), H, HKV, D, BS, ctx, seed=seed, kv=kind, extra_blocks=1)
        k, v, bt = _poison_unattended(inp["k"], inp["v"], inp["bt"], inp["ctx"], BS, kind)
        kref, vref, kvname = k, v, kind
        kd, vd = to_dev(k, kind, dev), to_dev(v, kind, dev)
        q = to_dev(inp["q"], inp["qt"], dev)
    assert not np.isfinite(oracle.to_float(kref, kvname)[0]).any()
    btd, ctxd = torch.from_numpy(bt).to(dev), torch.from_numpy(inp["ctx"]).to(dev)
    want = oracle.decode(inp["q_f32"], kref, vref, bt, inp["ctx"], scale, kvname)
    assert np.isfinite(want).all()
    tol = dict(atol=ATOL32, rtol=RTOL32) if kind == "f32" else {}
    for entry in ("v1", "v2", "v3auto", "v3s1", "v3s3", "v3s64", "v3s256"):
        got = to_host(run(pa, entry, q, kd, vd, btd, ctxd, scale))
        assert np.isfinite(got).all(), entry
        close(got, want, **tol)
    # Prefill of the last 3 positions of each sequence (chunked: ctx > S).
    S = 3
    qp = np.random.default_rng(seed).standard_normal((len(ctx), S, H, D), dtype=np.float32)
    wantp = oracle.prefill(qp, kref, vref, bt, inp["ctx"], scale, kvname)
    qpd = torch.from_numpy(qp).to(dev)
    got = to_host(pa.paged_attention_prefill(qpd, kd, vd, btd, ctxd, scale))
    assert np.isfinite(got).all()
    close(got, wantp, **tol)
    if kind in ("f16", "bf16"):
        got = to_host(pa.paged_attention_prefill_wmma(qpd, kd, vd, btd, ctxd, scale))
        assert np.isfinite(got).all()
        close(got, wantp)


@pytest.mark.parametrize("kind,D,qt", [("bf16", 128, "bf16"), ("f16", 128, "f16"), ("bf16", 64, "bf16"),
                                       ("f16", 128, "f32")])
def test_gqa4_two_kv_heads_per_work_group(pa, dev, kind, D, qt):
    """GQA groups of four over 16-bit caches whose heads are contiguous: a
    grid that fills the GPU serves two KV heads per work-group (one 2*D-element
    row per token, each lane computing its own KV head's four query heads).
    Ragged contexts with NaN and Inf planted in every unattended slot; the
    explicit split must dispatch the two-head kernel and match the oracle, as
    must the library's own plan."""
    B, H, HKV, BS = 64, 16, 4, 16
    ctx = np.random.default_rng(D + 5).integers(1, 700, B).astype(np.int32)
    inp = decode_case(B, H, HKV, D, BS, ctx, seed=D + 9, kv=kind, q=qt, extra_blocks=1)
    k, v, bt = _poison_unattended(inp["k"], inp["v"], inp["bt"], inp["ctx"], BS, kind)
    kd, vd = to_dev(k, kind, dev), to_dev(v, kind, dev)
    q = to_dev(inp["q"], inp["qt"], dev)
    btd, ctxd = torch.from_numpy(bt).to(dev), torch.from_numpy(inp["ctx"]).to(dev)
    scale = 1.0 / np.sqrt(D)
    want = oracle.decode(inp["q_f32"], k, v, bt, inp["ctx"], scale, kind)
    assert np.isfinite(want).all()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    for ns in (8, 0):
        got = to_host(pa.paged_attention_v3(q, kd, vd, btd, ctxd, scale, ns, out_dtype=torch.float32))
        if ns and B * (HKV // 2) * ns >= 3 * cus:
            assert f"{D}, 4, 2, " in pa.last_launch(), pa.last_launch()
        assert np.isfinite(got).all(), ns
        close(got, want)


@pytest.mark.parametrize("D,qt", [(128, torch.bfloat16), (128, torch.float32), (64, torch.float16)])
def test_fp8_gqa4_two_kv_heads_per_work_group(pa, dev, D, qt):
    """The FP8 group of four with two KV heads per work-group (the kernel held
    to three waves per SIMD for 16-bit q at D = 128): ragged contexts, NaN
    planted in every unattended slot, scaled cache, against the oracle."""
    B, H, HKV, BS = 64, 16, 4, 16
    ctx = np.random.default_rng(D + 11).integers(1, 700, B).astype(np.int32)
    inp, k8, v8, _, _ = fp8_case(B, H, HKV, D, BS, ctx, seed=D + 13, k_scale=0.05, v_scale=0.02)
    k8, v8 = np.concatenate([k8, k8[:1]]), np.concatenate([v8, v8[:1]])  # a spare block
    k8, v8, bt = _poison_unattended(k8, v8, inp["bt"], inp["ctx"], BS, "fp8")
    kf, vf = oracle.fp8_decode(k8) * np.float32(0.05), oracle.fp8_decode(v8) * np.float32(0.02)
    q = torch.from_numpy(inp["q_f32"]).to(dev).to(qt)
    qf = q.float().cpu().numpy()  # q as the kernel sees it
    btd, ctxd = torch.from_numpy(bt).to(dev), torch.from_numpy(inp["ctx"]).to(dev)
    want = oracle.decode(qf, kf, vf, bt, inp["ctx"], 0.1, "f32")
    assert np.isfinite(want).all()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    for ns in (8, 0):
        got = to_host(pa.paged_attention_v3(q, fp8_dev(k8, dev), fp8_dev(v8, dev), btd, ctxd, 0.1, ns,
                                            k_scale=0.05, v_scale=0.02))
        if ns and B * (HKV // 2) * ns >= 3 * cus:
            assert f"{D}, 4, 2, " in pa.last_launch(), pa.last_launch()
        assert np.isfinite(got).all(), ns
        close(got, want)


@pytest.mark.parametrize("kv,H,HKV,qt", [("f16", 4, 4, "f32"), ("bf16", 8, 2, "bf16"), ("f16", 8, 2, "f16")])
def test_compacted_grid_ragged_split(pa, dev, kv, H, HKV, qt):
    """The automatic v3 plan with fixed-length partitions over a ragged batch
    of at most 64 sequences, whose grid is numbered compactly (each sequence's
    needed partitions first, the idle work-groups last): an empty row, a row
    longer than the table, a one-token row, rows of one, several and all
    partitions in one launch, each against the oracle."""
    ctxs = [0, 48, 1, 300, 4096, 2049, 17]
    inp = decode_case(len(ctxs), H, HKV, 64, 16, ctxs, seed=31, kv=kv, q=qt, mb=256)
    q, k, v, bt, _ = dev_inputs(inp, dev)
    ctx = inp["ctx"].copy()
    ctx[1] = 256 * 16 + 1  # beyond MB*BS: NaN row, no read past the table
    assert pa.workspace_size(q, k, bt, 0) > 0, "the plan must split for this case"
    got = to_host(run(pa, "v3auto", q, k, v, bt, torch.from_numpy(ctx).to(dev), 0.125, out_dtype=torch.float32))
    assert np.all(got[0] == 0.0)
    assert np.all(np.isnan(got[1]))
    want = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], ctx, 0.125, kv)
    close(got[2:], want[2:])


@pytest.mark.parametrize("kv,H,HKV", [("f16", 8, 8), ("bf16", 16, 4)])
def test_explicit_long_split_longest_first(pa, dev, kv, H, HKV):
    """An explicit split into long partitions (at least 1024 tokens at the
    table's capacity) over a ragged batch dispatches the sequences longest
    first: every sequence still gets its own partitions (K = 0: each
    partition's l is exactly its token count, bit for bit) and the combined
    call matches the oracle, including an empty and an over-long context."""
    import ctypes as C
    ctx = [8192, 17, 3000, 0, 5000, 1, 8000, 4096, 2500]
    B, D, BS, S = len(ctx), 64, 16, 4
    inp = decode_case(B, H, HKV, D, BS, ctx, seed=61 + H, kv=kv, q=kv, mb=8192 // BS)
    q, k, v, bt, cd = dev_inputs(inp, dev)
    ctx_run = inp["ctx"].copy()
    ctx_run[1] = 8192 + 1  # beyond the table: NaN row
    cdr = torch.from_numpy(ctx_run).to(dev)
    got = to_host(pa.paged_attention_v3(q, k, v, bt, cdr, 0.125, S, out_dtype=torch.float32))
    want = oracle.decode(inp["q_f32"], inp["k"], inp["v"], inp["bt"], ctx_run, 0.125, kv)
    assert np.all(np.isnan(got[1])) and np.all(got[3] == 0.0)
    live = [b for b in range(B) if b not in (1, 3)]
    close(got[live], want[live])
    # Partition bounds through K = 0 (f32 data: l is exact).
    inp32 = decode_case(B, H, HKV, D, BS, ctx, seed=62, kv="f32", mb=8192 // BS)
    q32, _, v32, bt32, cd32 = dev_inputs(inp32, dev)
    k0 = torch.zeros_like(v32)
    out = torch.empty((B, H, D), dtype=torch.float32, device=dev)
    ws = torch.zeros(pa.workspace_size(q32, k0, bt32, S), dtype=torch.uint8, device=dev)
    V = pa.view
    pa.check(pa.lib().pa_v3_partition(C.byref(V(out)), C.byref(V(q32)), C.byref(V(k0)), C.byref(V(v32)),
                                      C.byref(V(bt32)), C.byref(V(cd32)), 1.0, S, ws.data_ptr(),
                                      ws.numel(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    rows = B * H * S
    up = lambda x: (x + 255) // 256 * 256
    w = ws.cpu().numpy()
    l = w[up(rows * D * 4) + up(rows * 4):][:rows * 4].view(np.float32).reshape(B, H, S)
    for b in range(B):
        if ctx[b] == 0:
            continue
        for s in range(S):
            st, en = oracle.partition_bounds(ctx[b], S, s)
            assert np.all(l[b, :, s] == max(0, en - st)), (b, s, l[b, :, s])
