// pa_decode.hpp -- gfx950 paged-attention decode kernel (context-split pass).
//
// Work unit: one work-group (4 waves of 64 lanes) per
//   (query row z, partition part, KV head kvh, head chunk hc), heads fastest.
// The GC query heads of one GQA group that share KV head kvh are served by
// the same work-group, so every K/V page is read from HBM once per KV head
// (the reference reads it once per query head, kernels/paged_attn_v3.cu:63).
//
// Gather.  A K (or V) row of one token is D * sizeof(KV) contiguous bytes.
// LPT = D / VEC consecutive lanes read it, VEC elements each (one 16-byte
// load; 8 bytes for FP8), so one load instruction fetches TPI = 64 / LPT
// whole rows (e.g. 8 rows of 128 B for D=64 fp16).  Physical addresses follow
// kernels/paged_attn_v3.cu:87-89 -- block id from the block table, then
// block/token/head strides -- computed in 64 bits.
//
// Softmax.  Each group of LPT lanes ("slot") runs its own online-softmax
// stream (m, l, acc) over the tokens it loads (kernels/paged_attn_v2.cu:103-115);
// the only per-token cross-lane work is the dot-product sum across the LPT
// lanes, done with DPP row operations.  Streams are combined with the
// log-sum-exp rule once at the end: across slots with lane shuffles, across
// waves through LDS.  Scores are kept in log2 units (q is pre-scaled by
// scale * log2 e) so every exponential is one v_exp_f32.
//
// Output.  direct: the normalised row (kernels/paged_attn_v2.cu:118-121);
// otherwise un-normalised partials acc/m/l for the LSE-reduce kernel
// (kernels/paged_attn_v3.cu:113-122).
#pragma once

#include "pa_device.hpp"

#include <atomic>

namespace pa {

// Ragged batches with fixed-length partitions: the grid holds `parts`
// partitions per (sequence, head unit), sized for the longest context a
// block-table row can hold, but a sequence of ctx tokens needs only
// ceil(ctx / part_tokens) of them (one for an empty or invalid row, which
// writes its fill).  In plain numbering the idle work-groups are spread
// through the grid and each holds a dispatch slot for a context-length load;
// compacted numbering gives the needed units the first ids, sequence by
// sequence (heads fastest, as before), and the idle ones the last.  Every
// wave derives the numbering from the context lengths itself: one load per
// lane and a prefix sum across the wave, hence at most 64 sequences.
__device__ inline bool compact_grid(const DecodeParams& p) {
  return p.part_tokens > 0 && p.Sq == 1 && p.B <= 64 && p.cu_q == nullptr;
}
// Unit `id` of the compacted numbering -> (z, part); false past the last one.
// Whole partitions come first, sequence by sequence (a context out of range
// is one unit: it writes its row), then each sequence's shorter last
// partition, longest first: the dispatcher hands out work-groups in id
// order, so the launch ends on its shortest units.  Config 3 (1044 units on
// 512 slots, partitions of 13 to 2048 tokens) had ended with half the slots
// idle for its last ~15 %.
__device__ inline bool compact_unit(const DecodeParams& p, int id, int lane, int& z, int& part) {
  const int maxctx = p.MB * p.BS;
  const int c = lane < p.B ? p.context_lens[lane] : 0;
  const bool valid = lane < p.B && c > 0 && c <= maxctx;
  const int whole = valid ? c / p.part_tokens : 0;
  const int nfull = lane < p.B ? (valid ? whole : 1) : 0;   // units of whole partitions
  const int rem = valid ? c - whole * p.part_tokens : 0;     // tokens of the last partition if shorter (0: none)
  int incl = nfull;  // inclusive prefix sum over sequences 0..lane
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o, 64);
    incl += lane >= o ? t : 0;
  }
  const int total_full = __builtin_amdgcn_readlane(incl, 63);
  if (id < total_full) {
    // Sequences whose whole partitions all precede id form a prefix of the lanes.
    const int zz = __builtin_popcountll(__builtin_amdgcn_ballot_w64(incl <= id));
    z = zz;
    part = id - __builtin_amdgcn_readlane(incl - nfull, zz);
    return true;
  }
  // The k-th shorter partition by length (descending; ties by sequence).
  const int k = id - total_full;
  int rank = 0;
  for (int j = 0; j < 64; ++j) {
    const int rj = __builtin_amdgcn_readlane(rem, j);
    rank += (rj > rem || (rj == rem && j < lane)) ? 1 : 0;
  }
  const uint64_t hit = __builtin_amdgcn_ballot_w64(rem > 0 && rank == k);
  if (hit == 0) return false;
  z = __builtin_ctzll(hit);
  part = __builtin_amdgcn_readlane(nfull, z);
  return true;
}

// Explicit splits into long partitions (DecodeParams::seq_order, set by the
// host): the sequences' work-groups are dispatched in order of context
// length, longest first (a sequence's partitions are all about equally
// long), so a ragged batch's launch ends on its shortest partitions instead
// of wherever a long sequence falls in the batch.  Rank r -> sequence (up to
// 64 single-row sequences).
__device__ inline int longest_first_seq(const DecodeParams& p, int r, int lane) {
  const int c = lane < p.B ? p.context_lens[lane] : -1;
  int rank = 0;
  for (int j = 0; j < p.B; ++j) {  // wave-uniform bound
    const int cj = __builtin_amdgcn_readlane(c, j);
    rank += (cj > c || (cj == c && j < lane)) ? 1 : 0;
  }
  const uint64_t hit = __builtin_amdgcn_ballot_w64(lane < p.B && rank == r);
  return hit ? __builtin_ctzll(hit) : r;
}

template <typename KV, int D, int NIO = 0>
struct DecodeShape {
  static constexpr int VEC = KV::kVec;         // elements per lane per load
  static constexpr int LPT = D / VEC;          // lanes per token row
  static_assert(LPT >= 1 && LPT <= 64 && (LPT & (LPT - 1)) == 0, "unsupported D/KV combination");
  static constexpr int TPI = 64 / LPT;         // token rows per load instruction
  static constexpr int NI = NIO > 0 ? NIO : 4;  // K (and V) loads per lane per tile
  static constexpr int TT = NI * TPI;          // tokens per wave tile
};

// The shape decode_kernel<KV, D, GC, HP, *> runs: one unpacked MHA head takes
// 2 loads per lane per tile (config 2 +0.8 % over 4).
template <typename KV, int D, int GC, int HP>
using DecodeShapeOf = DecodeShape<KV, D * HP, (GC == 1 && HP == 1) ? 2 : 0>;

// HP > 1 (MHA, or GQA groups of four): one work-group serves HP adjacent KV
// heads, whose rows of a token are contiguous in the pool, as one row of
// HP * D elements (up to 512 bytes); with GC > 1 the lanes of each head's
// part of the row serve that KV head's GC query heads.  A head's row shorter than a 128-byte line
// (FP8 at D = 64, 16-bit at D = 32) then costs whole-line requests instead of
// half-line ones, and longer packed rows keep more of each DRAM access
// useful; each head keeps its own softmax (the dot product is summed over
// the head's LPH lanes only).
// Groups of up to 4 heads are held to two waves per SIMD (<= 256 registers),
// which the loads in flight need; left to itself the allocator has tipped
// GC = 4 at D = 128 into one wave per SIMD (config 3: 415 -> 518 us).
// Register budget (waves per SIMD the allocator must fit): groups of up to 4
// heads two (above); the FP8 group of four at D = 128 packed two KV heads
// to a work-group three, which it fits with one spilled register outside
// the loop (170 registers otherwise: FP8 config 3 4550 -> 4753 GB/s); larger
// groups one.
template <typename KV, int D, int GC, int HP, int DQ>
constexpr int decode_waves_per_eu() {
  if (GC > 4) return 1;
  if (KV::kCode == kFP8 && GC == 4 && HP == 2 && D == 128 && DQ != 0) return 3;
  return 2;
}

// DQ (kF16 or kBF16): q is fp16 or bf16 and the cache provides element pairs
// of that type (the raw words of a cache of q's dtype; FP8 codes through one
// packed conversion per pair), so q is held as packed pairs (exact) and each
// score is VEC / 2 packed dot products (v_dot2c_f32_*), scaled afterwards,
// instead of widening K to fp32 and VEC fused multiply-adds: the score costs
// a quarter of the vector instructions (GQA groups are bound by them).
template <typename KV, int D, int GC, int HP = 1, int DQ = 0>
__global__ __launch_bounds__(kDecodeThreads) __attribute__((amdgpu_waves_per_eu(decode_waves_per_eu<KV, D, GC, HP, DQ>())))
void decode_kernel(const DecodeParams p) {
  static_assert(DQ == 0 || (pair_types<KV>::value & (1 << DQ)), "the cache cannot provide q's pairs");
  constexpr bool LAZY = GC >= 2;  // raise the softmax reference point only by more than 2^8
  using Sh = DecodeShapeOf<KV, D, GC, HP>;
  constexpr int VEC = Sh::VEC, LPT = Sh::LPT, TPI = Sh::TPI, NI = Sh::NI, TT = Sh::TT;
  // Packed P.V for GQA groups over fp16 or FP8 caches (V as fp16 pairs);
  // bf16 weights would be too coarse, so bf16 caches keep the fp32 path.
  // Groups of four heads whose KV head's row spans one 16-lane DPP row: each
  // lane of a quad finishes one head's score (transposing reduction) and its
  // exponential, shared across the quad.
  // The lane keeps its own head's row sum, shared across the quad once at the
  // end; with packed P.V the own weights are packed before they are shared.
  constexpr bool PBC = LAZY && GC == 4 && D / VEC == 16;
  constexpr bool PVP = LAZY && (Sh::NI % 2 == 0) && KV::kCode != kBF16 &&
                       ((pair_types<KV>::value >> kF16) & 1);
  constexpr int LPH = D / VEC;  // lanes per head's row
  constexpr int NW = kDecodeWaves;
  // Progress-ordered wave priority (one unpacked MHA head per work-group, and
  // only when the host found the whole grid resident at once, p.pprio).  A
  // SIMD issues the oldest ready wave first, so the three work-groups a CU
  // holds used to finish in age order (config 2: ~38, ~50, ~61 us of a 64 us
  // launch) and each CU ended with one work-group streaming alone.  Each wave
  // starts at priority 3 and steps down at 1/2, 3/4 and 7/8 of its tiles, so
  // waves that are behind win issue and a CU's work-groups finish together:
  // config 2 6276 -> 6368 GB/s.  With more work-groups than slots (the
  // dispatcher backfills) or packed and GQA rows it measured 1-3 % slower.
  constexpr bool PPRIO = GC == 1 && HP == 1;

  __shared__ int32_t s_bt[kBtChunk];
  __shared__ float s_acc[NW][GC][HP * D];
  __shared__ float s_m[NW][GC * HP];
  __shared__ float s_l[NW][GC * HP];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int slot = lane / LPT;
  const int sub = lane % LPT;
  const int hl = sub / LPH;   // this lane's head within the work-group's HP heads
  const int dsub = sub % LPH;

  // blockIdx.x -> (z, part, kvh, hc), heads fastest: the work-groups that
  // read the other heads' rows of the same pages are dispatched together, so
  // a page's DRAM rows are open for all of them (one KV head's row of a token
  // is a 128-256 byte slice of the page's token row).
  const int units_y = p.HKV / HP * p.head_chunks;
  int id = blockIdx.x;
  int y = id % units_y;
  id /= units_y;
  // Short explicit partitions (one is a few wave tiles, and a work-group per
  // partition would pay its start-up for each).  Wave-partition mode:
  // work-group `grp` serves partitions grp * NW + w, one per wave w.
  // Slot-partition mode: it serves `rounds` rounds of NW * TPI partitions,
  // round r's grp * gparts + r * NW * TPI + w * TPI + s for token slot s of
  // wave w: a slot's lanes stream their own partition's tokens, so the
  // wave's slot streams are the partials themselves, with no cross-slot
  // combine per partition.
  const bool wpm = p.wave_parts == kWavePart;
  const bool spm = p.wave_parts == kSlotPart;
  const int gparts = spm ? NW * TPI * p.rounds : wpm ? NW : 1;  // partitions per work-group
  const int ngrp = (p.parts + gparts - 1) / gparts;
  int part, z, grp = 0;  // part: per lane in the slot-partition mode
  if (compact_grid(p)) {
    if (!compact_unit(p, id, lane, z, part)) return;  // work-group uniform
  } else if (wpm || spm) {
    grp = id % ngrp;
    z = id / ngrp;
    part = grp * gparts + (spm ? wave * TPI + slot : wave);
  } else {
    part = id % p.parts;
    z = id / p.parts;
  }
  if (p.seq_order) z = longest_first_seq(p, z, lane);  // work-group uniform
  // One head per work-group (MHA, unpacked): rotate the head order by the
  // (sequence, partition) index.  Work-groups reach the 8 XCDs round robin,
  // so without it an XCD keeps reading the same few 128-byte head slices of
  // every token row (12 heads on 8 XCDs); rotated, each XCD's requests cover
  // all slice offsets: config 2 6.17 -> 6.40 TB/s.  GQA and packed groups
  // measured slightly slower with it (-0.3 to -0.8 %) and keep the plain order.
  if constexpr (GC == 1 && HP == 1) y = (y + (wpm || spm ? z * ngrp + grp : z * p.parts + part)) % units_y;
  const int kvh = y / p.head_chunks;  // first KV head: kvh * HP
  const int hc = y - kvh * p.head_chunks;
  const int b = z / p.Sq;
  const int sq = z - b * p.Sq;
  const int g0 = hc * GC;
  // q/out row: z, or in a variable-length batch the packed row of a sequence
  // that brings exactly one query row (others are the prefill kernel's).
  int64_t zq = z;
  if (p.cu_q) {
    const int qa = p.cu_q[b], qe = p.cu_q[b + 1];
    if (!(qa >= 0 && qe == qa + 1 && (int64_t)qe <= p.q_total)) return;  // work-group uniform
    zq = qa;
  }

  // The first block-table chunk of the partition is fetched before the
  // context length has arrived: the K/V loads then wait for one memory round
  // trip less at start-up (config 2 +0.2 %, FP8 config 3 +0.7 %).  Fixed-
  // length partitions know their first page; partitions of ceil(ctx / parts)
  // tokens take it from a context that fills the block table (maxctx), and
  // the staging below uses the prefetched entries only if that was right.
  // Packed 16-bit MHA rows (config 5) measured -2.5 % with it and keep the
  // plain order, except in the wave-partition mode, whose short partitions
  // are mostly start-up.
  const bool bt_early = !(GC == 1 && HP > 1 && KV::kCode != kFP8) || wpm || spm;  // work-group uniform
  const int64_t chunk_guess = ((int64_t)p.MB * p.BS + p.parts - 1) / p.parts;
  const int pg_early = p.part_tokens > 0 ? (int)(((int64_t)part * p.part_tokens) / p.BS)
                                         : (int)(((wpm || spm ? (int64_t)grp * gparts : (int64_t)part) * chunk_guess) / p.BS);
  int32_t bt_pre = 0;
  if (bt_early && pg_early + (int)threadIdx.x < p.MB)
    bt_pre = p.block_tables[(int64_t)b * p.bt_stride + pg_early + threadIdx.x];

  const int maxctx = p.MB * p.BS;
  const int ctx_b = p.context_lens[b];
  const int ctx = ctx_b - p.Sq + sq + 1;  // keys this query row attends
  const bool fixed = p.part_tokens > 0;
  const bool ok = ctx > 0 && ctx_b <= maxctx;
  const int nparts = fixed ? (ok ? (ctx + p.part_tokens - 1) / p.part_tokens : 0) : p.parts;
  // (fuse_final: a slot-partition work-group that covers every partition of
  // its unit, GC == 1, also merges them and writes the output.)
  const bool final_here = p.direct || (fixed && nparts <= 1) || p.fuse_final;

  if (!ok) {
    // Zero rows for an empty context, NaN rows for one longer than the table.
    if (final_here && (spm ? grp == 0 : part == 0)) {  // work-group uniform
      const float fillv = ctx <= 0 ? 0.0f : __builtin_nanf("");
      for (int idx = threadIdx.x; idx < GC * HP * D; idx += kDecodeThreads) {
        const int g = idx / (HP * D), dd = idx - g * (HP * D);
        const int d = dd % D, hh = dd / D;
        if (g0 + g >= p.G) continue;
        const int h = (kvh * HP + hh) * p.G + g0 + g;
        store_elem(p.out, p.out_dtype, (zq * p.H + h) * D + d, fillv);
      }
    }
    return;
  }
  if (wpm || spm ? grp * gparts >= nparts : part >= nparts) return;  // work-group uniform

  // This wave's (slot-partition mode: this lane's) tokens [t0, t1); the
  // work-group's [T0, T1) (wave- and slot-partition modes: its partitions
  // together; otherwise the same range).
  int t0, t1, T0, T1, chunk = 0;
  if (fixed) {
    t0 = part * p.part_tokens;
    t1 = min(t0 + p.part_tokens, ctx);
    T0 = t0;
    T1 = t1;
  } else {
    chunk = (ctx + p.parts - 1) / p.parts;  // kernels/paged_attn_v3.cu:65-68
    t0 = min(part * chunk, ctx);
    t1 = min(t0 + chunk, ctx);
    T0 = wpm || spm ? min(grp * gparts * chunk, ctx) : t0;
    T1 = wpm || spm ? min(T0 + gparts * chunk, ctx) : t1;
  }

  // This lane's slice of q for the GC heads, pre-scaled into log2 units.
  // PBC: lane j of each quad holds the heads in the order j, j^1, j^2, j^3
  // (slot g holds head g ^ j), so the transposing reduction below needs no
  // selects: at each exchange step the value a lane keeps and the value its
  // partner needs sit in fixed slots.
  float qr[GC][VEC];
  const int qperm = PBC ? (lane & 3) : 0;
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    const int gq = g ^ qperm;
    const bool hv = g0 + gq < p.G;
    const int h = (kvh * HP + hl) * p.G + g0 + (hv ? gq : 0);
    const int64_t qb = (zq * p.H + h) * D + dsub * VEC;
    load_elems<VEC>(p.q, p.q_dtype, qb, qr[g]);
  }
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    const bool hv = g0 + (g ^ qperm) < p.G;
#pragma unroll
    for (int e = 0; e < VEC; ++e) qr[g][e] = hv ? (DQ ? qr[g][e] : qr[g][e] * p.qscale) : 0.0f;
  }
  uint32_t qp[DQ ? GC : 1][DQ ? VEC / 2 : 1];
  if constexpr (DQ) {
#pragma unroll
    for (int g = 0; g < GC; ++g)
#pragma unroll
      for (int w = 0; w < VEC / 2; ++w) qp[g][w] = pack_pair_exact<DQ>(qr[g][2 * w], qr[g][2 * w + 1]);
  }

  float m[GC], l[GC], acc[GC][VEC], mx[GC];
  float m_own = kNegBig, mx_own = kNegBig;  // PBC: this lane's head's reference point and true maximum
  float l_own = 0.0f;                       // PBC: this lane's head's row sum
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    m[g] = kNegBig;
    mx[g] = kNegBig;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[g][e] = 0.0f;
  }
  int bad = 0;

  // Byte strides.  The host guarantees block and token strides (and BS times
  // the token stride) fit 32 bits, so a row address is one 64-bit
  // multiply-add on the block id plus a 32-bit in-block offset.
  const char* kbase = static_cast<const char*>(p.k) + (int64_t)kvh * HP * p.k_sh * KV::kBytes;
  const char* vbase = static_cast<const char*>(p.v) + (int64_t)kvh * HP * p.v_sh * KV::kBytes;
  const uint32_t k_sb = (uint32_t)(p.k_sb * KV::kBytes), k_st = (uint32_t)(p.k_st * KV::kBytes);
  const uint32_t v_sb = (uint32_t)(p.v_sb * KV::kBytes), v_st = (uint32_t)(p.v_st * KV::kBytes);
  const uint32_t lane_off = (uint32_t)(sub * VEC * KV::kBytes);
  const int32_t* bt_row = p.block_tables + (int64_t)b * p.bt_stride;
  const uint64_t nb = (uint64_t)p.num_blocks;
  // The same range check in 32 bits (a scalar compare for a wave-uniform
  // block id instead of a 64-bit vector one): block ids are int32, so a pool
  // of more than 2^31 blocks accepts every non-negative one, and a negative
  // id reads as >= 2^31.
  const uint32_t nb32 = nb > 0x80000000ull ? 0x80000000u : (uint32_t)nb;
  constexpr bool SADDR = GC > 1 || KV::kCode == kFP8;

  // One wave tile in flight: raw K/V rows of NI tokens per lane and which of
  // them are live (inside the partition, on a page with a valid block id).
  struct Tile {
    typename KV::Raw k[NI], v[NI];
    uint32_t live;
  };

  // Issue the loads of the tile starting at token `tile` (block ids from the
  // LDS-staged chunk starting at page cp).  Every lane loads: a token past
  // the partition end, or on a page with an invalid block id, reads row 0 of
  // block 0 (always in bounds, NB >= 1) and is masked out of the softmax.
  // tok(i): this lane's token of load i; ct1: this lane's end.
  auto issue_at = [&](auto&& tok, int cp, int ct1, Tile& T) {
    int blk[NI], off[NI];
    bool val[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int t = tok(i);
      val[i] = t < ct1;
      const int tt = val[i] ? t : ct1 - 1;
      const int pg = (int)fastdiv((uint32_t)tt, p.bs_div);
      off[i] = tt - pg * p.BS;
      blk[i] = s_bt[pg - cp];
    }
    uint32_t live = 0;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const bool okb = (uint64_t)(int64_t)blk[i] < nb;
      bad |= (val[i] && !okb) ? 1 : 0;
      const uint32_t bb = okb ? (uint32_t)blk[i] : 0u;
      const uint32_t oo = okb ? (uint32_t)off[i] : 0u;
      T.k[i] = load_raw<KV>(kbase, (uint64_t)bb * k_sb + (oo * k_st + lane_off));
      T.v[i] = load_raw<KV>(vbase, (uint64_t)bb * v_sb + (oo * v_st + lane_off));
      live |= (val[i] && okb) ? (1u << i) : 0u;
    }
    T.live = live;
    // Keep the loads here: the scheduler would otherwise sink them next to
    // their uses (to save registers) and serialise memory behind compute.
    __builtin_amdgcn_sched_barrier(0);
  };
  auto issue = [&](int tile, int cp, int ct1, Tile& T) {
    issue_at([&](int i) { return tile + i * TPI + slot; }, cp, ct1, T);
  };

  // Fast gather.  When BS is a multiple of TPI and tiles start on multiples
  // of TPI, the TPI rows of one load instruction lie in one page: the page's
  // block id and row base are wave-uniform (scalar registers) and a lane's
  // offset into the rows is loop-invariant, so issuing a load costs no
  // vector ALU work.  A row outside the partition or on an invalid block
  // reads row `slot` of block 0 (in bounds) and is masked.
  const uint32_t lane_row_k = (uint32_t)slot * k_st + lane_off;
  const uint32_t lane_row_v = (uint32_t)slot * v_st + lane_off;
  auto issue_fast = [&](int tile, int cp, int ct1, Tile& T) {
    // GQA groups and FP8 caches (bound by vector issue): the lanes' row
    // offsets re-enter the block through an empty asm, so the 32 -> 64-bit
    // extension of the address sits next to the loads and they take the
    // scalar-base form (SGPR base + 32-bit VGPR offset) instead of a 64-bit
    // VGPR address built by three vector instructions per load (FP8 config
    // 3 +2.7 %, FP8 config 2 +1 %; 16-bit MHA work-groups, bound by HBM,
    // measured -0.2 to -1 % and keep the plain form).
    uint32_t ork = lane_row_k, orv = lane_row_v;
    if constexpr (SADDR) asm volatile("" : "+v"(ork), "+v"(orv));
    int off0[NI], braw[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {  // all block-id reads first: one LDS round trip per tile
      const int ti = tile + i * TPI;  // wave-uniform first token of the instruction
      const int pg = (int)fastdiv((uint32_t)ti, p.bs_div);
      off0[i] = ti - pg * p.BS;
      braw[i] = s_bt[min(pg - cp, kBtChunk - 1)];
    }
    uint32_t live = 0;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int ti = tile + i * TPI;
      const int blk = __builtin_amdgcn_readfirstlane(braw[i]);
      const bool inrange = ti < ct1;
      const bool okb = inrange && (SADDR ? (uint32_t)blk < nb32 : (uint64_t)(int64_t)blk < nb);
      bad |= (inrange && !okb) ? 1 : 0;
      const uint32_t use = okb ? 1u : 0u;
      const uint64_t rk = (uint64_t)((uint32_t)blk * use) * k_sb + (uint32_t)off0[i] * use * k_st;
      const uint64_t rv = (uint64_t)((uint32_t)blk * use) * v_sb + (uint32_t)off0[i] * use * v_st;
      T.k[i] = load_raw<KV>(kbase + rk, ork);
      T.v[i] = load_raw<KV>(vbase + rv, orv);
      live |= (okb && ti + slot < ct1) ? (1u << i) : 0u;
    }
    T.live = live;
    __builtin_amdgcn_sched_barrier(0);
  };

  // Online-softmax update of this lane group's streams with one tile.
  auto consume = [&](const Tile& T) {
    float s[PBC ? 1 : NI][PBC ? 1 : GC];  // every head's score of each token
    float so[PBC ? NI : 1];                // PBC: this lane's head's score
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float d[GC];  // this lane's partial dot products
      if constexpr (DQ) {
        uint32_t kp[VEC / 2];
        KV::template to_pairs<DQ>(T.k[i], kp);
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          // GQA groups start each chain from the three-operand form (no zero
          // move: FP8 config 3 +3 %); one-head work-groups, bound by HBM
          // rather than vector issue, keep the builtin's code.
          if constexpr (GC > 1) {
            d[g] = dot2_first<DQ>(qp[g][0], kp[0]);
          } else {
            d[g] = dot2<DQ>(qp[g][0], kp[0], 0.0f);
          }
#pragma unroll
          for (int w = 1; w < VEC / 2; ++w) d[g] = dot2<DQ>(qp[g][w], kp[w], d[g]);
        }
      } else {
        float kf[VEC];
        KV::widen(T.k[i], kf);
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          d[g] = 0.0f;
#pragma unroll
          for (int e = 0; e < VEC; ++e) d[g] = fmaf(qr[g][e], kf[e], d[g]);
        }
      }
      const float sc = DQ ? p.qscale : 1.0f;
      if constexpr (PBC) {
        // Transposing sum over the 16-lane slot: after the two quad steps
        // lane j of each quad holds head j's sum over the quad, then the
        // four quads are added (row rotations by 4 and 8).
        // Slots hold heads j, j^1, j^2, j^3 (j = lane % 4): the xor-1
        // partner's slots 1 and 3 are this lane's heads j and j^2, and the
        // xor-2 partner's k1 is head j.
        const float k0 = d[0] + dpp<kDppXor1>(d[1]);
        const float k1 = d[2] + dpp<kDppXor1>(d[3]);
        float k = k0 + dpp<kDppXor2>(k1);
        // Rotation by 8 first: quad q then holds (P_q + P_q+2) + (P_q+1 + P_q+3)
        // in an order that differs between quads only by commuting operands,
        // so all four quads hold bitwise-identical sums.
        k += dpp<kDppRor8>(k);
        k += dpp<kDppRor4>(k);
        so[i] = k * sc;
      } else {
#pragma unroll
        for (int g = 0; g < GC; ++g) s[i][g] = group_sum<LPH>(d[g]) * sc;
      }
    }
    // A masked token has weight 0, but its V row may be the rest of the last
    // page past the context end, or row `slot` of block 0 substituted for a
    // token past the partition, and either may hold any bits: 0 * NaN is NaN.
    // Those rows are zeroed before P.V, one select per raw word (all-zero
    // bits are +0 in every KV type).  Unconditional selects: a wave-uniform
    // branch around them measured cheaper in instructions but cost 20-30
    // registers (and an occupancy step) in most kernels.
    typename KV::Raw vr[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const bool lv = (T.live >> i) & 1u;
#pragma unroll
      for (int w = 0; w < (int)(sizeof(vr[i]) / 4); ++w) vr[i][w] = lv ? T.v[i][w] : 0u;
    }
    // V for P.V: fp32 rows (vf), or, on the packed path, element pairs across
    // two tokens (vlo: element 2w of tokens 2u and 2u+1, vhi: element 2w+1).
    float vf[PVP ? 1 : NI][PVP ? 1 : VEC];
    uint32_t vlo[PVP ? NI / 2 : 1][PVP ? VEC / 2 : 1], vhi[PVP ? NI / 2 : 1][PVP ? VEC / 2 : 1];
    if constexpr (PVP && KV::kCode == kFP8) {
      // FP8: interleave the two tokens' codes byte by byte first (two
      // v_perm_b32 per code word of each token), so that each packed
      // conversion yields a cross-token fp16 pair directly.
#pragma unroll
      for (int u = 0; u < NI / 2; ++u)
#pragma unroll
        for (int j = 0; j < VEC / 4; ++j) {
          const uint32_t x0 = __builtin_amdgcn_perm(vr[2 * u + 1][j], vr[2 * u][j], 0x05010400u);
          const uint32_t x1 = __builtin_amdgcn_perm(vr[2 * u + 1][j], vr[2 * u][j], 0x07030602u);
          vlo[u][2 * j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x0, 1.0f, false));
          vhi[u][2 * j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x0, 1.0f, true));
          vlo[u][2 * j + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x1, 1.0f, false));
          vhi[u][2 * j + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x1, 1.0f, true));
        }
    } else if constexpr (PVP) {
      uint32_t vp[NI][VEC / 2];
#pragma unroll
      for (int i = 0; i < NI; ++i) KV::template to_pairs<kF16>(vr[i], vp[i]);
#pragma unroll
      for (int u = 0; u < NI / 2; ++u)
#pragma unroll
        for (int w = 0; w < VEC / 2; ++w) {
          vlo[u][w] = __builtin_amdgcn_perm(vp[2 * u + 1][w], vp[2 * u][w], 0x05040100u);
          vhi[u][w] = __builtin_amdgcn_perm(vp[2 * u + 1][w], vp[2 * u][w], 0x07060302u);
        }
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i) KV::widen(vr[i], vf[i]);
    }
    float pw[NI][GC];  // weights 2^(s - m) of each token and head
    uint32_t wp[PBC && PVP ? NI / 2 : 1][GC];  // PBC with packed P.V: the weights as fp16 pairs of two tokens
    if constexpr (PBC) {
      // The lane's own head: its tile maximum, the lazy test against its
      // reference point, and one exponential per token, shared across the quad.
      float mt = kNegBig;
#pragma unroll
      for (int i = 0; i < NI; ++i) mt = ((T.live >> i) & 1u) ? fmaxf(mt, so[i]) : mt;
      mx_own = fmaxf(mx_own, mt);
      const bool up = mt > m_own + 8.0f;
      if (__builtin_amdgcn_ballot_w64(up) != 0) {
        const float mtg[4] = {dpp_quad<0x00>(mt), dpp_quad<0x55>(mt), dpp_quad<0xAA>(mt), dpp_quad<0xFF>(mt)};
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          const float mn = mtg[g] > m[g] + 8.0f ? mtg[g] : m[g];
          const float corr = fast_exp2(m[g] - mn);
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[g][e] *= corr;
          m[g] = mn;
        }
        l_own *= fast_exp2(m_own - (up ? mt : m_own));
        m_own = up ? mt : m_own;
      }
      float pl[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) pl[i] = ((T.live >> i) & 1u) ? fast_exp2(so[i] - m_own) : 0.0f;
      if constexpr (PVP) {
        // The lane's own head: two tokens' weights as one fp16 pair, its row
        // sum over the rounded pair, and the pairs shared across the quad.
#pragma unroll
        for (int u = 0; u < NI / 2; ++u) {
          const uint32_t own =
              __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{pl[2 * u], pl[2 * u + 1]}, f16x2_t));
          l_own = dot2<kF16>(own, 0x3c003c00u, l_own);
          wp[u][0] = dpp_quad_u<0x00>(own);
          wp[u][1] = dpp_quad_u<0x55>(own);
          wp[u][2] = dpp_quad_u<0xAA>(own);
          wp[u][3] = dpp_quad_u<0xFF>(own);
        }
      } else {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          l_own += pl[i];
          pw[i][0] = dpp_quad<0x00>(pl[i]);
          pw[i][1] = dpp_quad<0x55>(pl[i]);
          pw[i][2] = dpp_quad<0xAA>(pl[i]);
          pw[i][3] = dpp_quad<0xFF>(pl[i]);
        }
      }
    } else {
      // Lazy rescale: a stream's reference point m is raised only when a tile
      // exceeds it by more than 2^8 (8 in log2 units), so every weight stays
      // <= 256 (softmax is invariant to the reference point).  The test is
      // wave-uniform, so the common case skips the correction exponentials and
      // the accumulator rescale.  mx tracks the true maximum; the streams are
      // rebased onto it once, after the last tile.  GQA groups only: for one
      // head per work-group (bound by HBM, not vector work) the branch costs
      // more than it saves.
      float mn[GC];
      uint32_t raise = 0;
#pragma unroll
      for (int g = 0; g < GC; ++g) {
        float mt = kNegBig;
#pragma unroll
        for (int i = 0; i < NI; ++i) mt = ((T.live >> i) & 1u) ? fmaxf(mt, s[i][g]) : mt;
        mn[g] = LAZY ? (mt > m[g] + 8.0f ? mt : m[g]) : fmaxf(m[g], mt);
        raise |= mn[g] != m[g] ? 1u : 0u;
        if constexpr (LAZY) mx[g] = fmaxf(mx[g], mt);
      }
      if (!LAZY || __builtin_amdgcn_ballot_w64(raise != 0) != 0) {
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          const float corr = fast_exp2(m[g] - mn[g]);
          l[g] *= corr;
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[g][e] *= corr;
          m[g] = mn[g];
        }
      }
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int g = 0; g < GC; ++g) pw[i][g] = ((T.live >> i) & 1u) ? fast_exp2(s[i][g] - m[g]) : 0.0f;
    }
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      float lg = l[g];
      if constexpr (PVP) {
        // Weights of two tokens as one fp16 pair (<= 256 by the lazy rescale;
        // 2^-12 relative rounding), the row sum over the same rounded weights,
        // then one packed dot product per element: acc[e] += p0 v0[e] + p1 v1[e].
#pragma unroll
        for (int u = 0; u < NI / 2; ++u) {
          uint32_t pp;
          if constexpr (PBC) {
            pp = wp[u][g];
          } else {
            const float p0 = pw[2 * u][g];
            const float p1 = pw[2 * u + 1][g];
            pp = __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{p0, p1}, f16x2_t));
            lg = dot2<kF16>(pp, 0x3c003c00u, lg);
          }
#pragma unroll
          for (int w = 0; w < VEC / 2; ++w) {
            acc[g][2 * w] = dot2<kF16>(vlo[u][w], pp, acc[g][2 * w]);
            acc[g][2 * w + 1] = dot2<kF16>(vhi[u][w], pp, acc[g][2 * w + 1]);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const float pi = pw[i][g];
          if constexpr (!PBC) lg += pi;
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[g][e] = fmaf(pi, vf[i][e], acc[g][e]);
        }
      }
      l[g] = lg;
    }
  };

  // Rebase each stream from its lazy reference point onto its true maximum
  // (the partials carry the maximum, kernels/paged_attn_v3.cu:113-122).
  auto rebase = [&]() {
    if constexpr (LAZY) {
      if constexpr (PBC) {  // the heads' maxima and row sums live in the quad's lanes
        mx[0] = dpp_quad<0x00>(mx_own);
        mx[1] = dpp_quad<0x55>(mx_own);
        mx[2] = dpp_quad<0xAA>(mx_own);
        mx[3] = dpp_quad<0xFF>(mx_own);
        l[0] = dpp_quad<0x00>(l_own);
        l[1] = dpp_quad<0x55>(l_own);
        l[2] = dpp_quad<0xAA>(l_own);
        l[3] = dpp_quad<0xFF>(l_own);
      }
#pragma unroll
      for (int g = 0; g < GC; ++g) {
        const float corr = fast_exp2(m[g] - mx[g]);
        l[g] *= corr;
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[g][e] *= corr;
        m[g] = mx[g];
      }
    }
  };

  // Combine the TPI slot streams of this wave (log-sum-exp rule).
  auto combine_slots = [&]() {
#pragma unroll
    for (int off = LPT; off < 64; off <<= 1) {
#pragma unroll
      for (int g = 0; g < GC; ++g) {
        const float mo = __shfl_xor(m[g], off, 64);
        const float lo = __shfl_xor(l[g], off, 64);
        const float mn = fmaxf(m[g], mo);
        const float a = fast_exp2(m[g] - mn);
        const float c = fast_exp2(mo - mn);
        l[g] = l[g] * a + lo * c;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float ao = __shfl_xor(acc[g][e], off, 64);
          acc[g][e] = acc[g][e] * a + ao * c;
        }
        m[g] = mn;
      }
    }
  };

  if (spm) {
    // The work-group's block-table entries in one staged chunk (the host
    // enables the mode only when they fit).  Each slot streams its own
    // partition of each round, NI consecutive tokens per tile (a token past
    // its end reads the masked safe row); the tile count is the chunk's,
    // wave-uniform, rounded up to even.  The two-tile pipeline runs on
    // across rounds: a round's first tile is issued before the previous
    // round's last is consumed.
    const int cp = T0 < T1 ? (int)fastdiv((uint32_t)T0, p.bs_div) : 0;
    if (T0 < T1) {
      const int np = (int)fastdiv((uint32_t)(T1 - 1), p.bs_div) + 1 - cp;
      if (bt_early && cp == pg_early) {
        static_assert(kBtChunk <= kDecodeThreads, "one prefetched entry per thread");
        if ((int)threadIdx.x < np) s_bt[threadIdx.x] = bt_pre;
      } else {
        for (int i = threadIdx.x; i < np; i += kDecodeThreads) s_bt[i] = bt_row[cp + i];
      }
      __syncthreads();
    }
    const int R = p.rounds;
    const int nt = ((chunk + NI - 1) / NI + 1) & ~1;  // tiles per round (even)
    // Fused output (GC == 1): each slot's partitions merged as they complete
    // (log-sum-exp rule), then the wave's slots and the waves as below.  A
    // bad block id poisons its own partition's partial and the output.
    float mT = kNegBig, lT = 0.0f, aT[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) aT[e] = 0.0f;
    int bad_all = 0;
    int cr = 0;  // round being consumed
    auto finish = [&]() __attribute__((always_inline)) {
      rebase();
      // This slot's partition: its partials from its lanes (dims dsub * VEC
      // .. of head hl), m and l from those of dsub 0.  The fused form keeps
      // them in registers only: the workspace is the split's scratch, and
      // the partials' writes (3 % of the bytes, 4-byte m and l stores among
      // them) took config 2 at 64 splits from 0.77 to 0.68 of 8 TB/s.
      const int pr = part + cr * NW * TPI;
      if (pr < nparts && !p.fuse_final) {
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          if (g0 + g >= p.G) continue;
          const int h = (kvh * HP + hl) * p.G + g0 + g;
          const int64_t pidx = ((int64_t)b * p.H + h) * p.parts + pr;
#pragma unroll
          for (int e = 0; e < VEC; ++e) p.ws_acc[pidx * D + dsub * VEC + e] = acc[g][e] * p.vscale;
          if (dsub == 0) {
            p.ws_m[pidx] = m[g];
            p.ws_l[pidx] = bad ? __builtin_nanf("") : l[g];
          }
        }
      }
      if constexpr (GC == 1) {
        if (p.fuse_final) {
          const float mn = fmaxf(mT, m[0]);
          const float ca = fast_exp2(mT - mn), cb = fast_exp2(m[0] - mn);
          lT = lT * ca + l[0] * cb;
#pragma unroll
          for (int e = 0; e < VEC; ++e) aT[e] = aT[e] * ca + acc[0][e] * cb;
          mT = mn;
        }
      }
#pragma unroll
      for (int g = 0; g < GC; ++g) {
        m[g] = kNegBig;
        mx[g] = kNegBig;
        l[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[g][e] = 0.0f;
      }
      m_own = kNegBig;
      mx_own = kNegBig;
      l_own = 0.0f;
      bad_all |= bad;
      bad = 0;
      ++cr;
    };
    if (T0 < T1) {
      // Issue position (round ir, token offset iu); past the last round a
      // tile reads the masked safe row of the last round's partition.  Each
      // tile carries the bad flag of its own loads, taken at consume time.
      int ir = 0, iu = 0;
      auto iss = [&](Tile& T, int& tb) __attribute__((always_inline)) {
        const int pr = part + min(ir, R - 1) * NW * TPI;
        const int r0 = min(pr * chunk, ctx), r1 = min(r0 + chunk, ctx);
        const int u = ir < R ? iu : chunk;
        const int keep = bad;
        bad = 0;
        issue_at([&](int i) { return r0 + u + i; }, cp, r1, T);
        tb = bad;
        bad = keep;
        iu += NI;
        if (iu >= nt * NI) {
          iu = 0;
          ++ir;
        }
      };
      const int ntot = nt * R;
      Tile A, B;
      int ba, bb, cu = 0;
      iss(A, ba);
      for (int j = 0; j < ntot; j += 2) {
        iss(B, bb);
        bad |= ba;
        consume(A);
        iss(A, ba);
        bad |= bb;
        consume(B);
        cu += 2;
        if (cu == nt) {
          finish();
          cu = 0;
        }
      }
    } else {
      for (int r = 0; r < R; ++r) finish();  // empty partitions: m = -3e38, l = 0
    }
    bad = bad_all;
    if constexpr (GC != 1) return;
    if (!p.fuse_final) return;  // work-group uniform
    m[0] = mT;
    mx[0] = mT;
    l[0] = lT;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[0][e] = aT[e];
  } else {
    const bool fast = (p.BS % TPI) == 0 && (t0 % TPI) == 0;
    if (T0 < T1) {
      const int pg0 = (int)fastdiv((uint32_t)T0, p.bs_div);
      const int pg1 = (int)fastdiv((uint32_t)(T1 - 1), p.bs_div) + 1;
      for (int cp = pg0; cp < pg1; cp += kBtChunk) {
        const int np = min(kBtChunk, pg1 - cp);
        __syncthreads();
        if (bt_early && cp == pg0 && pg0 == pg_early) {
          static_assert(kBtChunk <= kDecodeThreads, "one prefetched entry per thread");
          if ((int)threadIdx.x < np) s_bt[threadIdx.x] = bt_pre;
        } else {
          for (int i = threadIdx.x; i < np; i += kDecodeThreads) s_bt[i] = bt_row[cp + i];
        }
        __syncthreads();
        const int ct0 = max(t0, cp * p.BS);
        const int ct1 = min(t1, (cp + np) * p.BS);
        // Two tiles per wave in flight: the loads of the next tile are issued
        // before the current one is consumed.  The next-tile issue is
        // unconditional (past the end it reads the masked safe row), so every
        // path reaching a consume has the same loads outstanding and the wait
        // before it covers only the current tile.
        auto sweep = [&](auto&& iss) {
          const int kStep = wpm ? TT : NW * TT;  // this wave's tiles: its own partition's, or every NW-th
          const int first = wpm ? ct0 : ct0 + wave * TT;
          if (first < ct1) {
            // Counted, branch-free body: tile j+1 is issued before tile j is
            // consumed.  Every entry of the loop header has exactly one tile
            // (in A) outstanding, so the waits stay partial.
            const int ntw = (ct1 - first + kStep - 1) / kStep;  // tiles of this wave
            Tile A, B;
            int tile = first;
            const bool prio = PPRIO && p.pprio;  // work-group uniform
            if (prio) __builtin_amdgcn_s_setprio(3);
            const int e1 = (ntw / 2) & ~1, e2 = (3 * ntw / 4) & ~1, e3 = (7 * ntw / 8) & ~1;
            iss(tile, cp, ct1, A);
            for (int j = 0; j + 1 < ntw; j += 2) {
              if (prio) {
                if (j == e1) __builtin_amdgcn_s_setprio(2);
                if (j == e2) __builtin_amdgcn_s_setprio(1);
                if (j == e3) __builtin_amdgcn_s_setprio(0);
              }
              iss(tile + kStep, cp, ct1, B);
              consume(A);
              iss(tile + 2 * kStep, cp, ct1, A);
              consume(B);
              tile += 2 * kStep;
            }
            if (ntw & 1) consume(A);
          }
        };
        if (fast) {
          sweep(issue_fast);
        } else {
          sweep(issue);
        }
      }
    }
  }  // slot-partition mode / plain sweep
  rebase();
  combine_slots();
  if (wpm) {
    // This wave's partition complete: its partials straight from the lanes
    // of slot 0 (dims dsub * VEC .. of head hl), m and l from those of dsub 0.
    const bool wbad = __builtin_amdgcn_ballot_w64(bad != 0) != 0;
    if (slot == 0 && part < nparts) {
#pragma unroll
      for (int g = 0; g < GC; ++g) {
        if (g0 + g >= p.G) continue;
        const int h = (kvh * HP + hl) * p.G + g0 + g;
        const int64_t pidx = ((int64_t)b * p.H + h) * p.parts + part;
#pragma unroll
        for (int e = 0; e < VEC; ++e) p.ws_acc[pidx * D + dsub * VEC + e] = acc[g][e] * p.vscale;
        if (dsub == 0) {
          p.ws_m[pidx] = m[g];
          p.ws_l[pidx] = wbad ? __builtin_nanf("") : l[g];
        }
      }
    }
    return;
  }
  if (slot == 0) {
#pragma unroll
    for (int g = 0; g < GC; ++g)
#pragma unroll
      for (int e = 0; e < VEC; ++e) s_acc[wave][g][sub * VEC + e] = acc[g][e];
  }
  if (slot == 0 && dsub == 0) {
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      s_m[wave][g * HP + hl] = m[g];
      s_l[wave][g * HP + hl] = l[g];
    }
  }
  bad = __syncthreads_or(bad);

  // Combine the waves and write out.
  for (int idx = threadIdx.x; idx < GC * HP * D; idx += kDecodeThreads) {
    const int g = idx / (HP * D), dd = idx - g * (HP * D);
    const int d = dd % D, hh = dd / D;
    if (g0 + g >= p.G) continue;
    const int gh = g * HP + hh;
    float M = kNegBig;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][gh]);
    float L = 0.0f, A = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = fast_exp2(s_m[w][gh] - M);
      L += s_l[w][gh] * wt;
      A += s_acc[w][g][dd] * wt;
    }
    const int h = (kvh * HP + hh) * p.G + g0 + g;
    if (final_here) {
      store_elem(p.out, p.out_dtype, (zq * p.H + h) * D + d,
                 bad ? __builtin_nanf("") : A * p.vscale / L);
    } else {
      const int64_t pidx = ((int64_t)b * p.H + h) * p.parts + part;
      p.ws_acc[pidx * D + d] = A * p.vscale;
      if (d == 0) {
        p.ws_m[pidx] = M;
        p.ws_l[pidx] = bad ? __builtin_nanf("") : L;
      }
    }
  }
}

// Work-groups of `kernel` resident at once on the current device (CUs x
// work-groups per CU), cached per device; 0 when the runtime cannot say.
template <typename F>
inline int64_t decode_residency(F kernel, std::atomic<int64_t> (&cache)[64]) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64) {
    const int64_t c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0, k = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&k, kernel, kDecodeThreads, 0) != hipSuccess || k <= 0) return 0;
  const int64_t r = (int64_t)n * k;
  if (dev < 64) cache[dev].store(r, std::memory_order_relaxed);
  return r;
}

template <typename KV, int D, int GC, int HP, int DQ>
hipError_t launch_decode_one(const DecodeParams& p, int64_t blocks, hipStream_t stream) {
  const auto kernel = decode_kernel<KV, D, GC, HP, DQ>;
  DecodeParams q = p;
  q.pprio = 0;
  if constexpr (GC == 1 && HP == 1) {
    static std::atomic<int64_t> cache[64];
    const int64_t res = decode_residency(kernel, cache);
    q.pprio = res > 0 && blocks <= res ? 1 : 0;
  }
  note_launch("pa::decode_kernel<%s, %d, %d, %d, %d>", KV::kName, D, GC, HP, DQ);
  hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(kDecodeThreads), 0, stream, q);
  return hipGetLastError();
}

template <typename KV, int D, int GC, int HP = 1>
hipError_t launch_decode_dg(const DecodeParams& p0, hipStream_t stream) {
  DecodeParams p = p0;
  // Short explicit partitions.  A call whose host plan fuses
  // (decode_fuse_rounds(), GC == 1) takes the slot-partition mode in rounds:
  // one work-group per unit.  Otherwise one partition per token slot when
  // every slot of a work-group has one (parts >= kDecodeWaves * TPI) and the
  // work-group's pages fit one staged block-table chunk; else one per wave.
  constexpr int TPI = DecodeShapeOf<KV, D, GC, HP>::TPI;
  const int fr = GC == 1 && p.fuse_final && p.wave_parts ? decode_fuse_rounds(p.parts, p.MB, p.BS, TPI) : 0;
  p.fuse_final = fr > 0 ? 1 : 0;
  p.rounds = 1;
  if (fr > 0) {
    p.wave_parts = kSlotPart;
    p.rounds = fr;
    t_decode_fused = 1;
  } else if (p.wave_parts) {
    const int64_t chunk_max = ((int64_t)p.MB * p.BS + p.parts - 1) / p.parts;
    const int64_t pages = ((int64_t)kDecodeWaves * TPI * chunk_max + p.BS - 1) / p.BS + 1;
    p.wave_parts = p.parts >= kDecodeWaves * TPI && pages <= kBtChunk ? kSlotPart : kWavePart;
  }
  const int64_t gparts = p.wave_parts == kSlotPart ? (int64_t)kDecodeWaves * TPI * p.rounds
                                                   : p.wave_parts ? kDecodeWaves : 1;
  const int64_t groups = (p.parts + gparts - 1) / gparts;
  const int64_t blocks = (int64_t)p.B * p.Sq * (p.HKV / HP) * p.head_chunks * groups;
  constexpr int PTS = pair_types<KV>::value;
  if constexpr ((PTS >> kF16) & 1) {
    if (p.q_dtype == kF16) return launch_decode_one<KV, D, GC, HP, kF16>(p, blocks, stream);
  }
  if constexpr ((PTS >> kBF16) & 1) {
    if (p.q_dtype == kBF16) return launch_decode_one<KV, D, GC, HP, kBF16>(p, blocks, stream);
  }
  return launch_decode_one<KV, D, GC, HP, 0>(p, blocks, stream);
}

template <typename KV, int D>
hipError_t launch_decode_d(const DecodeParams& p, int gc, hipStream_t stream) {
  // Packed heads (the plan's choice) need K's and V's heads contiguous.
  if (gc == 1 && p.hp > 1 && p.k_sh == D && p.v_sh == D && p.HKV % p.hp == 0) {
    if constexpr (D * KV::kBytes * 4 <= kPackRowBytes) {
      if (p.hp == 4) return launch_decode_dg<KV, D, 1, 4>(p, stream);
    }
    if constexpr (D * KV::kBytes * 2 <= kPackRowBytes) {
      if (p.hp == 2) return launch_decode_dg<KV, D, 1, 2>(p, stream);
    }
  }
  // GQA groups of four with two KV heads per work-group (one head chunk).
  if (gc == 4 && p.G == 4 && p.hp == 2 && p.k_sh == D && p.v_sh == D && p.HKV % 2 == 0) {
    static_assert(kPackGqaMax == 2, "GQA groups of four pack at most two KV heads");
    if constexpr (KV::kBytes <= 2 && D * KV::kBytes * 2 <= kPackRowBytes) return launch_decode_dg<KV, D, 4, 2>(p, stream);
  }
  switch (gc) {
    case 1: return launch_decode_dg<KV, D, 1>(p, stream);
    case 2: return launch_decode_dg<KV, D, 2>(p, stream);
    case 4: return launch_decode_dg<KV, D, 4>(p, stream);
    case 8: return launch_decode_dg<KV, D, 8>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

template <typename KV>
hipError_t launch_decode_kv(const DecodeParams& p, int gc, hipStream_t stream) {
  switch (p.D) {
    case 32: return launch_decode_d<KV, 32>(p, gc, stream);
    case 64: return launch_decode_d<KV, 64>(p, gc, stream);
    case 128: return launch_decode_d<KV, 128>(p, gc, stream);
    case 256:
      if constexpr (KV::kBytes <= 4) return launch_decode_d<KV, 256>(p, gc, stream);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pa
