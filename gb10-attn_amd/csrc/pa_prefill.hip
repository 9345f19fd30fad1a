// pa_prefill.hip -- causal paged prefill on CDNA4 matrix cores (gfx950).
//
// Replaces the reference's WMMA tile kernel (kernels/paged_attn_wmma.cu:36-210)
// with a design built around v_mfma_f32_32x32x16_{f16,bf16}:
//
//  * A work-group (4 waves) owns one (sequence b, query head h, block of 128
//    query rows); wave w owns 32 of those rows, one MFMA n-tile.  The kernel
//    is sized for two work-groups per CU (<= 256 registers per lane, 68 KB of
//    LDS), so every SIMD holds two waves and one wave's softmax arithmetic
//    overlaps the other's matrix work.
//  * Key tiles (64 keys for D <= 128, 32 for D = 256) are gathered from the
//    paged pool (block table -> page -> row, 64-bit offsets) straight into
//    LDS with global_load_lds_dwordx4: no registers or VALU stores on the way,
//    and the next tile's loads are in flight while the current one is used.
//    Rows are XOR-swizzled in 16-byte chunks (the swizzle is applied on the
//    global side, since a wave's direct load fills 1 KB of LDS in lane order).
//  * Scores are computed transposed, S^T = K . Q^T: K rows are the MFMA A
//    operand read from LDS (16 bytes per lane), the wave's 32 query rows are
//    the B operand held in registers for the whole loop.  In the 32x32 S^T
//    accumulator layout a lane holds 16 keys of one query column, eight of
//    which are exactly the B operand slots of one 16-key step of
//    O^T += V^T . P^T -- probabilities never leave registers.  The V^T A
//    operand is two ds_read_b64_tr_b16 per step.
//  * The softmax is done in log2 units with the scale folded into one FMA per
//    score; the running max is only raised when a tile's max exceeds it by
//    more than 2^8 (probabilities stay <= 256, exact in fp16/bf16 range), so
//    the O^T rescale is a rare wave-uniform branch instead of a per-tile
//    multiply.  Masking runs only on tiles that cross a wave's diagonal.
//  * Work-groups are ordered by query block, longest first, across all
//    (sequence, head) pairs.  (Grouping one (sequence, head)'s blocks on one
//    XCD, for L2 reuse, put three blocks of the same length on each CU when
//    all work-groups are resident: config 4a ran 22 % slower.)
//
// Semantics follow kernels/paged_attn_wmma.cu:80-205: query row r of the
// chunk sits at ctx - S + r and sees keys [0, ctx - S + r]; accumulation and
// the softmax are fp32; a row that sees no key is written as zeros (:200).
// Precision: P is carried in fp16 (11-bit significand) as the reference does.
// A bf16 V tile is converted to fp16 while it is staged, so P.V runs in fp16
// too; if any staged |v| reaches 65520 (fp16 overflow, or inf) the
// work-group restarts in a mode that keeps V in bf16 and carries P as a bf16
// hi + lo pair (two P.V products, ~16-bit significand).  q that does not
// arrive in the KV type is likewise split into hi + lo for Q.K^T.
#include "pa_device.hpp"

#include <atomic>

namespace pa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;
typedef __attribute__((address_space(3))) void lds_void_t;
typedef uint64_t u64x2_t __attribute__((ext_vector_type(2)));

// 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4):
// lane i writes lds + 16*i; lds must be wave-uniform.  (A function of its own:
// used directly in the kernel template, the builtin stops the host pass from
// emitting the launch stubs.)
__device__ inline void lds_dma16(const void* g, lds_void_t* lds) {
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}

// The same load as inline asm (M0 set by the compiler from the operand).  The
// compiler does not see it write LDS, so it places no wait for it before later
// LDS reads; the caller waits (vmcnt) before the barrier that publishes the data.
__device__ inline void lds_dma16_async(const void* g, lds_void_t* lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "{m0}"(m));
}

template <bool kBf16>
__device__ inline f32x16_t mfma32(const u32x4_t& a, const u32x4_t& b, const f32x16_t& c) {
  if constexpr (kBf16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a),
                                                  __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
  }
}

// Two fp32 values -> one packed 16-bit pair, round to nearest even.
template <bool kBf16>
__device__ inline uint32_t pack2(float x, float y) {
  if constexpr (kBf16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{x, y}, bf16x2_t));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{x, y}, half2_t));
  }
}

// The two fp32 values of a packed 16-bit pair.
template <bool kBf16>
__device__ inline float2_t unpack2(uint32_t w) {
  if constexpr (kBf16) {
    return float2_t{__builtin_bit_cast(float, w << 16), __builtin_bit_cast(float, w & 0xffff0000u)};
  } else {
    const half2_t h = __builtin_bit_cast(half2_t, w);
    return float2_t{(float)h[0], (float)h[1]};
  }
}

// Eight consecutive q elements (16-byte aligned) as fp32.
__device__ inline void load8f(const void* q, int dtype, int64_t idx, float (&x)[8]) {
  if (dtype == kF32) {
    const float4_t a = *reinterpret_cast<const float4_t*>(static_cast<const float*>(q) + idx);
    const float4_t b = *reinterpret_cast<const float4_t*>(static_cast<const float*>(q) + idx + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = a[e];
      x[4 + e] = b[e];
    }
  } else {
    const u32x4_t r = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(q) + idx);
    if (dtype == kF16) {
      KvF16::widen(r, x);
    } else {
      KvBF16::widen(r, x);
    }
  }
}

constexpr int kPfThreads = 256;   // 4 waves
constexpr int kVlMaxSeqs = 256;   // variable-length batches numbered compactly (four per lane)
constexpr int kPfBtStage = 1024;  // block-table entries staged in LDS
constexpr float kLazyRescale = 8.0f;  // raise the running max only past 2^8
constexpr float kWeightCap = 32768.0f;  // 8-wave kernel: raise it when a lane's weights sum past 2^15
                                        // (weights up to 2^15 are exact in fp16 and bf16 range)


// How a tile's P.V product is formed.
enum PvMode : int {
  kPvDirect = 0,   // V tile loaded straight into LDS; P and V in fp16
  kPvConvert = 1,  // bf16 V converted to fp16 while staged; P and V in fp16
  kPvSplit = 2,    // bf16 V in LDS; P as bf16 hi + lo, two products
  kPvF8 = 3,       // FP8 K and V codes staged in registers, written to LDS as fp16 (exact)
};
template <int M>
struct PvTag {
  static constexpr int value = M;
};

// FP8 (E4M3) caches: the codes convert exactly to fp16 and to bf16, so K tiles
// take q's 16-bit type (no hi + lo split of a bf16 q) and V tiles fp16 (P
// stays fp16).  KvFP8 serves fp16 and fp32 q, KvFP8QkBf16 bf16 q.
struct KvFP8QkBf16 : KvFP8 {
  static constexpr const char* kName = "pa::KvFP8QkBf16";
};
template <typename KV>
struct QkBf16 {  // Q.K^T on bf16 MFMA
  static constexpr bool value = KV::kCode == kBF16;
};
template <>
struct QkBf16<KvFP8QkBf16> {
  static constexpr bool value = true;
};

template <int D>
struct PfShape {
  static constexpr int QW = 32;                  // query rows per wave (one MFMA n-tile)
  static constexpr int QB = 4 * QW;              // query rows per work-group
  static constexpr int KB = D <= 128 ? 64 : 32;  // keys per tile
  static constexpr int MT = KB / 32;             // 32-key m-tiles of S^T
  static constexpr int KS = D / 16;              // 16-dim k-steps of Q.K^T
  static constexpr int DT = D / 32;              // 32-dim m-tiles of O^T
  static constexpr int NCH = D / 8;              // 16-byte chunks per row
  // LDS chunk swizzles (chunk cc of row r sits at position cc ^ f(r)), one per
  // read pattern, so that every 256-byte LDS pass hits 64 distinct banks:
  //  K, read as the S^T A operand (16 consecutive rows, one chunk):
  //    f(r) = (r >> KSH) & KSW;
  //  V, read transposed (4 consecutive rows x 4 consecutive chunks per 32
  //  lanes): f(r) = ((r >> VSH) & VSW) << 2.
  static constexpr int KSW = (NCH < 16 ? NCH : 16) - 1;
  static constexpr int KSH = NCH >= 16 ? 0 : NCH == 8 ? 1 : 2;
  static constexpr int VSW = NCH >= 16 ? 3 : NCH == 8 ? 1 : 0;
  static constexpr int VSH = NCH >= 16 ? 0 : 1;
  static constexpr int CPT = KB * NCH / kPfThreads;    // chunks per thread per tile
  static constexpr int WAVES_PER_EU = D <= 128 ? 2 : 1;
  static_assert(KB * NCH % kPfThreads == 0, "tile chunks must divide the work-group");
};

// LDS element offsets of (row, chunk cc) in the swizzled [KB][D] K and V tiles.
template <int D>
__device__ inline int kpos(int row, int cc) {
  return cc ^ ((row >> PfShape<D>::KSH) & PfShape<D>::KSW);
}
template <int D>
__device__ inline int vpos(int row, int cc) {
  return cc ^ (((row >> PfShape<D>::VSH) & PfShape<D>::VSW) << 2);
}
template <int D>
__device__ inline int swk(int row, int cc) {
  return row * D + (kpos<D>(row, cc) << 3);
}
template <int D>
__device__ inline int swv(int row, int cc) {
  return row * D + (vpos<D>(row, cc) << 3);
}

// kSplit (key-split mode, tiles of two 32-key m-tiles): a work-group serves
// 64 query rows; waves 0-1 own rows 0-31 / 32-63 over the first 32 keys of
// every tile, waves 2-3 the same rows over the second 32, and the two halves
// are merged through LDS at the end (log-sum-exp rule).  The loads and the
// LDS layout are those of the plain mode; each wave does half of a tile's
// work, so a query block's chain of tiles takes half as long and twice as
// many work-groups share the work.  Chosen when the plain grid is too short
// for the dispatcher to balance causal blocks (config 4a: 768 work-groups,
// chains of 2 to 16 tiles, on 768 slots).
template <typename KV, int D, bool kSplitQ, bool kSplit>
__global__ __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(PfShape<D>::WAVES_PER_EU)))
void prefill_mfma_kernel(const PrefillParams p) {
  using Sh = PfShape<D>;
  constexpr int QW = Sh::QW, KB = Sh::KB, MT = Sh::MT, KS = Sh::KS, DT = Sh::DT;
  static_assert(!kSplit || MT == 2, "the key-split mode halves tiles of two m-tiles");
  constexpr int MTW = kSplit ? 1 : MT;           // 32-key m-tiles of each tile this wave computes
  constexpr int QB = kSplit ? 2 * QW : Sh::QB;   // query rows per work-group
  constexpr int NCH = Sh::NCH, CPT = Sh::CPT;
  constexpr bool kBf16 = QkBf16<KV>::value;  // Q.K^T operand type (and the type of a split q)
  constexpr bool kF8 = KV::kCode == kFP8;    // tiles converted from FP8 codes; P.V in fp16
  constexpr int EB = KV::kBytes;

  __shared__ __attribute__((aligned(16))) uint16_t sK0[KB * D];
  __shared__ __attribute__((aligned(16))) uint16_t sK1[KB * D];
  __shared__ __attribute__((aligned(16))) uint16_t sV0[KB * D];
  __shared__ __attribute__((aligned(16))) uint16_t sV1[KB * D];
  __shared__ int32_t s_bt[kPfBtStage];  // window of the work-group's block ids
  __shared__ int s_badkey;              // first key whose page has an invalid block id
  __shared__ u64x2_t s_off0[KB];        // per-row K/V byte offsets of a tile (even / odd tiles)
  __shared__ u64x2_t s_off1[KB];
  __shared__ int s_ovf;                 // the fp16 pass produced a non-finite O

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rw = kSplit ? (wave & 1) : wave;   // this wave's 32 query rows of the block
  const int par = kSplit ? (wave >> 1) : 0;    // key half of every tile (key-split mode)
  const int n = lane & 31;   // query column of this lane (S^T, O^T) / key row (K operand)
  const int hh = lane >> 5;  // lane half: k-slot block of the operands

  // Work-group -> unit (b, h, query block).  Units are numbered with the
  // query block as the slow index, longest first across all (sequence, head)
  // pairs.  When the grid is more than one resident wave, work-group x takes
  // unit x: the dispatcher hands the longest remaining unit to each CU slot
  // that frees.  When every work-group is resident at once (p.wg_cus = C
  // CUs), the dispatcher places work-groups x, x + C, x + 2C, ... on one CU;
  // odd generations then take their units mirrored, so each CU's units add
  // up to about the same number of key tiles (config 4a: 27-28 per CU instead
  // of 20-34).  The mirror keeps x mod 8 (work-groups go to the 8 XCDs round
  // robin), so a (sequence, head) pair's blocks, which read the same keys,
  // stay on one XCD's L2.
  const int nq = p.q_tiles;
  const int64_t nbh = (int64_t)p.B * p.H;
  int qt, h, b;
  if (p.vl_compact) {
    // Variable-length batch, compacted grid: the work-groups take only the
    // (query block, sequence, head) units that have rows -- query blocks
    // from the last (longest) down, then sequences, then heads -- and those
    // past the last unit exit.  A grid sized by the longest sequence would
    // dispatch a work-group for every block of every sequence, most of them
    // (decode rows of a mixed batch, blocks past a short sequence's rows)
    // exiting only after a memory round trip, and spread the working ones
    // across the launch.  Per-sequence block counts sit in the lanes
    // (kVlMaxSeqs / 64 per lane); each level costs one ballot per chunk.
    int nbk[kVlMaxSeqs / 64];
#pragma unroll
    for (int c = 0; c < kVlMaxSeqs / 64; ++c) {
      const int i = c * 64 + lane;
      nbk[c] = 0;
      if (i < p.B) {
        const int qa = p.cu_q[i], qb = p.cu_q[i + 1];
        int len = qa >= 0 && qb >= qa && (int64_t)qb <= p.q_total ? qb - qa : 0;
        if (p.skip_single && len == 1) len = 0;
        nbk[c] = (min(len, p.S) + QB - 1) / QB;
      }
    }
    int64_t rem = blockIdx.x;
    int fb = -1, ft = 0, fh = 0;
    for (int t = nq - 1; t >= 0 && fb < 0; --t) {  // wave-uniform
#pragma unroll
      for (int c = 0; c < kVlMaxSeqs / 64; ++c) {
        const uint64_t m = __builtin_amdgcn_ballot_w64(nbk[c] > t);
        const int64_t cnt = (int64_t)__builtin_popcountll(m) * p.H;
        if (fb < 0) {
          if (rem < cnt) {
            const int k = (int)(rem / p.H);
            const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
            const uint64_t sel = __builtin_amdgcn_ballot_w64(((m >> lane) & 1u) != 0 && rank == k);
            fb = c * 64 + __builtin_ctzll(sel);
            ft = t;
            fh = (int)(rem - (int64_t)k * p.H);
          } else {
            rem -= cnt;
          }
        }
      }
    }
    if (fb < 0) return;  // past the last unit (work-group uniform)
    qt = ft;
    h = fh;
    b = fb;
  } else {
    int64_t x = blockIdx.x;
    if (p.wg_cus > 0) {
      const int64_t C = p.wg_cus, g = x / C, j = x - g * C;
      if ((g & 1) && (g + 1) * C <= nbh * nq) x = g * C + (C % 8 == 0 ? C - 8 - (j & ~(int64_t)7) + (j & 7) : C - 1 - j);
    }
    qt = nq - 1 - (int)(x / nbh);
    const int64_t bh = x % nbh;
    h = (int)(bh % p.H);
    b = (int)(bh / p.H);
  }
  const int kvh = h / p.G;

  // This sequence's query rows: S of them (row r at position ctx - S + r)
  // starting at token tok0 of q/out, of which the first Sr are served.
  // Uniform batches: S = Sr = p.S.  Variable-length batches: rows cu_q[b] ..
  // cu_q[b+1] of the packed [T, H, D] q/out, at most p.S (the caller's
  // max_q_len) of them served; a malformed range (negative, decreasing or
  // past T) is treated as empty.
  int S = p.S;
  int64_t tok0 = (int64_t)b * p.S;
  if (p.cu_q) {
    const int qa = p.cu_q[b], qb = p.cu_q[b + 1];
    const bool ok = qa >= 0 && qb >= qa && (int64_t)qb <= p.q_total;
    S = ok ? qb - qa : 0;
    tok0 = ok ? qa : 0;
    if (p.skip_single && S == 1) return;  // the decode kernel serves it (work-group uniform)
  }
  const int Sr = min(S, p.S);
  const int ctx = p.context_lens[b];
  const int maxctx = p.MB * p.BS;
  const int qs0 = qt * QB;
  if (qs0 >= Sr) return;            // no served rows of this sequence here (work-group uniform)
  const int qw0 = qs0 + rw * QW;    // this wave's first query row
  const int qrow = qw0 + n;
  const bool live = qrow < Sr;

  if (ctx > maxctx) {  // context longer than the block table: poison rows that attend keys
    if (live && hh == 0) {
      const float fillv = ctx - S + qrow < 0 ? 0.0f : __builtin_nanf("");
      const int64_t orow = ((tok0 + qrow) * p.H + h) * D;
      for (int d = 0; d < D; ++d) store_elem(p.out, p.out_dtype, orow + d, fillv);
    }
    return;
  }
  if (threadIdx.x == 0) {
    s_badkey = 0x7fffffff;
    s_ovf = 0;
  }

  // Keys the work-group's rows can see: [0, kend); this wave's rows: [0, wave_kend).
  const int kend = min(ctx, ctx - S + min(qs0 + QB, Sr));
  const int ntiles = kend > 0 ? (kend + KB - 1) / KB : 0;
  const int wave_last = min(qw0 + QW - 1, Sr - 1);
  const int wave_kend = qw0 < Sr ? min(ctx, ctx - S + wave_last + 1) : 0;
  const int wave_kfull = ctx - S + qw0 + 1;  // keys below this are visible to every row of the wave
  const int qpos = ctx - S + qrow;
  const int qlim = min(qpos, kend - 1);        // last key this column may see

  // Q^T operand (row qrow, dims ks*16 + hh*8 .. +8) in the KV type.  The sign of
  // the scale is applied here (exactly), so the softmax scale below is positive.
  u32x4_t qf[KS], qf_lo[kSplitQ ? KS : 1];
  {
    const int64_t qoff = ((tok0 + (live ? qrow : 0)) * p.H + h) * D + hh * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (!kSplitQ) {
        u32x4_t r = u32x4_t{0u, 0u, 0u, 0u};
        if (live) r = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p.q) + qoff + ks * 16);
        qf[ks] = (r & p.q_and) ^ p.q_xor;
      } else {
        float xv[8];
        if (live) {
          load8f(p.q, p.q_dtype, qoff + ks * 16, xv);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) xv[e] = 0.0f;
        }
        uint32_t w[4], wl[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x0 = xv[2 * j] * p.q_sign, x1 = xv[2 * j + 1] * p.q_sign;
          w[j] = pack2<kBf16>(x0, x1);
          const float2_t r = unpack2<kBf16>(w[j]);
          wl[j] = pack2<kBf16>(x0 - r[0], x1 - r[1]);
        }
        qf[ks] = u32x4_t{w[0], w[1], w[2], w[3]};
        qf_lo[ks] = u32x4_t{wl[0], wl[1], wl[2], wl[3]};
      }
    }
  }
  const float qscale = p.qscale;

  const int32_t* bt_row = p.block_tables + (int64_t)b * p.bt_stride;
  // Block ids of the pages this work-group reads live in an LDS window of
  // kPfBtStage pages starting at page win0, so a tile's loads never wait
  // behind a dependent block-table load.  The window moves (at a tile
  // boundary, between barriers) when the next tile to load leaves it.
  const int npages = kend > 0 ? (int)fastdiv((uint32_t)(kend - 1), p.bs_div) + 1 : 0;
  int win0 = 0;
  auto stage = [&](int first) {
    win0 = first;
    const int cnt = min(kPfBtStage, npages - first);
    for (int i = threadIdx.x; i < cnt; i += kPfThreads) s_bt[i] = bt_row[first + i];
  };
  auto ensure_window = [&](int t) {  // work-group uniform
    const int last = min(t * KB + KB, kend) - 1;
    const int plast = (int)fastdiv((uint32_t)last, p.bs_div);
    if (plast >= win0 + kPfBtStage) {
      __syncthreads();
      stage((int)fastdiv((uint32_t)(t * KB), p.bs_div));
      __syncthreads();
    }
  };

  const char* kbase = static_cast<const char*>(p.k) + (int64_t)kvh * p.k_sh * EB;
  const char* vbase = static_cast<const char*>(p.v) + (int64_t)kvh * p.v_sh * EB;
  const uint32_t k_sbb = (uint32_t)(p.k_sb * EB), k_stb = (uint32_t)(p.k_st * EB);
  const uint32_t v_sbb = (uint32_t)(p.v_sb * EB), v_stb = (uint32_t)(p.v_st * EB);
  const uint64_t nb = (uint64_t)p.num_blocks;

  // This thread's chunks of a tile: chunk c fills LDS chunk position
  // pos = (c*4 + wave)*64 + lane (wave-contiguous 1 KB per direct load), i.e.
  // row pos / NCH at swizzled position pos % NCH; it loads the source chunk
  // whose swizzled position that is (an involution: the same XOR).
  int prow[CPT], ksrc[CPT], vsrc[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int pos = (c * 4 + wave) * 64 + lane;
    prow[c] = pos / NCH;
    ksrc[c] = kpos<D>(prow[c], pos % NCH) * 8 * EB;  // byte offset of the 8-element source chunk
    vsrc[c] = vpos<D>(prow[c], pos % NCH) * 8 * EB;
  }
  int badkey = 0x7fffffff;

  // Row offsets of a tile, built once per tile by the first KB / 64 waves (one
  // row per lane) two tiles ahead, so the other waves' loads cost one LDS read and an add
  // per chunk.  Entry r = {K byte offset, V byte offset | use}; a row past
  // kend, or on a page with an invalid block id, points at row 0 of block 0
  // (in bounds, NB >= 1) with use = 0.  Offsets are multiples of 16 bytes, so
  // bit 0 of the V offset is free for the flag.
  auto build = [&](int t, u64x2_t* tb) {
    if (wave * 64 + lane < KB) {
      const int row = wave * 64 + lane;
      const int kabs = t * KB + row;
      const bool valid = kabs < kend;
      const int kk = valid ? kabs : 0;
      const int pg = (int)fastdiv((uint32_t)kk, p.bs_div);
      const int off = kk - pg * p.BS;
      const int blk = s_bt[valid ? pg - win0 : 0];
      const bool okb = (uint64_t)(int64_t)blk < nb;
      if (valid && !okb) badkey = min(badkey, kabs);
      const bool use = valid && okb;
      const uint32_t ub = use ? (uint32_t)blk : 0u, uo = use ? (uint32_t)off : 0u;
      tb[row] = u64x2_t{(uint64_t)ub * k_sbb + uo * k_stb,
                        ((uint64_t)ub * v_sbb + uo * v_stb) | (use ? 1u : 0u)};
    }
  };

  f32x16_t o[DT];
  float m = -__builtin_inff(), l = 0.0f;  // running max (log2 units); this lane half's row sum

  // One pass over the key tiles in PV mode kMode.  Returns false (work-group
  // uniform) when kPvConvert produced a non-finite O (a V value that fp16
  // cannot hold, or non-finite data): the caller reruns in kPvSplit.
  auto run = [&](auto mode_tag) -> bool {
    constexpr int kMode = decltype(mode_tag)::value;
    constexpr bool kDirectV = kMode != kPvConvert && kMode != kPvF8;
    constexpr bool kPvBf16 = kMode == kPvSplit;

#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] = 0.0f;
    }
    m = -__builtin_inff();
    l = 0.0f;

    u32x4_t vreg[kDirectV || kMode == kPvF8 ? 1 : CPT];
    u32x2_t kreg8[kMode == kPvF8 ? CPT : 1], vreg8[kMode == kPvF8 ? CPT : 1];  // FP8 codes of this thread's chunks
    uint32_t umask = 0;

    // Loads of a tile into (dK, dV) from its offset table: entries() reads
    // this thread's table entries, chunk(c) issues chunk c's K (and V unless
    // converted) loads straight to LDS.
    u64x2_t ent[CPT];
    auto entries = [&](const u64x2_t* tb) {
#pragma unroll
      for (int c = 0; c < CPT; ++c) ent[c] = tb[prow[c]];
      umask = 0;
    };
    auto chunk = [&](int c, uint16_t* dK, uint16_t* dV) {
      const uint32_t use = (uint32_t)ent[c][1] & 1u;
      umask |= use << c;
      const char* va = vbase + (ent[c][1] - use) + vsrc[c];
      if constexpr (kMode == kPvF8) {
        kreg8[c] = *reinterpret_cast<const u32x2_t*>(kbase + ent[c][0] + ksrc[c]);
        vreg8[c] = *reinterpret_cast<const u32x2_t*>(va);
        return;
      }
      lds_dma16(kbase + ent[c][0] + ksrc[c], (lds_void_t*)(dK + (c * 4 + wave) * 512));
      if constexpr (kDirectV) {
        lds_dma16(va, (lds_void_t*)(dV + (c * 4 + wave) * 512));
      } else {
        vreg[c] = *reinterpret_cast<const u32x4_t*>(va);
      }
    };
    auto issue = [&](const u64x2_t* tb, uint16_t* dK, uint16_t* dV) {
      entries(tb);
#pragma unroll
      for (int c = 0; c < CPT; ++c) chunk(c, dK, dV);
      __builtin_amdgcn_sched_barrier(0);
    };
    // After a tile's loads are complete: zero V rows that were substituted
    // (their probabilities are 0, but substituted data may not be finite),
    // or convert the register-staged bf16 V to fp16 (exact for
    // 2^-17 <= |v| < 65504; smaller values round to fp16 subnormals).
    auto finish = [&](uint16_t* dK, uint16_t* dV) {
      if constexpr (kMode == kPvF8) {
        // Codes -> 16-bit pairs (v_cvt_scalef32_pk_{f16,bf16}_fp8 at scale 1:
        // exact for every code), K in the Q.K^T type, V in fp16; V rows that were
        // substituted are zeroed (their codes may be NaN), K rows need not be
        // (their scores are masked).
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
          uint32_t wk[4], wv[4];
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            if constexpr (kBf16) {
              wk[2 * j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(kreg8[c][j], 1.0f, false));
              wk[2 * j + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(kreg8[c][j], 1.0f, true));
            } else {
              wk[2 * j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(kreg8[c][j], 1.0f, false));
              wk[2 * j + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(kreg8[c][j], 1.0f, true));
            }
            wv[2 * j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(vreg8[c][j], 1.0f, false));
            wv[2 * j + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(vreg8[c][j], 1.0f, true));
          }
          const bool used = (umask >> c) & 1u;
#pragma unroll
          for (int j = 0; j < 4; ++j) wv[j] = used ? wv[j] : 0u;
          const int at = ((c * 4 + wave) * 64 + lane) * 8;
          *reinterpret_cast<u32x4_t*>(dK + at) = u32x4_t{wk[0], wk[1], wk[2], wk[3]};
          *reinterpret_cast<u32x4_t*>(dV + at) = u32x4_t{wv[0], wv[1], wv[2], wv[3]};
        }
      } else if constexpr (kDirectV) {
        if (umask != (1u << CPT) - 1u) {
#pragma unroll
          for (int c = 0; c < CPT; ++c) {
            if (!((umask >> c) & 1u))
              *reinterpret_cast<u32x4_t*>(dV + ((c * 4 + wave) * 64 + lane) * 8) = u32x4_t{0u, 0u, 0u, 0u};
          }
        }
      } else {
        // Rows are substituted only at the end of the keys or on a bad block
        // id: the zeroing selects run only when some lane of the wave has one.
        const bool all_used = __builtin_amdgcn_ballot_w64(umask != (1u << CPT) - 1u) == 0;
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
          u32x4_t w;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t x = vreg[c][j];
            w[j] = pack2<false>(__builtin_bit_cast(float, x << 16), __builtin_bit_cast(float, x & 0xffff0000u));
          }
          if (!all_used) {
            asm volatile("");
            if (!((umask >> c) & 1u)) w = u32x4_t{0u, 0u, 0u, 0u};
          }
          *reinterpret_cast<u32x4_t*>(dV + ((c * 4 + wave) * 64 + lane) * 8) = w;
        }
      }
    };

    // S^T, softmax and O^T update for tile t from LDS (cK, cV).
    auto compute = [&](int t, const uint16_t* cK, const uint16_t* cV) {
      // Key-split mode: this wave's 32 keys are rows par*32 .. of the tile;
      // the swizzles depend on row bits below 32 only, so its m-tile is the
      // tile's shifted by par*32 rows.
      cK += par * 32 * D;
      cV += par * 32 * D;
      f32x16_t st[MTW];
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) st[mt][r] = 0.0f;
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt) {
          const u32x4_t a = *reinterpret_cast<const u32x4_t*>(cK + swk<D>(mt * 32 + n, 2 * ks + hh));
          st[mt] = mfma32<kBf16>(a, qf[ks], st[mt]);
          if constexpr (kSplitQ) st[mt] = mfma32<kBf16>(a, qf_lo[ks], st[mt]);
        }
      }
      // Keys of this lane: t*KB + mt*32 + 8*(r/4) + 4*hh + r%4.  Only tiles
      // that cross the wave's diagonal (or the end of the keys) are masked;
      // the empty asm keeps this a branch rather than selects on every tile.
      const int tk0 = t * KB + par * 32;
      if (tk0 + MTW * 32 > wave_kfull) {
        asm volatile("");
        const int thr = qlim - tk0 - 4 * hh;
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            if (mt * 32 + 8 * (r >> 2) + (r & 3) > thr) st[mt][r] = -__builtin_inff();
          }
        }
      }
      // Max over this lane half's keys of the column; the other half holds the
      // column's other keys.  The two halves share m, and m only has to move
      // when some half exceeds m + 2^8, so the cross-half max is formed only
      // on that (rare) branch.
      float mx = -__builtin_inff();
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[mt][r]);
      }
      const float mxh = mx * qscale;
      if (__builtin_amdgcn_ballot_w64(mxh > m + kLazyRescale) != 0) {
        asm volatile("");  // rare: keep the O^T rescale behind the branch
        const float mxs = fmaxf(mxh, __shfl_xor(mxh, 32, 64));
        const float mn = fmaxf(m, mxs);
        const float corr = mn == -__builtin_inff() ? 1.0f : fast_exp2(m - mn);
        m = mn;
        l *= corr;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] *= corr;
      }
      const float negm = m == -__builtin_inff() ? 0.0f : -m;

      // Per 32-key m-tile: P^T operands of its two 16-key steps (accumulator
      // slots 8s .. 8s+7 of step s), then O^T += V^T . P^T.  V^T operand of
      // step (mt, s): lane l of 16-lane group g supplies row
      // mt*32 + 16s + 4*hh + (l%16)/4 (and +8), dims dt*32 + 16*(g%2) +
      // (l%4)*4 .. +4, and receives dim dt*32 + lane%32.
      const int li = lane & 15;
      const int trow = 4 * hh + (li >> 2);
      const int tcol = 16 * ((lane >> 4) & 1) + (li & 3) * 4;
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) {
        u32x4_t pb[2], pb_lo[kPvBf16 ? 2 : 1];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          uint32_t w[4], wl[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float p0 = fast_exp2(fmaf(st[mt][8 * s + 2 * j], qscale, negm));
            const float p1 = fast_exp2(fmaf(st[mt][8 * s + 2 * j + 1], qscale, negm));
            w[j] = pack2<kPvBf16>(p0, p1);
            if constexpr (kPvBf16) {
              const float2_t r = unpack2<true>(w[j]);
              wl[j] = pack2<true>(p0 - r[0], p1 - r[1]);
              l += p0 + p1;
            } else {
              l = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w[j]), half2_t{1.0f16, 1.0f16}, l, false);
            }
          }
          pb[s] = u32x4_t{w[0], w[1], w[2], w[3]};
          if constexpr (kPvBf16) pb_lo[s] = u32x4_t{wl[0], wl[1], wl[2], wl[3]};
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            const int r0 = mt * 32 + 16 * s + trow;
            const int col = dt * 32 + tcol;
            const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_short4_t*)(cV + swv<D>(r0, col >> 3) + (col & 7)));
            const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_short4_t*)(cV + swv<D>(r0 + 8, col >> 3) + (col & 7)));
            const uint64_t lo64 = __builtin_bit_cast(uint64_t, lo), hi64 = __builtin_bit_cast(uint64_t, hi);
            const u32x4_t a = u32x4_t{(uint32_t)lo64, (uint32_t)(lo64 >> 32), (uint32_t)hi64,
                                      (uint32_t)(hi64 >> 32)};
            o[dt] = mfma32<kPvBf16>(a, pb[s], o[dt]);
            if constexpr (kPvBf16) o[dt] = mfma32<true>(a, pb_lo[s], o[dt]);
          }
        }
      }
    };

    // Double-buffered tiles, unrolled by two so each LDS buffer (and offset
    // table) is a distinct object: tile t+1's loads and tile t+2's offset
    // table are produced while tile t is computed; one barrier per tile.
    stage(0);
    __syncthreads();
    build(0, s_off0);
    if (ntiles > 1) {
      ensure_window(1);
      build(1, s_off1);
    }
    __syncthreads();
    if (ntiles > 0) {
      issue(s_off0, sK0, sV0);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's loads are in LDS
      finish(sK0, sV0);
    }
    __syncthreads();
    for (int t = 0; t < ntiles; t += 2) {
      if (t + 2 < ntiles) ensure_window(t + 2);
      if (t + 2 < ntiles) build(t + 2, s_off0);
      const bool more1 = t + 1 < ntiles;
      if (more1) issue(s_off1, sK1, sV1);
      if (t * KB + par * 32 < wave_kend) compute(t, sK0, sV0);
      if (more1) {
        __builtin_amdgcn_s_waitcnt(0x0F70);
        finish(sK1, sV1);
      }
      __syncthreads();
      if (!more1) break;
      if (t + 3 < ntiles) ensure_window(t + 3);
      if (t + 3 < ntiles) build(t + 3, s_off1);
      const bool more2 = t + 2 < ntiles;
      if (more2) issue(s_off0, sK0, sV0);
      if ((t + 1) * KB + par * 32 < wave_kend) compute(t + 1, sK1, sV1);
      if (t + 2 < ntiles) {
        __builtin_amdgcn_s_waitcnt(0x0F70);
        finish(sK0, sV0);
      }
      __syncthreads();
    }
    if constexpr (kMode == kPvConvert) {
      bool bad = false;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) bad |= !__builtin_isfinite(o[dt][r]);
      }
      if (bad) s_ovf = 1;
      __syncthreads();
      if (s_ovf) return false;
    }
    return true;
  };

  if constexpr (kF8) {
    run(PvTag<kPvF8>{});
  } else if constexpr (kBf16) {
    if (!run(PvTag<kPvConvert>{})) {
      badkey = 0x7fffffff;
      run(PvTag<kPvSplit>{});
    }
  } else {
    run(PvTag<kPvDirect>{});
  }

  if (badkey != 0x7fffffff) atomicMin(&s_badkey, badkey);
  __syncthreads();
  const int bad_from = s_badkey;

  // Key-split mode: waves 2-3 hand their (m, l, O^T) to waves 0-1 through
  // the (now idle) tile buffers; the lanes of the two waves hold the same
  // rows and dims, so the merge is lane by lane (log-sum-exp rule on the
  // reference points m, which are -inf where a wave saw no key).
  if constexpr (kSplit) {
    float* xo = reinterpret_cast<float*>(rw == 0 ? sK0 : sK1);  // [DT * 16][64]: KB * D halves hold it
    float* xm = reinterpret_cast<float*>(sV0) + rw * 128;       // m [64], l [64]
    if (par == 1) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) xo[(dt * 16 + r) * 64 + lane] = o[dt][r];
      }
      xm[lane] = m;
      xm[64 + lane] = l;
    }
    __syncthreads();
    if (par == 1) return;
    const float m2 = xm[lane], l2 = xm[64 + lane];
    const float mn = fmaxf(m, m2);
    const float a = m == -__builtin_inff() ? 0.0f : fast_exp2(m - mn);
    const float c = m2 == -__builtin_inff() ? 0.0f : fast_exp2(m2 - mn);
    l = l * a + l2 * c;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] = o[dt][r] * a + xo[(dt * 16 + r) * 64 + lane] * c;
    }
  }

  // Row sum over the two lane halves, normalise, write.  O^T slot r of lane
  // (n, hh) in m-tile dt is dim dt*32 + 8*(r/4) + 4*hh + r%4 of row qrow.
  const float lt = l + __shfl_xor(l, 32, 64);
  if (!live) return;
  const bool bad = bad_from <= qpos;
  const float inv = lt > 0.0f ? p.vscale / lt : 0.0f;
  const int64_t orow = ((tok0 + qrow) * p.H + h) * D;
  // Slots 4j .. 4j+3 of m-tile dt are 4 consecutive dims: one 8-byte (16-bit
  // out) or 16-byte (fp32 out) store when the output base allows it.
  const uintptr_t oa = reinterpret_cast<uintptr_t>(p.out);
  const bool vec = (p.out_dtype == kF32 ? (oa & 15) == 0 : (oa & 7) == 0);
  if (!vec) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = dt * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
        store_elem(p.out, p.out_dtype, orow + d, bad ? __builtin_nanf("") : o[dt][r] * inv);
      }
    }
    return;
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = bad ? __builtin_nanf("") : o[dt][4 * j + i] * inv;
      const int64_t e = orow + dt * 32 + 8 * j + 4 * hh;
      if (p.out_dtype == kF32) {
        u64x2_t w = u64x2_t{(uint64_t)__builtin_bit_cast(uint32_t, v[0]) | ((uint64_t)__builtin_bit_cast(uint32_t, v[1]) << 32),
                            (uint64_t)__builtin_bit_cast(uint32_t, v[2]) | ((uint64_t)__builtin_bit_cast(uint32_t, v[3]) << 32)};
        *reinterpret_cast<u64x2_t*>(static_cast<float*>(p.out) + e) = w;
      } else {
        const uint32_t w0 = p.out_dtype == kF16 ? pack2<false>(v[0], v[1]) : pack2<true>(v[0], v[1]);
        const uint32_t w1 = p.out_dtype == kF16 ? pack2<false>(v[2], v[3]) : pack2<true>(v[2], v[3]);
        const uint64_t w = (uint64_t)w0 | ((uint64_t)w1 << 32);
        *reinterpret_cast<uint64_t*>(static_cast<uint16_t*>(p.out) + e) = w;
      }
    }
  }
}

// Ping-pong prefill (64-key tiles; 16-bit caches with q in the KV type, or
// FP8 caches with fp16 or bf16 q, the codes staged in registers).  A
// work-group of 8 waves serves 256 query rows (wave w owns rows 32w ..) and
// is the only one on its CU, so each SIMD holds wave s of group 0 (waves 0-3)
// and wave s + 4 of group 1.  Every phase ends at a work-group barrier, and
// group 1 runs one phase behind group 0: in each phase one group does its
// matrix step (O^T += V^T . P^T of tile j - 1, then S^T = K . Q^T of tile j)
// while the other does its vector step (the softmax of its S^T of tile j),
// so each SIMD issues one wave's MFMAs against the other wave's vector work.
// In the four-wave kernel the two waves of a SIMD belong to different
// work-groups, drift into the same step and queue behind each other.
//
// Phase ph, group g: step e = ph - g; even e = matrix step e / 2, odd e =
// vector step e / 2.  Tile j's K is read in phases 2j (group 0) and 2j + 1
// (group 1), its V (by the P.V of step j + 1) in 2j + 2 and 2j + 3.  Loads
// (at D >= 64 every thread of both groups loads its share of every K and V
// tile, so the two groups' vector steps carry the same work; at D = 32, one
// 16-byte chunk per thread of a group, group 1 loads K and group 0 V):
//  * in its vector step j (phase 2j + 1 + g) a thread issues its chunks of K
//    of tile j + 2 and of V of tile j + 1: direct to LDS, except a bf16 V
//    tile and FP8 codes, which go to registers -- both buffers were last
//    read in phase 2j - 1;
//  * at the end of its matrix step j + 1 (phase 2j + 2 + g) it waits for
//    them and finishes them (bf16 V converted to fp16, FP8 K and V codes to
//    16-bit pairs, and stored; substituted V rows zeroed), before the
//    barrier ahead of their first read (phase 2j + 4).
// Per-row offset tables (three, tile t in t % 3) are built by wave 0 in its
// vector step j for tile j + 3.
template <int N>
struct Slot {  // a compile-time buffer index
  static constexpr int value = N;
};

constexpr int kPpThreads = 512;  // 8 waves
constexpr int kPpRows = 256;     // query rows per work-group

template <typename KV, int D>
__global__ __launch_bounds__(kPpThreads) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_pp_kernel(const PrefillParams p) {
  using Sh = PfShape<D>;
  static_assert(Sh::KB == 64 && Sh::MT == 2, "64-key tiles");
  constexpr int QW = 32, QB = kPpRows, KB = 64, MT = 2, KS = Sh::KS, DT = Sh::DT, NCH = Sh::NCH;
  constexpr int CPT = Sh::CPT;  // chunks per thread of one group (256 threads) per tile
  constexpr bool kBf16 = QkBf16<KV>::value;  // Q.K^T operand type
  constexpr bool kF8 = KV::kCode == kFP8;    // tiles converted from FP8 codes; P.V in fp16
  constexpr int EB = KV::kBytes;
  static_assert(EB == 2 || kF8, "16-bit or FP8 caches");

  __shared__ __attribute__((aligned(16))) uint16_t sK[3][KB * D];
  __shared__ __attribute__((aligned(16))) uint16_t sV[3][KB * D];
  __shared__ int32_t s_bt[kPfBtStage];
  __shared__ u64x2_t s_off[3][KB];
  __shared__ int s_badkey;
  __shared__ int s_ovf;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;
  const int n = lane & 31;
  const int hh = lane >> 5;

  // Work-group -> unit (b, h, query block), as the four-wave kernel.
  const int nq = p.q_tiles;
  const int64_t nbh = (int64_t)p.B * p.H;
  int64_t x = blockIdx.x;
  if (p.wg_cus > 0) {
    const int64_t C = p.wg_cus, g = x / C, jj = x - g * C;
    if ((g & 1) && (g + 1) * C <= nbh * nq) x = g * C + (C % 8 == 0 ? C - 8 - (jj & ~(int64_t)7) + (jj & 7) : C - 1 - jj);
  }
  const int qt = nq - 1 - (int)(x / nbh);
  const int64_t bh = x % nbh;
  const int h = (int)(bh % p.H);
  const int b = (int)(bh / p.H);
  const int kvh = h / p.G;

  int S = p.S;
  int64_t tok0 = (int64_t)b * p.S;
  if (p.cu_q) {
    const int qa = p.cu_q[b], qb = p.cu_q[b + 1];
    const bool ok = qa >= 0 && qb >= qa && (int64_t)qb <= p.q_total;
    S = ok ? qb - qa : 0;
    tok0 = ok ? qa : 0;
    if (p.skip_single && S == 1) return;
  }
  const int Sr = min(S, p.S);
  const int qs0 = qt * QB;
  if (qs0 >= Sr) return;
  const int qw0 = qs0 + wave * QW;
  const int qrow = qw0 + n;
  const bool live = qrow < Sr;

  // Issued before the context length arrives: the block table's first
  // min(MB, kPfBtStage) entries (the window; the host serves only tables that
  // fit it) and this lane's q.
  const int32_t* bt_row = p.block_tables + (int64_t)b * p.bt_stride;
  const int nbt = min(p.MB, kPfBtStage);
  static_assert(kPfBtStage == 2 * kPpThreads, "two entries per thread");
  int32_t btp0 = 0, btp1 = 0;
  if ((int)threadIdx.x < nbt) btp0 = bt_row[threadIdx.x];
  if ((int)threadIdx.x + kPpThreads < nbt) btp1 = bt_row[threadIdx.x + kPpThreads];
  u32x4_t qf[KS];
  {
    const int64_t qoff = ((tok0 + (live ? qrow : 0)) * p.H + h) * D + hh * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4_t r = u32x4_t{0u, 0u, 0u, 0u};
      if (live) r = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p.q) + qoff + ks * 16);
      qf[ks] = (r & p.q_and) ^ p.q_xor;
    }
  }
  const int ctx = p.context_lens[b];
  const int maxctx = p.MB * p.BS;

  if (ctx > maxctx) {
    if (live && hh == 0) {
      const float fillv = ctx - S + qrow < 0 ? 0.0f : __builtin_nanf("");
      const int64_t orow = ((tok0 + qrow) * p.H + h) * D;
      for (int d = 0; d < D; ++d) store_elem(p.out, p.out_dtype, orow + d, fillv);
    }
    return;
  }
  if (threadIdx.x == 0) {
    s_badkey = 0x7fffffff;
    s_ovf = 0;
  }

  const int kend = min(ctx, ctx - S + min(qs0 + QB, Sr));
  const int ntiles = kend > 0 ? (kend + KB - 1) / KB : 0;
  const int wave_last = min(qw0 + QW - 1, Sr - 1);
  const int wave_kend = qw0 < Sr ? min(ctx, ctx - S + wave_last + 1) : 0;
  const int wave_kfull = ctx - S + qw0 + 1;
  const int qpos = ctx - S + qrow;
  const int qlim = min(qpos, kend - 1);

  const float qscale = p.qscale;

  // The block ids of every page the work-group reads.
  const int npages = kend > 0 ? min((int)fastdiv((uint32_t)(kend - 1), p.bs_div) + 1, nbt) : 0;
  if ((int)threadIdx.x < npages) s_bt[threadIdx.x] = btp0;
  if ((int)threadIdx.x + kPpThreads < npages) s_bt[threadIdx.x + kPpThreads] = btp1;

  const char* kbase = static_cast<const char*>(p.k) + (int64_t)kvh * p.k_sh * EB;
  const char* vbase = static_cast<const char*>(p.v) + (int64_t)kvh * p.v_sh * EB;
  const uint32_t k_sbb = (uint32_t)(p.k_sb * EB), k_stb = (uint32_t)(p.k_st * EB);
  const uint32_t v_sbb = (uint32_t)(p.v_sb * EB), v_stb = (uint32_t)(p.v_st * EB);
  const uint64_t nb = (uint64_t)p.num_blocks;

  // This thread's chunks of a tile.  With two or more chunks per thread of a
  // group (D >= 64), both groups load half of every K tile and half of every
  // V tile (CH chunks of each per thread), so the two groups' vector steps
  // carry the same work; at D = 32 (one chunk) group 1 loads K, group 0 V.
  constexpr bool kHalves = CPT % 2 == 0;
  constexpr int CH = kHalves ? CPT / 2 : CPT;
  auto cpos = [&](int c) { return kHalves ? c * 8 + wave : c * 4 + (wave & 3); };  // 64-chunk group of chunk c
  const bool do_k = kHalves || grp == 1, do_v = kHalves || grp == 0;  // wave-uniform
  int prow[CH], ksrc[CH], vsrc[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int pos = cpos(c) * 64 + lane;
    prow[c] = pos / NCH;
    ksrc[c] = kpos<D>(prow[c], pos % NCH) * 8 * EB;
    vsrc[c] = vpos<D>(prow[c], pos % NCH) * 8 * EB;
  }
  int badkey = 0x7fffffff;

  // Wave 0: the offset table of tile t (entry r = {K byte offset, V byte
  // offset | use}; a row past kend or on an invalid block id reads row 0 of
  // block 0 with use = 0).
  auto build = [&](auto slot, int t) {
    const int row = lane;
    const int kabs = t * KB + row;
    const bool valid = kabs < kend;
    const int kk = valid ? kabs : 0;
    const int pg = (int)fastdiv((uint32_t)kk, p.bs_div);
    const int off = kk - pg * p.BS;
    const int blk = s_bt[valid ? pg : 0];
    const bool okb = (uint64_t)(int64_t)blk < nb;
    if (valid && !okb) badkey = min(badkey, kabs);
    const bool use = valid && okb;
    const uint32_t ub = use ? (uint32_t)blk : 0u, uo = use ? (uint32_t)off : 0u;
    s_off[decltype(slot)::value][row] = u64x2_t{(uint64_t)ub * k_sbb + uo * k_stb,
                                ((uint64_t)ub * v_sbb + uo * v_stb) | (use ? 1u : 0u)};
  };

  f32x16_t o[DT];
  float m = -__builtin_inff(), l = 0.0f;

  auto run = [&](auto mode_tag) -> bool {
    constexpr int kMode = decltype(mode_tag)::value;
    constexpr bool kDirectV = kMode != kPvConvert && kMode != kPvF8;
    constexpr bool kPvBf16 = kMode == kPvSplit;

#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] = 0.0f;
    }
    m = -__builtin_inff();
    l = 0.0f;

    u32x4_t vreg[kDirectV || kF8 ? 1 : CH];
    u32x2_t kreg8[kF8 ? CH : 1], vreg8[kF8 ? CH : 1];  // FP8 codes of this thread's chunks
    uint32_t umask = 0;

    // This thread's K chunks of tile t: straight to LDS, or (FP8) codes into
    // registers `kr`.
    auto issue_k = [&](auto slot, u32x2_t (&kr)[kF8 ? CH : 1]) {
      if (!do_k) return;
      const u64x2_t* tb = s_off[decltype(slot)::value];
      uint16_t* dK = sK[decltype(slot)::value];
      uint64_t e[CH];  // the K halves of the table entries first: one LDS round trip
#pragma unroll
      for (int c = 0; c < CH; ++c) e[c] = reinterpret_cast<const uint64_t*>(tb + prow[c])[0];
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        if constexpr (kF8) {
          kr[c] = *reinterpret_cast<const u32x2_t*>(kbase + e[c] + ksrc[c]);
        } else {
          lds_dma16_async(kbase + e[c] + ksrc[c], (lds_void_t*)(dK + cpos(c) * 512));
        }
      }
    };
    // FP8, after this thread's K loads of tile t are complete: codes -> Q.K^T
    // type pairs (exact for every code; rows past the keys need no zeroing:
    // their scores are masked).
    auto finish_k = [&](auto slot, const u32x2_t (&kr)[kF8 ? CH : 1]) {
      if constexpr (kF8) {
        if (!do_k) return;
        uint16_t* dK = sK[decltype(slot)::value];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          uint32_t w[4];
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            if constexpr (kBf16) {
              w[2 * j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(kr[c][j], 1.0f, false));
              w[2 * j + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(kr[c][j], 1.0f, true));
            } else {
              w[2 * j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(kr[c][j], 1.0f, false));
              w[2 * j + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(kr[c][j], 1.0f, true));
            }
          }
          *reinterpret_cast<u32x4_t*>(dK + (cpos(c) * 64 + lane) * 8) = u32x4_t{w[0], w[1], w[2], w[3]};
        }
      }
    };
    // This thread's V chunks of tile t (to LDS, or to registers for conversion).
    auto issue_v = [&](auto slot) {
      if (!do_v) return;
      const u64x2_t* tb = s_off[decltype(slot)::value];
      uint16_t* dV = sV[decltype(slot)::value];
      umask = 0;
      uint64_t e[CH];  // the V halves of the table entries first: one LDS round trip
#pragma unroll
      for (int c = 0; c < CH; ++c) e[c] = reinterpret_cast<const uint64_t*>(tb + prow[c])[1];
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const uint32_t use = (uint32_t)e[c] & 1u;
        umask |= use << c;
        const char* va = vbase + (e[c] - use) + vsrc[c];
        if constexpr (kF8) {
          vreg8[c] = *reinterpret_cast<const u32x2_t*>(va);
        } else if constexpr (kDirectV) {
          lds_dma16_async(va, (lds_void_t*)(dV + cpos(c) * 512));
        } else {
          vreg[c] = *reinterpret_cast<const u32x4_t*>(va);
        }
      }
    };
    // After this thread's V loads are complete: zero substituted rows, or
    // convert the staged bf16 V to fp16 (exact for 2^-17 <= |v| < 65504), or
    // the FP8 codes to fp16 (exact; substituted rows zeroed: their codes may
    // be NaN).
    auto finish_v = [&](auto slot) {
      if (!do_v) return;
      uint16_t* dV = sV[decltype(slot)::value];
      if constexpr (kF8) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          uint32_t w[4];
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            w[2 * j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(vreg8[c][j], 1.0f, false));
            w[2 * j + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(vreg8[c][j], 1.0f, true));
          }
          const bool used = (umask >> c) & 1u;
#pragma unroll
          for (int j = 0; j < 4; ++j) w[j] = used ? w[j] : 0u;
          *reinterpret_cast<u32x4_t*>(dV + (cpos(c) * 64 + lane) * 8) = u32x4_t{w[0], w[1], w[2], w[3]};
        }
      } else if constexpr (kDirectV) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the direct loads are not tracked by the compiler
        if (umask != (1u << CH) - 1u) {
#pragma unroll
          for (int c = 0; c < CH; ++c) {
            if (!((umask >> c) & 1u))
              *reinterpret_cast<u32x4_t*>(dV + (cpos(c) * 64 + lane) * 8) = u32x4_t{0u, 0u, 0u, 0u};
          }
        }
      } else {
        const bool all_used = __builtin_amdgcn_ballot_w64(umask != (1u << CH) - 1u) == 0;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          u32x4_t w;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t xv = vreg[c][j];
            w[j] = pack2<false>(__builtin_bit_cast(float, xv << 16), __builtin_bit_cast(float, xv & 0xffff0000u));
          }
          if (!all_used) {
            asm volatile("");
            if (!((umask >> c) & 1u)) w = u32x4_t{0u, 0u, 0u, 0u};
          }
          *reinterpret_cast<u32x4_t*>(dV + (cpos(c) * 64 + lane) * 8) = w;
        }
      }
    };

    f32x16_t st[MT];
    u32x4_t pb[MT][2], pb_lo[kPvBf16 ? MT : 1][2];
    // Softmax of tile t: mask, lazy maximum, P^T operands (see the four-wave kernel).
    auto softmax = [&](int t) {
      const int tk0 = t * KB;
      if (tk0 + KB > wave_kfull) {
        asm volatile("");
        const int thr = qlim - tk0 - 4 * hh;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            if (mt * 32 + 8 * (r >> 2) + (r & 3) > thr) st[mt][r] = -__builtin_inff();
          }
        }
      }
      // Weights against the running maximum m, packed as the P^T operands,
      // and their row sum over the rounded weights (four chains, added at the
      // end): each lane's sum over its 16 keys of the row.
      auto weights = [&](float negm) __attribute__((always_inline)) {
        float ls[MT][2];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            uint32_t w[4], wl[4];
            float lc = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float p0 = fast_exp2(fmaf(st[mt][8 * s2 + 2 * j], qscale, negm));
              const float p1 = fast_exp2(fmaf(st[mt][8 * s2 + 2 * j + 1], qscale, negm));
              w[j] = pack2<kPvBf16>(p0, p1);
              if constexpr (kPvBf16) {
                const float2_t r = unpack2<true>(w[j]);
                wl[j] = pack2<true>(p0 - r[0], p1 - r[1]);
                lc += p0 + p1;
              } else {
                lc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w[j]), half2_t{1.0f16, 1.0f16}, lc, false);
              }
            }
            ls[mt][s2] = lc;
            pb[mt][s2] = u32x4_t{w[0], w[1], w[2], w[3]};
            if constexpr (kPvBf16) pb_lo[mt][s2] = u32x4_t{wl[0], wl[1], wl[2], wl[3]};
          }
        }
        return (ls[0][0] + ls[0][1]) + (ls[1][0] + ls[1][1]);
      };
      // The maximum is raised only when needed: on the first tile (every
      // live row sees key 0), or when a lane's weights could leave the range
      // they are exact in (a sum above 2^15, or not finite: a weight past
      // 2^15).  The tile maximum is computed only then.
      float lsum = weights(m == -__builtin_inff() ? 0.0f : -m);
      if (__builtin_amdgcn_ballot_w64(t == 0 || !(lsum <= kWeightCap)) != 0) {
        asm volatile("");
        // Maximum over four independent chains (short dependency chains).
        float mc[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          mc[c] = st[c >> 1][(c & 1) * 8];
#pragma unroll
          for (int r = 1; r < 8; ++r) mc[c] = fmaxf(mc[c], st[c >> 1][(c & 1) * 8 + r]);
        }
        const float mxh = fmaxf(fmaxf(mc[0], mc[1]), fmaxf(mc[2], mc[3])) * qscale;
        const float mxs = fmaxf(mxh, __shfl_xor(mxh, 32, 64));
        const float mn = fmaxf(m, mxs);
        const float corr = mn == -__builtin_inff() ? 1.0f : fast_exp2(m - mn);
        m = mn;
        l *= corr;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] *= corr;
        lsum = weights(m == -__builtin_inff() ? 0.0f : -m);
      }
      l += lsum;
    };
    // Matrix step: O^T += V^T . P^T of tile j - 1 (V in slot SV), then
    // S^T = K . Q^T of tile j (K in slot SK).  Each LDS operand is read two
    // MFMAs ahead into a ring of three, in this order (fences keep the
    // scheduler from regrouping the reads next to their uses), and the first
    // two K operands are read before the P.V products.
    const int li = lane & 15;
    const int trow = 4 * hh + (li >> 2);
    const int tcol = 16 * ((lane >> 4) & 1) + (li & 3) * 4;
    auto mstep = [&](auto sk, auto sv, bool do_pv, bool do_qk) {
      const uint16_t* cK = sK[decltype(sk)::value];
      const uint16_t* cV = sV[decltype(sv)::value];
      u32x4_t ka[3][MT];
      auto rdk = [&](int ks, u32x4_t (&dst)[MT]) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          dst[mt] = *reinterpret_cast<const u32x4_t*>(cK + swk<D>(mt * 32 + n, 2 * ks + hh));
      };
      if (do_qk) {
        rdk(0, ka[0]);
        rdk(1, ka[1]);
      }
      if (do_pv) {
        // Product i: m-tile mt = i / (2 DT), step s2 = (i / DT) % 2, dims dt = i % DT.
        constexpr int NP = MT * 2 * DT;
        u32x4_t va[3];
        auto rdv = [&](int i, u32x4_t& dst) {
          const int mt = i / (2 * DT), s2 = (i / DT) % 2, dt = i % DT;
          const int r0 = mt * 32 + 16 * s2 + trow;
          const int col = dt * 32 + tcol;
          const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_short4_t*)(cV + swv<D>(r0, col >> 3) + (col & 7)));
          const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_short4_t*)(cV + swv<D>(r0 + 8, col >> 3) + (col & 7)));
          const uint64_t lo64 = __builtin_bit_cast(uint64_t, lo), hi64 = __builtin_bit_cast(uint64_t, hi);
          dst = u32x4_t{(uint32_t)lo64, (uint32_t)(lo64 >> 32), (uint32_t)hi64, (uint32_t)(hi64 >> 32)};
        };
        rdv(0, va[0]);
        rdv(1, va[1]);
#pragma unroll
        for (int i = 0; i < NP; ++i) {
          if (i + 2 < NP) rdv(i + 2, va[(i + 2) % 3]);
          __builtin_amdgcn_sched_barrier(0);
          const int mt = i / (2 * DT), s2 = (i / DT) % 2, dt = i % DT;
          o[dt] = mfma32<kPvBf16>(va[i % 3], pb[mt][s2], o[dt]);
          if constexpr (kPvBf16) o[dt] = mfma32<true>(va[i % 3], pb_lo[mt][s2], o[dt]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if (do_qk) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int r = 0; r < 16; ++r) st[mt][r] = 0.0f;
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          if (ks + 2 < KS) rdk(ks + 2, ka[(ks + 2) % 3]);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) st[mt] = mfma32<kBf16>(ka[ks % 3][mt], qf[ks], st[mt]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };

    // Prologue: tables 0-2, K of tiles 0 and 1, V of tile 0.
    __syncthreads();
    if (wave == 0) {
      if (ntiles > 0) build(Slot<0>{}, 0);
      if (ntiles > 1) build(Slot<1>{}, 1);
      if (ntiles > 2) build(Slot<2>{}, 2);
    }
    __syncthreads();
    if (ntiles > 0) {
      u32x2_t kreg8b[kF8 ? CH : 1];
      issue_k(Slot<0>{}, kreg8);
      if (ntiles > 1) issue_k(Slot<1>{}, kreg8b);
      issue_v(Slot<0>{});
      finish_k(Slot<0>{}, kreg8);
      if (ntiles > 1) finish_k(Slot<1>{}, kreg8b);
      finish_v(Slot<0>{});
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();

    // Step j (buffer slot j % 3, a compile-time index: every LDS address is a
    // loop-invariant lane offset plus an immediate).  Every wave runs the
    // same steps; group 1 passes one barrier first, so its k-th barrier of
    // the loop meets group 0's (k + 1)-th: one phase behind.  Loads for a
    // later tile start at the top of a vector step and are finished at the
    // end of the next matrix step, two phases later.
    auto step = [&](auto slot, int j) {
      constexpr int B0 = decltype(slot)::value;  // tile j
      constexpr int B1 = (B0 + 1) % 3;           // tile j + 1
      constexpr int B2 = (B0 + 2) % 3;           // tiles j + 2 and j - 1
      // Matrix step j.
      // The matrix step issues at a raised wave priority: a SIMD otherwise
      // issues the older wave (group 0) first, so group 1's MFMAs queued
      // behind group 0's vector work (config 4b +0.7 %, FP8 +0.4 %).
      __builtin_amdgcn_s_setprio(1);
      mstep(Slot<B0>{}, Slot<B2>{}, j >= 1 && (j - 1) * KB < wave_kend, j < ntiles && j * KB < wave_kend);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
      // This thread's loads of vector step j - 1: V of tile j and K of tile j + 1.
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the direct loads are not tracked by the compiler
      if (j >= 1 && j + 1 < ntiles) finish_k(Slot<B1>{}, kreg8);
      if (j >= 1 && j < ntiles) finish_v(Slot<B0>{});
      __syncthreads();
      // Vector step j.
      if (j + 1 < ntiles) issue_v(Slot<B1>{});
      if (j + 2 < ntiles) issue_k(Slot<B2>{}, kreg8);
      if (j < ntiles && j * KB < wave_kend) softmax(j);
      if (wave == 0 && j + 3 < ntiles) build(Slot<B0>{}, j + 3);
      __syncthreads();
    };
    if (grp == 1) __syncthreads();
    for (int j = 0; j <= ntiles; j += 3) {  // work-group uniform exits
      step(Slot<0>{}, j);
      if (j + 1 > ntiles) break;
      step(Slot<1>{}, j + 1);
      if (j + 2 > ntiles) break;
      step(Slot<2>{}, j + 2);
    }
    if (grp == 0) __syncthreads();
    if constexpr (kMode == kPvConvert) {
      bool bad = false;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) bad |= !__builtin_isfinite(o[dt][r]);
      }
      if (bad) s_ovf = 1;
      __syncthreads();
      if (s_ovf) return false;
    }
    return true;
  };

  if constexpr (kF8) {
    run(PvTag<kPvF8>{});
  } else if constexpr (KV::kCode == kBF16) {
    if (!run(PvTag<kPvConvert>{})) {
      badkey = 0x7fffffff;
      run(PvTag<kPvSplit>{});
    }
  } else {
    run(PvTag<kPvDirect>{});
  }

  if (badkey != 0x7fffffff) atomicMin(&s_badkey, badkey);
  __syncthreads();
  const int bad_from = s_badkey;

  const float lt = l + __shfl_xor(l, 32, 64);
  if (!live) return;
  const bool bad = bad_from <= qpos;
  const float inv = lt > 0.0f ? p.vscale / lt : 0.0f;
  const int64_t orow = ((tok0 + qrow) * p.H + h) * D;
  const uintptr_t oa = reinterpret_cast<uintptr_t>(p.out);
  const bool vec = (p.out_dtype == kF32 ? (oa & 15) == 0 : (oa & 7) == 0);
  if (!vec) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = dt * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
        store_elem(p.out, p.out_dtype, orow + d, bad ? __builtin_nanf("") : o[dt][r] * inv);
      }
    }
    return;
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = bad ? __builtin_nanf("") : o[dt][4 * j + i] * inv;
      const int64_t e = orow + dt * 32 + 8 * j + 4 * hh;
      if (p.out_dtype == kF32) {
        u64x2_t w = u64x2_t{(uint64_t)__builtin_bit_cast(uint32_t, v[0]) | ((uint64_t)__builtin_bit_cast(uint32_t, v[1]) << 32),
                            (uint64_t)__builtin_bit_cast(uint32_t, v[2]) | ((uint64_t)__builtin_bit_cast(uint32_t, v[3]) << 32)};
        *reinterpret_cast<u64x2_t*>(static_cast<float*>(p.out) + e) = w;
      } else {
        const uint32_t w0 = p.out_dtype == kF16 ? pack2<false>(v[0], v[1]) : pack2<true>(v[0], v[1]);
        const uint32_t w1 = p.out_dtype == kF16 ? pack2<false>(v[2], v[3]) : pack2<true>(v[2], v[3]);
        const uint64_t w = (uint64_t)w0 | ((uint64_t)w1 << 32);
        *reinterpret_cast<uint64_t*>(static_cast<uint16_t*>(p.out) + e) = w;
      }
    }
  }
}

// CU count of the current device and resident work-groups per CU of one
// kernel instance, cached per device; {0, 0} if unknown.
template <typename F>
static void residency(F kernel, std::atomic<int64_t> (&cache)[64], int64_t* cus, int64_t* per_cu,
                      int threads = kPfThreads) {
  *cus = *per_cu = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return;
  if (dev < 64) {
    const int64_t c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) {
      *cus = c >> 8;
      *per_cu = c & 0xff;
      return;
    }
  }
  int n = 0, k = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&k, kernel, threads, 0) != hipSuccess || k <= 0 ||
      k > 0xff)
    return;
  if (dev < 64) cache[dev].store(((int64_t)n << 8) | k, std::memory_order_relaxed);
  *cus = n;
  *per_cu = k;
}

template <typename KV, int D, bool kSplitQ, bool kSplit>
static hipError_t launch_pf_q(const PrefillParams& p, hipStream_t stream) {
  static std::atomic<int64_t> cache[64];
  const auto kernel = prefill_mfma_kernel<KV, D, kSplitQ, kSplit>;
  PrefillParams q = p;
  constexpr int QB = kSplit ? 2 * PfShape<D>::QW : PfShape<D>::QB;
  q.q_tiles = (p.S + QB - 1) / QB;
  int64_t units = (int64_t)q.B * q.H * q.q_tiles;
  int64_t cus = 0, per_cu = 0;
  residency(kernel, cache, &cus, &per_cu);
  q.wg_cus = units > cus && units <= cus * per_cu ? (int32_t)cus : 0;  // one resident wave
  // Variable-length batches of up to kVlMaxSeqs sequences: a compacted grid
  // of at most the units with rows (sum over sequences of ceil(rows / QB) <
  // T / QB + sequences).
  q.vl_compact = 0;
  if (p.cu_q && p.B <= kVlMaxSeqs) {
    const int64_t ub = (p.q_total + QB - 1) / QB + std::min<int64_t>(p.B, p.q_total);
    units = (int64_t)q.H * std::min<int64_t>((int64_t)q.B * q.q_tiles, ub);
    q.vl_compact = 1;
    q.wg_cus = 0;
  }
  note_launch("pa::prefill_mfma_kernel<%s, %d, %s, %s>", KV::kName, D, kSplitQ ? "true" : "false",
              kSplit ? "true" : "false");
  hipLaunchKernelGGL(kernel, dim3((unsigned)units), dim3(kPfThreads), 0, stream, q);
  return hipGetLastError();
}

template <typename KV, int D>
static hipError_t launch_pp(const PrefillParams& p, hipStream_t stream) {
  static std::atomic<int64_t> cache[64];
  const auto kernel = prefill_pp_kernel<KV, D>;
  PrefillParams q = p;
  q.q_tiles = (p.S + kPpRows - 1) / kPpRows;
  const int64_t units = (int64_t)q.B * q.H * q.q_tiles;
  int64_t cus = 0, per_cu = 0;
  residency(kernel, cache, &cus, &per_cu, kPpThreads);
  q.wg_cus = units > cus && units <= cus * per_cu ? (int32_t)cus : 0;  // one resident wave
  note_launch("pa::prefill_pp_kernel<%s, %d>", KV::kName, D);
  hipLaunchKernelGGL(kernel, dim3((unsigned)units), dim3(kPpThreads), 0, stream, q);
  return hipGetLastError();
}

// Key-split mode when the plain grid (blocks of 128 query rows) has fewer
// work-groups than CUs: chunks of a long context
// (the reference's 512-token chunk at context 2048: 192 work-groups, +19 %).
// Above that, twice the tiles cost more than the shorter chains save
// (config 4a, 768 work-groups: -17 %).
// The choice counts the work-groups that have rows to serve: a uniform
// batch's B * ceil(S / rows) per head; a variable-length batch brings T rows
// in all (its grid is sized by the longest sequence, and the work-groups past
// a sequence's rows exit at once), so about ceil(T / rows) of its blocks carry
// work.  (A mixed batch of 64 decode rows and four 256-row chunks had taken
// the 8-wave kernel for its 816-block grid: 48 blocks with rows, on 256 CUs.)
template <typename KV, int D>
static hipError_t launch_pf(const PrefillParams& p, hipStream_t stream) {
  if constexpr (PfShape<D>::MT == 2) {
    static std::atomic<int64_t> cache[64];
    int64_t cus = 0, per_cu = 0;
    residency(prefill_mfma_kernel<KV, D, false, false>, cache, &cus, &per_cu);
    auto busy = [&](int rows) {
      const int64_t grid = (int64_t)p.B * ((p.S + rows - 1) / rows);
      return (int64_t)p.H * (p.cu_q ? std::min<int64_t>(grid, (p.q_total + rows - 1) / rows) : grid);
    };
    const int64_t plain = busy(PfShape<D>::QB);
    if (cus > 0 && plain < cus)
      return p.q_split ? launch_pf_q<KV, D, true, true>(p, stream) : launch_pf_q<KV, D, false, true>(p, stream);
    // The 8-wave kernel (one work-group per CU) for grids of at least two
    // of its work-groups per CU; below that its 256-row blocks leave CUs
    // idle at the end of the launch (config 4a: 384 work-groups, -20 %).
    if constexpr (KV::kCode == kF16 || KV::kCode == kBF16 || KV::kCode == kFP8) {
      const int64_t pp_units = busy(kPpRows);
      if (!p.q_split && p.MB <= kPfBtStage && cus > 0 && pp_units >= 2 * cus) return launch_pp<KV, D>(p, stream);
    }
  }
  return p.q_split ? launch_pf_q<KV, D, true, false>(p, stream) : launch_pf_q<KV, D, false, false>(p, stream);
}

template <typename KV>
static hipError_t launch_pf_kv(const PrefillParams& p, hipStream_t stream) {
  switch (p.D) {
    case 32: return launch_pf<KV, 32>(p, stream);
    case 64: return launch_pf<KV, 64>(p, stream);
    case 128: return launch_pf<KV, 128>(p, stream);
    case 256: return launch_pf<KV, 256>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_prefill_mfma(const PrefillParams& p, int kv_dtype, hipStream_t stream) {
  if (kv_dtype == kF16) return launch_pf_kv<KvF16>(p, stream);
  if (kv_dtype == kBF16) return launch_pf_kv<KvBF16>(p, stream);
  if (kv_dtype == kFP8) return p.q_dtype == kBF16 ? launch_pf_kv<KvFP8QkBf16>(p, stream) : launch_pf_kv<KvFP8>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace pa
