// pa_prefill.hip -- causal paged prefill on CDNA4 matrix cores (gfx950).
//
// Replaces the reference's WMMA tile kernel (kernels/paged_attn_wmma.cu:36-210)
// with a design built around v_mfma_f32_16x16x32_{f16,bf16}:
//
//  * A work-group (4 waves) owns one (sequence b, query head h, block of 64
//    query rows); wave w owns 16 of those rows.  Key tiles of 64 keys are
//    gathered from the paged pool (block table -> page -> row, 64-bit offsets)
//    into LDS once per work-group and shared by the 4 waves; the next tile's
//    global loads are in flight while the current one is computed.
//  * Scores are computed transposed, S^T = K . Q^T: K rows are the MFMA A
//    operand read straight from LDS (16 contiguous bytes per lane) and the
//    wave's Q rows are the B operand, held in registers for the whole loop.
//    In the S^T accumulator layout each lane holds 4 consecutive keys of one
//    query column, which is exactly the layout the B operand of the
//    following O^T += V^T . P^T product needs -- the probabilities never
//    leave registers, and the O^T rescale by the per-query correction is a
//    per-lane multiply (the reference round-trips O through shared memory for
//    it, kernels/paged_attn_wmma.cu:167-181).
//  * V is stored transposed in LDS ([D][keys]) so the V^T A operand is two
//    8-byte LDS reads per MFMA.
//  * Causal work skipping: a work-group stops at the last key its last query
//    row can see; a wave skips tiles beyond its own rows; masking is applied
//    only on tiles that cross a wave's diagonal.
//  * Work-groups are ordered longest-first within a (sequence, head) and the
//    (sequence, head) ranges are laid out so that consecutive ranges land on
//    the same XCD (work-group i runs on XCD i mod 8), keeping a head's K/V
//    pages in one L2.
//
// Semantics follow kernels/paged_attn_wmma.cu:80-205: query row r of the
// chunk sits at ctx - S + r and sees keys [0, ctx - S + r]; accumulation and
// the softmax are fp32; a row that sees no key is written as zeros (:200).
// Precision: fp16 carries P and Q as the reference does (one rounding to
// fp16, 11-bit significand).  bf16 has an 8-bit significand, too coarse for
// the fp32-oracle tolerance, so P is carried as a bf16 hi + lo pair (two
// P.V products, ~16-bit significand), and Q likewise whenever it does not
// arrive in the KV type.
#include "pa_device.hpp"

namespace pa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

template <typename KV>
__device__ inline float4_t mfma16x16x32(const u32x4_t& a, const u32x4_t& b, const float4_t& c) {
  if constexpr (KV::kCode == kF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
                                                  __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
}

// fp32 -> 16-bit KV element bits, round to nearest even.
template <typename KV>
__device__ inline uint32_t to_bits16(float x) {
  if constexpr (KV::kCode == kF16) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
  } else {
    return (uint32_t)f32_to_bf16_bits(x);
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

template <typename KV>
__device__ inline float from_bits16(uint32_t h) {
  if constexpr (KV::kCode == kF16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  } else {
    return __builtin_bit_cast(float, h << 16);
  }
}

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

constexpr int kPfThreads = 256;  // 4 waves
constexpr int kPfBtStage = 1024;  // block-table entries staged in LDS

// Query rows per wave for head dims up to 128 (compile-time knob): 32 gives
// each LDS K/V fragment two uses, 16 halves the registers.
#ifndef PA_PF_QW
#define PA_PF_QW 32
#endif

template <int D>
struct PfShape {
  static constexpr int QW = D <= 128 ? PA_PF_QW : 16;  // query rows per wave
  static constexpr int NT = QW / 16;             // 16-column n-tiles per wave
  static constexpr int QB = 4 * QW;              // query rows per work-group
  static constexpr int KB = D <= 128 ? 64 : 32;  // keys per tile
  static constexpr int MT = KB / 16;             // 16-key m-tiles per tile
  static constexpr int NSLAB = D / 32;           // 32-wide k-slabs of Q.K^T
  static constexpr int NDT = D / 16;             // 16-row tiles of O^T
  static constexpr int NCH = D / 8;              // 16-byte chunks per row
  static constexpr int SWZ = NCH >= 8 ? 7 : NCH - 1;  // chunk swizzle mask
  static constexpr int CPT = KB * NCH / kPfThreads;    // chunks per thread per tile
  static_assert(KB * NCH % kPfThreads == 0, "tile chunks must divide the work-group");
};

// LDS element offset of (row, chunk cc) in a swizzled [KB][D] tile: chunk cc of
// row r lives at chunk position cc ^ (r & SWZ), which spreads the 16-byte
// reads of 16 consecutive rows (same cc) over distinct banks.
template <int D>
__device__ inline int swz(int row, int cc) {
  return row * D + ((cc ^ (row & PfShape<D>::SWZ)) << 3);
}

template <typename KV, int D, bool kSplitQ>
__global__ __launch_bounds__(kPfThreads) void prefill_mfma_kernel(const PrefillParams p) {
  using Sh = PfShape<D>;
  constexpr int QW = Sh::QW, NT = Sh::NT, QB = Sh::QB, KB = Sh::KB, MT = Sh::MT;
  constexpr int NSLAB = Sh::NSLAB, NDT = Sh::NDT, NCH = Sh::NCH, CPT = Sh::CPT;

  __shared__ __attribute__((aligned(16))) uint16_t sK[2][KB * D];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][KB * D];
  __shared__ int s_badkey;  // first key whose page has an invalid block id
  __shared__ int32_t s_bt[kPfBtStage];  // the work-group's block ids, when they fit

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;  // query column (S^T / O^T) or key row (K operand)
  const int kg = lane >> 4;   // lane group: k-index block of the operands

  // Work-group -> (b, h, query block): XCD-contiguous, longest block first.
  const int nq = p.q_tiles;
  const int64_t total = (int64_t)p.B * p.H * nq;
  int64_t x = blockIdx.x;
  if ((total & 7) == 0) x = (x & 7) * (total >> 3) + (x >> 3);
  const int qt = nq - 1 - (int)(x % nq);
  const int64_t bh = x / nq;
  const int h = (int)(bh % p.H);
  const int b = (int)(bh / p.H);
  const int kvh = h / p.G;

  const int ctx = p.context_lens[b];
  const int maxctx = p.MB * p.BS;
  const int qs0 = qt * QB;
  const int qw0 = qs0 + wave * QW;  // this wave's first query row

  if (ctx > maxctx) {  // context longer than the block table: poison rows that attend keys
    for (int nt = 0; nt < NT; ++nt) {
      const int qrow = qw0 + nt * 16 + col;
      if (qrow < p.S && kg == 0) {
        const float fillv = ctx - p.S + qrow < 0 ? 0.0f : __builtin_nanf("");
        const int64_t orow = (((int64_t)b * p.S + qrow) * p.H + h) * D;
        for (int d = 0; d < D; ++d) store_elem(p.out, p.out_dtype, orow + d, fillv);
      }
    }
    return;
  }
  if (threadIdx.x == 0) s_badkey = 0x7fffffff;

  // Keys the work-group's rows can see: [0, kend); this wave's rows: [0, wave_kend).
  const int kend = min(ctx, ctx - p.S + min(qs0 + QB, p.S));
  const int ntiles = kend > 0 ? (kend + KB - 1) / KB : 0;
  const int wave_last = min(qw0 + QW - 1, p.S - 1);
  const int wave_kend = min(ctx, ctx - p.S + wave_last + 1);
  const int wave_kfull = ctx - p.S + qw0 + 1;  // keys below this are visible to every row
  const bool wave_padded = qw0 + QW > p.S;

  // Q^T operands (rows qw0 + nt*16 + col, dims c*32 + kg*8 .. +8), rounded to
  // the KV type, with the rounding residual for the low-part product.
  u32x4_t qf[NT][NSLAB], qf_lo[kSplitQ ? NT : 1][NSLAB];
  int qpos[NT];
  bool live[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int qrow = qw0 + nt * 16 + col;
    live[nt] = qrow < p.S;
    qpos[nt] = ctx - p.S + qrow;
    const int64_t qrow_off = (((int64_t)b * p.S + qrow) * p.H + h) * D;
#pragma unroll
    for (int c = 0; c < NSLAB; ++c) {
      uint32_t w[4], wl[4];
      float xv[8];
      if (live[nt]) {
        load8f(p.q, p.q_dtype, qrow_off + c * 32 + kg * 8, xv);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[e] = 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float x0 = xv[2 * j], x1 = xv[2 * j + 1];
        const uint32_t h0 = to_bits16<KV>(x0), h1 = to_bits16<KV>(x1);
        w[j] = h0 | (h1 << 16);
        wl[j] = to_bits16<KV>(x0 - from_bits16<KV>(h0)) | (to_bits16<KV>(x1 - from_bits16<KV>(h1)) << 16);
      }
      qf[nt][c] = u32x4_t{w[0], w[1], w[2], w[3]};
      if constexpr (kSplitQ) qf_lo[nt][c] = u32x4_t{wl[0], wl[1], wl[2], wl[3]};
    }
  }
  constexpr bool kSplitP = KV::kCode == kBF16;

  float4_t o[NDT][NT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) o[dt][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m[NT], l[NT];  // l: this lane group's share of the row sum
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m[nt] = kNegBig;
    l[nt] = 0.0f;
  }

  const int32_t* bt_row = p.block_tables + (int64_t)b * p.bt_stride;
  // Block ids of the pages this work-group reads live in an LDS window of
  // kPfBtStage pages starting at page win0, so a tile's K/V loads never wait
  // behind a dependent block-table load.  The window moves (at a tile
  // boundary, behind a barrier) when the next tile to load leaves it.
  const int npages = kend > 0 ? (int)fastdiv((uint32_t)(kend - 1), p.bs_div) + 1 : 0;
  int win0 = 0;
  auto stage = [&](int first) {
    win0 = first;
    const int n = min(kPfBtStage, npages - first);
    for (int i = threadIdx.x; i < n; i += kPfThreads) s_bt[i] = bt_row[first + i];
  };
  auto ensure_window = [&](int t) {  // uniform; call with every thread, then barrier
    const int last = min(t * KB + KB, kend) - 1;
    const int plast = (int)fastdiv((uint32_t)last, p.bs_div);
    if (plast >= win0 + kPfBtStage) {
      __syncthreads();  // every gload of the old window is done
      stage((int)fastdiv((uint32_t)(t * KB), p.bs_div));
      __syncthreads();
    }
  };
  stage(0);
  __syncthreads();
  const int64_t k_sb = p.k_sb * 2, k_st = p.k_st * 2, k_sh = (int64_t)kvh * p.k_sh * 2;
  const int64_t v_sb = p.v_sb * 2, v_st = p.v_st * 2, v_sh = (int64_t)kvh * p.v_sh * 2;
  const uint64_t nb = (uint64_t)p.num_blocks;
  int badkey = 0x7fffffff;

  // Global -> registers for tile t (16-byte chunks), registers -> LDS (swizzled).
  // Global -> registers for tile t.  Branch-free: a row past kend, or on a
  // page with an invalid block id, loads row 0 of block 0 (in bounds, NB >= 1)
  // and is zeroed when stored to LDS.
  u32x4_t rk[CPT], rv[CPT];
  uint32_t rmask = 0;
  const char* kbase = static_cast<const char*>(p.k) + k_sh;
  const char* vbase = static_cast<const char*>(p.v) + v_sh;
  auto gload = [&](int t) {
    int blk[CPT], off[CPT];
    bool val[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int idx = (int)threadIdx.x + c * kPfThreads;
      const int row = idx / NCH;
      const int kabs = t * KB + row;
      val[c] = kabs < kend;
      const int pg = (int)fastdiv((uint32_t)(val[c] ? kabs : 0), p.bs_div);
      off[c] = (val[c] ? kabs : 0) - pg * p.BS;
      blk[c] = s_bt[val[c] ? pg - win0 : 0];
    }
    uint32_t mask = 0;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int idx = (int)threadIdx.x + c * kPfThreads;
      const int cc = idx - (idx / NCH) * NCH;
      const bool okb = (uint64_t)(int64_t)blk[c] < nb;
      if (val[c] && !okb) badkey = min(badkey, t * KB + idx / NCH);
      const bool use = val[c] && okb;
      const int64_t bb = use ? blk[c] : 0;
      const int64_t oo = use ? off[c] : 0;
      rk[c] = load16(kbase, bb * k_sb + oo * k_st + cc * 16);
      rv[c] = load16(vbase, bb * v_sb + oo * v_st + cc * 16);
      mask |= use ? (1u << c) : 0u;
    }
    rmask = mask;
  };
  auto sstore = [&](int buf) {
    const u32x4_t zero = u32x4_t{0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int idx = (int)threadIdx.x + c * kPfThreads;
      const int row = idx / NCH, cc = idx - (idx / NCH) * NCH;
      const bool use = (rmask >> c) & 1u;
      *reinterpret_cast<u32x4_t*>(&sK[buf][swz<D>(row, cc)]) = use ? rk[c] : zero;
      *reinterpret_cast<u32x4_t*>(&sV[buf][swz<D>(row, cc)]) = use ? rv[c] : zero;
    }
  };

  auto compute = [&](int t, int buf) {
    const int tk0 = t * KB;
    // S^T = K . Q^T: MT x NT tiles of 16 keys x 16 queries.
    float4_t st[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) st[mt][nt] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NSLAB; ++c) {
        const int row = mt * 16 + col;
        const u32x4_t a = *reinterpret_cast<const u32x4_t*>(&sK[buf][swz<D>(row, c * 4 + kg)]);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          st[mt][nt] = mfma16x16x32<KV>(a, qf[nt][c], st[mt][nt]);
          if constexpr (kSplitQ) st[mt][nt] = mfma16x16x32<KV>(a, qf_lo[nt][c], st[mt][nt]);
        }
      }
    }
    // Online softmax per query column; keys of this lane: tk0 + mt*16 + kg*4 + i.
    const bool need_mask = tk0 + KB > wave_kfull || wave_padded;
    u32x4_t pb[KB / 32][NT], pb_lo[KB / 32][NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float mx = kNegBig;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float sv = st[mt][nt][i] * p.qscale;
          if (need_mask) {
            const int key = tk0 + mt * 16 + kg * 4 + i;
            if (!(live[nt] && key <= qpos[nt])) sv = kNegBig;
          }
          st[mt][nt][i] = sv;
          mx = fmaxf(mx, sv);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mn = fmaxf(m[nt], mx);
      const float corr = fast_exp2(m[nt] - mn);
      m[nt] = mn;
      float ls = l[nt] * corr;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[dt][nt] *= corr;
      // P^T operand per 32-key chunk c2: keys c2*32 + kg*4 + {0..3} (m-tile 2*c2)
      // then c2*32 + 16 + kg*4 + {0..3} (m-tile 2*c2+1), matching the V^T reads.
#pragma unroll
      for (int c2 = 0; c2 < KB / 32; ++c2) {
        uint32_t w[4], wl[4];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const float s0 = st[2 * c2 + half][nt][2 * j];
            const float s1 = st[2 * c2 + half][nt][2 * j + 1];
            const float p0 = s0 > kNegBig ? fast_exp2(s0 - mn) : 0.0f;
            const float p1 = s1 > kNegBig ? fast_exp2(s1 - mn) : 0.0f;
            const uint32_t h0 = to_bits16<KV>(p0), h1 = to_bits16<KV>(p1);
            w[half * 2 + j] = h0 | (h1 << 16);
            if constexpr (kSplitP) {
              ls += p0 + p1;
              wl[half * 2 + j] = to_bits16<KV>(p0 - from_bits16<KV>(h0)) |
                                 (to_bits16<KV>(p1 - from_bits16<KV>(h1)) << 16);
            } else {
              ls += from_bits16<KV>(h0) + from_bits16<KV>(h1);
            }
          }
        }
        pb[c2][nt] = u32x4_t{w[0], w[1], w[2], w[3]};
        if constexpr (kSplitP) pb_lo[c2][nt] = u32x4_t{wl[0], wl[1], wl[2], wl[3]};
      }
      l[nt] = ls;
    }
    // O^T += V^T . P^T.  V^T operand for (c2, dt): two transposing 8-byte LDS
    // reads; lane j of each 16-lane group supplies row key_base + j/4, dims
    // dt*16 + (j%4)*4 .. +4, and receives dim dt*16 + j for the 4 rows.
    const int trow = col >> 2, tcol = (col & 3) * 4;
#pragma unroll
    for (int c2 = 0; c2 < KB / 32; ++c2) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const int r0 = c2 * 32 + kg * 4 + trow;
        const int r1 = r0 + 16;
        const int dcol = dt * 16 + tcol;
        const int e0 = swz<D>(r0, dcol >> 3) + (dcol & 7);
        const int e1 = swz<D>(r1, dcol >> 3) + (dcol & 7);
        const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(&sV[buf][e0]));
        const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(&sV[buf][e1]));
        const uint64_t lo64 = __builtin_bit_cast(uint64_t, lo), hi64 = __builtin_bit_cast(uint64_t, hi);
        const u32x4_t a = u32x4_t{(uint32_t)lo64, (uint32_t)(lo64 >> 32), (uint32_t)hi64,
                                  (uint32_t)(hi64 >> 32)};
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          o[dt][nt] = mfma16x16x32<KV>(a, pb[c2][nt], o[dt][nt]);
          if constexpr (kSplitP) o[dt][nt] = mfma16x16x32<KV>(a, pb_lo[c2][nt], o[dt][nt]);
        }
      }
    }
  };

  // Double-buffered tiles: the next tile's global loads are in flight while
  // the current tile is computed; one barrier per tile.
  if (ntiles > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) {
      ensure_window(t + 1);
      gload(t + 1);
    }
    if (t * KB < wave_kend) compute(t, buf);
    if (t + 1 < ntiles) sstore(buf ^ 1);
    __syncthreads();
  }
  if (badkey != 0x7fffffff) atomicMin(&s_badkey, badkey);
  __syncthreads();
  const int bad_from = s_badkey;

  // Row sums over the 4 lane groups, normalise, write 4 dims per lane per O^T tile.
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float lt = l[nt] + __shfl_xor(l[nt], 16, 64);
    lt += __shfl_xor(lt, 32, 64);
    if (!live[nt]) continue;
    const bool bad = bad_from <= qpos[nt];
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    const int qrow = qw0 + nt * 16 + col;
    const int64_t orow = (((int64_t)b * p.S + qrow) * p.H + h) * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = dt * 16 + kg * 4 + i;
        store_elem(p.out, p.out_dtype, orow + d, bad ? __builtin_nanf("") : o[dt][nt][i] * inv);
      }
    }
  }
}

template <typename KV, int D>
static hipError_t launch_pf(const PrefillParams& p, hipStream_t stream) {
  PrefillParams q = p;
  q.q_tiles = (p.S + PfShape<D>::QB - 1) / PfShape<D>::QB;
  const int64_t blocks = (int64_t)q.B * q.H * q.q_tiles;
  if (p.q_split)
    hipLaunchKernelGGL((prefill_mfma_kernel<KV, D, true>), dim3((unsigned)blocks), dim3(kPfThreads),
                       0, stream, q);
  else
    hipLaunchKernelGGL((prefill_mfma_kernel<KV, D, false>), dim3((unsigned)blocks), dim3(kPfThreads),
                       0, stream, q);
  return hipGetLastError();
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
  return hipErrorInvalidValue;
}

}  // namespace pa
