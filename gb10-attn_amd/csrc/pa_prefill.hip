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

constexpr int kPfQB = 64;  // query rows per work-group
constexpr int kPfKB = 64;  // keys per tile
constexpr int kPfThreads = 256;

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

template <typename KV>
__device__ inline float from_bits16(uint32_t h) {
  if constexpr (KV::kCode == kF16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  } else {
    return __builtin_bit_cast(float, h << 16);
  }
}

template <typename KV, int D>
__global__ __launch_bounds__(kPfThreads) void prefill_mfma_kernel(const PrefillParams p) {
  constexpr int NSLAB = D / 32;         // 32-wide k-slabs of the QK^T product
  constexpr int NDT = D / 16;           // 16-row tiles of O^T
  constexpr int KROW = D + 8;           // sK row pitch (elements): 16-byte pad
  constexpr int VROW = kPfKB + 8;       // sV row pitch (keys)
  constexpr int CHUNKS = kPfKB * D / 8; // 16-byte pieces per K (or V) tile
  constexpr int CPT = (CHUNKS + kPfThreads - 1) / kPfThreads;
  static_assert(D % 32 == 0, "D must be a multiple of 32");

  __shared__ __attribute__((aligned(16))) uint16_t sK[kPfKB * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t sV[D * VROW];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;  // query column (S^T / O^T) or key row (K operand)
  const int kg = lane >> 4;   // lane group: k-index block of the operands

  // Work-group -> (b, h, query tile): XCD-contiguous, longest tile first.
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
  const int qs0 = qt * kPfQB;
  const int qrow = qs0 + wave * 16 + col;           // this lane's query row
  const bool row_live = qrow < p.S;
  const int qpos = ctx - p.S + qrow;                // absolute position
  const int64_t out_row = (((int64_t)b * p.S + qrow) * p.H + h) * D;

  if (ctx > maxctx) {  // context longer than the block table: poison the rows that attend keys
    if (row_live && kg == 0) {
      const float fillv = qpos < 0 ? 0.0f : __builtin_nanf("");
      for (int d = 0; d < D; ++d) store_elem(p.out, p.out_dtype, out_row + d, fillv);
    }
    return;
  }
  __shared__ int s_badkey;  // first key whose page has an invalid block id
  if (threadIdx.x == 0) s_badkey = 0x7fffffff;
  __syncthreads();
  // Keys the whole work-group can see: [0, kend).
  const int kend = min(ctx, ctx - p.S + min(qs0 + kPfQB, p.S));
  const int ntiles = kend > 0 ? (kend + kPfKB - 1) / kPfKB : 0;
  // Keys this wave's rows can see.
  const int wave_last = min(qs0 + wave * 16 + 15, p.S - 1);
  const int wave_kend = min(ctx, ctx - p.S + wave_last + 1);
  const int wave_kfull = ctx - p.S + qs0 + wave * 16 + 1;  // keys < this are visible to all rows

  // Q^T operand: row qrow, dims c*32 + kg*8 .. +8, rounded to the KV type
  // (qf) with the rounding residual in qf_lo.
  u32x4_t qf[NSLAB], qf_lo[NSLAB];
#pragma unroll
  for (int c = 0; c < NSLAB; ++c) {
    uint32_t w[4], wl[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float x0 = 0.0f, x1 = 0.0f;
      if (row_live) {
        const int64_t qi = out_row + c * 32 + kg * 8 + 2 * j;
        x0 = load_elem(p.q, p.q_dtype, qi);
        x1 = load_elem(p.q, p.q_dtype, qi + 1);
      }
      const uint32_t h0 = to_bits16<KV>(x0), h1 = to_bits16<KV>(x1);
      w[j] = h0 | (h1 << 16);
      wl[j] = to_bits16<KV>(x0 - from_bits16<KV>(h0)) | (to_bits16<KV>(x1 - from_bits16<KV>(h1)) << 16);
    }
    qf[c] = u32x4_t{w[0], w[1], w[2], w[3]};
    qf_lo[c] = u32x4_t{wl[0], wl[1], wl[2], wl[3]};
  }
  const bool q_split = p.q_split != 0;
  constexpr bool kSplitP = KV::kCode == kBF16;

  float4_t o[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) o[t] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m = kNegBig;
  float l = 0.0f;  // this lane group's share of the row sum

  const int32_t* bt_row = p.block_tables + (int64_t)b * p.bt_stride;
  const int64_t k_sb = p.k_sb * 2, k_st = p.k_st * 2, k_sh = (int64_t)kvh * p.k_sh * 2;
  const int64_t v_sb = p.v_sb * 2, v_st = p.v_st * 2, v_sh = (int64_t)kvh * p.v_sh * 2;
  const uint64_t nb = (uint64_t)p.num_blocks;

  u32x4_t rk[CPT], rv[CPT];
  auto gload = [&](int tile) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int idx = (int)threadIdx.x + c * kPfThreads;
      rk[c] = u32x4_t{0, 0, 0, 0};
      rv[c] = u32x4_t{0, 0, 0, 0};
      if (idx < CHUNKS) {
        const int key = idx / (D / 8);
        const int dg = idx - key * (D / 8);
        const int kabs = tile * kPfKB + key;
        if (kabs < kend) {
          const int pg = (int)fastdiv((uint32_t)kabs, p.bs_div);
          const int off = kabs - pg * p.BS;
          const int blk = bt_row[pg];
          if ((uint64_t)(int64_t)blk >= nb) {
            atomicMin(&s_badkey, kabs);
          } else {
            rk[c] = load16(p.k, (int64_t)blk * k_sb + (int64_t)off * k_st + k_sh + dg * 16);
            rv[c] = load16(p.v, (int64_t)blk * v_sb + (int64_t)off * v_st + v_sh + dg * 16);
          }
        }
      }
    }
  };

  if (ntiles > 0) gload(0);
  for (int t = 0; t < ntiles; ++t) {
    // Stage the tile: K as [key][D], V transposed as [D][key].
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int idx = (int)threadIdx.x + c * kPfThreads;
      if (idx < CHUNKS) {
        const int key = idx / (D / 8);
        const int dg = idx - key * (D / 8);
        *reinterpret_cast<u32x4_t*>(&sK[key * KROW + dg * 8]) = rk[c];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          sV[(dg * 8 + 2 * j) * VROW + key] = (uint16_t)(rv[c][j] & 0xffffu);
          sV[(dg * 8 + 2 * j + 1) * VROW + key] = (uint16_t)(rv[c][j] >> 16);
        }
      }
    }
    __syncthreads();
    if (t + 1 < ntiles) gload(t + 1);

    const int tk0 = t * kPfKB;
    if (tk0 < wave_kend) {
      // S^T tile: 4 blocks of 16 keys x 16 query columns.
      float4_t st[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NSLAB; ++c) {
          const u32x4_t a =
              *reinterpret_cast<const u32x4_t*>(&sK[(mt * 16 + col) * KROW + c * 32 + kg * 8]);
          acc = mfma16x16x32<KV>(a, qf[c], acc);
          if (q_split) acc = mfma16x16x32<KV>(a, qf_lo[c], acc);
        }
        st[mt] = acc;
      }
      const bool need_mask = tk0 + kPfKB > wave_kfull || !row_live;
      float mx = kNegBig;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float s = st[mt][i] * p.qscale;
          if (need_mask) {
            const int key = tk0 + mt * 16 + kg * 4 + i;
            if (!(row_live && key <= qpos)) s = kNegBig;
          }
          st[mt][i] = s;
          mx = fmaxf(mx, s);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mn = fmaxf(m, mx);
      const float corr = fast_exp2(m - mn);
      l *= corr;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[dt] *= corr;
      // P^T operand, one per 32-key chunk: keys c2*32 + kg*4 + {0..3} and
      // c2*32 + 16 + kg*4 + {0..3}, matching the V^T reads below.
      u32x4_t pb[2], pb_lo[2];
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        uint32_t w[4], wl[4];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const float s0 = st[2 * c2 + half][2 * j];
            const float s1 = st[2 * c2 + half][2 * j + 1];
            const float p0 = s0 > kNegBig ? fast_exp2(s0 - mn) : 0.0f;
            const float p1 = s1 > kNegBig ? fast_exp2(s1 - mn) : 0.0f;
            const uint32_t h0 = to_bits16<KV>(p0), h1 = to_bits16<KV>(p1);
            w[half * 2 + j] = h0 | (h1 << 16);
            if constexpr (kSplitP) {
              l += p0 + p1;
              wl[half * 2 + j] = to_bits16<KV>(p0 - from_bits16<KV>(h0)) |
                                 (to_bits16<KV>(p1 - from_bits16<KV>(h1)) << 16);
            } else {
              l += from_bits16<KV>(h0) + from_bits16<KV>(h1);
            }
          }
        }
        pb[c2] = u32x4_t{w[0], w[1], w[2], w[3]};
        if constexpr (kSplitP) pb_lo[c2] = u32x4_t{wl[0], wl[1], wl[2], wl[3]};
      }
      m = mn;
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const uint16_t* vr = &sV[(dt * 16 + col) * VROW + c2 * 32 + kg * 4];
          const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(vr);
          const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(vr + 16);
          const u32x4_t a = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
          o[dt] = mfma16x16x32<KV>(a, pb[c2], o[dt]);
          if constexpr (kSplitP) o[dt] = mfma16x16x32<KV>(a, pb_lo[c2], o[dt]);
        }
      }
    }
    __syncthreads();
  }
  __syncthreads();
  const bool bad = s_badkey <= qpos;  // this row read a page with an invalid block id

  // Row sum over the 4 lane groups, normalise, write 4 dims per lane per O^T tile.
  float lt = l + __shfl_xor(l, 16, 64);
  lt += __shfl_xor(lt, 32, 64);
  if (!row_live) return;
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = dt * 16 + kg * 4 + i;
      store_elem(p.out, p.out_dtype, out_row + d, bad ? __builtin_nanf("") : o[dt][i] * inv);
    }
  }
}

template <typename KV, int D>
static hipError_t launch_pf(const PrefillParams& p, hipStream_t stream) {
  const int64_t blocks = (int64_t)p.B * p.H * p.q_tiles;
  hipLaunchKernelGGL((prefill_mfma_kernel<KV, D>), dim3((unsigned)blocks), dim3(kPfThreads), 0,
                     stream, p);
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
