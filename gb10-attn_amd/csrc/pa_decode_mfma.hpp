// pa_decode_mfma.hpp -- GQA decode on CDNA4 matrix cores (gfx950).
//
// For a GQA group of GC >= 8 query heads per KV head, the VALU decode kernel
// spends GC dot products, GC softmax streams and GC weighted-V updates per
// lane on every K/V row and runs out of issue slots before HBM bandwidth.
// Here the group is the n-dimension of v_mfma_f32_16x16x32_{f16,bf16}:
//
//  * Work unit as the VALU kernel: one work-group (4 waves) per (query row,
//    partition, KV head, head chunk), heads fastest.  The waves take 32-token
//    tiles of the partition round robin, each with its own online-softmax
//    state, and merge by the log-sum-exp rule at the end.
//  * S^T = K . Q^T: a lane loads its K operand straight from the paged pool
//    (token lane%16 of a 16-token m-tile, dims (lane/16)*8 + 32*ks .. +8, one
//    16-byte load); Q^T (the GC heads, zero-padded to 16 columns) stays in
//    registers.  A 16-token m-tile lies in one page (block size a multiple of
//    16, tiles 16-aligned), so page lookups are wave-uniform.
//  * O^T += V^T . P^T: the V tile goes to the wave's own LDS buffer with
//    global_load_lds_dwordx4 and is read transposed (ds_read_b64_tr_b16);
//    the probabilities never leave registers.  P is carried as a 16-bit
//    hi + lo pair (two products; ~22/16-bit significand for fp16/bf16), and q
//    likewise when it does not arrive in the KV type, so the result keeps the
//    fp32-softmax precision of the reference's decode (kernels/paged_attn_v3.cu:93-111).
//  * Two tiles in flight per wave (K in registers, V in a double-buffered LDS
//    area); rows past the partition end, or on pages with an invalid block id,
//    load row 0 of block 0, are masked, and their V rows are zeroed in LDS.
// Semantics (partition bounds, partials, NaN / zero rows) are the VALU
// kernel's: same DecodeParams, same outputs.
#pragma once

#include "pa_decode.hpp"

namespace pa {

typedef __bf16 bf16x8m_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void_m_t;
typedef short short4m_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4m_t lds_short4m_t;
typedef _Float16 half2m_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2m_t __attribute__((ext_vector_type(2)));

template <bool kBf16>
__device__ inline float4_t mfma16(const u32x4_t& a, const u32x4_t& b, const float4_t& c) {
  if constexpr (kBf16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8m_t, a),
                                                   __builtin_bit_cast(bf16x8m_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
                                                  __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
  }
}

template <bool kBf16>
__device__ inline uint32_t pack2m(float x, float y) {
  if constexpr (kBf16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{x, y}, bf16x2m_t));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{x, y}, half2m_t));
  }
}

template <bool kBf16>
__device__ inline float2_t unpack2m(uint32_t w) {
  if constexpr (kBf16) {
    return float2_t{__builtin_bit_cast(float, w << 16), __builtin_bit_cast(float, w & 0xffff0000u)};
  } else {
    const half2m_t h = __builtin_bit_cast(half2m_t, w);
    return float2_t{(float)h[0], (float)h[1]};
  }
}

__device__ inline void dma16(const void* g, lds_void_m_t* lds) { __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0); }

template <int D>
struct DmShape {
  static constexpr int KT = 32;              // tokens per wave tile (two 16-token m-tiles)
  static constexpr int KS = D / 32;          // 32-dim k-steps of S^T
  static constexpr int NDT = D / 16;         // 16-dim m-tiles of O^T
  static constexpr int NCH = D / 8;          // 16-byte chunks per V row
  static constexpr int TPD = 1024 / (D * 2); // V rows per direct load (1 KB)
  static constexpr int NDMA = KT / TPD;      // direct loads per V tile
  static constexpr int VSW = NCH >= 16 ? 3 : NCH == 8 ? 1 : 0;  // V swizzle (as the prefill's V tiles)
  static constexpr int VSH = NCH >= 16 ? 0 : 1;
  static constexpr int TILE = KT * D;        // 16-bit elements per V tile
};

// Chunk position of chunk cc of V row r: conflict-free transposed reads.
template <int D>
__device__ inline int dm_vpos(int r, int cc) {
  return cc ^ (((r >> DmShape<D>::VSH) & DmShape<D>::VSW) << 2);
}

constexpr float kDmLazy = 8.0f;  // raise the running max only past 2^8


// SQ: q may need the hi + lo split (q's dtype is not the cache's).  A
// separate instance for q of the cache's dtype keeps the run-time test out of
// the k-step loop, where it put a branch between consecutive MFMAs.
template <typename KV, int D, int GC, bool SQ>
__global__ __launch_bounds__(256) void decode_mfma_kernel(const DecodeParams p) {
  using Sh = DmShape<D>;
  constexpr int KT = Sh::KT, KS = Sh::KS, NDT = Sh::NDT, NCH = Sh::NCH, TPD = Sh::TPD, NDMA = Sh::NDMA;
  constexpr int NW = 4;
  constexpr bool kBf16 = KV::kCode == kBF16;
  static_assert(GC <= 16, "the GQA group is one 16-column MFMA n-tile");

  // Per-wave double-buffered V tiles; reused for the cross-wave merge.
  __shared__ __attribute__((aligned(16))) uint16_t s_v[NW][2][Sh::TILE];
  __shared__ int32_t s_bt[kBtChunk];
  __shared__ float s_m[NW][16];
  __shared__ float s_l[NW][16];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;  // head column (S^T, O^T, Q^T) / token row (K operand)
  const int kg = lane >> 4;   // lane group: k-slot block of the operands

  const int units_y = p.HKV * p.head_chunks;
  int id = blockIdx.x;
  const int y = id % units_y;
  id /= units_y;
  int part, z;
  if (compact_grid(p)) {
    if (!compact_unit(p, id, lane, z, part)) return;  // work-group uniform
  } else {
    part = id % p.parts;
    z = id / p.parts;
  }
  const int kvh = y / p.head_chunks;
  const int hc = y - kvh * p.head_chunks;
  const int b = z / p.Sq;
  const int sq = z - b * p.Sq;
  const int g0 = hc * GC;

  const int maxctx = p.MB * p.BS;
  const int ctx_b = p.context_lens[b];
  const int ctx = ctx_b - p.Sq + sq + 1;
  const bool fixed = p.part_tokens > 0;
  const bool ok = ctx > 0 && ctx_b <= maxctx;
  const int nparts = fixed ? (ok ? (ctx + p.part_tokens - 1) / p.part_tokens : 0) : p.parts;
  const bool final_here = p.direct || (fixed && nparts <= 1);

  if (!ok) {
    if (final_here && part == 0) {
      const float fillv = ctx <= 0 ? 0.0f : __builtin_nanf("");
      for (int idx = threadIdx.x; idx < GC * D; idx += 256) {
        const int g = idx / D, d = idx - (idx / D) * D;
        if (g0 + g >= p.G) continue;
        const int h = kvh * p.G + g0 + g;
        store_elem(p.out, p.out_dtype, ((int64_t)z * p.H + h) * D + d, fillv);
      }
    }
    return;
  }
  if (part >= nparts) return;
  int t0, t1;
  if (fixed) {
    t0 = part * p.part_tokens;
    t1 = min(t0 + p.part_tokens, ctx);
  } else {
    const int chunk = (ctx + p.parts - 1) / p.parts;
    t0 = part * chunk;
    t1 = min(t0 + chunk, ctx);
  }

  // Q^T operand: head column col (zero past the group), dims 32*ks + kg*8 .. +8,
  // in the KV type (hi + lo when q is another type).
  const bool qlive = col < GC && g0 + col < p.G;
  const bool split_q = SQ && p.q_dtype != KV::kCode;
  u32x4_t qf[KS], qlo[KS];
  {
    const int64_t qb = ((int64_t)z * p.H + kvh * p.G + g0 + (qlive ? col : 0)) * D + kg * 8;
    float xq[KS][8];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) load_elems<8>(p.q, p.q_dtype, qb + 32 * ks, xq[ks]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      uint32_t w[4], wl[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float x0 = qlive ? xq[ks][2 * j] : 0.0f;
        const float x1 = qlive ? xq[ks][2 * j + 1] : 0.0f;
        w[j] = pack2m<kBf16>(x0, x1);
        const float2_t r = unpack2m<kBf16>(w[j]);
        wl[j] = pack2m<kBf16>(x0 - r[0], x1 - r[1]);
      }
      qf[ks] = u32x4_t{w[0], w[1], w[2], w[3]};
      qlo[ks] = u32x4_t{wl[0], wl[1], wl[2], wl[3]};
    }
  }
  const float qscale = p.qscale;

  const char* kbase = static_cast<const char*>(p.k) + (int64_t)kvh * p.k_sh * 2;
  const char* vbase = static_cast<const char*>(p.v) + (int64_t)kvh * p.v_sh * 2;
  const uint32_t k_sb = (uint32_t)(p.k_sb * 2), k_st = (uint32_t)(p.k_st * 2);
  const uint32_t v_sb = (uint32_t)(p.v_sb * 2), v_st = (uint32_t)(p.v_st * 2);
  const int32_t* bt_row = p.block_tables + (int64_t)b * p.bt_stride;
  const uint64_t nb = (uint64_t)p.num_blocks;
  // Lane-invariant parts of the addresses: K row col of an m-tile at dims
  // kg*8 (+32*ks); V direct loads: row lane/NCH of each 1 KB piece, source
  // chunk at the swizzled position lane%NCH.
  const uint32_t k_lane = (uint32_t)col * k_st + (uint32_t)kg * 16;
  const int vrow = lane / NCH;
  const uint32_t v_lane = (uint32_t)vrow * v_st;

  float4_t o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m = -__builtin_inff(), l = 0.0f;
  int bad = 0;

  struct Tile {
    u32x4_t k[2][KS];
    uint32_t live;    // bit mt: m-tile mt is on a valid page
    int first;        // first token of the tile
  };

  // Loads of the tile at token `tile` (pages staged from cp): K into
  // registers, V straight into LDS buffer dv.
  auto issue = [&](int tile, int cp, int ct1, Tile& T, uint16_t* dv) {
    uint32_t live = 0;
    uint64_t base_k[2], base_v[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int ti = tile + mt * 16;  // wave-uniform
      const bool inrange = ti < ct1;
      const int pg = (int)fastdiv((uint32_t)(inrange ? ti : tile), p.bs_div);
      const int off0 = (inrange ? ti : tile) - pg * p.BS;
      const int blk = __builtin_amdgcn_readfirstlane(s_bt[min(pg - cp, kBtChunk - 1)]);
      const bool okb = (uint64_t)(int64_t)blk < nb;
      bad |= (inrange && !okb) ? 1 : 0;
      const uint32_t use = (inrange && okb) ? 1u : 0u;
      live |= use << mt;
      base_k[mt] = (uint64_t)((uint32_t)blk * use) * k_sb + (uint32_t)off0 * use * k_st;
      base_v[mt] = (uint64_t)((uint32_t)blk * use) * v_sb + (uint32_t)off0 * use * v_st;
    }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        T.k[mt][ks] = load16(kbase + base_k[mt], k_lane + ks * 64);  // cacheable: the other half of the line is the next k-step's
    }
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int mt = (i * TPD) / 16;
      // This lane fills chunk position lane%NCH of tile row i*TPD + vrow.
      const uint32_t src = (uint32_t)dm_vpos<D>(i * TPD + vrow, lane % NCH) * 16;
      dma16(vbase + base_v[mt] + (uint32_t)((i * TPD) % 16) * v_st + v_lane + src,
            (lds_void_m_t*)(dv + i * 512));
    }
    T.live = live;
    T.first = tile;
    __builtin_amdgcn_sched_barrier(0);
  };

  // After the tile's loads landed: zero V rows that are masked (past the
  // partition or on a substituted page) -- their probabilities are 0, but the
  // data there may not be finite.
  auto fix_v = [&](const Tile& T, int ct1, uint16_t* dv) {
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int r = i * TPD + vrow;  // token row of this lane's chunk in the tile
      const bool masked = !((T.live >> (r / 16)) & 1u) || T.first + r >= ct1;
      if (masked) *reinterpret_cast<u32x4_t*>(dv + i * 512 + lane * 8) = u32x4_t{0u, 0u, 0u, 0u};
    }
  };

  auto compute = [&](const Tile& T, int ct1, const uint16_t* cv) {
    float4_t st[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      st[mt] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        st[mt] = mfma16<kBf16>(T.k[mt][ks], qf[ks], st[mt]);
        if (split_q) st[mt] = mfma16<kBf16>(T.k[mt][ks], qlo[ks], st[mt]);
      }
    }
    // Scores in log2 units (any sign of the scale).  Lane (col, kg) holds
    // tokens first + mt*16 + kg*4 + i of head column col.
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) st[mt] *= qscale;
    if (T.first + KT > ct1 || T.live != 3u) {
      asm volatile("");
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = mt * 16 + kg * 4 + i;
          if (!((T.live >> mt) & 1u) || T.first + r >= ct1) st[mt][i] = -__builtin_inff();
        }
      }
    }
    float mx = fmaxf(fmaxf(fmaxf(st[0][0], st[0][1]), fmaxf(st[0][2], st[0][3])),
                     fmaxf(fmaxf(st[1][0], st[1][1]), fmaxf(st[1][2], st[1][3])));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mxs = mx;
    if (__builtin_amdgcn_ballot_w64(mxs > m + kDmLazy) != 0) {
      asm volatile("");
      const float mn = fmaxf(m, mxs);
      const float corr = mn == -__builtin_inff() ? 1.0f : fast_exp2(m - mn);
      m = mn;
      l *= corr;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[dt] *= corr;
    }
    const float negm = m == -__builtin_inff() ? 0.0f : -m;
    // P^T operand: slots 0..3 = m-tile 0 (tokens kg*4 + i), 4..7 = m-tile 1.
    uint32_t w[4], wl[4];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float p0 = fast_exp2(st[mt][2 * j] + negm);
        const float p1 = fast_exp2(st[mt][2 * j + 1] + negm);
        l += p0 + p1;
        const uint32_t h = pack2m<kBf16>(p0, p1);
        const float2_t r = unpack2m<kBf16>(h);
        w[mt * 2 + j] = h;
        wl[mt * 2 + j] = pack2m<kBf16>(p0 - r[0], p1 - r[1]);
      }
    }
    const u32x4_t pb = u32x4_t{w[0], w[1], w[2], w[3]};
    const u32x4_t pl = u32x4_t{wl[0], wl[1], wl[2], wl[3]};
    // V^T operand of dim tile dt: rows kg*4 + (col/4) and 16 + kg*4 + (col/4),
    // dims dt*16 + (col%4)*4 .. +4; lane receives dim dt*16 + col.
    const int r0 = kg * 4 + (col >> 2);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int c = dt * 16 + (col & 3) * 4;
      const short4m_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_short4m_t*)(cv + r0 * D + (dm_vpos<D>(r0, c >> 3) << 3) + (c & 7)));
      const short4m_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_short4m_t*)(cv + (r0 + 16) * D + (dm_vpos<D>(r0 + 16, c >> 3) << 3) + (c & 7)));
      const uint64_t lo64 = __builtin_bit_cast(uint64_t, lo), hi64 = __builtin_bit_cast(uint64_t, hi);
      const u32x4_t a = u32x4_t{(uint32_t)lo64, (uint32_t)(lo64 >> 32), (uint32_t)hi64, (uint32_t)(hi64 >> 32)};
      o[dt] = mfma16<kBf16>(a, pb, o[dt]);
      o[dt] = mfma16<kBf16>(a, pl, o[dt]);
    }
  };

  uint16_t* vb0 = s_v[wave][0];
  uint16_t* vb1 = s_v[wave][1];
  if (t0 < t1) {
    const int pg0 = (int)fastdiv((uint32_t)t0, p.bs_div);
    const int pg1 = (int)fastdiv((uint32_t)(t1 - 1), p.bs_div) + 1;
    for (int cp = pg0; cp < pg1; cp += kBtChunk) {
      const int np = min(kBtChunk, pg1 - cp);
      __syncthreads();
      for (int i = threadIdx.x; i < np; i += 256) s_bt[i] = bt_row[cp + i];
      __syncthreads();
      const int ct0 = max(t0, cp * p.BS);
      const int ct1 = min(t1, (cp + np) * p.BS);
      const int first = ct0 + wave * KT;
      if (first < ct1) {
        constexpr int kStep = NW * KT;
        const int ntw = (ct1 - first + kStep - 1) / kStep;
        Tile A, B;
        int tile = first;
        issue(tile, cp, ct1, A, vb0);
        for (int j = 0; j + 1 < ntw; j += 2) {
          issue(tile + kStep, cp, ct1, B, vb1);
          __builtin_amdgcn_s_waitcnt(0x0F70 | ((2 * KS + NDMA) & 15) | (((2 * KS + NDMA) >> 4) << 14));
          fix_v(A, ct1, vb0);
          compute(A, ct1, vb0);
          issue(tile + 2 * kStep, cp, ct1, A, vb0);
          __builtin_amdgcn_s_waitcnt(0x0F70 | ((2 * KS + NDMA) & 15) | (((2 * KS + NDMA) >> 4) << 14));
          fix_v(B, ct1, vb1);
          compute(B, ct1, vb1);
          tile += 2 * kStep;
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);
        if (ntw & 1) {
          fix_v(A, ct1, vb0);
          compute(A, ct1, vb0);
        }
      }
    }
  }

  // Row sums over the four lane groups; every lane of a column then holds the
  // column's (m, l).  Merge the waves through LDS (the V buffers are free now).
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  __syncthreads();
  float* s_acc = reinterpret_cast<float*>(&s_v[0][0][0]);  // [NW][16][D]
  static_assert(sizeof(s_v) >= sizeof(float) * NW * 16 * D, "merge area");
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) s_acc[(wave * 16 + col) * D + dt * 16 + kg * 4 + i] = o[dt][i];
  }
  if (kg == 0) {
    s_m[wave][col] = m;
    s_l[wave][col] = l;
  }
  bad = __syncthreads_or(bad);

  for (int idx = threadIdx.x; idx < GC * D; idx += 256) {
    const int g = idx / D, d = idx - (idx / D) * D;
    if (g0 + g >= p.G) continue;
    float M = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][g]);
    float L = 0.0f, A = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = M == -__builtin_inff() ? 0.0f : fast_exp2(s_m[w][g] - M);
      L += s_l[w][g] * wt;
      A += s_acc[(w * 16 + g) * D + d] * wt;
    }
    const int h = kvh * p.G + g0 + g;
    if (final_here) {
      store_elem(p.out, p.out_dtype, ((int64_t)z * p.H + h) * D + d,
                 bad ? __builtin_nanf("") : (L > 0.0f ? A * p.vscale / L : 0.0f));
    } else {
      const int64_t pidx = ((int64_t)b * p.H + h) * p.parts + part;
      p.ws_acc[pidx * D + d] = A * p.vscale;
      if (d == 0) {
        p.ws_m[pidx] = M == -__builtin_inff() ? kNegBig : M;
        p.ws_l[pidx] = bad ? __builtin_nanf("") : L;
      }
    }
  }
}

template <typename KV, int D, int GC>
hipError_t launch_decode_mfma_dg(const DecodeParams& p, hipStream_t stream) {
  const int64_t blocks = (int64_t)p.B * p.Sq * p.HKV * p.head_chunks * p.parts;
  const bool sq = p.q_dtype != KV::kCode;
  note_launch("pa::decode_mfma_kernel<%s, %d, %d, %s>", KV::kName, D, GC, sq ? "true" : "false");
  if (!sq)
    hipLaunchKernelGGL((decode_mfma_kernel<KV, D, GC, false>), dim3((unsigned)blocks), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_mfma_kernel<KV, D, GC, true>), dim3((unsigned)blocks), dim3(256), 0, stream, p);
  return hipGetLastError();
}

// The matrix-core path serves 16-bit caches, GQA groups of >= 8 heads (at 4
// the VALU kernel is as fast: config 3 4856 vs 4866 GB/s; at 8 the VALU
// kernel's per-lane work halves its rate: 2735 vs 5127 GB/s), one query
// position, 16-aligned pages and partitions; everything else stays on the
// VALU kernel.
template <typename KV>
bool decode_mfma_eligible(const DecodeParams& p, int gc) {
  if constexpr (KV::kCode != kF16 && KV::kCode != kBF16) {
    return false;
  } else {
    const bool aligned = p.part_tokens > 0 ? p.part_tokens % 16 == 0 : p.parts == 1;
    return gc >= 8 && p.Sq == 1 && p.BS % 16 == 0 && aligned && !p.cu_q;
  }
}

template <typename KV>
hipError_t launch_decode_mfma(const DecodeParams& p, int gc, hipStream_t stream) {
  if constexpr (KV::kCode != kF16 && KV::kCode != kBF16) {
    return hipErrorInvalidValue;
  } else {
#define PA_DM_D(DD)                                                       \
  case DD:                                                                \
    return launch_decode_mfma_dg<KV, DD, 8>(p, stream);
    switch (p.D) {
      PA_DM_D(32)
      PA_DM_D(64)
      PA_DM_D(128)
      PA_DM_D(256)
      default: return hipErrorInvalidValue;
    }
#undef PA_DM_D
  }
}

}  // namespace pa
