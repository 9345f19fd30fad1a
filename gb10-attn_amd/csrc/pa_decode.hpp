// pa_decode.hpp -- gfx950 paged-attention decode kernel (context-split pass).
//
// Work unit: one work-group (4 waves of 64 lanes) per
//   (query row z, KV head kvh, head chunk hc, partition part).
// The GC query heads of one GQA group that share KV head kvh are served by
// the same work-group, so every K/V page is read from HBM once per KV head
// (the reference reads it once per query head, kernels/paged_attn_v3.cu:63).
//
// Gather.  A K (or V) row of one token is D * sizeof(KV) contiguous bytes.
// LPT = D * sizeof(KV) / 16 consecutive lanes read it with one 16-byte load
// each, so one global_load_dwordx4 instruction fetches TPI = 64 / LPT whole
// rows (e.g. 8 rows of 128 B for D=64 fp16).  Physical addresses follow
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

namespace pa {

template <typename KV, int D>
struct DecodeShape {
  static constexpr int VEC = KV::kVec;         // elements per lane per load
  static constexpr int LPT = D / VEC;          // lanes per token row
  static_assert(LPT >= 1 && LPT <= 64 && (LPT & (LPT - 1)) == 0, "unsupported D/KV combination");
  static constexpr int TPI = 64 / LPT;         // token rows per load instruction
  static constexpr int NI_RAW = 32 / TPI;
  static constexpr int NI = NI_RAW < 1 ? 1 : (NI_RAW > 8 ? 8 : NI_RAW);  // loads per K tile
  static constexpr int TT = NI * TPI;          // tokens per wave tile
};

constexpr int kDecodeWaves = 4;
constexpr int kDecodeThreads = 64 * kDecodeWaves;
constexpr int kBtChunk = 256;  // block-table entries staged in LDS at a time

template <typename KV, int D, int GC>
__global__ __launch_bounds__(kDecodeThreads) void decode_kernel(const DecodeParams p) {
  using Sh = DecodeShape<KV, D>;
  constexpr int VEC = Sh::VEC, LPT = Sh::LPT, TPI = Sh::TPI, NI = Sh::NI, TT = Sh::TT;
  constexpr int NW = kDecodeWaves;

  __shared__ int32_t s_bt[kBtChunk];
  __shared__ float s_acc[NW][GC][D];
  __shared__ float s_m[NW][GC];
  __shared__ float s_l[NW][GC];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int slot = lane / LPT;
  const int sub = lane % LPT;

  // blockIdx.x -> (z, kvh, hc, part), partition fastest.
  const int units_y = p.HKV * p.head_chunks;
  int id = blockIdx.x;
  const int part = id % p.parts;
  id /= p.parts;
  const int y = id % units_y;
  const int z = id / units_y;
  const int kvh = y / p.head_chunks;
  const int hc = y - kvh * p.head_chunks;
  const int b = z / p.Sq;
  const int sq = z - b * p.Sq;
  const int g0 = hc * GC;

  const int maxctx = p.MB * p.BS;
  const int ctx_b = p.context_lens[b];
  const int ctx = ctx_b - p.Sq + sq + 1;  // keys this query row attends
  const bool fixed = p.part_tokens > 0;
  const bool ok = ctx > 0 && ctx_b <= maxctx;
  const int nparts = fixed ? (ok ? (ctx + p.part_tokens - 1) / p.part_tokens : 0) : p.parts;
  const bool final_here = p.direct || (fixed && nparts <= 1);

  if (!ok) {
    // Zero rows for an empty context, NaN rows for one longer than the table.
    if (final_here && part == 0) {
      const float fillv = ctx <= 0 ? 0.0f : __builtin_nanf("");
      for (int idx = threadIdx.x; idx < GC * D; idx += kDecodeThreads) {
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
    const int chunk = (ctx + p.parts - 1) / p.parts;  // kernels/paged_attn_v3.cu:65-68
    t0 = part * chunk;
    t1 = min(t0 + chunk, ctx);
  }

  // This lane's slice of q for the GC heads, pre-scaled into log2 units.
  float qr[GC][VEC];
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    const bool hv = g0 + g < p.G;
    const int h = kvh * p.G + g0 + g;
    const int64_t qb = ((int64_t)z * p.H + h) * D + sub * VEC;
#pragma unroll
    for (int e = 0; e < VEC; ++e) qr[g][e] = hv ? load_elem(p.q, p.q_dtype, qb + e) * p.qscale : 0.0f;
  }

  float m[GC], l[GC], acc[GC][VEC];
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    m[g] = kNegBig;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[g][e] = 0.0f;
  }
  int bad = 0;

  const int64_t k_lane = ((int64_t)kvh * p.k_sh + sub * VEC) * KV::kBytes;
  const int64_t v_lane = ((int64_t)kvh * p.v_sh + sub * VEC) * KV::kBytes;
  const int64_t k_sb = p.k_sb * KV::kBytes, k_st = p.k_st * KV::kBytes;
  const int64_t v_sb = p.v_sb * KV::kBytes, v_st = p.v_st * KV::kBytes;
  const int32_t* bt_row = p.block_tables + (int64_t)b * p.bt_stride;
  const uint64_t nb = (uint64_t)p.num_blocks;

  if (t0 < t1) {
    const int pg0 = (int)fastdiv((uint32_t)t0, p.bs_div);
    const int pg1 = (int)fastdiv((uint32_t)(t1 - 1), p.bs_div) + 1;
    for (int cp = pg0; cp < pg1; cp += kBtChunk) {
      const int np = min(kBtChunk, pg1 - cp);
      __syncthreads();
      if ((int)threadIdx.x < np) s_bt[threadIdx.x] = bt_row[cp + threadIdx.x];
      __syncthreads();
      const int ct0 = max(t0, cp * p.BS);
      const int ct1 = min(t1, (cp + np) * p.BS);
      for (int tile = ct0 + wave * TT; tile < ct1; tile += NW * TT) {
        u32x4_t rk[NI], rv[NI];
        bool val[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const int t = tile + i * TPI + slot;
          val[i] = t < ct1;
          rk[i] = u32x4_t{0, 0, 0, 0};
          rv[i] = u32x4_t{0, 0, 0, 0};
          if (val[i]) {
            const int pg = (int)fastdiv((uint32_t)t, p.bs_div);
            const int off = t - pg * p.BS;
            const int blk = s_bt[pg - cp];
            if ((uint64_t)(int64_t)blk >= nb) {
              bad = 1;
              val[i] = false;
            } else {
              rk[i] = load16(p.k, (int64_t)blk * k_sb + (int64_t)off * k_st + k_lane);
              rv[i] = load16(p.v, (int64_t)blk * v_sb + (int64_t)off * v_st + v_lane);
            }
          }
        }
        float s[NI][GC];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          float kf[VEC];
          KV::widen(rk[i], kf);
#pragma unroll
          for (int g = 0; g < GC; ++g) {
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < VEC; ++e) d = fmaf(qr[g][e], kf[e], d);
            s[i][g] = group_sum<LPT>(d);
          }
        }
        float vf[NI][VEC];
#pragma unroll
        for (int i = 0; i < NI; ++i) KV::widen(rv[i], vf[i]);
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          float mt = kNegBig;
#pragma unroll
          for (int i = 0; i < NI; ++i) mt = val[i] ? fmaxf(mt, s[i][g]) : mt;
          const float mn = fmaxf(m[g], mt);
          const float corr = fast_exp2(m[g] - mn);
          float lg = l[g] * corr;
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[g][e] *= corr;
#pragma unroll
          for (int i = 0; i < NI; ++i) {
            const float pi = val[i] ? fast_exp2(s[i][g] - mn) : 0.0f;
            lg += pi;
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[g][e] = fmaf(pi, vf[i][e], acc[g][e]);
          }
          l[g] = lg;
          m[g] = mn;
        }
      }
    }
  }

  // Combine the TPI slot streams of this wave (log-sum-exp rule).
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
  if (slot == 0) {
#pragma unroll
    for (int g = 0; g < GC; ++g)
#pragma unroll
      for (int e = 0; e < VEC; ++e) s_acc[wave][g][sub * VEC + e] = acc[g][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      s_m[wave][g] = m[g];
      s_l[wave][g] = l[g];
    }
  }
  bad = __syncthreads_or(bad);

  // Combine the waves and write out.
  for (int idx = threadIdx.x; idx < GC * D; idx += kDecodeThreads) {
    const int g = idx / D, d = idx - (idx / D) * D;
    if (g0 + g >= p.G) continue;
    float M = kNegBig;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][g]);
    float L = 0.0f, A = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = fast_exp2(s_m[w][g] - M);
      L += s_l[w][g] * wt;
      A += s_acc[w][g][d] * wt;
    }
    const int h = kvh * p.G + g0 + g;
    if (final_here) {
      store_elem(p.out, p.out_dtype, ((int64_t)z * p.H + h) * D + d,
                 bad ? __builtin_nanf("") : A / L);
    } else {
      const int64_t pidx = ((int64_t)b * p.H + h) * p.parts + part;
      p.ws_acc[pidx * D + d] = A;
      if (d == 0) {
        p.ws_m[pidx] = M;
        p.ws_l[pidx] = bad ? __builtin_nanf("") : L;
      }
    }
  }
}

template <typename KV, int D, int GC>
hipError_t launch_decode_dg(const DecodeParams& p, hipStream_t stream) {
  const int64_t blocks = (int64_t)p.B * p.Sq * p.HKV * p.head_chunks * p.parts;
  hipLaunchKernelGGL((decode_kernel<KV, D, GC>), dim3((unsigned)blocks), dim3(kDecodeThreads), 0,
                     stream, p);
  return hipGetLastError();
}

template <typename KV, int D>
hipError_t launch_decode_d(const DecodeParams& p, int gc, hipStream_t stream) {
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
