// pa_reduce.hip -- log-sum-exp reduce of the context-split partials, the
// separate second launch of the split decode (kernels/paged_attn_v3.cu:128-166):
//   M = max_s m_s,  w_s = 2^(m_s - M),  out = sum_s w_s acc_s / sum_s w_s l_s
// (m in log2 units).  One wave per (sequence, query head): lanes load the
// partition states in parallel, reduce them with cross-lane operations, then
// stream the D-wide partial rows with the weights broadcast from SGPRs.
#include "pa_device.hpp"

namespace pa {

constexpr int kReduceWaves = 4;

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int D>
__global__ __launch_bounds__(64 * kReduceWaves) void reduce_kernel(const ReduceParams p) {
  constexpr int DPL = (D + 63) / 64;  // dims per lane
  constexpr int CH = 8;               // partial rows whose loads are issued together
  const int lane = threadIdx.x & 63;
  const int64_t f = (int64_t)blockIdx.x * kReduceWaves + (threadIdx.x >> 6);
  if (f >= (int64_t)p.B * p.H) return;
  const int b = (int)(f / p.H);
  const int P = p.parts;
  const int64_t base = f * P;

  // The kernel is latency-bound (a few hundred KB of partials), so the
  // context length, the partition states and the first CH partial rows are
  // loaded in one round trip, before the partition count is known.  Entries
  // past the count (never written by this call's partition pass) are loaded
  // -- they lie inside the workspace -- but only ever selected away.
  const int ctx = p.context_lens[b];
  float mv = lane < P ? p.ws_m[base + lane] : kNegBig;
  float lv = lane < P ? p.ws_l[base + lane] : 0.0f;
  float rows[CH][DPL];
#pragma unroll
  for (int i = 0; i < CH; ++i)
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const int d = lane + 64 * j;
      rows[i][j] = (i < P && d < D) ? p.ws_acc[(base + i) * D + d] : 0.0f;
    }

  const int maxctx = p.MB * p.BS;
  const bool fixed = p.part_tokens > 0;
  const bool ok = ctx > 0 && ctx <= maxctx;
  int n;
  if (fixed) {
    if (!ok) return;  // the partition kernel wrote this row
    n = (ctx + p.part_tokens - 1) / p.part_tokens;
    if (n <= 1) return;
  } else {
    if (!ok) {
      const float fillv = ctx <= 0 ? 0.0f : __builtin_nanf("");
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        const int d = lane + 64 * j;
        if (d < D) store_elem(p.out, p.out_dtype, f * D + d, fillv);
      }
      return;
    }
    n = P;
  }

  // Global max over the n partition maxima (lanes hold partitions 0..63).
  float M = lane < n ? mv : kNegBig;
  for (int s0 = 64; s0 < n; s0 += 64) {
    const int s = s0 + lane;
    M = fmaxf(M, s < n ? p.ws_m[base + s] : kNegBig);
  }
  M = wave_max(M);

  // Partitions 0..63: weights in their lanes, rows from registers (first CH)
  // or loaded CH at a time.
  float w = lane < n ? fast_exp2(mv - M) : 0.0f;
  float L = lane < n ? w * lv : 0.0f;
  float acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] = 0.0f;
  auto add_rows = [&](int s0, const float (&r)[CH][DPL], float wl) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const float wi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), i));
      if (s0 + i < n) {
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[j] = fmaf(wi, r[i][j], acc[j]);
      }
    }
  };
  auto load_rows = [&](int s0, float (&r)[CH][DPL]) {
#pragma unroll
    for (int i = 0; i < CH; ++i)
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        const int d = lane + 64 * j;
        r[i][j] = (s0 + i < n && d < D) ? p.ws_acc[(base + s0 + i) * D + d] : 0.0f;
      }
  };
  add_rows(0, rows, w);
  for (int s0 = CH; s0 < n; s0 += CH) {
    if ((s0 & 63) == 0) {  // next 64 partitions: their weights into the lanes
      const int s = s0 + lane;
      const float m2 = s < n ? p.ws_m[base + s] : kNegBig;
      const float l2 = s < n ? p.ws_l[base + s] : 0.0f;
      w = s < n ? fast_exp2(m2 - M) : 0.0f;
      L += s < n ? w * l2 : 0.0f;
    }
    load_rows(s0, rows);
    // Lane i of the 64-lane window holds the weight of partition (s0 & ~63) + i.
    const int wl0 = s0 & 63;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const float wi = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), wl0 + i));
      if (s0 + i < n) {
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[j] = fmaf(wi, rows[i][j], acc[j]);
      }
    }
  }
  L = wave_sum(L);
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = lane + 64 * j;
    if (d < D) store_elem(p.out, p.out_dtype, f * D + d, acc[j] / L);
  }
}

hipError_t launch_reduce(const ReduceParams& p, hipStream_t stream) {
  const int64_t waves = (int64_t)p.B * p.H;
  const dim3 grid((unsigned)((waves + kReduceWaves - 1) / kReduceWaves));
  const dim3 block(64 * kReduceWaves);
  note_launch("pa::reduce_kernel<%d>", p.D);
  switch (p.D) {
    case 32: hipLaunchKernelGGL(reduce_kernel<32>, grid, block, 0, stream, p); break;
    case 64: hipLaunchKernelGGL(reduce_kernel<64>, grid, block, 0, stream, p); break;
    case 128: hipLaunchKernelGGL(reduce_kernel<128>, grid, block, 0, stream, p); break;
    case 256: hipLaunchKernelGGL(reduce_kernel<256>, grid, block, 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace pa
