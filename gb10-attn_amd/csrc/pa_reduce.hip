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
  const int lane = threadIdx.x & 63;
  const int64_t f = (int64_t)blockIdx.x * kReduceWaves + (threadIdx.x >> 6);
  if (f >= (int64_t)p.B * p.H) return;
  const int b = (int)(f / p.H);

  const int ctx = p.context_lens[b];
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
    n = p.parts;
  }

  const int64_t base = f * p.parts;
  // Global max over the n partition maxima.
  float M = kNegBig;
  for (int s0 = 0; s0 < n; s0 += 64) {
    const int s = s0 + lane;
    M = fmaxf(M, s < n ? p.ws_m[base + s] : kNegBig);
  }
  M = wave_max(M);

  float L = 0.0f;
  float acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] = 0.0f;
  for (int s0 = 0; s0 < n; s0 += 64) {
    const int s = s0 + lane;
    const float w = s < n ? fast_exp2(p.ws_m[base + s] - M) : 0.0f;
    L += s < n ? w * p.ws_l[base + s] : 0.0f;
    const int cnt = min(64, n - s0);
    for (int i = 0; i < cnt; ++i) {
      const float wi = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), i));
      const float* row = p.ws_acc + (base + s0 + i) * D;
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        const int d = lane + 64 * j;
        if (d < D) acc[j] = fmaf(wi, row[d], acc[j]);
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
