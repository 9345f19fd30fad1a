// pa_reduce.hip -- log-sum-exp reduce of the context-split partials, the
// separate second launch of the split decode (kernels/paged_attn_v3.cu:128-166):
//   M = max_s m_s,  w_s = 2^(m_s - M),  out = sum_s w_s acc_s / sum_s w_s l_s
// (m in log2 units).  One wave per (sequence, query head).  Lane (r, c)
// covers dims 4c .. 4c + 3 of the partial rows (LR = D / 4 lanes per row) for
// every RI-th partition (RI = 64 / LR rows per load instruction), so a round
// of NL loads per lane reads NL * RI whole rows at once; the partition states
// sit one per lane, and each weight reaches the lanes that read its row by a
// lane permute.  The kernel is latency-bound (a few MB of partials): the
// context length, the first 64 partition states and the first round of rows
// are loaded in one round trip, and a split of up to 64 partitions (D <= 64;
// 32 at D = 128, 16 at D = 256) needs no other.
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
  constexpr int LR = D / 4;                  // lanes per partial row
  constexpr int RI = 64 / LR;                // rows per load instruction
  constexpr int NL = 64 / RI < 16 ? 64 / RI : 16;  // loads per lane per round
  constexpr int PR = NL * RI;                // partitions per round (divides 64)
  static_assert(LR >= 1 && LR <= 64 && 64 % PR == 0, "unsupported head_dim");
  const int lane = threadIdx.x & 63;
  const int r = lane / LR, c = lane % LR;
  const int64_t f = (int64_t)blockIdx.x * kReduceWaves + (threadIdx.x >> 6);
  if (f >= (int64_t)p.B * p.H) return;
  const int b = (int)(f / p.H);
  const int P = p.parts;
  const int64_t base = f * P;

  // One round trip: the context length, partition states 0..63, the first
  // round of rows (partitions past this call's count are not loaded).
  const int ctx = p.context_lens[b];
  float mv = lane < P ? p.ws_m[base + lane] : kNegBig;
  float lv = lane < P ? p.ws_l[base + lane] : 0.0f;
  float4_t rows[NL];
  auto load_rows = [&](int s0, int lim) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int s = s0 + i * RI + r;
      rows[i] = s < lim ? *reinterpret_cast<const float4_t*>(p.ws_acc + (base + s) * D + 4 * c)
                        : float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };
  load_rows(0, P);

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
      if (r == 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) store_elem(p.out, p.out_dtype, f * D + 4 * c + e, fillv);
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

  float4_t acc = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float L = 0.0f;
  for (int w0 = 0; w0 < n; w0 += 64) {  // windows of 64 partitions: their weights in the lanes
    if (w0 > 0) {
      const int s = w0 + lane;
      mv = s < n ? p.ws_m[base + s] : kNegBig;
      lv = s < n ? p.ws_l[base + s] : 0.0f;
    }
    const float w = w0 + lane < n ? fast_exp2(mv - M) : 0.0f;
    L += w0 + lane < n ? w * lv : 0.0f;
    for (int k0 = 0; k0 < 64 && w0 + k0 < n; k0 += PR) {
      if (w0 + k0 > 0) load_rows(w0 + k0, n);
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        const int j = k0 + i * RI + r;  // this row's partition within the window
        const float wi = __shfl(w, j, 64);
        // Rows past the count may hold anything (0 * NaN is NaN): selected away.
        const float4_t x = w0 + j < n ? rows[i] : float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = fmaf(wi, x[e], acc[e]);
      }
    }
  }
  // Sum the RI row groups (lanes c, c + LR, ...), then the row sums.
#pragma unroll
  for (int off = LR; off < 64; off <<= 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += __shfl_xor(acc[e], off, 64);
  }
  L = wave_sum(L);
  if (r == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) store_elem(p.out, p.out_dtype, f * D + 4 * c + e, acc[e] / L);
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
