// pa_write.hip -- KV-cache write ("reshape and cache") on gfx950.
//
// Writes T new tokens' K and V rows ([T, HKV, D], any token/head strides)
// into the paged pool ([NB, BS, HKV, D] views) at the slots of a slot
// mapping: token t goes to block slot[t] / BS, row slot[t] % BS.  This is the
// write the reference's serving engine does with TorchBlockAllocator.write_kv
// (external; call sites harness/repro_crash.py:52-58 and
// results/c001-20260901-223111/bench_b64_c2048.txt:16-22), where a
// sequence's [n_head, ctx, head_dim] layer slice is exactly a strided
// [T, HKV, D] source and slot[t] = block_ids[t / BS] * BS + t % BS.
//
// HBM-bound byte work: each thread moves 8 elements of one (token, head) row
// (one 16-byte store for a 16-bit cache, 8 bytes for FP8), converting the
// element type on the way (round to nearest even, as the oracle's codecs).  A
// negative slot is skipped (padding tokens), as is a slot past the pool;
// 64-bit offsets.  With per-tensor scales the cache receives key / k_scale
// and value / v_scale (fp32 division, correctly rounded), the form the
// scaled decode entry point reads back.
#include "pa_device.hpp"

#include <algorithm>

namespace pa {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kWriteThreads = 256;

// Eight source elements (16-byte aligned) as fp32, or as raw 16-bit words
// when source and cache share a 16-bit type.
template <int SRC>
__device__ inline void load8(const void* base, int64_t idx, float (&x)[8]) {
  if constexpr (SRC == kF32) {
    const float4_t a = *reinterpret_cast<const float4_t*>(static_cast<const float*>(base) + idx);
    const float4_t b = *reinterpret_cast<const float4_t*>(static_cast<const float*>(base) + idx + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = a[e];
      x[4 + e] = b[e];
    }
  } else {
    const u32x4_t r = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(base) + idx);
    if constexpr (SRC == kF16) {
      KvF16::widen(r, x);
    } else {
      KvBF16::widen(r, x);
    }
  }
}

// fp32 -> FP8 E4M3 (OCP, "fn": no infinities) code, round to nearest even,
// saturating at +-448 (the largest finite value; infinities too), NaN ->
// 0x7f, -0 -> 0x80.  Normal range: the fp32 bits rounded to 3 mantissa bits
// and rebiased (exponent bias 127 -> 7); below 2^-6 the code is the integer
// nearest |x| * 2^9 (subnormal steps of 2^-9; 8 is the smallest normal).
__device__ inline uint32_t fp8_e4m3_code(float x) {
  const uint32_t b = __builtin_bit_cast(uint32_t, x);
  const uint32_t sign = (b >> 24) & 0x80u;
  const uint32_t a = b & 0x7fffffffu;
  if (a > 0x7f800000u) return 0x7fu;        // NaN
  if (a >= 0x43e00000u) return sign | 0x7eu;  // |x| >= 448
  if (a >= 0x3c800000u) {                   // |x| >= 2^-6
    const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
    return sign | ((r >> 20) - ((127u - 7u) << 3));
  }
  return sign | (uint32_t)__builtin_rintf(__builtin_bit_cast(float, a) * 512.0f);
}

// x / s rounded to nearest, from r = RN(1 / s): q = RN(x r) is within one ulp
// of x / s, the residual x - q s is exact in one FMA, and RN(q + (x - q s) r)
// is the correctly rounded quotient (Markstein's theorem) while x, r and q
// stay in the normal range.  fast: |r| in [2^-60, 2^60] (host-checked); then
// |x| in [2^-60, 2^61) keeps q normal.  Otherwise (zero, subnormal, huge,
// NaN, infinite operands) the full-precision division is taken.
__device__ inline float div_rn(float x, float s, float r, bool fast) {
  const float q = x * r;
  const uint32_t e = (__builtin_bit_cast(uint32_t, x) >> 23) & 0xffu;  // biased exponent of x
  if (fast && e - 67u <= 120u) return __builtin_fmaf(__builtin_fmaf(-q, s, x), r, q);
  return (x == 0.0f || x != x) ? q : __fdiv_rn(x, s);
}

template <int DST>
__device__ inline void store8(void* base, int64_t idx, const float (&x)[8]) {
  if constexpr (DST == kFP8) {
    u32x2_t w;
    bool nan = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) nan |= x[e] != x[e];
    if (!nan) {
      // v_cvt_pk_fp8_f32 (round to nearest even) on values clamped to +-448,
      // so that every finite or infinite input saturates as fp8_e4m3_code does.
      float c[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) c[e] = __builtin_fminf(__builtin_fmaxf(x[e], -448.0f), 448.0f);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(c[4 * j], c[4 * j + 1], 0, false);
        w[j] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c[4 * j + 2], c[4 * j + 3], lo, true);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j)
        w[j] = fp8_e4m3_code(x[4 * j]) | (fp8_e4m3_code(x[4 * j + 1]) << 8) |
               (fp8_e4m3_code(x[4 * j + 2]) << 16) | (fp8_e4m3_code(x[4 * j + 3]) << 24);
    }
    *reinterpret_cast<u32x2_t*>(static_cast<uint8_t*>(base) + idx) = w;
  } else if constexpr (DST == kF32) {
    float* p = static_cast<float*>(base) + idx;
    *reinterpret_cast<float4_t*>(p) = float4_t{x[0], x[1], x[2], x[3]};
    *reinterpret_cast<float4_t*>(p + 4) = float4_t{x[4], x[5], x[6], x[7]};
  } else {
    u32x4_t w;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float2_t f = float2_t{x[2 * j], x[2 * j + 1]};
      if constexpr (DST == kF16) {
        w[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, half2_t));
      } else {
        w[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
      }
    }
    *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(base) + idx) = w;
  }
}

template <int SRC, int DST, bool kSlot64>
__global__ __launch_bounds__(kWriteThreads) void write_kv_kernel(const WriteParams p) {
  // Work item -> (token, head, 8-element chunk) in 32-bit arithmetic (a launch
  // covers fewer than 2^31 items; the host splits larger writes by tokens).
  const uint32_t idx = blockIdx.x * kWriteThreads + threadIdx.x;
  const uint32_t th = fastdiv(idx, p.chunk_div);  // (token, head) row of this launch
  if (th >= (uint32_t)p.T * (uint32_t)p.HKV) return;
  const int c = (int)(idx - th * p.chunk_div.d);
  const uint32_t tl = fastdiv(th, p.hkv_div);
  const int h = (int)(th - tl * (uint32_t)p.HKV);
  const int64_t t = (int64_t)p.t_base + tl;

  const int64_t ks = t * p.key_st + (int64_t)h * p.key_sh + c * 8;
  const int64_t vs = t * p.val_st + (int64_t)h * p.val_sh + c * 8;
  const int64_t slot = kSlot64 ? static_cast<const int64_t*>(p.slots)[t]
                               : (int64_t) static_cast<const int32_t*>(p.slots)[t];
  auto dest = [&](int64_t& kd, int64_t& vd) {
    const uint32_t s32 = (uint32_t)slot;
    const uint32_t blk = fastdiv(s32, p.bs_div);
    const uint32_t off = s32 - blk * (uint32_t)p.BS;
    kd = (int64_t)blk * p.kc_sb + (int64_t)off * p.kc_st + (int64_t)h * p.kc_sh + c * 8;
    vd = (int64_t)blk * p.vc_sb + (int64_t)off * p.vc_st + (int64_t)h * p.vc_sh + c * 8;
  };
  if constexpr (SRC == DST && SRC != kF32) {
    if (p.unit_scale) {
      // Same 16-bit type: copy the bits (NaN payloads included), K's row then
      // V's (one read and one write stream at a time: the four streams at
      // once measured 2-5 % slower).
      if (slot < 0 || slot >= p.nslots) return;
      int64_t kd, vd;
      dest(kd, vd);
      *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(p.kc) + kd) =
          *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p.key) + ks);
      *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(p.vc) + vd) =
          *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p.value) + vs);
      return;
    }
  }
  // Converting writes: the slot and both source rows are loaded in one round
  // trip (FP8 config 4b +8 %).
  float kx[8], vx[8];
  load8<SRC>(p.key, ks, kx);
  load8<SRC>(p.value, vs, vx);
  if (slot < 0 || slot >= p.nslots) return;
  int64_t kd, vd;
  dest(kd, vd);
  if (!p.unit_scale) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      kx[e] = div_rn(kx[e], p.k_scale, p.k_rcp, p.k_fast);
      vx[e] = div_rn(vx[e], p.v_scale, p.v_rcp, p.v_fast);
    }
  }
  store8<DST>(p.kc, kd, kx);
  store8<DST>(p.vc, vd, vx);
}

// Tokens per launch: fewer than 2^30 work items each.
constexpr int64_t kWriteMaxItems = (int64_t)1 << 30;

template <int SRC, int DST>
static hipError_t launch_w(const WriteParams& p0, hipStream_t stream) {
  WriteParams p = p0;
  const int64_t per_token = (int64_t)p.HKV * (p.D >> 3);
  const int64_t step = std::max<int64_t>(1, kWriteMaxItems / per_token);
  p.chunk_div = make_fastdiv((uint32_t)(p.D >> 3));
  p.hkv_div = make_fastdiv((uint32_t)p.HKV);
  note_launch("pa::write_kv_kernel<%d, %d, %s>", SRC, DST, p.slot_i64 ? "true" : "false");
  for (int64_t t = 0; t < p0.T; t += step) {
    p.t_base = (int32_t)t;
    p.T = (int32_t)std::min<int64_t>(step, p0.T - t);
    const int64_t work = p.T * per_token;
    const unsigned blocks = (unsigned)((work + kWriteThreads - 1) / kWriteThreads);
    if (p.slot_i64)
      hipLaunchKernelGGL((write_kv_kernel<SRC, DST, true>), dim3(blocks), dim3(kWriteThreads), 0, stream, p);
    else
      hipLaunchKernelGGL((write_kv_kernel<SRC, DST, false>), dim3(blocks), dim3(kWriteThreads), 0, stream, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <int SRC>
static hipError_t launch_w_src(const WriteParams& p, hipStream_t stream) {
  switch (p.cache_dtype) {
    case kF16: return launch_w<SRC, kF16>(p, stream);
    case kBF16: return launch_w<SRC, kBF16>(p, stream);
    case kF32: return launch_w<SRC, kF32>(p, stream);
    case kFP8: return launch_w<SRC, kFP8>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_write_kv(const WriteParams& p, hipStream_t stream) {
  switch (p.src_dtype) {
    case kF16: return launch_w_src<kF16>(p, stream);
    case kBF16: return launch_w_src<kBF16>(p, stream);
    case kF32: return launch_w_src<kF32>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pa
