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
// (one 16-byte store for a 16-bit cache), converting the element type on the
// way (round to nearest even, as the oracle's codecs).  A negative slot is
// skipped (padding tokens), as is a slot past the pool; 64-bit offsets.
#include "pa_device.hpp"

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

template <int DST>
__device__ inline void store8(void* base, int64_t idx, const float (&x)[8]) {
  if constexpr (DST == kF32) {
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
  const int chunks = p.D >> 3;
  const int64_t idx = (int64_t)blockIdx.x * kWriteThreads + threadIdx.x;
  const int64_t rows = (int64_t)p.T * p.HKV;
  if (idx >= rows * chunks) return;
  const int c = (int)(idx % chunks);
  const int64_t th = idx / chunks;
  const int h = (int)(th % p.HKV);
  const int64_t t = th / p.HKV;

  const int64_t slot = kSlot64 ? static_cast<const int64_t*>(p.slots)[t]
                               : (int64_t) static_cast<const int32_t*>(p.slots)[t];
  if (slot < 0 || slot >= p.nslots) return;
  const uint32_t s32 = (uint32_t)slot;
  const uint32_t blk = fastdiv(s32, p.bs_div);
  const uint32_t off = s32 - blk * (uint32_t)p.BS;

  const int64_t ks = t * p.key_st + (int64_t)h * p.key_sh + c * 8;
  const int64_t vs = t * p.val_st + (int64_t)h * p.val_sh + c * 8;
  const int64_t kd = (int64_t)blk * p.kc_sb + (int64_t)off * p.kc_st + (int64_t)h * p.kc_sh + c * 8;
  const int64_t vd = (int64_t)blk * p.vc_sb + (int64_t)off * p.vc_st + (int64_t)h * p.vc_sh + c * 8;
  if constexpr (SRC == DST && SRC != kF32) {
    // Same 16-bit type: copy the bits (NaN payloads included).
    *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(p.kc) + kd) =
        *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p.key) + ks);
    *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(p.vc) + vd) =
        *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p.value) + vs);
  } else {
    float x[8];
    load8<SRC>(p.key, ks, x);
    store8<DST>(p.kc, kd, x);
    load8<SRC>(p.value, vs, x);
    store8<DST>(p.vc, vd, x);
  }
}

template <int SRC, int DST>
static hipError_t launch_w(const WriteParams& p, hipStream_t stream) {
  const int64_t work = (int64_t)p.T * p.HKV * (p.D >> 3);
  const unsigned blocks = (unsigned)((work + kWriteThreads - 1) / kWriteThreads);
  note_launch("pa::write_kv_kernel<%d, %d, %s>", SRC, DST, p.slot_i64 ? "true" : "false");
  if (p.slot_i64)
    hipLaunchKernelGGL((write_kv_kernel<SRC, DST, true>), dim3(blocks), dim3(kWriteThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((write_kv_kernel<SRC, DST, false>), dim3(blocks), dim3(kWriteThreads), 0, stream, p);
  return hipGetLastError();
}

template <int SRC>
static hipError_t launch_w_src(const WriteParams& p, hipStream_t stream) {
  switch (p.cache_dtype) {
    case kF16: return launch_w<SRC, kF16>(p, stream);
    case kBF16: return launch_w<SRC, kBF16>(p, stream);
    case kF32: return launch_w<SRC, kF32>(p, stream);
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
