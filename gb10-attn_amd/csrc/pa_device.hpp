// pa_device.hpp -- device helpers for the gfx950 kernels: KV element codecs,
// DPP lane reductions, dtype-generic loads/stores.
#pragma once

#include <type_traits>

#include "pa_common.hpp"

namespace pa {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- KV types --
// Each KV storage type is read 16 bytes per lane (one global_load_dwordx4;
// FP8: 8 bytes) and widened to fp32 in registers.

struct KvF16 {
  static constexpr const char* kName = "pa::KvF16";
  using Raw = u32x4_t;
  static constexpr int kBytes = 2;
  static constexpr int kVec = 8;
  static constexpr int kCode = kF16;
  __device__ static inline void widen(const u32x4_t& r, float (&o)[kVec]) {
    const half8_t h = __builtin_bit_cast(half8_t, r);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (float)h[e];
  }
  // Element pairs for packed dot products: the raw words already are.
  static constexpr int kPairs = 1 << kF16;
  template <int PT>
  __device__ static inline void to_pairs(const u32x4_t& r, uint32_t (&o)[kVec / 2]) {
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = r[w];
  }
};

struct KvBF16 {
  static constexpr const char* kName = "pa::KvBF16";
  using Raw = u32x4_t;
  static constexpr int kBytes = 2;
  static constexpr int kVec = 8;
  static constexpr int kCode = kBF16;
  __device__ static inline void widen(const u32x4_t& r, float (&o)[kVec]) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      o[2 * w] = __builtin_bit_cast(float, r[w] << 16);
      o[2 * w + 1] = __builtin_bit_cast(float, r[w] & 0xffff0000u);
    }
  }
  static constexpr int kPairs = 1 << kBF16;
  template <int PT>
  __device__ static inline void to_pairs(const u32x4_t& r, uint32_t (&o)[kVec / 2]) {
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = r[w];
  }
};

struct KvF32 {
  static constexpr const char* kName = "pa::KvF32";
  using Raw = u32x4_t;
  static constexpr int kBytes = 4;
  static constexpr int kVec = 4;
  static constexpr int kCode = kF32;
  __device__ static inline void widen(const u32x4_t& r, float (&o)[kVec]) {
    // Cast the whole vector: bit-casting single vector elements miscompiles
    // to one dword load reused for every element.
    const float4_t f = __builtin_bit_cast(float4_t, r);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = f[e];
  }
};

struct KvF64 {
  static constexpr const char* kName = "pa::KvF64";
  using Raw = u32x4_t;
  static constexpr int kBytes = 8;
  static constexpr int kVec = 2;
  static constexpr int kCode = kF64;
  __device__ static inline void widen(const u32x4_t& r, float (&o)[kVec]) {
    const uint64_t a = ((uint64_t)r[1] << 32) | r[0];
    const uint64_t b = ((uint64_t)r[3] << 32) | r[2];
    o[0] = (float)__builtin_bit_cast(double, a);
    o[1] = (float)__builtin_bit_cast(double, b);
  }
};

// OCP FP8 E4M3 ("e4m3fn": no infinities, S.1111.111 = NaN); v_cvt_pk_f32_fp8
// widens two at a time (exact: every code is an fp32 value).  Lanes load 8
// bytes (8 elements), so per-lane state matches the 16-bit caches.
struct KvFP8 {
  static constexpr const char* kName = "pa::KvFP8";
  static constexpr int kBytes = 1;
  static constexpr int kVec = 8;
  static constexpr int kCode = kFP8;
  using Raw = u32x2_t;
  __device__ static inline void widen(const Raw& r, float (&o)[kVec]) {
#pragma unroll
    for (int w = 0; w < kVec / 4; ++w) {
      const float2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)r[w], false);
      const float2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)r[w], true);
      o[4 * w] = lo[0];
      o[4 * w + 1] = lo[1];
      o[4 * w + 2] = hi[0];
      o[4 * w + 3] = hi[1];
    }
  }
  // Element pairs in fp16 or bf16 (v_cvt_scalef32_pk_{f16,bf16}_fp8 with
  // scale 1: exact for every code, NaN included).
  static constexpr int kPairs = (1 << kF16) | (1 << kBF16);
  template <int PT>
  __device__ static inline void to_pairs(const Raw& r, uint32_t (&o)[kVec / 2]) {
#pragma unroll
    for (int w = 0; w < kVec / 4; ++w) {
      if constexpr (PT == kF16) {
        o[2 * w] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(r[w], 1.0f, false));
        o[2 * w + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(r[w], 1.0f, true));
      } else {
        o[2 * w] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r[w], 1.0f, false));
        o[2 * w + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r[w], 1.0f, true));
      }
    }
  }
};

// Packed dot products over 16-bit element pairs (PT = kF16 or kBF16):
// c + a.lo * b.lo + a.hi * b.hi (v_dot2c_f32_f16 / v_dot2c_f32_bf16), and the
// pair of two fp32 values that PT represents exactly (element 0 low).
template <int PT>
__device__ inline float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (PT == kF16)
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c, false);
  else
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                          false);
}
// The first product of a chain: a.lo * b.lo + a.hi * b.hi from a zero
// accumulator.  Through the builtin the compiler materialises the zero with a
// v_mov_b32 and then uses the accumulating v_dot2c form; the three-operand
// form takes the zero as an inline constant.
template <int PT>
__device__ inline float dot2_first(uint32_t a, uint32_t b) {
  float r;
  if constexpr (PT == kF16)
    asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  else
    asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
template <int PT>
__device__ inline uint32_t pack_pair_exact(float x, float y) {
  if constexpr (PT == kF16)
    return __builtin_bit_cast(uint32_t, f16x2_t{(_Float16)x, (_Float16)y});
  else
    return (__builtin_bit_cast(uint32_t, x) >> 16) | (__builtin_bit_cast(uint32_t, y) & 0xffff0000u);
}

// Which 16-bit pair types a cache type provides (0: none).
template <typename KV, typename = void>
struct pair_types { static constexpr int value = 0; };
template <typename KV>
struct pair_types<KV, std::void_t<decltype(KV::kPairs)>> { static constexpr int value = KV::kPairs; };

__device__ inline u32x4_t load16(const void* base, int64_t byte_off) {
  return *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const char*>(base) + byte_off);
}

// One lane's raw K/V load of a KV type (16 bytes, or 8 for FP8), with the
// non-temporal (streaming) hint: each K/V row is read once per work-group.
template <typename KV>
__device__ inline typename KV::Raw load_raw(const void* base, int64_t byte_off) {
  using Raw = typename KV::Raw;
  return __builtin_nontemporal_load(reinterpret_cast<const Raw*>(reinterpret_cast<const char*>(base) + byte_off));
}

// ------------------------------------------------------- scalar element I/O --

__device__ inline float load_elem(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case kF16: return (float)reinterpret_cast<const _Float16*>(p)[i];
    case kBF16:
      return __builtin_bit_cast(float, (uint32_t)reinterpret_cast<const uint16_t*>(p)[i] << 16);
    case kF64: return (float)reinterpret_cast<const double*>(p)[i];
    default: return reinterpret_cast<const float*>(p)[i];
  }
}

// N consecutive elements p[i .. i+N) as fp32, i a multiple of N.  All loads
// of the row are issued before any is used, with the widest vector the base
// alignment allows (the branch is uniform: it depends on p and dtype only).
// A kernel's prologue then costs one memory round trip for its q row instead
// of one per element, which matters when the loads queue behind other
// work-groups' K/V streams.
typedef _Float16 f16x2v_t __attribute__((ext_vector_type(2)));
template <int N>
__device__ inline void load_elems(const void* p, int dtype, int64_t i, float (&o)[N]) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  if (dtype == kF32) {
    const float* f = static_cast<const float*>(p) + i;
    if constexpr (N % 4 == 0) {
      if ((a & 15) == 0) {
        float4_t v[N / 4];
#pragma unroll
        for (int k = 0; k < N / 4; ++k) v[k] = reinterpret_cast<const float4_t*>(f)[k];
#pragma unroll
        for (int k = 0; k < N / 4; ++k) {
#pragma unroll
          for (int e = 0; e < 4; ++e) o[4 * k + e] = v[k][e];
        }
        return;
      }
    }
    if constexpr (N % 2 == 0) {
      if ((a & 7) == 0) {
        float2_t v[N / 2];
#pragma unroll
        for (int k = 0; k < N / 2; ++k) v[k] = reinterpret_cast<const float2_t*>(f)[k];
#pragma unroll
        for (int k = 0; k < N / 2; ++k) {
          o[2 * k] = v[k][0];
          o[2 * k + 1] = v[k][1];
        }
        return;
      }
    }
  } else if (dtype == kF16 || dtype == kBF16) {
    const bool bf = dtype == kBF16;
    const uint16_t* h = static_cast<const uint16_t*>(p) + i;
    auto widen2 = [&](uint32_t w, float& x0, float& x1) {
      if (bf) {
        x0 = __builtin_bit_cast(float, w << 16);
        x1 = __builtin_bit_cast(float, w & 0xffff0000u);
      } else {
        const f16x2v_t hv = __builtin_bit_cast(f16x2v_t, w);
        x0 = (float)hv[0];
        x1 = (float)hv[1];
      }
    };
    if constexpr (N % 8 == 0) {
      if ((a & 15) == 0) {
        u32x4_t v[N / 8];
#pragma unroll
        for (int k = 0; k < N / 8; ++k) v[k] = reinterpret_cast<const u32x4_t*>(h)[k];
#pragma unroll
        for (int k = 0; k < N / 8; ++k) {
#pragma unroll
          for (int w = 0; w < 4; ++w) widen2(v[k][w], o[8 * k + 2 * w], o[8 * k + 2 * w + 1]);
        }
        return;
      }
    }
    if constexpr (N % 4 == 0) {
      if ((a & 7) == 0) {
        u32x2_t v[N / 4];
#pragma unroll
        for (int k = 0; k < N / 4; ++k) v[k] = reinterpret_cast<const u32x2_t*>(h)[k];
#pragma unroll
        for (int k = 0; k < N / 4; ++k) {
#pragma unroll
          for (int w = 0; w < 2; ++w) widen2(v[k][w], o[4 * k + 2 * w], o[4 * k + 2 * w + 1]);
        }
        return;
      }
    }
  }
#pragma unroll
  for (int e = 0; e < N; ++e) o[e] = load_elem(p, dtype, i + e);
}

// fp32 -> bf16 with round-to-nearest-even (NaN kept quiet).
__device__ inline uint16_t f32_to_bf16_bits(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ inline void store_elem(void* p, int dtype, int64_t i, float x) {
  switch (dtype) {
    case kF16: reinterpret_cast<_Float16*>(p)[i] = (_Float16)x; break;
    case kBF16: reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(x); break;
    default: reinterpret_cast<float*>(p)[i] = x; break;
  }
}

// ------------------------------------------------------- lane reductions --
// DPP row operations stay inside 16-lane rows and need no LDS traffic.

template <int CTRL>
__device__ inline float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// A quad permutation as a plain move (a broadcast whose result feeds no
// add): every lane reads a lane of its own quad, so the value a lane would
// keep without a source is never needed, and the mov form leaves it
// undefined instead of materialising a zero (one v_mov_b32 per use).  dpp()
// keeps the zero: the compiler folds that form into a following add.
template <int CTRL>
__device__ inline uint32_t dpp_quad_u(uint32_t v) {
  static_assert(CTRL >= 0 && CTRL <= 0xff, "quad permutations only");
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ inline float dpp_quad(float v) {
  static_assert(CTRL >= 0 && CTRL <= 0xff, "quad permutations only");
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i inside each 8-lane half row
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i inside each 16-lane row
constexpr int kDppRor4 = 0x124;       // lane i reads lane (i - 4) mod 16 of its 16-lane row
constexpr int kDppRor8 = 0x128;       // lane i reads lane (i - 8) mod 16 of its 16-lane row

// Sum over aligned groups of N consecutive lanes (N a power of two <= 64);
// every lane of a group receives the group's total.
template <int N>
__device__ inline float group_sum(float v) {
  if constexpr (N >= 2) v += dpp<kDppXor1>(v);
  if constexpr (N >= 4) v += dpp<kDppXor2>(v);
  if constexpr (N >= 8) v += dpp<kDppHalfMirror>(v);
  if constexpr (N >= 16) v += dpp<kDppMirror>(v);
  if constexpr (N >= 32) v += __shfl_xor(v, 16, 64);
  if constexpr (N >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace pa
