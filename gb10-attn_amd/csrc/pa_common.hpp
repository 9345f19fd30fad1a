// pa_common.hpp -- types shared by the host launchers and the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pa {

enum Dtype : int32_t { kF32 = 0, kF16 = 1, kBF16 = 2, kF64 = 3, kI32 = 4, kI64 = 5, kFP8 = 6 };

constexpr float kNegBig = -3.0e38f;          // empty-softmax sentinel (kernels/paged_attn_v3.cu:21)
constexpr float kLog2e = 1.4426950408889634f;

// Unsigned division by a runtime constant d (1 <= d < 2^31) for n < 2^31:
// q = (umulhi(n, m) + n) >> s with s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1
// (Granlund & Montgomery, "Division by invariant integers using multiplication", 1994).
struct FastDiv {
  uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  f.s = 0;
  while ((1ull << f.s) < d) ++f.s;
  f.m = (uint32_t)(((1ull << 32) * ((1ull << f.s) - d)) / d + 1);
  return f;
}

__host__ __device__ inline uint32_t fastdiv(uint32_t n, const FastDiv& f) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t hi = __umulhi(n, f.m);
#else
  const uint32_t hi = (uint32_t)(((uint64_t)n * f.m) >> 32);
#endif
  return (hi + n) >> f.s;
}

// Everything one decode launch needs.  q/out are [Bq, Sq, H, D] contiguous;
// decode has Sq = 1.  For the fp32 prefill path every query row is its own
// decode problem with context ctx_b - Sq + s + 1 (kernels/paged_attn_prefill.cu:62-65).
struct DecodeParams {
  const void* q;
  void* out;
  const void* k;
  const void* v;
  const int32_t* block_tables;
  const int32_t* context_lens;
  float* ws_acc;  // [B][H][parts][D]
  float* ws_m;    // [B][H][parts]
  float* ws_l;    // [B][H][parts]
  int64_t k_sb, k_st, k_sh;  // element strides of k_cache: block, token, head
  int64_t v_sb, v_st, v_sh;
  int64_t bt_stride;   // elements between block-table rows
  int64_t num_blocks;  // NB: valid block ids are [0, NB)
  int32_t B, Sq, H, HKV, G, D, BS, MB;
  int32_t head_chunks;  // ceil(G / GC): WGs per KV head
  int32_t q_dtype, out_dtype;
  int32_t parts;        // partitions per (sequence, KV head) in the grid
  int32_t part_tokens;  // > 0: fixed partition length; 0: chunk = ceil(ctx / parts)
  int32_t direct;       // 1: one partition, every WG writes the normalised output
  int32_t hp;           // KV heads per work-group (head packing: MHA, or GQA groups of four); <= 1: one
  int32_t pprio;        // 1: the whole grid is resident at once; waves lower their priority as they progress
  int32_t wave_parts;   // explicit splits into short chunks: 1 from the host (the launcher picks the
                        // mode: a partition per wave or per token slot); 0 otherwise
  int32_t rounds;       // slot-partition mode: partitions each token slot serves in turn
  int32_t fuse_final;   // host: the call wants the output too and decode_fuse_rounds() allows it;
                        // kernel: the work-group covers every partition of its unit and writes it
  int32_t seq_order;    // explicit split into long partitions, B <= 64, Sq = 1: sequences dispatched
                        // longest first
  FastDiv bs_div;
  float qscale;         // scale * k_scale * log2(e): scores come out in log2 units
  float vscale;         // v_scale (FP8 caches): applied to the weighted V sum
  // Variable-length batches (Sq = 1): [B + 1] row offsets into packed [T, H, D]
  // q/out; only sequences of exactly one row are served (else null).
  const int32_t* cu_q;
  int64_t q_total;
};

struct ReduceParams {
  void* out;
  const float* ws_acc;
  const float* ws_m;
  const float* ws_l;
  const int32_t* context_lens;
  int32_t B, H, D, MB, BS;
  int32_t out_dtype;
  int32_t parts;
  int32_t part_tokens;
};

struct PrefillParams {
  const void* q;   // [B, S, H, D]
  void* out;       // [B, S, H, D]
  const void* k;
  const void* v;
  const int32_t* block_tables;
  const int32_t* context_lens;
  int64_t k_sb, k_st, k_sh;
  int64_t v_sb, v_st, v_sh;
  int64_t bt_stride;
  int64_t num_blocks;
  int32_t B, S, H, HKV, G, D, BS, MB;
  int32_t q_dtype, out_dtype;
  int32_t q_tiles;   // ceil(S / QBLOCK)
  int32_t wg_cus;    // > 0: the whole grid is resident on this many CUs (work-group order)
  const int32_t* cu_q;  // variable-length batches: [B + 1] row offsets into [T, H, D] q/out (else null)
  int64_t q_total;      // T (variable-length batches)
  int32_t skip_single;  // variable-length batches: sequences of one row are served by the decode kernel
  int32_t vl_compact;   // variable-length batches (B <= kVlMaxSeqs): the grid holds only units with rows
  int32_t q_split;   // q is not exactly the KV type: add a low-part product
  FastDiv bs_div;
  float qscale;      // |scale| * log2(e), or 1 when scale == 0 (always positive)
  float q_sign;      // sign of scale applied to q (+1, -1, or 0 when scale == 0)
  float vscale;      // v_scale of a scaled (FP8) cache: multiplies the output rows
  uint32_t q_and;    // the same on packed 16-bit q: bits & q_and ^ q_xor
  uint32_t q_xor;
};

// KV-cache write: new [T, HKV, D] rows -> paged pool slots (element strides).
struct WriteParams {
  void* kc;            // k_cache / v_cache [NB, BS, HKV, D]
  void* vc;
  const void* key;     // [T, HKV, D]
  const void* value;
  const void* slots;   // [T] int32 or int64
  int64_t kc_sb, kc_st, kc_sh;
  int64_t vc_sb, vc_st, vc_sh;
  int64_t key_st, key_sh;
  int64_t val_st, val_sh;
  int64_t nslots;      // NB * BS (< 2^31)
  int32_t T, HKV, D, BS;
  int32_t src_dtype, cache_dtype, slot_i64;
  int32_t unit_scale;  // 1: k_scale == v_scale == 1 (no division)
  float k_scale, v_scale;  // the cache holds key / k_scale and value / v_scale
  float k_rcp, v_rcp;      // 1 / k_scale, 1 / v_scale rounded to nearest (fp32)
  int32_t k_fast, v_fast;  // |k_rcp|, |v_rcp| in [2^-60, 2^60]: the reciprocal-based division applies
  FastDiv bs_div;
  FastDiv chunk_div, hkv_div;  // D / 8 and HKV (work item -> token, head, chunk)
  int32_t t_base;              // first token of this launch (large writes take several)
};

constexpr int kDecodeWaves = 4;
constexpr int kDecodeThreads = 64 * kDecodeWaves;
constexpr int kBtChunk = 256;  // block-table entries a decode work-group stages in LDS at a time

// Explicit short partitions (DecodeParams::wave_parts): one per wave, or one
// per token slot of a wave (TPI per wave).
constexpr int kWavePart = 1;
constexpr int kSlotPart = 2;
constexpr int kMaxSlotRounds = 8;  // most partitions per token slot in the fused mode

// Token rows one decode load instruction covers (TPI: 64 lanes over rows of
// HP * D elements, 16 bytes per lane, FP8 8), as the kernels are built.
inline int decode_tpi(int D, int HP, int kv_bytes) {
  const int vec = kv_bytes == 1 ? 8 : 16 / kv_bytes;
  const int lpt = D * HP / vec;
  return lpt >= 64 ? 1 : 64 / lpt;
}

// Fused explicit split: one work-group per (sequence, head group) serves all
// `parts` partitions in rounds of kDecodeWaves * tpi (a partition per token
// slot), merges each one's partials into the output in registers (none are
// written), with no reduce launch.  The rounds it takes, or 0 when there are fewer
// partitions than slots, more rounds than kMaxSlotRounds, or the
// work-group's pages would not fit one staged block-table chunk.
inline int decode_fuse_rounds(int64_t parts, int MB, int BS, int tpi) {
  const int64_t gp1 = (int64_t)kDecodeWaves * tpi;
  if (parts < gp1 || MB <= 0 || BS <= 0) return 0;
  const int64_t R = (parts + gp1 - 1) / gp1;
  const int64_t chunk_max = ((int64_t)MB * BS + parts - 1) / parts;
  const int64_t pages = (R * gp1 * chunk_max + BS - 1) / BS + 1;
  return R <= kMaxSlotRounds && pages <= kBtChunk ? (int)R : 0;
}

// Records the kernel instance a launcher is about to dispatch, as profilers
// print its demangled name, for pa_last_launch() (host side, per thread).
void note_launch(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// Host launchers (defined in the kernel translation units).
hipError_t launch_decode(const DecodeParams& p, int kv_dtype, int gc, hipStream_t stream);
// Set by the decode launcher when a launch wrote the output itself although
// the plan splits (fuse_final took effect): no reduce launch is needed.
extern thread_local int t_decode_fused;
hipError_t launch_reduce(const ReduceParams& p, hipStream_t stream);
hipError_t launch_prefill_mfma(const PrefillParams& p, int kv_dtype, hipStream_t stream);
hipError_t launch_write_kv(const WriteParams& p, hipStream_t stream);

// Head packing (heads contiguous in the pool; MHA, or GQA groups of four over
// 16-bit caches): one decode work-group
// serves HP adjacent KV heads, whose rows of a token are contiguous, as one
// row of HP * D elements.  Wider contiguous reads keep more of each DRAM row
// access useful: at B = 256, ctx 2048, fp16 D = 64 one head per work-group
// streams 6.42 TB/s, two 6.66, four 6.80.  Rows shorter than a 128-byte line
// are always packed (two heads at least), since a half-line request costs
// a whole line.  The planner chooses HP per call (DecodeParams::hp); it sees
// only K (the workspace-size query has no V), and the kernel also needs V's
// heads contiguous, else it serves one head per work-group under the same
// plan.
constexpr int kPackRowBytes = 512;  // widest packed row
constexpr int kPackMax = 4;         // most KV heads per work-group
constexpr int kPackGqaMax = 2;      // most KV heads per work-group for GQA groups of four

// Widest packing the layout allows (1 = none).  GQA groups of four query
// heads over 8/16-bit caches pack too: each lane still serves one KV head's
// group, so the vector work per lane is unchanged and only the rows read
// together get wider (two KV heads: config 3 5819 -> 5968 GB/s, FP8 config 3
// 4550 -> 4753).
inline int decode_pack_max(int D, int kv_bytes, int G, int HKV, int64_t k_sh) {
  if (k_sh != D || !(G == 1 || (G == 4 && kv_bytes <= 2))) return 1;
  const int most = G == 1 ? kPackMax : kPackGqaMax;
  const int64_t row = kPackRowBytes;
  int hp = 1;
  for (int c = 2; c <= most; c *= 2)
    if ((int64_t)D * kv_bytes * c <= row && HKV % c == 0) hp = c;
  return hp;
}

// Narrowest packing worth running: two heads when a row is under a line.
inline int decode_pack_min(int D, int kv_bytes, int G, int HKV, int64_t k_sh) {
  return (D * kv_bytes < 128 && decode_pack_max(D, kv_bytes, G, HKV, k_sh) >= 2) ? 2 : 1;
}

// Heads per decode work-group for a GQA group of G query heads.
inline int decode_heads_per_wg(int G) {
  if (G <= 1) return 1;
  if (G <= 2) return 2;
  if (G <= 4) return 4;
  if (G <= 8) return 8;
  if (G % 8 == 0) return 8;
  if (G % 4 == 0) return 4;
  if (G % 2 == 0) return 2;
  return 1;
}

}  // namespace pa
