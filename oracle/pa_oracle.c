/*
 * pa_oracle.c -- CPU restatement of gb10-attn's paged-attention arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the GPU library is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product path never does.
 *
 * Every function cites the reference lines it follows (paths relative to the
 * gb10-attn repository root).  The arithmetic is plain fp32, in the
 * reference's loop order, with libm expf (the reference's std::exp(float)),
 * built with -ffp-contract=off and no vectorisation so that it matches the
 * reference's scalar code bit for bit where the two share a loop order.
 *
 * Conventions the reference leaves open (fixed here and in the library):
 *   - ctx <= 0 produces zero output rows;
 *   - ctx > MB*BS, or a block id outside [0, NB) on a live page, produces NaN
 *     output rows.
 * The split/merge functions keep the reference's literal behaviour instead
 * (an all-empty merge divides by zero, kernels/paged_attn_v3.cu:162).
 *
 * Pinning of each function is recorded in the header of tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { OR_F32 = 0, OR_F16 = 1, OR_BF16 = 2, OR_F64 = 3 };

#define OR_NEG_BIG (-3.0e38f) /* kernels/paged_attn_v3.cu:21 */

/* ---------------------------------------------------------------- codecs -- */

/* IEEE-754 binary16 -> binary32, exact (written from the bit layout). */
float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (h >> 15) & 1u;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  float v;
  if (e == 0) {
    v = ldexpf((float)man, -24); /* zero or subnormal: man * 2^-24 */
  } else if (e == 31) {
    v = man ? NAN : INFINITY;
  } else {
    v = ldexpf((float)(man | 0x400u), (int)e - 25); /* (1024+man) * 2^(e-15-10) */
  }
  return sign ? -v : v;
}

/* binary32 -> binary16, round to nearest even. */
uint16_t oracle_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u); /* NaN */
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
  const uint32_t e = ax >> 23;
  if (e < 113) {
    /* result is a binary16 subnormal: round(m * 2^(e-150) / 2^-24) */
    if (e < 101) return (uint16_t)sign; /* below 2^-26: rounds to zero */
    const uint64_t m = (uint64_t)((ax & 0x7fffffu) | 0x800000u);
    const int s = 126 - (int)e; /* 14..25 */
    uint64_t r = m >> s;
    const uint64_t rem = m & ((1ull << s) - 1);
    const uint64_t half = 1ull << (s - 1);
    if (rem > half || (rem == half && (r & 1))) r++;
    return (uint16_t)(sign | (uint32_t)r);
  }
  uint32_t h = ((e - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* carry may reach the exponent */
  return (uint16_t)(sign | h);
}

/* bfloat16 -> binary32, exact. */
float oracle_bf16_to_f32(uint16_t h) {
  const uint32_t x = (uint32_t)h << 16;
  float f;
  memcpy(&f, &x, 4);
  return f;
}

/* binary32 -> bfloat16, round to nearest even. */
uint16_t oracle_f32_to_bf16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(((x >> 16) & 0x8000u) | 0x7fc0u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

void oracle_f16_decode(float* dst, const uint16_t* src, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = oracle_f16_to_f32(src[i]);
}
void oracle_f16_encode(uint16_t* dst, const float* src, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = oracle_f32_to_f16(src[i]);
}
void oracle_bf16_decode(float* dst, const uint16_t* src, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = oracle_bf16_to_f32(src[i]);
}
void oracle_bf16_encode(uint16_t* dst, const float* src, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = oracle_f32_to_bf16(src[i]);
}

/* An element of a K/V cache as the reference's kernels read it:
 * static_cast<float>(k_ptr[i]) (kernels/paged_attn_v3.cu:94). */
static inline float ld(const void* p, int dt, int64_t i) {
  switch (dt) {
    case OR_F16: return oracle_f16_to_f32(((const uint16_t*)p)[i]);
    case OR_BF16: return oracle_bf16_to_f32(((const uint16_t*)p)[i]);
    case OR_F64: return (float)((const double*)p)[i];
    default: return ((const float*)p)[i];
  }
}

/* A paged K/V cache view: element (blk, off, kvh, d) is at
 * blk*sb + off*st + kvh*sh + d, all in 64 bits. */
typedef struct {
  const void* k;
  const void* v;
  int32_t dtype;
  int32_t pad_;
  int64_t num_blocks;
  int64_t sb, st, sh; /* element strides: block, token, head */
} oracle_kv_t;

/* ------------------------------------------------------- partitioning -- */

/* Partition s of S over a context of ctx tokens: [s*chunk, min(s*chunk+chunk, ctx))
 * with chunk = ceil(ctx / S), in C int arithmetic (kernels/paged_attn_v3.cu:65-68). */
void oracle_partition_bounds(int ctx, int S, int s, int* start, int* end) {
  const int chunk = (ctx + S - 1) / S;
  const int st = s * chunk;
  const int en = (st + chunk < ctx) ? st + chunk : ctx;
  *start = st;
  *end = en;
}

/* kernels/paged_attn_v3.cu:170-190 with the SM count as an argument. */
int64_t oracle_choose_num_splits(int64_t num_seqs, int64_t num_heads, int64_t max_context,
                                 int64_t sms) {
  int64_t have = num_seqs * num_heads;
  if (have < 1) have = 1;
  int64_t by_chain = max_context / 32;
  if (by_chain < 1) by_chain = 1;
  int64_t fill = (sms * 8 + have - 1) / have;
  if (fill < 1) fill = 1;
  int64_t s = by_chain > fill ? by_chain : fill;
  if (s > 64) s = 64;
  if (s < 1) s = 1;
  return s;
}

/* Bytes a decode call must move at minimum: K and V of every live token of
 * every KV head, read once (docs/REPORT.md:35-37, with HKV in place of H so
 * that GQA counts each KV head once). */
double oracle_decode_min_bytes(const int32_t* ctx, int B, int HKV, int D, int kv_itemsize) {
  double tok = 0.0;
  for (int b = 0; b < B; ++b) tok += ctx[b] > 0 ? (double)ctx[b] : 0.0;
  return 2.0 * tok * HKV * D * kv_itemsize;
}

/* ---------------------------------------------------------------- gather -- */

/* Physical location of token j of sequence b (kernels/paged_attn_v3.cu:87-89):
 * copies the K and V rows of KV head kvh for j in [0, n) into dk/dv [n][D].
 * Returns 0, or -1 if a block id is outside [0, NB). */
int oracle_gather(float* dk, float* dv, const oracle_kv_t* kv, const int32_t* bt_row,
                  int n, int kvh, int D, int BS) {
  for (int j = 0; j < n; ++j) {
    const int blk = bt_row[j / BS];
    const int off = j % BS;
    if (blk < 0 || blk >= kv->num_blocks) return -1;
    const int64_t base = (int64_t)blk * kv->sb + (int64_t)off * kv->st + (int64_t)kvh * kv->sh;
    for (int d = 0; d < D; ++d) {
      dk[(int64_t)j * D + d] = ld(kv->k, kv->dtype, base + d);
      dv[(int64_t)j * D + d] = ld(kv->v, kv->dtype, base + d);
    }
  }
  return 0;
}

static int live_pages_ok(const oracle_kv_t* kv, const int32_t* bt_row, int n, int BS) {
  for (int p = 0; p < (n + BS - 1) / BS; ++p)
    if (bt_row[p] < 0 || bt_row[p] >= kv->num_blocks) return 0;
  return 1;
}

static void fill(float* o, int D, float x) {
  for (int d = 0; d < D; ++d) o[d] = x;
}

/* ---------------------------------------------------------------- decode -- */

/* Scalar fp32 paged decode, loop for loop rocm/hip/paged_attn_v1_hip.cpp:104-141
 * (cpu_reference): scores, max, expf, denominator, out[d] = sum_j s_j v_j[d] / denom.
 * q [B,H,D] fp32; out [B,H,D] fp32; bt row stride bt_stride. */
void oracle_decode(float* out, const float* q, const oracle_kv_t* kv, const int32_t* bt,
                   int64_t bt_stride, const int32_t* ctx, int B, int H, int HKV, int D, int BS,
                   int MB, float scale) {
  const int64_t maxctx = (int64_t)MB * BS;
  float* score = (float*)malloc(sizeof(float) * (size_t)(maxctx > 0 ? maxctx : 1));
  for (int b = 0; b < B; ++b) {
    const int32_t* row = bt + (int64_t)b * bt_stride;
    for (int h = 0; h < H; ++h) {
      const int kv_h = h / (H / HKV);
      const int n = ctx[b];
      float* o = out + ((int64_t)b * H + h) * D;
      if (n <= 0) { fill(o, D, 0.0f); continue; }
      if (n > maxctx || !live_pages_ok(kv, row, n, BS)) { fill(o, D, NAN); continue; }
      const float* qv = q + ((int64_t)b * H + h) * D;
      float mx = OR_NEG_BIG;
      for (int j = 0; j < n; ++j) {
        const int blk = row[j / BS], off = j % BS;
        const int64_t base = (int64_t)blk * kv->sb + (int64_t)off * kv->st + (int64_t)kv_h * kv->sh;
        float dot = 0.0f;
        for (int d = 0; d < D; ++d) dot += qv[d] * ld(kv->k, kv->dtype, base + d);
        score[j] = dot * scale;
        mx = mx < score[j] ? score[j] : mx;
      }
      float denom = 0.0f;
      for (int j = 0; j < n; ++j) {
        score[j] = expf(score[j] - mx);
        denom += score[j];
      }
      for (int d = 0; d < D; ++d) {
        float acc = 0.0f;
        for (int j = 0; j < n; ++j) {
          const int blk = row[j / BS], off = j % BS;
          const int64_t base = (int64_t)blk * kv->sb + (int64_t)off * kv->st + (int64_t)kv_h * kv->sh;
          acc += score[j] * ld(kv->v, kv->dtype, base + d);
        }
        o[d] = acc / denom;
      }
    }
  }
  free(score);
}

/* One online-softmax stream over tokens [start, end) of one (b, h), the
 * per-warp loop of kernels/paged_attn_v2.cu:89-116 / kernels/paged_attn_v3.cu:86-110
 * with the dot product summed in dimension order. */
static void online_stream(float* acc, float* m_out, float* l_out, const float* qv,
                          const oracle_kv_t* kv, const int32_t* row, int start, int end,
                          int kv_h, int D, int BS, float scale) {
  float m = OR_NEG_BIG, l = 0.0f;
  for (int d = 0; d < D; ++d) acc[d] = 0.0f;
  for (int j = start; j < end; ++j) {
    const int blk = row[j / BS], off = j % BS;
    const int64_t base = (int64_t)blk * kv->sb + (int64_t)off * kv->st + (int64_t)kv_h * kv->sh;
    float dot = 0.0f;
    for (int d = 0; d < D; ++d) dot += qv[d] * ld(kv->k, kv->dtype, base + d);
    const float s = dot * scale;
    const float m_new = fmaxf(m, s);
    const float corr = expf(m - m_new);
    const float p = expf(s - m_new);
    l = l * corr + p;
    for (int d = 0; d < D; ++d) acc[d] = acc[d] * corr + p * ld(kv->v, kv->dtype, base + d);
    m = m_new;
  }
  *m_out = m;
  *l_out = l;
}

/* Online-softmax decode, kernels/paged_attn_v2.cu:40-122: out = acc * (1/l). */
void oracle_decode_online(float* out, const float* q, const oracle_kv_t* kv, const int32_t* bt,
                          int64_t bt_stride, const int32_t* ctx, int B, int H, int HKV, int D,
                          int BS, int MB, float scale) {
  const int64_t maxctx = (int64_t)MB * BS;
  float* acc = (float*)malloc(sizeof(float) * (size_t)D);
  for (int b = 0; b < B; ++b) {
    const int32_t* row = bt + (int64_t)b * bt_stride;
    for (int h = 0; h < H; ++h) {
      float* o = out + ((int64_t)b * H + h) * D;
      const int n = ctx[b];
      if (n <= 0) { fill(o, D, 0.0f); continue; }
      if (n > maxctx || !live_pages_ok(kv, row, n, BS)) { fill(o, D, NAN); continue; }
      float m, l;
      online_stream(acc, &m, &l, q + ((int64_t)b * H + h) * D, kv, row, 0, n, h / (H / HKV), D,
                    BS, scale);
      const float inv = 1.0f / l;
      for (int d = 0; d < D; ++d) o[d] = acc[d] * inv;
    }
  }
  free(acc);
}

/* Split pass, kernels/paged_attn_v3.cu:33-123: un-normalised partials
 * pacc [B,H,S,D], natural-log running max pm [B,H,S] and sum pl [B,H,S]. */
void oracle_decode_partials(float* pacc, float* pm, float* pl, const float* q,
                            const oracle_kv_t* kv, const int32_t* bt, int64_t bt_stride,
                            const int32_t* ctx, int B, int H, int HKV, int D, int BS, int S,
                            float scale) {
  for (int b = 0; b < B; ++b) {
    const int32_t* row = bt + (int64_t)b * bt_stride;
    for (int h = 0; h < H; ++h) {
      for (int s = 0; s < S; ++s) {
        int start, end;
        oracle_partition_bounds(ctx[b], S, s, &start, &end);
        const int64_t pidx = ((int64_t)b * H + h) * S + s;
        online_stream(pacc + pidx * D, pm + pidx, pl + pidx, q + ((int64_t)b * H + h) * D, kv,
                      row, start, end, h / (H / HKV), D, BS, scale);
      }
    }
  }
}

/* Merge pass, kernels/paged_attn_v3.cu:128-166 (log-sum-exp combine). */
void oracle_merge(float* out, const float* pacc, const float* pm, const float* pl, int B, int H,
                  int S, int D) {
  float* acc = (float*)malloc(sizeof(float) * (size_t)D);
  for (int64_t f = 0; f < (int64_t)B * H; ++f) {
    const int64_t base = f * S;
    float m_g = OR_NEG_BIG;
    for (int s = 0; s < S; ++s) m_g = fmaxf(m_g, pm[base + s]);
    float l_g = 0.0f;
    for (int d = 0; d < D; ++d) acc[d] = 0.0f;
    for (int s = 0; s < S; ++s) {
      const float w = expf(pm[base + s] - m_g);
      l_g += pl[base + s] * w;
      for (int d = 0; d < D; ++d) acc[d] += pacc[(base + s) * D + d] * w;
    }
    const float inv = 1.0f / l_g;
    for (int d = 0; d < D; ++d) out[f * D + d] = acc[d] * inv;
  }
  free(acc);
}

/* --------------------------------------------------------------- prefill -- */

/* Causal chunked prefill, kernels/paged_attn_prefill.cu:33-118: query s of
 * sequence b sits at q_pos = ctx_b - S + s and attends keys [0, q_pos];
 * q_pos < 0 gives zeros (:62-74).  q/out [B,S,H,D] fp32. */
void oracle_prefill(float* out, const float* q, const oracle_kv_t* kv, const int32_t* bt,
                    int64_t bt_stride, const int32_t* ctx, int B, int S, int H, int HKV, int D,
                    int BS, int MB, float scale) {
  const int64_t maxctx = (int64_t)MB * BS;
  float* acc = (float*)malloc(sizeof(float) * (size_t)D);
  for (int b = 0; b < B; ++b) {
    const int32_t* row = bt + (int64_t)b * bt_stride;
    for (int s = 0; s < S; ++s) {
      for (int h = 0; h < H; ++h) {
        const int64_t idx = (((int64_t)b * S + s) * H + h) * D;
        const int q_pos = ctx[b] - S + s;
        const int end = q_pos + 1;
        if (end <= 0) { fill(out + idx, D, 0.0f); continue; }
        /* NaN when the context exceeds the table or a page this row reads is invalid */
        if (ctx[b] > maxctx || !live_pages_ok(kv, row, end, BS)) { fill(out + idx, D, NAN); continue; }
        float m, l;
        online_stream(acc, &m, &l, q + idx, kv, row, 0, end, h / (H / HKV), D, BS, scale);
        const float inv = 1.0f / l;
        for (int d = 0; d < D; ++d) out[idx + d] = acc[d] * inv;
      }
    }
  }
  free(acc);
}

/* Non-paged scalar primitives of arm_cpu/src/scalar.cpp:9-46 (dot in index
 * order; softmax as max, expf, sum, multiply by 1/sum). */
float oracle_dot(const float* a, const float* b, int64_t n) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; ++i) s += a[i] * b[i];
  return s;
}

void oracle_softmax_inplace(float* x, int64_t n) {
  if (n == 0) return;
  float mx = -INFINITY;
  for (int64_t i = 0; i < n; ++i) mx = mx < x[i] ? x[i] : mx;
  float sum = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    x[i] = expf(x[i] - mx);
    sum += x[i];
  }
  const float inv = 1.0f / sum;
  for (int64_t i = 0; i < n; ++i) x[i] *= inv;
}
