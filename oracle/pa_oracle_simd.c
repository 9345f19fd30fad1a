/* pa_oracle_simd.c -- vectorised, multi-threaded CPU port of the reference's
 * paged decode (rocm/hip/paged_attn_v1_hip.cpp:104-141), used only as the
 * "SIMD variant on all host cores" CPU baseline that bench.py times beside
 * the GPU, and checked against the scalar oracle in tests/.  TEST AND
 * BASELINE INFRASTRUCTURE ONLY: the product path never loads it.
 *
 * Same algorithm and index formula as cpu_reference (scores, max, exp,
 * denominator, weighted V sum; kernels/paged_attn_v3.cu:87-89 addressing),
 * parallel over (sequence, head) with OpenMP and vectorised over the head
 * dimension with AVX2/FMA; fp16 K/V are widened with F16C, bf16 by a shift.
 * Summation order differs from the scalar loop, so results agree within
 * fp32 rounding, not bit for bit.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include <omp.h>

/* Eight consecutive elements as fp32: dtype 0 = f32, 1 = f16, 2 = bf16. */
static inline __m256 load8(const void* base, int dtype, int64_t idx) {
  if (dtype == 1) {
    return _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)((const uint16_t*)base + idx)));
  } else if (dtype == 2) {
    const __m128i h = _mm_loadu_si128((const __m128i*)((const uint16_t*)base + idx));
    return _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16));
  }
  return _mm256_loadu_ps((const float*)base + idx);
}

static inline float hsum8(__m256 v) {
  __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
  lo = _mm_add_ps(lo, hi);
  lo = _mm_hadd_ps(lo, lo);
  lo = _mm_hadd_ps(lo, lo);
  return _mm_cvtss_f32(lo);
}

/* out[B,H,D] f32; q[B,H,D] f32; k/v pools of `dtype` with element strides
 * (block sb, token st, head sh); D a multiple of 8.  Rows with ctx <= 0 are
 * zeros.  Returns 0, or -1 for an unsupported D. */
int oracle_decode_simd(float* out, const float* q, const void* k, const void* v, int dtype, int64_t sb,
                       int64_t st, int64_t sh, const int32_t* bt, int64_t bt_stride, const int32_t* ctx,
                       int B, int H, int HKV, int D, int BS, int MB, float scale, int threads) {
  if (D % 8 != 0 || D > 512) return -1;
  const int64_t maxctx = (int64_t)MB * BS;
#pragma omp parallel num_threads(threads)
  {
    float* score = (float*)malloc(sizeof(float) * (size_t)(maxctx > 0 ? maxctx : 1));
#pragma omp for schedule(dynamic, 1)
    for (int64_t bh = 0; bh < (int64_t)B * H; ++bh) {
      const int b = (int)(bh / H), h = (int)(bh % H);
      const int kvh = h / (H / HKV);
      const int n = ctx[b] < maxctx ? ctx[b] : (int)maxctx;
      float* o = out + bh * D;
      if (n <= 0) {
        for (int d = 0; d < D; ++d) o[d] = 0.0f;
        continue;
      }
      const int32_t* row = bt + (int64_t)b * bt_stride;
      const float* qv = q + bh * D;
      float mx = -INFINITY;
      for (int j = 0; j < n; ++j) {
        const int64_t base = (int64_t)row[j / BS] * sb + (int64_t)(j % BS) * st + (int64_t)kvh * sh;
        __m256 acc = _mm256_setzero_ps();
        for (int d = 0; d < D; d += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(qv + d), load8(k, dtype, base + d), acc);
        score[j] = hsum8(acc) * scale;
        mx = score[j] > mx ? score[j] : mx;
      }
      float denom = 0.0f;
      for (int j = 0; j < n; ++j) {
        score[j] = expf(score[j] - mx);
        denom += score[j];
      }
      __m256 accv[64];
      for (int c = 0; c < D / 8; ++c) accv[c] = _mm256_setzero_ps();
      for (int j = 0; j < n; ++j) {
        const int64_t base = (int64_t)row[j / BS] * sb + (int64_t)(j % BS) * st + (int64_t)kvh * sh;
        const __m256 p = _mm256_set1_ps(score[j]);
        for (int c = 0; c < D / 8; ++c) accv[c] = _mm256_fmadd_ps(p, load8(v, dtype, base + 8 * c), accv[c]);
      }
      const __m256 inv = _mm256_set1_ps(1.0f / denom);
      for (int c = 0; c < D / 8; ++c) _mm256_storeu_ps(o + 8 * c, _mm256_mul_ps(accv[c], inv));
    }
    free(score);
  }
  return 0;
}
