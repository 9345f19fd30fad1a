// ref_shim.cpp -- exposes the reference's own scalar CPU code as a C ABI.
//
// TEST INFRASTRUCTURE ONLY (builds oracle/_ref/libgb10_ref.so).  Nothing of
// the reference is copied here: the reference source files are compiled where
// they lie under the reference checkout (REF_ROOT, passed by oracle/Makefile),
// and this unit only adds extern "C" entry points around functions that are
// otherwise file-static or namespaced.
//
//   ref_cpu_reference   -> cpu_reference, rocm/hip/paged_attn_v1_hip.cpp:104-141
//   ref_selftest_inputs -> the self-test inputs of rocm/hip/paged_attn_v1_hip.cpp:151-162
//                          (same std::mt19937 seed, distribution and draw order)
//   ref_dot_scalar / ref_softmax_inplace / ref_attention_scores
//                       -> arm_cpu/src/scalar.cpp:9-46
//   ref_scalar_smoke_inputs -> inputs of arm_cpu/src/bench.cpp:60-63 (mt19937(2026))
#include <cstdint>
#include <random>
#include <vector>

// The HIP self-test defines main(); rename it so this library exports no main.
#define main gb10_ref_hip_selftest_main
#include REF_HIP_SOURCE
#undef main

#include "gb10_arm/attention.hpp"

extern "C" {

void ref_cpu_reference(float* out, const float* k, const float* v, const float* q,
                       const int* bt, const int* ctx, int B, int H, int HKV, int D, int BS,
                       int MB, int NB, float scale) {
  const size_t kv_elems = (size_t)NB * BS * HKV * D;
  std::vector<float> vk(k, k + kv_elems), vv(v, v + kv_elems), vq(q, q + (size_t)B * H * D);
  std::vector<int> vbt(bt, bt + (size_t)B * MB), vctx(ctx, ctx + B);
  std::vector<float> vout((size_t)B * H * D);
  cpu_reference(vout, vk, vv, vq, vbt, vctx, B, H, HKV, D, BS, MB, scale);
  for (size_t i = 0; i < vout.size(); ++i) out[i] = vout[i];
}

// A prepared call of cpu_reference, so a timing loop measures the reference
// function alone and not the copies into its std::vector arguments.
struct RefCall {
  std::vector<float> k, v, q, out;
  std::vector<int> bt, ctx;
  int B, H, HKV, D, BS, MB;
  float scale;
};

void* ref_call_create(const float* k, const float* v, const float* q, const int* bt,
                      const int* ctx, int B, int H, int HKV, int D, int BS, int MB, int NB,
                      float scale) {
  const size_t kv_elems = (size_t)NB * BS * HKV * D;
  RefCall* c = new RefCall{std::vector<float>(k, k + kv_elems), std::vector<float>(v, v + kv_elems),
                           std::vector<float>(q, q + (size_t)B * H * D),
                           std::vector<float>((size_t)B * H * D),
                           std::vector<int>(bt, bt + (size_t)B * MB), std::vector<int>(ctx, ctx + B),
                           B, H, HKV, D, BS, MB, scale};
  return c;
}

void ref_call_run(void* h, float* out) {
  RefCall* c = static_cast<RefCall*>(h);
  cpu_reference(c->out, c->k, c->v, c->q, c->bt, c->ctx, c->B, c->H, c->HKV, c->D, c->BS, c->MB,
                c->scale);
  if (out) std::copy(c->out.begin(), c->out.end(), out);
}

void ref_call_free(void* h) { delete static_cast<RefCall*>(h); }

// Inputs of the reference HIP self-test (B=2, H=4, HKV=2, D=32, BS=16, MB=4,
// NB=8, ctx=48): q [B*H*D], k/v [NB*BS*HKV*D], bt [B*MB], ctx [B].
void ref_selftest_inputs(float* q, float* k, float* v, int* bt, int* ctx) {
  const int B = 2, H = 4, HKV = 2, D = 32, BS = 16, MB = 4, NB = 8, NCTX = 48;
  std::mt19937 rng(7);
  std::uniform_real_distribution<float> dist(-0.25f, 0.25f);
  for (int i = 0; i < B * H * D; ++i) q[i] = dist(rng);
  for (int i = 0; i < NB * BS * HKV * D; ++i) k[i] = dist(rng);
  for (int i = 0; i < NB * BS * HKV * D; ++i) v[i] = dist(rng);
  for (int b = 0; b < B; ++b)
    for (int m = 0; m < MB; ++m) bt[b * MB + m] = (b * MB + m) % NB;
  for (int b = 0; b < B; ++b) ctx[b] = NCTX;
}

float ref_dot_scalar(const float* a, const float* b, int64_t n) {
  return gb10::arm::dot_scalar(a, b, (size_t)n);
}

void ref_softmax_inplace(float* x, int64_t n) { gb10::arm::softmax_inplace(x, (size_t)n); }

void ref_attention_scores(const float* query, const float* keys, float* scores, int64_t tokens,
                          int64_t dim) {
  gb10::arm::attention_scores(query, keys, scores, (size_t)tokens, (size_t)dim,
                              gb10::arm::dot_scalar);
}

// Inputs of the arm scalar_smoke bench: query [dim], keys [tokens*dim].
void ref_scalar_smoke_inputs(float* query, float* keys, int64_t tokens, int64_t dim) {
  std::mt19937 rng(2026);
  std::uniform_real_distribution<float> dist(-0.25f, 0.25f);
  for (int64_t i = 0; i < dim; ++i) query[i] = dist(rng);
  for (int64_t i = 0; i < tokens * dim; ++i) keys[i] = dist(rng);
}

}  // extern "C"
