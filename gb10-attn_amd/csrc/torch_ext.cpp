// torch_ext.cpp -- the reference's torch::Tensor launchers as PyTorch
// operators (torch.ops.gb10_attn.*), served by libpagedattn.so through the
// C-ABI of include/pagedattn.h.
//
// Same names, argument order, argument meaning, output (a new fp32 tensor)
// and error behaviour (TORCH_CHECK -> RuntimeError) as kernels/*.h:
//   paged_attention        kernels/paged_attn_v1.h:13-15
//   paged_attention_v2     kernels/paged_attn_v2.h:13-15
//   paged_attention_v3     kernels/paged_attn_v3.h:13-16
//   choose_num_splits      kernels/paged_attn_v3.h:17
//   paged_attention_prefill       kernels/paged_attn_prefill.h:13-15
//   paged_attention_prefill_wmma  kernels/paged_attn_wmma.h:13-15
// plus paged_attention_prefill_varlen (mixed decode + prefill batches) and
// write_kv / write_kv_scaled (the engine's KV-cache write, pa_write_kv and
// pa_write_kv_scaled).  As in the
// reference, inputs are made contiguous (K/V only when the kernels cannot
// address the given strides), block tables and context lengths are cast to
// int32, and the v3 scratch comes from the caching allocator per call.  Work
// goes to torch's current stream of q's device.  Host code only.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "../../include/pagedattn.h"

namespace {

int pa_dtype(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return PA_DTYPE_F32;
    case at::kHalf: return PA_DTYPE_F16;
    case at::kBFloat16: return PA_DTYPE_BF16;
    case at::kDouble: return PA_DTYPE_F64;
    case at::kInt: return PA_DTYPE_I32;
    case at::kLong: return PA_DTYPE_I64;
    case at::kFloat8_e4m3fn: return PA_DTYPE_FP8_E4M3;
    default: TORCH_CHECK(false, "unsupported dtype ", t);
  }
  return -1;
}

pa_tensor_t view(const at::Tensor& t) {
  TORCH_CHECK(t.dim() <= PA_MAX_DIMS, "tensors of at most ", PA_MAX_DIMS, " dims");
  pa_tensor_t v;
  std::memset(&v, 0, sizeof(v));
  v.data = t.data_ptr();
  v.dtype = pa_dtype(t.scalar_type());
  v.ndim = (int32_t)t.dim();
  for (int64_t i = 0; i < t.dim(); ++i) {
    v.shape[i] = t.size(i);
    v.stride[i] = t.stride(i);
  }
  return v;
}

void check(int rc) { TORCH_CHECK(rc == PA_OK, pa_last_error()); }

void* stream_of(const at::Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

// K/V views the kernels address in place: last dim contiguous, 16-byte
// aligned base and strides (one layer of a larger pool qualifies).
bool kv_addressable(const at::Tensor& t) {
  if (t.dim() != 4 || t.stride(3) != 1 || reinterpret_cast<uintptr_t>(t.data_ptr()) % 16) return false;
  for (int i = 0; i < 3; ++i)
    if ((t.stride(i) * t.element_size()) % 16 != 0 && t.size(i) != 1) return false;
  return true;
}

struct Args {
  at::Tensor q, k, v, bt, ctx;
};

Args prep(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& bt,
          const at::Tensor& ctx, int64_t qdim, const char* qlayout) {
  TORCH_CHECK(q.is_cuda(), "q must be on CUDA");
  TORCH_CHECK(k.is_cuda() && v.is_cuda(), "kv cache must be on CUDA");
  TORCH_CHECK(q.dim() == qdim, "q must be ", qlayout);
  TORCH_CHECK(k.dim() == 4, "k_cache must be [NB, BS, H, D]");
  Args a;
  a.q = q.contiguous();
  a.k = kv_addressable(k) ? k : k.contiguous();
  a.v = kv_addressable(v) ? v : v.contiguous();
  a.bt = bt.to(q.device(), at::kInt).contiguous();
  a.ctx = ctx.to(q.device(), at::kInt).contiguous();
  return a;
}

using SimpleFn = int (*)(pa_tensor_t*, const pa_tensor_t*, const pa_tensor_t*, const pa_tensor_t*,
                         const pa_tensor_t*, const pa_tensor_t*, double, void*);

at::Tensor call_simple(SimpleFn fn, const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                       const at::Tensor& bt, const at::Tensor& ctx, double scale, int64_t qdim,
                       const char* qlayout) {
  Args a = prep(q, k, v, bt, ctx, qdim, qlayout);
  c10::DeviceGuard guard(a.q.device());
  at::Tensor out = at::empty(a.q.sizes(), a.q.options().dtype(at::kFloat));
  pa_tensor_t o = view(out), qq = view(a.q), kk = view(a.k), vv = view(a.v), bb = view(a.bt), cc = view(a.ctx);
  check(fn(&o, &qq, &kk, &vv, &bb, &cc, scale, stream_of(a.q)));
  return out;
}

at::Tensor op_paged_attention(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                              const at::Tensor& bt, const at::Tensor& ctx, double scale) {
  return call_simple(&paged_attention, q, k, v, bt, ctx, scale, 3, "[B, H, D]");
}

at::Tensor op_paged_attention_v2(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                 const at::Tensor& bt, const at::Tensor& ctx, double scale) {
  return call_simple(&paged_attention_v2, q, k, v, bt, ctx, scale, 3, "[B, H, D]");
}

at::Tensor op_paged_attention_prefill(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                      const at::Tensor& bt, const at::Tensor& ctx, double scale) {
  return call_simple(&paged_attention_prefill, q, k, v, bt, ctx, scale, 4, "[B, S, H, D]");
}

at::Tensor op_paged_attention_prefill_wmma(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                           const at::Tensor& bt, const at::Tensor& ctx, double scale) {
  return call_simple(&paged_attention_prefill_wmma, q, k, v, bt, ctx, scale, 4, "[B, S, H, D]");
}

at::Tensor op_paged_attention_prefill_wmma_scaled(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                                  const at::Tensor& bt, const at::Tensor& ctx, double scale,
                                                  double k_scale, double v_scale) {
  Args a = prep(q, k, v, bt, ctx, 4, "[B, S, H, D]");
  c10::DeviceGuard guard(a.q.device());
  at::Tensor out = at::empty(a.q.sizes(), a.q.options().dtype(at::kFloat));
  pa_tensor_t o = view(out), qq = view(a.q), kk = view(a.k), vv = view(a.v), bb = view(a.bt), cc = view(a.ctx);
  check(paged_attention_prefill_wmma_scaled(&o, &qq, &kk, &vv, &bb, &cc, scale, k_scale, v_scale,
                                            stream_of(a.q)));
  return out;
}

at::Tensor op_paged_attention_v3(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                 const at::Tensor& bt, const at::Tensor& ctx, double scale, int64_t num_splits) {
  Args a = prep(q, k, v, bt, ctx, 3, "[B, H, D]");
  c10::DeviceGuard guard(a.q.device());
  at::Tensor out = at::empty(a.q.sizes(), a.q.options().dtype(at::kFloat));
  pa_tensor_t o = view(out), qq = view(a.q), kk = view(a.k), vv = view(a.v), bb = view(a.bt), cc = view(a.ctx);
  const size_t ws = paged_attention_v3_workspace_size(&qq, &kk, &bb, num_splits);
  TORCH_CHECK(ws != (size_t)-1, pa_last_error());
  at::Tensor scratch;
  void* wp = nullptr;
  if (ws > 0) {
    scratch = at::empty({(int64_t)ws + 256}, a.q.options().dtype(at::kByte));
    wp = reinterpret_cast<void*>((reinterpret_cast<uintptr_t>(scratch.data_ptr()) + 255) & ~uintptr_t(255));
  }
  check(paged_attention_v3(&o, &qq, &kk, &vv, &bb, &cc, scale, num_splits, wp, ws, stream_of(a.q)));
  return out;
}

at::Tensor op_paged_attention_v3_scaled(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                        const at::Tensor& bt, const at::Tensor& ctx, double scale,
                                        int64_t num_splits, double k_scale, double v_scale) {
  Args a = prep(q, k, v, bt, ctx, 3, "[B, H, D]");
  c10::DeviceGuard guard(a.q.device());
  at::Tensor out = at::empty(a.q.sizes(), a.q.options().dtype(at::kFloat));
  pa_tensor_t o = view(out), qq = view(a.q), kk = view(a.k), vv = view(a.v), bb = view(a.bt), cc = view(a.ctx);
  const size_t ws = paged_attention_v3_workspace_size(&qq, &kk, &bb, num_splits);
  TORCH_CHECK(ws != (size_t)-1, pa_last_error());
  at::Tensor scratch;
  void* wp = nullptr;
  if (ws > 0) {
    scratch = at::empty({(int64_t)ws + 256}, a.q.options().dtype(at::kByte));
    wp = reinterpret_cast<void*>((reinterpret_cast<uintptr_t>(scratch.data_ptr()) + 255) & ~uintptr_t(255));
  }
  check(paged_attention_v3_scaled(&o, &qq, &kk, &vv, &bb, &cc, scale, k_scale, v_scale, num_splits, wp, ws,
                                  stream_of(a.q)));
  return out;
}

at::Tensor op_paged_attention_prefill_varlen_scaled(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                                    const at::Tensor& bt, const at::Tensor& ctx, const at::Tensor& cu,
                                                    int64_t max_q_len, double scale, double k_scale,
                                                    double v_scale) {
  Args a = prep(q, k, v, bt, ctx, 3, "[T, H, D]");
  at::Tensor cuq = cu.to(a.q.device(), at::kInt).contiguous();
  c10::DeviceGuard guard(a.q.device());
  at::Tensor out = at::empty(a.q.sizes(), a.q.options().dtype(at::kFloat));
  pa_tensor_t o = view(out), qq = view(a.q), kk = view(a.k), vv = view(a.v), bb = view(a.bt), cc = view(a.ctx),
              uu = view(cuq);
  check(paged_attention_prefill_varlen_scaled(&o, &qq, &kk, &vv, &bb, &cc, &uu, max_q_len, scale, k_scale, v_scale,
                                              stream_of(a.q)));
  return out;
}

at::Tensor op_paged_attention_prefill_varlen(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                             const at::Tensor& bt, const at::Tensor& ctx, const at::Tensor& cu,
                                             int64_t max_q_len, double scale) {
  return op_paged_attention_prefill_varlen_scaled(q, k, v, bt, ctx, cu, max_q_len, scale, 1.0, 1.0);
}

int64_t op_choose_num_splits(int64_t num_seqs, int64_t num_heads, int64_t max_context) {
  const int64_t s = choose_num_splits(num_seqs, num_heads, max_context);
  TORCH_CHECK(s > 0, pa_last_error());
  return s;
}

void op_write_kv_scaled(at::Tensor& k_cache, at::Tensor& v_cache, const at::Tensor& key, const at::Tensor& value,
                        const at::Tensor& slot_mapping, double k_scale, double v_scale) {
  TORCH_CHECK(k_cache.is_cuda() && v_cache.is_cuda() && key.is_cuda() && value.is_cuda(),
              "k_cache, v_cache, key and value must be on CUDA");
  TORCH_CHECK(kv_addressable(k_cache) && kv_addressable(v_cache),
              "k_cache/v_cache must be 16-byte aligned [NB, BS, HKV, D] views with a contiguous last dim");
  at::Tensor kk = key.stride(-1) == 1 && reinterpret_cast<uintptr_t>(key.data_ptr()) % 16 == 0 ? key : key.contiguous();
  at::Tensor vv = value.stride(-1) == 1 && reinterpret_cast<uintptr_t>(value.data_ptr()) % 16 == 0 ? value : value.contiguous();
  at::Tensor sm = slot_mapping.to(key.device()).contiguous();
  if (sm.scalar_type() != at::kInt && sm.scalar_type() != at::kLong) sm = sm.to(at::kLong);
  c10::DeviceGuard guard(key.device());
  pa_tensor_t kc = view(k_cache), vc = view(v_cache), ks = view(kk), vs = view(vv), ss = view(sm);
  check(pa_write_kv_scaled(&kc, &vc, &ks, &vs, &ss, k_scale, v_scale, stream_of(kk)));
}

void op_write_kv(at::Tensor& k_cache, at::Tensor& v_cache, const at::Tensor& key, const at::Tensor& value,
                 const at::Tensor& slot_mapping) {
  op_write_kv_scaled(k_cache, v_cache, key, value, slot_mapping, 1.0, 1.0);
}

}  // namespace

TORCH_LIBRARY(gb10_attn, m) {
  m.def("paged_attention(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, "
        "Tensor context_lens, float scale) -> Tensor", &op_paged_attention);
  m.def("paged_attention_v2(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, "
        "Tensor context_lens, float scale) -> Tensor", &op_paged_attention_v2);
  m.def("paged_attention_v3(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, "
        "Tensor context_lens, float scale, int num_splits) -> Tensor", &op_paged_attention_v3);
  m.def("paged_attention_v3_scaled(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, "
        "Tensor context_lens, float scale, int num_splits, float k_scale, float v_scale) -> Tensor",
        &op_paged_attention_v3_scaled);
  m.def("choose_num_splits(int num_seqs, int num_heads, int max_context) -> int", &op_choose_num_splits);
  m.def("paged_attention_prefill(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, "
        "Tensor context_lens, float scale) -> Tensor", &op_paged_attention_prefill);
  m.def("paged_attention_prefill_wmma(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, "
        "Tensor context_lens, float scale) -> Tensor", &op_paged_attention_prefill_wmma);
  m.def("paged_attention_prefill_wmma_scaled(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, "
        "Tensor context_lens, float scale, float k_scale, float v_scale) -> Tensor",
        &op_paged_attention_prefill_wmma_scaled);
  m.def("paged_attention_prefill_varlen(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, "
        "Tensor context_lens, Tensor cu_seqlens_q, int max_q_len, float scale) -> Tensor",
        &op_paged_attention_prefill_varlen);
  m.def("paged_attention_prefill_varlen_scaled(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, "
        "Tensor context_lens, Tensor cu_seqlens_q, int max_q_len, float scale, float k_scale, float v_scale) -> Tensor",
        &op_paged_attention_prefill_varlen_scaled);
  m.def("write_kv(Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor key, Tensor value, Tensor slot_mapping) -> ()",
        &op_write_kv);
  m.def("write_kv_scaled(Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor key, Tensor value, Tensor slot_mapping, "
        "float k_scale, float v_scale) -> ()",
        &op_write_kv_scaled);
}
