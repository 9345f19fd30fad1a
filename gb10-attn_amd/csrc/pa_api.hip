// pa_api.hip -- the extern "C" entry points of include/pagedattn.h.
//
// Host-side work only: argument checks (every check runs before any HIP
// call, so a rejected call has no device side effect), the partition plan,
// parameter packing, and kernel launches on the caller's stream.  Nothing
// here allocates device memory; scratch comes from the caller's workspace.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/pagedattn.h"
#include "pa_common.hpp"

// Split scratch of paged_attention_v3_noalloc: a fixed device array, one copy
// per GPU, held until the process ends.  Host code never passes `scratch`
// itself to a kernel (on the host it names a stand-in, not device memory):
// its device address is read per device with hipGetSymbolAddress.
static __device__ __align__(256) unsigned char scratch[PA_NOALLOC_SCRATCH_BYTES];

namespace pa {
// Kernel instances dispatched by the last launching call on this thread.
thread_local std::string g_launches;

void note_launch(const char* fmt, ...) {
  char buf[160];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  if (!g_launches.empty()) g_launches += "; ";
  g_launches += buf;
}

hipError_t launch_decode_f16(const DecodeParams& p, int gc, hipStream_t stream);
hipError_t launch_decode_bf16(const DecodeParams& p, int gc, hipStream_t stream);
hipError_t launch_decode_f32(const DecodeParams& p, int gc, hipStream_t stream);
hipError_t launch_decode_f64(const DecodeParams& p, int gc, hipStream_t stream);
hipError_t launch_decode_fp8(const DecodeParams& p, int gc, hipStream_t stream);

thread_local int t_decode_fused = 0;

hipError_t launch_decode(const DecodeParams& p, int kv_dtype, int gc, hipStream_t stream) {
  switch (kv_dtype) {
    case kF16: return launch_decode_f16(p, gc, stream);
    case kBF16: return launch_decode_bf16(p, gc, stream);
    case kF32: return launch_decode_f32(p, gc, stream);
    case kF64: return launch_decode_f64(p, gc, stream);
    case kFP8: return launch_decode_fp8(p, gc, stream);
    default: return hipErrorInvalidValue;
  }
}
}  // namespace pa

namespace {

using namespace pa;

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int dtype_bytes(int dt) {
  switch (dt) {
    case kF32: case kI32: return 4;
    case kF16: case kBF16: return 2;
    case kF64: case kI64: return 8;
    case kFP8: return 1;
    default: return 0;
  }
}

const char* dtype_name(int dt) {
  switch (dt) {
    case kF32: return "float32";
    case kF16: return "float16";
    case kBF16: return "bfloat16";
    case kF64: return "float64";
    case kI32: return "int32";
    case kI64: return "int64";
    case kFP8: return "float8_e4m3fn";
    default: return "unknown";
  }
}

bool is_contiguous(const pa_tensor_t* t) {
  int64_t s = 1;
  for (int i = t->ndim - 1; i >= 0; --i) {
    if (t->shape[i] != 1 && t->stride[i] != s) return false;
    s *= t->shape[i];
  }
  return true;
}

int64_t numel(const pa_tensor_t* t) {
  int64_t n = 1;
  for (int i = 0; i < t->ndim; ++i) n *= t->shape[i];
  return n;
}

int check_tensor(const pa_tensor_t* t, const char* name, int ndim, const char* layout) {
  if (!t) return fail(PA_ERR_INVALID_ARGUMENT, "%s is NULL", name);
  if (t->ndim != ndim) return fail(PA_ERR_INVALID_ARGUMENT, "%s must be %s", name, layout);
  for (int i = 0; i < ndim; ++i)
    if (t->shape[i] < 0) return fail(PA_ERR_INVALID_ARGUMENT, "%s has a negative size", name);
  if (!t->data && numel(t) > 0) return fail(PA_ERR_INVALID_ARGUMENT, "%s has a NULL data pointer", name);
  return PA_OK;
}

// ------------------------------------------------------------ device info --

int device_cu_count(int* cus) {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0)
    return fail(PA_ERR_HIP, "no HIP device is available");
  if (dev < 64) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) { *cus = c; return PA_OK; }
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    return fail(PA_ERR_HIP, "cannot read the compute-unit count of device %d", dev);
  if (dev < 64) cached[dev].store(n, std::memory_order_relaxed);
  *cus = n;
  return PA_OK;
}

// Device address of the current device's `scratch`, looked up once per
// device (the first paged_attention_v3_noalloc call on it) with that device
// current, and kept.
constexpr int kMaxDevices = 64;
struct ScratchSlot {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t err = hipSuccess;
};
ScratchSlot g_scratch[kMaxDevices];

int scratch_address(void** ptr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return fail(PA_ERR_HIP, "no HIP device is available");
  if (dev >= kMaxDevices) return fail(PA_ERR_UNSUPPORTED, "device %d: at most %d devices are served", dev, kMaxDevices);
  ScratchSlot& s = g_scratch[dev];
  std::call_once(s.once, [&s] { s.err = hipGetSymbolAddress(&s.ptr, HIP_SYMBOL(scratch)); });
  if (s.err != hipSuccess || !s.ptr)
    return fail(PA_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(s.err));
  *ptr = s.ptr;
  return PA_OK;
}

// Tuning constants of the partition planner: target resident work-groups
// per CU; the shortest partition worth a work-group (and the same for tiny
// grids, whose time is latency, not bandwidth) and the longest (bounds ragged
// imbalance), in tokens.  Config 3 (ragged GQA-4, contexts to 32768) measured
// 1024-token partitions 2.6 % slower than 2048, 3072 3.5 % slower, 4096 17 %.
// Longest explicit partition (tokens, at the block table's capacity) served
// in the wave-partition mode.
constexpr int64_t kWavePartTokens = 256;
// Shortest explicit partition (tokens, at the block table's capacity) whose
// split dispatches its sequences longest first.
constexpr int64_t kLongestFirstTokens = 1024;

struct PlanKnobs {
  int64_t wgs_per_cu = 3;
  int64_t min_part = 256;
  int64_t min_part_tiny = 64;
  int64_t max_part = 2048;
  // A split pays for its reduce launch only when the unsplit work-groups'
  // streams are long: contexts (in 64-element rows) of at least
  // split_min_tokens, and ctx^2 * CUs >= split_pay * units.  Measured on 256
  // CUs, GPT-2 heads (D = 64, fp16), B = 1-48 x ctx 256-2048, whole calls
  // back to back: the unsplit launch won below 1024 tokens at every B (B = 1
  // ctx 512: 10.0 vs 11.0 us; B = 16 ctx 512: 11.1 vs 14.9 us), at 1024 from
  // B = 8 on (equal at 8; B = 32: 22.6 vs 25.9 us), at 1536 from B = 16 on
  // (20.4 vs 22.5 us) and at 2048 from B = 32 on (38.6 vs 41.5 us); the split
  // won from 1024 tokens at B <= 4 (B = 1 ctx 1024: 11.6 vs 14.0 us) and at
  // 1536 at B = 8 (17.4 vs 19.2 us); B = 16 at 2048 sits at the boundary
  // (either by 3-4 %, run to run).
  int64_t split_min_tokens = 1024;
  int64_t split_pay = 21845 * 256;
};

const PlanKnobs& knobs() {
  static constexpr PlanKnobs k{};
  return k;
}

// ---------------------------------------------------------- decode checks --

struct DecodeArgs {
  DecodeParams p;
  int kv_dtype;
  int gc;
};

// The kernels take scales as fp32: a finite double past FLT_MAX would become
// inf there, so every scale (and the folded softmax scale) is checked as fp32.
static bool finite_f32(double x) { return std::isfinite((float)x); }


// Shared checks of every entry point (the TORCH_CHECKs of
// kernels/paged_attn_v3.cu:199-216 and kernels/paged_attn_prefill.cu:128-146,
// plus the layout rules of this ABI).  prefill selects q [B,S,H,D].
int check_args(const pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k,
               const pa_tensor_t* v, const pa_tensor_t* bt, const pa_tensor_t* ctx, double scale,
               bool prefill, DecodeArgs* a) {
  int rc;
  const int qnd = prefill ? 4 : 3;
  const char* qlay = prefill ? "[B, S, H, D]" : "[B, H, D]";
  if ((rc = check_tensor(q, "q", qnd, qlay))) return rc;
  if ((rc = check_tensor(out, "out", qnd, qlay))) return rc;
  if ((rc = check_tensor(k, "k_cache", 4, "[NB, BS, H, D]"))) return rc;
  if ((rc = check_tensor(v, "v_cache", 4, "[NB, BS, H, D]"))) return rc;
  if ((rc = check_tensor(bt, "block_tables", 2, "[B, MB]"))) return rc;
  if ((rc = check_tensor(ctx, "context_lens", 1, "[B]"))) return rc;

  for (int i = 0; i < qnd; ++i)
    if (out->shape[i] != q->shape[i])
      return fail(PA_ERR_INVALID_ARGUMENT, "out must have the shape of q");
  if (q->dtype != kF32 && q->dtype != kF16 && q->dtype != kBF16)
    return fail(PA_ERR_INVALID_ARGUMENT, "q must be float32, float16 or bfloat16 (got %s)", dtype_name(q->dtype));
  if (out->dtype != kF32 && out->dtype != kF16 && out->dtype != kBF16)
    return fail(PA_ERR_INVALID_ARGUMENT, "out must be float32, float16 or bfloat16 (got %s)", dtype_name(out->dtype));
  if (k->dtype != kF32 && k->dtype != kF16 && k->dtype != kBF16 && k->dtype != kF64 && k->dtype != kFP8)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "k_cache must be float32, float16, bfloat16, float64 or float8_e4m3fn (got %s)", dtype_name(k->dtype));
  if (v->dtype != k->dtype) return fail(PA_ERR_INVALID_ARGUMENT, "v_cache must have the dtype of k_cache");
  if (bt->dtype != kI32) return fail(PA_ERR_INVALID_ARGUMENT, "block_tables must be int32");
  if (ctx->dtype != kI32) return fail(PA_ERR_INVALID_ARGUMENT, "context_lens must be int32");
  if (!is_contiguous(q)) return fail(PA_ERR_INVALID_ARGUMENT, "q must be contiguous");
  if (!is_contiguous(out)) return fail(PA_ERR_INVALID_ARGUMENT, "out must be contiguous");
  for (int i = 0; i < 4; ++i)
    if (v->shape[i] != k->shape[i]) return fail(PA_ERR_INVALID_ARGUMENT, "v_cache must have the shape of k_cache");
  if (!std::isfinite(scale) || !finite_f32(scale * 1.4426950408889634))
    return fail(PA_ERR_INVALID_ARGUMENT, "scale must be finite");

  const int64_t B = q->shape[0];
  const int64_t S = prefill ? q->shape[1] : 1;
  const int64_t H = q->shape[prefill ? 2 : 1];
  const int64_t D = q->shape[prefill ? 3 : 2];
  const int64_t NB = k->shape[0], BS = k->shape[1], HKV = k->shape[2];
  const int64_t MB = bt->shape[1];
  if (bt->shape[0] != B) return fail(PA_ERR_INVALID_ARGUMENT, "block_tables must have B rows");
  if (ctx->shape[0] != B) return fail(PA_ERR_INVALID_ARGUMENT, "context_lens must have B entries");
  if (k->shape[3] != D) return fail(PA_ERR_INVALID_ARGUMENT, "k_cache head_dim (%lld) != q head_dim (%lld)",
                                    (long long)k->shape[3], (long long)D);
  if (HKV <= 0 || H <= 0 || H % HKV != 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "n_head must be divisible by n_kv_head");
  if (BS <= 0) return fail(PA_ERR_INVALID_ARGUMENT, "block_size must be positive");
  if (D != 32 && D != 64 && D != 128 && D != 256)
    return fail(PA_ERR_UNSUPPORTED, "unsupported head_dim %lld", (long long)D);
  if (k->dtype == kF64 && D > 128)
    return fail(PA_ERR_UNSUPPORTED, "float64 KV caches support head_dim <= 128");
  if (MB * BS >= (1LL << 31) || B * S >= (1LL << 31) || B >= (1LL << 31) || H >= (1 << 16))
    return fail(PA_ERR_UNSUPPORTED, "problem too large for 32-bit token indices");
  if (bt->stride[1] != 1 || (B > 1 && bt->stride[0] < MB))
    return fail(PA_ERR_INVALID_ARGUMENT, "block_tables rows must be contiguous");
  if (ctx->stride[0] != 1 && B > 1) return fail(PA_ERR_INVALID_ARGUMENT, "context_lens must be contiguous");
  if (NB < 1) return fail(PA_ERR_INVALID_ARGUMENT, "k_cache must hold at least one block");
  const int es = dtype_bytes(k->dtype);
  for (const pa_tensor_t* t : {k, v}) {
    if (t->stride[3] != 1)
      return fail(PA_ERR_INVALID_ARGUMENT, "k_cache/v_cache must have a contiguous last dimension");
    for (int i = 0; i < 3; ++i)
      if (t->stride[i] < 0) return fail(PA_ERR_UNSUPPORTED, "k_cache/v_cache strides must be non-negative");
    // Kernels address a row as block * block_stride (64-bit) + token * token_stride
    // + lane offset (32-bit): the block stride and one block's extent must fit 32 bits.
    if (t->stride[0] * es >= (1LL << 32) || (BS * t->stride[1] + D) * es >= (1LL << 32))
      return fail(PA_ERR_UNSUPPORTED, "k_cache/v_cache block or token stride too large");
    for (int i = 0; i < 3; ++i)
      if (((t->stride[i] * es) & 15) != 0 && t->shape[i] > 1)
        return fail(PA_ERR_UNSUPPORTED, "k_cache/v_cache strides must be multiples of 16 bytes");
    if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0)
      return fail(PA_ERR_UNSUPPORTED, "k_cache/v_cache must be 16-byte aligned");
  }

  DecodeParams& p = a->p;
  memset(&p, 0, sizeof(p));
  p.q = q->data;
  p.out = out->data;
  p.k = k->data;
  p.v = v->data;
  p.block_tables = static_cast<const int32_t*>(bt->data);
  p.context_lens = static_cast<const int32_t*>(ctx->data);
  p.k_sb = k->stride[0]; p.k_st = k->stride[1]; p.k_sh = k->stride[2];
  p.v_sb = v->stride[0]; p.v_st = v->stride[1]; p.v_sh = v->stride[2];
  p.bt_stride = B > 1 ? bt->stride[0] : MB;
  p.num_blocks = NB;
  p.B = (int)B; p.Sq = (int)S; p.H = (int)H; p.HKV = (int)HKV; p.G = (int)(H / HKV);
  p.D = (int)D; p.BS = (int)BS; p.MB = (int)MB;
  p.q_dtype = q->dtype;
  p.out_dtype = out->dtype;
  p.bs_div = make_fastdiv((uint32_t)BS);
  p.qscale = (float)(scale * 1.4426950408889634);
  p.vscale = 1.0f;
  a->kv_dtype = k->dtype;
  a->gc = decode_heads_per_wg(p.G);
  p.head_chunks = (p.G + a->gc - 1) / a->gc;
  return PA_OK;
}

struct Plan {
  int64_t parts;
  int64_t part_tokens;  // 0 = reference count mode
  bool direct;
  int hp;  // KV heads per work-group (head packing)
};

// Head packing for a plan with `splits` partitions per (sequence, KV head):
// the widest packing whose work-groups still fill the GPU (target resident
// work-groups), else the narrowest one.
int pack_for(const DecodeParams& p, int kv_bytes, int64_t splits, int cus) {
  const int lo = decode_pack_min(p.D, kv_bytes, p.G, p.HKV, p.k_sh);
  const int hi = decode_pack_max(p.D, kv_bytes, p.G, p.HKV, p.k_sh);
  const int64_t target = (int64_t)cus * knobs().wgs_per_cu;
  for (int c = hi; c > lo; c /= 2)
    if ((int64_t)p.B * p.Sq * (p.HKV / c) * splits >= target) return c;
  return lo;
}

// The plan of a v3 call.  An explicit split needs no device query (the
// workspace-size query runs without one); its packing is chosen at launch
// (hp = 0 here).
int make_plan(const DecodeParams& p, int gc, int kv_bytes, int64_t num_splits, Plan* plan) {
  (void)gc;
  if (num_splits > 0) {
    if (num_splits > (1 << 20)) return fail(PA_ERR_INVALID_ARGUMENT, "num_splits too large");
    plan->parts = num_splits;
    plan->part_tokens = 0;
    plan->direct = num_splits == 1;
    plan->hp = 0;
    return PA_OK;
  }
  int cus = 0;
  int rc = device_cu_count(&cus);
  if (rc) return rc;
  // Auto plan: partitions for the narrowest packing, then the widest packing
  // that needs no more partitions than that (packing divides the work-groups
  // per sequence; a plan that must split anyway for length absorbs it).
  const int lo = decode_pack_min(p.D, kv_bytes, p.G, p.HKV, p.k_sh);
  const int hi = decode_pack_max(p.D, kv_bytes, p.G, p.HKV, p.k_sh);
  const int64_t maxctx = (int64_t)p.MB * p.BS;
  // (A unit of c packed heads streams c * D elements per token: its head
  // dimension for the planner's stream-length rule.)
  auto parts_for = [&](int c, int64_t* ptok) {
    int64_t np = 0;
    pa_plan_partitions(p.B, (p.HKV / c) * p.G, p.HKV / c, (int64_t)p.D * c, maxctx, cus, ptok, &np);
    return np;
  };
  int64_t ptok = 0;
  const int64_t nparts = parts_for(lo, &ptok);
  int hp = lo;
  // A grid that does not fill the GPU even unpacked keeps every work-group
  // it can get (latency-bound: more loads in flight beat wider rows).
  const bool fills = (int64_t)p.B * p.Sq * (p.HKV / lo) * nparts >= (int64_t)cus * knobs().wgs_per_cu;
  // The packed grid must fill the GPU too (an unsplit plan at the packed
  // width can leave it short: config 2 at two heads per work-group would be
  // 384 work-groups on 256 CUs).
  for (int c = hi; fills && c > lo; c /= 2) {
    int64_t pt = 0;
    if (parts_for(c, &pt) == nparts && pt == ptok &&
        (int64_t)p.B * p.Sq * (p.HKV / c) * nparts >= (int64_t)cus * knobs().wgs_per_cu) {
      hp = c;
      break;
    }
  }
  plan->parts = nparts;
  plan->part_tokens = nparts > 1 ? ptok : 0;
  plan->direct = nparts <= 1;
  plan->hp = hp;
  return PA_OK;
}

size_t workspace_bytes_for(int64_t B, int64_t H, int64_t D, const Plan& plan) {
  if (plan.direct) return 0;
  const size_t rows = (size_t)B * H * plan.parts;
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  return up(rows * D * 4) + 2 * up(rows * 4);
}

void bind_workspace(DecodeParams* p, void* ws, const Plan& plan) {
  const size_t rows = (size_t)p->B * p->H * plan.parts;
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  char* base = static_cast<char*>(ws);
  p->ws_acc = reinterpret_cast<float*>(base);
  p->ws_m = reinterpret_cast<float*>(base + up(rows * p->D * 4));
  p->ws_l = reinterpret_cast<float*>(base + up(rows * p->D * 4) + up(rows * 4));
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return PA_OK;
  return fail(PA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// One direct decode launch (one partition per sequence): v1, v2 and the
// fp32 prefill path.
int run_direct(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k, const pa_tensor_t* v,
               const pa_tensor_t* bt, const pa_tensor_t* ctx, double scale, bool prefill,
               void* stream) {
  g_launches.clear();
  DecodeArgs a;
  int rc = check_args(out, q, k, v, bt, ctx, scale, prefill, &a);
  if (rc) return rc;
  if ((int64_t)a.p.B * a.p.Sq * a.p.H == 0) return PA_OK;
  a.p.parts = 1;
  a.p.part_tokens = 0;
  a.p.direct = 1;
  int cus = 0;
  if ((rc = device_cu_count(&cus))) return rc;
  a.p.hp = pack_for(a.p, dtype_bytes(a.kv_dtype), 1, cus);
  return hip_status(launch_decode(a.p, a.kv_dtype, a.gc, static_cast<hipStream_t>(stream)),
                    "decode kernel launch");
}

enum V3Phase { kBoth = 3, kPartition = 1, kReduce = 2 };

int run_v3(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k, const pa_tensor_t* v,
           const pa_tensor_t* bt, const pa_tensor_t* ctx, double scale, int64_t num_splits,
           void* ws, size_t ws_bytes, void* stream, int phases, double k_scale = 1.0,
           double v_scale = 1.0, bool noalloc = false) {
  g_launches.clear();
  DecodeArgs a;
  int rc = check_args(out, q, k, v, bt, ctx, scale, false, &a);
  if (rc) return rc;
  if (noalloc) ws_bytes = PA_NOALLOC_SCRATCH_BYTES;  // the split scratch is this device's fixed array
  if (!finite_f32(k_scale) || !finite_f32(v_scale))
    return fail(PA_ERR_INVALID_ARGUMENT, "k_scale and v_scale must be finite");
  if (!finite_f32(scale * k_scale * 1.4426950408889634))
    return fail(PA_ERR_INVALID_ARGUMENT, "scale * k_scale must be finite");
  // Dequantisation scales of the cache (FP8): k_scale joins the softmax
  // scale, v_scale multiplies the weighted V sum.
  a.p.qscale = (float)(scale * k_scale * 1.4426950408889634);
  a.p.vscale = (float)v_scale;
  if ((int64_t)a.p.B * a.p.H == 0) return PA_OK;
  Plan plan;
  if ((rc = make_plan(a.p, a.gc, dtype_bytes(a.kv_dtype), num_splits, &plan))) return rc;
  const size_t need = workspace_bytes_for(a.p.B, a.p.H, a.p.D, plan);
  if (noalloc && need > ws_bytes)
    return fail(PA_ERR_WORKSPACE,
                "paged_attention_v3_noalloc: this call's split needs %zu bytes of scratch, more than the "
                "fixed %zu (PA_NOALLOC_SCRATCH_BYTES); use paged_attention_v3 with a workspace",
                need, ws_bytes);
  if (noalloc && (rc = scratch_address(&ws))) return rc;
  if (need > 0 && (!ws || ws_bytes < need))
    return fail(PA_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", need, ws ? ws_bytes : 0);
  if (need > 0 && (reinterpret_cast<uintptr_t>(ws) & 255) != 0)
    return fail(PA_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  a.p.parts = (int)plan.parts;
  a.p.part_tokens = (int)plan.part_tokens;
  a.p.direct = plan.direct ? 1 : 0;
  // Explicit splits into short chunks (the reference's own count at long
  // contexts: 64 splits of 32 tokens at ctx 2048) run with a partition per
  // wave or per token slot, each written as its own partials.  A call that
  // wants the output too, over groups of one query head per KV head chunk,
  // fuses when decode_fuse_rounds() allows it and one work-group per (row,
  // head) at the narrowest packing still fills the GPU: that work-group
  // serves every partition of its unit in rounds, merges each partition's
  // partials into the output in registers (they are not written), and the
  // reduce launch is skipped (config 2 at 64 splits: partition kernel +
  // reduce 79.0 us per call, fused 65.6 us).
  const int64_t maxctx = (int64_t)a.p.MB * a.p.BS;
  a.p.wave_parts = num_splits > 0 && !plan.direct && (maxctx + plan.parts - 1) / plan.parts <= kWavePartTokens;
  a.p.hp = plan.hp;
  a.p.fuse_final = 0;
  if (a.p.wave_parts && phases == kBoth && a.gc == 1) {
    int cus = 0;
    if ((rc = device_cu_count(&cus))) return rc;
    const int kvb = dtype_bytes(a.kv_dtype);
    const int hp = pack_for(a.p, kvb, 1, cus);
    if ((int64_t)a.p.B * a.p.Sq * (a.p.HKV / hp) * a.p.head_chunks >= cus &&
        decode_fuse_rounds(plan.parts, a.p.MB, a.p.BS, decode_tpi(a.p.D, hp, kvb)) > 0) {
      a.p.fuse_final = 1;
      a.p.hp = hp;
    }
  }
  if (a.p.hp == 0) {
    int cus = 0;
    if ((rc = device_cu_count(&cus))) return rc;
    a.p.hp = pack_for(a.p, dtype_bytes(a.kv_dtype), plan.parts, cus);
  }
  // An explicit split into long partitions over up to 64 sequences orders
  // the sequences longest first (the kernel ranks the context lengths; one
  // more memory round trip per work-group, which short partitions do not
  // repay): config 3's ragged batch at 8 splits (partitions up to 4096
  // tokens) 5.33 -> 6.17 TB/s; at 64 splits (up to 512) -2 %, and config 2's
  // uniform batch at 8 or 64 splits -3.7 %, hence the bound.
  a.p.seq_order = num_splits > 0 && !plan.direct && a.p.B <= 64 && a.p.Sq == 1 &&
                  (maxctx + plan.parts - 1) / plan.parts >= kLongestFirstTokens ? 1 : 0;
  if (!plan.direct) bind_workspace(&a.p, ws, plan);
  hipStream_t s = static_cast<hipStream_t>(stream);
  t_decode_fused = 0;
  if (phases & kPartition) {
    if ((rc = hip_status(launch_decode(a.p, a.kv_dtype, a.gc, s), "partition kernel launch"))) return rc;
  }
  if ((phases & kReduce) && !plan.direct && !t_decode_fused) {
    ReduceParams r;
    r.out = a.p.out;
    r.ws_acc = a.p.ws_acc;
    r.ws_m = a.p.ws_m;
    r.ws_l = a.p.ws_l;
    r.context_lens = a.p.context_lens;
    r.B = a.p.B; r.H = a.p.H; r.D = a.p.D; r.MB = a.p.MB; r.BS = a.p.BS;
    r.out_dtype = a.p.out_dtype;
    r.parts = a.p.parts;
    r.part_tokens = a.p.part_tokens;
    if ((rc = hip_status(launch_reduce(r, s), "reduce kernel launch"))) return rc;
  }
  return PA_OK;
}

// MFMA prefill launch for checked arguments; cu != null selects the
// variable-length layout (rows cu[b] .. cu[b+1] of a packed [T, H, D] q/out).
int run_prefill_mfma(DecodeArgs& a, const pa_tensor_t* q, const int32_t* cu, int64_t T, double scale,
                     void* stream, bool route_single = false, double v_scale = 1.0) {
  if (!route_single) g_launches.clear();
  // kernels/paged_attn_wmma.cu:220-223 requires fp16; bf16 and FP8 (E4M3, read
  // as fp16) are served as well.
  if (a.kv_dtype != kF16 && a.kv_dtype != kBF16 && a.kv_dtype != kFP8)
    return fail(PA_ERR_INVALID_ARGUMENT, "the MFMA path needs an fp16, bf16 or float8_e4m3fn KV cache");
  if (a.p.D > 256) return fail(PA_ERR_UNSUPPORTED, "unsupported head_dim for the MFMA path: %d", a.p.D);
  if ((int64_t)a.p.B * a.p.Sq * a.p.H == 0) return PA_OK;
  if ((reinterpret_cast<uintptr_t>(q->data) & 15) != 0)
    return fail(PA_ERR_UNSUPPORTED, "the MFMA path needs a 16-byte aligned q");
  PrefillParams pp;
  memset(&pp, 0, sizeof(pp));
  const DecodeParams& p = a.p;
  pp.q = p.q; pp.out = p.out; pp.k = p.k; pp.v = p.v;
  pp.block_tables = p.block_tables; pp.context_lens = p.context_lens;
  pp.k_sb = p.k_sb; pp.k_st = p.k_st; pp.k_sh = p.k_sh;
  pp.v_sb = p.v_sb; pp.v_st = p.v_st; pp.v_sh = p.v_sh;
  pp.bt_stride = p.bt_stride; pp.num_blocks = p.num_blocks;
  pp.B = p.B; pp.S = p.Sq; pp.H = p.H; pp.HKV = p.HKV; pp.G = p.G; pp.D = p.D; pp.BS = p.BS; pp.MB = p.MB;
  pp.q_dtype = p.q_dtype; pp.out_dtype = p.out_dtype;
  // FP8 K tiles take q's type when q is fp16 or bf16 (the codes convert exactly to both).
  pp.q_split = a.kv_dtype == kFP8 ? p.q_dtype == kF32 : p.q_dtype != a.kv_dtype;
  pp.bs_div = p.bs_div;
  pp.cu_q = cu;
  pp.q_total = T;
  pp.skip_single = route_single ? 1 : 0;
  pp.vscale = (float)v_scale;
  // The kernel applies the sign of the scale to q (exactly) and keeps the
  // softmax scale positive, so the running max of raw scores orders as the scaled ones.
  const double log2e = 1.4426950408889634;
  pp.q_and = 0xffffffffu;
  pp.q_xor = 0u;
  pp.q_sign = 1.0f;
  pp.qscale = (float)(scale * log2e);
  if (scale < 0) {
    pp.q_xor = 0x80008000u;
    pp.q_sign = -1.0f;
    pp.qscale = (float)(-scale * log2e);
  } else if (scale == 0) {
    pp.q_and = 0u;
    pp.q_sign = 0.0f;
    pp.qscale = 1.0f;
  }
  return hip_status(launch_prefill_mfma(pp, a.kv_dtype, static_cast<hipStream_t>(stream)),
                    "prefill kernel launch");
}

}  // namespace

extern "C" {

int pa_abi_version(void) { return PA_ABI_VERSION; }

const char* pa_last_error(void) { return g_last_error.c_str(); }

const char* pa_last_launch(void) { return pa::g_launches.c_str(); }

int64_t choose_num_splits_for(int64_t num_seqs, int64_t num_heads, int64_t max_context,
                              int64_t num_compute_units) {
  // kernels/paged_attn_v3.cu:170-190, compute units in place of SMs.
  const int64_t have = std::max<int64_t>(num_seqs * num_heads, 1);
  const int64_t by_chain = std::max<int64_t>(max_context / 32, 1);
  const int64_t to_fill = std::max<int64_t>((num_compute_units * 8 + have - 1) / have, 1);
  const int64_t s = std::max(by_chain, to_fill);
  return std::max<int64_t>(1, std::min<int64_t>(s, 64));
}

int64_t choose_num_splits(int64_t num_seqs, int64_t num_heads, int64_t max_context) {
  int cus = 0;
  if (device_cu_count(&cus)) return -1;
  return choose_num_splits_for(num_seqs, num_heads, max_context, cus);
}

int pa_plan_partitions(int64_t num_seqs, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                       int64_t max_context, int64_t num_compute_units, int64_t* partition_tokens,
                       int64_t* num_partitions) {
  if (!partition_tokens || !num_partitions)
    return fail(PA_ERR_INVALID_ARGUMENT, "NULL output pointer");
  if (num_seqs < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads || max_context < 0 ||
      num_compute_units <= 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "invalid planning arguments");
  const PlanKnobs& kn = knobs();
  const int64_t G = num_heads / num_kv_heads;
  const int64_t gc = decode_heads_per_wg((int)G);
  const int64_t units = std::max<int64_t>(1, num_seqs * num_kv_heads * ((G + gc - 1) / gc));
  const int64_t target = num_compute_units * kn.wgs_per_cu;
  const double ctx_rows = (double)max_context * (double)std::max<int64_t>(head_dim, 1) / 64.0;
  if (ctx_rows < (double)kn.split_min_tokens ||
      ctx_rows * ctx_rows * (double)num_compute_units < (double)kn.split_pay * (double)units) {
    *partition_tokens = std::max<int64_t>(max_context, 1);
    *num_partitions = 1;
    return PA_OK;
  }
  int64_t S = (target + units - 1) / units;                             // fill the GPU
  S = std::max(S, (max_context + kn.max_part - 1) / kn.max_part);       // bound partition length
  // Tiny grids (the units with partitions of min_part tokens still cannot
  // fill the GPU: a few short sequences) take shorter partitions, so that
  // more work-groups have their loads in flight at once.
  const bool tiny = units * std::max<int64_t>(1, max_context / kn.min_part) < target;
  const int64_t min_part = tiny ? kn.min_part_tiny : kn.min_part;
  S = std::min(S, std::max<int64_t>(1, max_context / min_part));        // keep partitions long enough
  if (S <= 1 || max_context <= 0) {
    *partition_tokens = std::max<int64_t>(max_context, 1);
    *num_partitions = 1;
    return PA_OK;
  }
  int64_t ptok = (max_context + S - 1) / S;
  const int64_t gran = ptok > 64 ? 128 : 64;  // whole wave tiles for all 4 waves
  ptok = (ptok + gran - 1) / gran * gran;
  *partition_tokens = ptok;
  *num_partitions = (max_context + ptok - 1) / ptok;
  if (*num_partitions <= 1) *partition_tokens = std::max<int64_t>(max_context, 1);
  return PA_OK;
}

int paged_attention(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                    const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                    const pa_tensor_t* context_lens, double scale, void* stream) {
  return run_direct(out, q, k_cache, v_cache, block_tables, context_lens, scale, false, stream);
}

int paged_attention_v2(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                       const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                       const pa_tensor_t* context_lens, double scale, void* stream) {
  return run_direct(out, q, k_cache, v_cache, block_tables, context_lens, scale, false, stream);
}

int paged_attention_v3(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                       const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                       const pa_tensor_t* context_lens, double scale, int64_t num_splits,
                       void* workspace, size_t workspace_bytes, void* stream) {
  return run_v3(out, q, k_cache, v_cache, block_tables, context_lens, scale, num_splits, workspace,
                workspace_bytes, stream, kBoth);
}

int paged_attention_v3_scaled(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                              const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                              const pa_tensor_t* context_lens, double scale, double k_scale, double v_scale,
                              int64_t num_splits, void* workspace, size_t workspace_bytes, void* stream) {
  return run_v3(out, q, k_cache, v_cache, block_tables, context_lens, scale, num_splits, workspace,
                workspace_bytes, stream, kBoth, k_scale, v_scale);
}

int paged_attention_v3_noalloc(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                               const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                               const pa_tensor_t* context_lens, double scale, int64_t num_splits,
                               void* stream) {
  return run_v3(out, q, k_cache, v_cache, block_tables, context_lens, scale, num_splits, nullptr, 0, stream,
                kBoth, 1.0, 1.0, true);
}

int pa_v3_partition(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                    const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                    const pa_tensor_t* context_lens, double scale, int64_t num_splits,
                    void* workspace, size_t workspace_bytes, void* stream) {
  return run_v3(out, q, k_cache, v_cache, block_tables, context_lens, scale, num_splits, workspace,
                workspace_bytes, stream, kPartition);
}

int pa_v3_reduce(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                 const pa_tensor_t* block_tables, const pa_tensor_t* context_lens,
                 int64_t num_splits, void* workspace, size_t workspace_bytes, void* stream) {
  return run_v3(out, q, k_cache, k_cache, block_tables, context_lens, 1.0, num_splits, workspace,
                workspace_bytes, stream, kReduce);
}

size_t paged_attention_v3_workspace_size(const pa_tensor_t* q, const pa_tensor_t* k_cache,
                                         const pa_tensor_t* block_tables, int64_t num_splits) {
  if (check_tensor(q, "q", 3, "[B, H, D]") || check_tensor(k_cache, "k_cache", 4, "[NB, BS, H, D]") ||
      check_tensor(block_tables, "block_tables", 2, "[B, MB]"))
    return (size_t)-1;
  const int64_t B = q->shape[0], H = q->shape[1], D = q->shape[2];
  const int64_t BS = k_cache->shape[1], HKV = k_cache->shape[2], MB = block_tables->shape[1];
  if (HKV <= 0 || H % HKV) {
    fail(PA_ERR_INVALID_ARGUMENT, "n_head must be divisible by n_kv_head");
    return (size_t)-1;
  }
  DecodeParams p;
  memset(&p, 0, sizeof(p));
  p.B = (int)B; p.H = (int)H; p.HKV = (int)HKV; p.G = (int)(H / HKV); p.D = (int)D; p.BS = (int)BS;
  p.MB = (int)MB;
  p.k_sh = k_cache->stride[2];
  Plan plan;
  if (make_plan(p, decode_heads_per_wg(p.G), dtype_bytes(k_cache->dtype), num_splits, &plan)) return (size_t)-1;
  return workspace_bytes_for(B, H, D, plan);
}

int paged_attention_prefill(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                            const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                            const pa_tensor_t* context_lens, double scale, void* stream) {
  return run_direct(out, q, k_cache, v_cache, block_tables, context_lens, scale, true, stream);
}

int paged_attention_prefill_wmma(pa_tensor_t* out, const pa_tensor_t* q,
                                 const pa_tensor_t* k_cache, const pa_tensor_t* v_cache,
                                 const pa_tensor_t* block_tables,
                                 const pa_tensor_t* context_lens, double scale, void* stream) {
  DecodeArgs a;
  int rc = check_args(out, q, k_cache, v_cache, block_tables, context_lens, scale, true, &a);
  if (rc) return rc;
  return run_prefill_mfma(a, q, nullptr, 0, scale, stream);
}

int paged_attention_prefill_wmma_scaled(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                                        const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                                        const pa_tensor_t* context_lens, double scale, double k_scale,
                                        double v_scale, void* stream) {
  if (!finite_f32(k_scale) || !finite_f32(v_scale))
    return fail(PA_ERR_INVALID_ARGUMENT, "k_scale and v_scale must be finite");
  // k_scale joins the softmax scale (q . (k_scale k) = (scale k_scale) q . k),
  // v_scale multiplies the output rows.
  DecodeArgs a;
  int rc = check_args(out, q, k_cache, v_cache, block_tables, context_lens, scale * k_scale, true, &a);
  if (rc) return rc;
  return run_prefill_mfma(a, q, nullptr, 0, scale * k_scale, stream, false, v_scale);
}

int paged_attention_prefill_varlen(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                                   const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                                   const pa_tensor_t* context_lens, const pa_tensor_t* cu_seqlens_q,
                                   int64_t max_q_len, double scale, void* stream) {
  return paged_attention_prefill_varlen_scaled(out, q, k_cache, v_cache, block_tables, context_lens, cu_seqlens_q,
                                               max_q_len, scale, 1.0, 1.0, stream);
}

int paged_attention_prefill_varlen_scaled(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                                          const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                                          const pa_tensor_t* context_lens, const pa_tensor_t* cu_seqlens_q,
                                          int64_t max_q_len, double scale, double k_scale, double v_scale,
                                          void* stream) {
  int rc;
  if (!finite_f32(k_scale) || !finite_f32(v_scale))
    return fail(PA_ERR_INVALID_ARGUMENT, "k_scale and v_scale must be finite");
  if ((rc = check_tensor(q, "q", 3, "[T, H, D]"))) return rc;
  if ((rc = check_tensor(out, "out", 3, "[T, H, D]"))) return rc;
  if ((rc = check_tensor(block_tables, "block_tables", 2, "[B, MB]"))) return rc;
  if ((rc = check_tensor(cu_seqlens_q, "cu_seqlens_q", 1, "[B + 1]"))) return rc;
  for (int i = 0; i < 3; ++i)
    if (out->shape[i] != q->shape[i]) return fail(PA_ERR_INVALID_ARGUMENT, "out must have the shape of q");
  if (!is_contiguous(q)) return fail(PA_ERR_INVALID_ARGUMENT, "q must be contiguous");
  if (!is_contiguous(out)) return fail(PA_ERR_INVALID_ARGUMENT, "out must be contiguous");
  const int64_t B = block_tables->shape[0], T = q->shape[0];
  if (cu_seqlens_q->dtype != kI32) return fail(PA_ERR_INVALID_ARGUMENT, "cu_seqlens_q must be int32");
  if (cu_seqlens_q->shape[0] != B + 1) return fail(PA_ERR_INVALID_ARGUMENT, "cu_seqlens_q must have B + 1 entries");
  if (cu_seqlens_q->stride[0] != 1) return fail(PA_ERR_INVALID_ARGUMENT, "cu_seqlens_q must be contiguous");
  if (max_q_len < 0) return fail(PA_ERR_INVALID_ARGUMENT, "max_q_len must be non-negative");
  if (T >= (1LL << 31)) return fail(PA_ERR_UNSUPPORTED, "too many query tokens");
  // The attention checks run on [B, max_q_len, H, D] descriptors of the packed
  // q/out (shape and type checks only; rows are addressed through cu_seqlens_q).
  const int64_t mq = std::max<int64_t>(max_q_len, 1);
  pa_tensor_t q4 = {q->data, q->dtype, 4, {B, mq, q->shape[1], q->shape[2]},
                    {mq * q->shape[1] * q->shape[2], q->shape[1] * q->shape[2], q->shape[2], 1}};
  pa_tensor_t o4 = q4;
  o4.data = out->data;
  o4.dtype = out->dtype;
  DecodeArgs a;
  rc = check_args(&o4, &q4, k_cache, v_cache, block_tables, context_lens, scale * k_scale, true, &a);
  if (rc) return rc;
  if (max_q_len == 0 || T == 0) return PA_OK;
  g_launches.clear();
  const int32_t* cu = static_cast<const int32_t*>(cu_seqlens_q->data);
  // Sequences that bring one query row (decode steps of the batch) go to the
  // decode kernel, one launch over every sequence in which the others' work-
  // groups exit at once; the prefill kernel then skips them.  The rows are
  // told apart on the device (cu_seqlens_q is device memory: no host sync).
  const bool prefill_ok = (a.kv_dtype == kF16 || a.kv_dtype == kBF16 || a.kv_dtype == kFP8) && a.p.D <= 256 &&
                          (reinterpret_cast<uintptr_t>(q->data) & 15) == 0 && (int64_t)a.p.B * a.p.H > 0;
  if (prefill_ok) {  // (otherwise the prefill call below reports why, before any launch)
    DecodeArgs d = a;  // check_args folded k_scale into d.p.qscale
    d.p.vscale = (float)v_scale;
    d.p.Sq = 1;
    d.p.cu_q = cu;
    d.p.q_total = T;
    d.p.parts = 1;
    d.p.part_tokens = 0;
    d.p.direct = 1;
    int cus = 0;
    if ((rc = device_cu_count(&cus))) return rc;
    d.p.hp = pack_for(d.p, dtype_bytes(d.kv_dtype), 1, cus);
    if ((rc = hip_status(launch_decode(d.p, d.kv_dtype, d.gc, static_cast<hipStream_t>(stream)),
                         "decode kernel launch")))
      return rc;
  }
  return run_prefill_mfma(a, q, cu, T, scale * k_scale, stream, true, v_scale);
}

int pa_write_kv(pa_tensor_t* k_cache, pa_tensor_t* v_cache, const pa_tensor_t* key,
                const pa_tensor_t* value, const pa_tensor_t* slot_mapping, void* stream) {
  return pa_write_kv_scaled(k_cache, v_cache, key, value, slot_mapping, 1.0, 1.0, stream);
}

int pa_write_kv_scaled(pa_tensor_t* k_cache, pa_tensor_t* v_cache, const pa_tensor_t* key,
                       const pa_tensor_t* value, const pa_tensor_t* slot_mapping, double k_scale,
                       double v_scale, void* stream) {
  g_launches.clear();
  int rc;
  if ((rc = check_tensor(k_cache, "k_cache", 4, "[NB, BS, HKV, D]"))) return rc;
  if ((rc = check_tensor(v_cache, "v_cache", 4, "[NB, BS, HKV, D]"))) return rc;
  if ((rc = check_tensor(key, "key", 3, "[T, HKV, D]"))) return rc;
  if ((rc = check_tensor(value, "value", 3, "[T, HKV, D]"))) return rc;
  if ((rc = check_tensor(slot_mapping, "slot_mapping", 1, "[T]"))) return rc;
  const int cd = k_cache->dtype, sd = key->dtype;
  if (cd != kF16 && cd != kBF16 && cd != kF32 && cd != kFP8)
    return fail(PA_ERR_INVALID_ARGUMENT, "k_cache must be float16, bfloat16, float32 or float8_e4m3fn (got %s)",
                dtype_name(cd));
  if (!finite_f32(k_scale) || !finite_f32(v_scale) || (float)k_scale == 0.0f || (float)v_scale == 0.0f)
    return fail(PA_ERR_INVALID_ARGUMENT, "k_scale and v_scale must be finite and nonzero");
  if (v_cache->dtype != cd) return fail(PA_ERR_INVALID_ARGUMENT, "v_cache must have the dtype of k_cache");
  if (sd != kF16 && sd != kBF16 && sd != kF32)
    return fail(PA_ERR_INVALID_ARGUMENT, "key must be float16, bfloat16 or float32 (got %s)", dtype_name(sd));
  if (value->dtype != sd) return fail(PA_ERR_INVALID_ARGUMENT, "value must have the dtype of key");
  if (slot_mapping->dtype != kI32 && slot_mapping->dtype != kI64)
    return fail(PA_ERR_INVALID_ARGUMENT, "slot_mapping must be int32 or int64");
  for (int i = 0; i < 4; ++i)
    if (v_cache->shape[i] != k_cache->shape[i])
      return fail(PA_ERR_INVALID_ARGUMENT, "v_cache must have the shape of k_cache");
  const int64_t NB = k_cache->shape[0], BS = k_cache->shape[1], HKV = k_cache->shape[2], D = k_cache->shape[3];
  const int64_t T = key->shape[0];
  for (int i = 0; i < 3; ++i)
    if (value->shape[i] != key->shape[i]) return fail(PA_ERR_INVALID_ARGUMENT, "value must have the shape of key");
  if (key->shape[1] != HKV || key->shape[2] != D)
    return fail(PA_ERR_INVALID_ARGUMENT, "key must be [T, %lld, %lld] to match k_cache", (long long)HKV,
                (long long)D);
  if (slot_mapping->shape[0] != T) return fail(PA_ERR_INVALID_ARGUMENT, "slot_mapping must have T entries");
  if (T > 1 && slot_mapping->stride[0] != 1) return fail(PA_ERR_INVALID_ARGUMENT, "slot_mapping must be contiguous");
  if (D <= 0 || D % 8 != 0) return fail(PA_ERR_UNSUPPORTED, "head_dim must be a positive multiple of 8");
  if (BS <= 0) return fail(PA_ERR_INVALID_ARGUMENT, "block_size must be positive");
  if (NB * BS >= (1LL << 31) || T * HKV * (D / 8) >= (1LL << 40))
    return fail(PA_ERR_UNSUPPORTED, "problem too large for 32-bit slot indices");
  const int ces = dtype_bytes(cd), ses = dtype_bytes(sd);
  for (const pa_tensor_t* t : {(const pa_tensor_t*)k_cache, (const pa_tensor_t*)v_cache}) {
    if (t->stride[3] != 1) return fail(PA_ERR_INVALID_ARGUMENT, "k_cache/v_cache must have a contiguous last dimension");
    for (int i = 0; i < 3; ++i) {
      if (t->stride[i] < 0) return fail(PA_ERR_UNSUPPORTED, "k_cache/v_cache strides must be non-negative");
      if (((t->stride[i] * ces) & 15) != 0 && t->shape[i] > 1)
        return fail(PA_ERR_UNSUPPORTED, "k_cache/v_cache strides must be multiples of 16 bytes");
    }
    if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0)
      return fail(PA_ERR_UNSUPPORTED, "k_cache/v_cache must be 16-byte aligned");
  }
  for (const pa_tensor_t* t : {key, value}) {
    if (t->stride[2] != 1) return fail(PA_ERR_INVALID_ARGUMENT, "key/value must have a contiguous last dimension");
    for (int i = 0; i < 2; ++i) {
      if (t->stride[i] < 0) return fail(PA_ERR_UNSUPPORTED, "key/value strides must be non-negative");
      if (((t->stride[i] * ses) & 15) != 0 && t->shape[i] > 1)
        return fail(PA_ERR_UNSUPPORTED, "key/value token and head strides must be multiples of 16 bytes");
    }
    if ((reinterpret_cast<uintptr_t>(t->data) & 15) != 0)
      return fail(PA_ERR_UNSUPPORTED, "key/value must be 16-byte aligned");
  }
  if (T == 0 || NB == 0 || HKV == 0) return PA_OK;
  WriteParams p;
  memset(&p, 0, sizeof(p));
  p.kc = k_cache->data; p.vc = v_cache->data;
  p.key = key->data; p.value = value->data; p.slots = slot_mapping->data;
  p.kc_sb = k_cache->stride[0]; p.kc_st = k_cache->stride[1]; p.kc_sh = k_cache->stride[2];
  p.vc_sb = v_cache->stride[0]; p.vc_st = v_cache->stride[1]; p.vc_sh = v_cache->stride[2];
  p.key_st = key->stride[0]; p.key_sh = key->stride[1];
  p.val_st = value->stride[0]; p.val_sh = value->stride[1];
  p.nslots = NB * BS;
  p.T = (int32_t)std::min<int64_t>(T, INT32_MAX);
  if (T > INT32_MAX) return fail(PA_ERR_UNSUPPORTED, "too many tokens for one call");
  p.HKV = (int32_t)HKV; p.D = (int32_t)D; p.BS = (int32_t)BS;
  p.src_dtype = sd; p.cache_dtype = cd; p.slot_i64 = slot_mapping->dtype == kI64;
  p.k_scale = (float)k_scale; p.v_scale = (float)v_scale;
  p.k_rcp = 1.0f / p.k_scale; p.v_rcp = 1.0f / p.v_scale;  // IEEE single division: correctly rounded
  auto in_range = [](float r) { return std::fabs(r) >= 0x1p-60f && std::fabs(r) <= 0x1p60f; };
  p.k_fast = in_range(p.k_rcp); p.v_fast = in_range(p.v_rcp);
  p.unit_scale = p.k_scale == 1.0f && p.v_scale == 1.0f;
  p.bs_div = make_fastdiv((uint32_t)BS);
  return hip_status(launch_write_kv(p, static_cast<hipStream_t>(stream)), "KV write kernel launch");
}

}  // extern "C"
