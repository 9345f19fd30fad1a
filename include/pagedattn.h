/*
 * pagedattn.h -- C-ABI of the MI355X (gfx950) paged-attention library.
 *
 * Drop-in boundary for the reference's torch::Tensor launchers declared in
 * kernels/paged_attn_v1.h, kernels/paged_attn_v2.h, kernels/paged_attn_v3.h,
 * kernels/paged_attn_prefill.h and kernels/paged_attn_wmma.h (gb10-attn).
 *
 * Every reference launcher takes (q, k_cache, v_cache, block_tables,
 * context_lens, scale[, num_splits]) and returns a freshly allocated fp32
 * tensor.  A C ABI cannot return a tensor, so here:
 *   - each tensor argument is a pa_tensor_t view (device pointer, dtype,
 *     shape, element strides) -- plain C, no torch types;
 *   - the output is a caller-allocated pa_tensor_t (fp32 as in the reference,
 *     or fp16/bf16);
 *   - scratch for the context split is a caller-provided workspace whose size
 *     is queried with paged_attention_v3_workspace_size();
 *   - work is enqueued asynchronously on the given HIP stream (hipStream_t,
 *     NULL = the null stream, which is where the reference launches);
 *   - the return value is a pa_status_t; on failure pa_last_error() returns a
 *     thread-local message.  Every argument check runs on the host before any
 *     HIP call, so a rejected call touches no device state.
 *
 * Layouts (the reference's, kernels/paged_attn_v3.cu:51-55):
 *   decode q / out      [B, H, D]
 *   prefill q / out     [B, S, H, D]
 *   k_cache / v_cache   [NB, BS, HKV, D]   (any element strides; the last dim
 *                                           must be contiguous; all offsets are
 *                                           computed in 64 bits).  Decode paths
 *                                           take fp32, fp16, bf16, fp64 or FP8
 *                                           E4M3; the MFMA prefill fp16 / bf16.
 *   block_tables        int32 [B, MB]      (row stride may exceed MB)
 *   context_lens        int32 [B]
 * Token j of sequence b, KV head kvh, lives at
 *   k_cache[block_tables[b][j / BS], j % BS, kvh, :]
 * and query head h reads KV head h / (H / HKV) (kernels/paged_attn_v3.cu:63,87-89).
 *
 * Behaviour the reference leaves undefined, fixed here:
 *   - context_lens[b] <= 0: the output rows of sequence b are written as zeros
 *     (reference: v1/v2 leave garbage, v3 writes NaN);
 *   - context_lens[b] > MB*BS, or a block id outside [0, NB) on the sequence's
 *     live pages: the output rows of that sequence are NaN and no out-of-range
 *     memory is read (reference: out-of-bounds reads).
 */
#ifndef PAGEDATTN_H_
#define PAGEDATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PA_ABI_VERSION 2
#define PA_MAX_DIMS 4

typedef enum pa_dtype {
  PA_DTYPE_F32 = 0,
  PA_DTYPE_F16 = 1,
  PA_DTYPE_BF16 = 2,
  PA_DTYPE_F64 = 3,
  PA_DTYPE_I32 = 4,
  PA_DTYPE_I64 = 5,
  PA_DTYPE_FP8_E4M3 = 6  /* OCP FP8 E4M3 (torch.float8_e4m3fn): KV caches of the decode paths */
} pa_dtype_t;

typedef enum pa_status {
  PA_OK = 0,
  PA_ERR_INVALID_ARGUMENT = 1, /* shape / dtype / null-pointer errors (TORCH_CHECK in the reference) */
  PA_ERR_UNSUPPORTED = 2,      /* valid request this build does not serve (e.g. head_dim 96) */
  PA_ERR_WORKSPACE = 3,        /* workspace missing or too small */
  PA_ERR_HIP = 4               /* a HIP runtime call or kernel launch failed */
} pa_status_t;

/* A strided view of device memory, the C counterpart of a torch::Tensor argument. */
typedef struct pa_tensor {
  void* data;                   /* device pointer to element [0, ..., 0] */
  int32_t dtype;                /* pa_dtype_t */
  int32_t ndim;                 /* 1..PA_MAX_DIMS */
  int64_t shape[PA_MAX_DIMS];
  int64_t stride[PA_MAX_DIMS];  /* in elements, not bytes */
} pa_tensor_t;

/* ABI version this library was built with (PA_ABI_VERSION). */
int pa_abi_version(void);

/* Message for the last failed call on this thread ("" if none). */
const char* pa_last_error(void);

/* Kernel instances the last launching call on this thread dispatched, named
 * as profilers print them (e.g. "pa::decode_kernel<pa::KvF16, 64, 1, 1, 1>"),
 * separated by "; " ("" when that call launched nothing).  A diagnostic with
 * no reference counterpart: it lets a benchmark report the kernel it timed. */
const char* pa_last_launch(void);

/* Decode, naive-fused semantics.  Replaces paged_attention(),
 * kernels/paged_attn_v1.h:13-15 (kernels/paged_attn_v1.cu:112-159).
 * q [B,H,D] f32|f16|bf16; k/v [NB,BS,HKV,D] f32|f16|bf16|f64; out [B,H,D] f32|f16|bf16. */
int paged_attention(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                    const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                    const pa_tensor_t* context_lens, double scale, void* stream);

/* Decode, online-softmax semantics.  Replaces paged_attention_v2(),
 * kernels/paged_attn_v2.h:13-15 (kernels/paged_attn_v2.cu:124-177). */
int paged_attention_v2(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                       const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                       const pa_tensor_t* context_lens, double scale, void* stream);

/* Decode with a FlashDecoding context split followed by a separate
 * log-sum-exp reduce kernel.  Replaces paged_attention_v3(),
 * kernels/paged_attn_v3.h:13-16 (kernels/paged_attn_v3.cu:192-261).
 * num_splits > 0: sequence b is cut into num_splits partitions
 *   [s*chunk, min((s+1)*chunk, ctx_b)), chunk = ceil(ctx_b / num_splits),
 *   exactly as kernels/paged_attn_v3.cu:65-68.
 * num_splits <= 0: the library plans fixed-size partitions from MB*BS, the
 *   batch size and the device's CU count (see pa_plan_partitions); when the
 *   batch alone fills the GPU no split and no reduce launch happen.
 * An explicit split into short partitions (at most 256 tokens at MB*BS),
 * with one query head per work-group head chunk (MHA, or odd GQA group
 * sizes above 8), whose one-work-group-per-(sequence, head) grid fills the GPU,
 * runs fused: one launch computes every partition and merges them by the
 * same rule in registers, and the workspace is not written.
 * workspace must be device memory of at least
 *   paged_attention_v3_workspace_size(...) bytes (NULL allowed when that is 0). */
int paged_attention_v3(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                       const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                       const pa_tensor_t* context_lens, double scale, int64_t num_splits,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes paged_attention_v3 needs for these arguments on the current
 * device (0 when no split is planned).  Returns (size_t)-1 on invalid arguments. */
size_t paged_attention_v3_workspace_size(const pa_tensor_t* q, const pa_tensor_t* k_cache,
                                         const pa_tensor_t* block_tables, int64_t num_splits);

/* The two launches paged_attention_v3 makes, exported for callers that time
 * or interleave them.  pa_v3_partition writes per-partition softmax state
 * into the workspace (or, for sequences that fit one partition, the final
 * output); pa_v3_reduce merges it.  Calling both back to back on one stream
 * computes what paged_attention_v3 computes: the same partitions and merge
 * rule (the one-call form may run them fused, as described there).
 * Workspace layout for a plan with P partitions per sequence:
 *   float acc[B][H][P][D]   un-normalised sum_j p_j v_j   (kernels/paged_attn_v3.cu:113-122)
 *   float m  [B][H][P]      running max, in log2 units (score * scale * log2 e)
 *   float l  [B][H][P]      sum_j p_j
 * An empty partition has m = -3e38 and l = 0 (kernels/paged_attn_v3.cu:76-77). */
int pa_v3_partition(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                    const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                    const pa_tensor_t* context_lens, double scale, int64_t num_splits,
                    void* workspace, size_t workspace_bytes, void* stream);
int pa_v3_reduce(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                 const pa_tensor_t* block_tables, const pa_tensor_t* context_lens,
                 int64_t num_splits, void* workspace, size_t workspace_bytes, void* stream);

/* Split count of the reference heuristic, kernels/paged_attn_v3.cu:170-190:
 *   clamp(max(max_context / 32, ceil(8 * CUs / (num_seqs * num_heads))), 1, 64)
 * with the current device's compute-unit count in place of the SM count.
 * Returns -1 (and sets pa_last_error) when no device can be queried. */
int64_t choose_num_splits(int64_t num_seqs, int64_t num_heads, int64_t max_context);

/* The same formula for an explicit compute-unit count; pure, needs no GPU. */
int64_t choose_num_splits_for(int64_t num_seqs, int64_t num_heads, int64_t max_context,
                              int64_t num_compute_units);

/* The partition plan paged_attention_v3 uses when num_splits <= 0, for an
 * explicit CU count; pure, needs no GPU.  Writes the partition length in
 * tokens and the number of partitions per sequence (1 = no split).  It
 * sees no cache layout: for MHA caches whose head rows are shorter than 128
 * bytes (served two heads per work-group) paged_attention_v3 plans with
 * num_kv_heads / 2 units; paged_attention_v3_workspace_size always matches
 * the call. */
int pa_plan_partitions(int64_t num_seqs, int64_t num_heads, int64_t num_kv_heads,
                       int64_t head_dim, int64_t max_context, int64_t num_compute_units,
                       int64_t* partition_tokens, int64_t* num_partitions);

/* Causal (chunked) prefill, fp32 arithmetic.  Replaces paged_attention_prefill(),
 * kernels/paged_attn_prefill.h:13-15 (kernels/paged_attn_prefill.cu:122-175).
 * Query s of sequence b sits at q_pos = ctx_b - S + s and attends keys
 * [0, q_pos]; q_pos < 0 gives a zero row (kernels/paged_attn_prefill.cu:62-74). */
int paged_attention_prefill(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                            const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                            const pa_tensor_t* context_lens, double scale, void* stream);

/* Causal (chunked) prefill on CDNA4 matrix cores.  Replaces
 * paged_attention_prefill_wmma(), kernels/paged_attn_wmma.h:13-15
 * (kernels/paged_attn_wmma.cu:212-274).  K/V fp16 (as the reference), bf16
 * or FP8 E4M3 (read as fp16, exactly); Q is rounded to the tile type (split
 * hi + lo when it arrives in another type), the probabilities to fp16 (bf16
 * hi + lo when a bf16 V value does not fit fp16), accumulation is fp32.
 * D in {32, 64, 128, 256}. */
int paged_attention_prefill_wmma(pa_tensor_t* out, const pa_tensor_t* q,
                                 const pa_tensor_t* k_cache, const pa_tensor_t* v_cache,
                                 const pa_tensor_t* block_tables,
                                 const pa_tensor_t* context_lens, double scale, void* stream);

/* paged_attention_v3 over a quantised KV cache: the cache holds K / k_scale
 * and V / v_scale (per-tensor scales, e.g. a float8_e4m3fn cache), and the
 * result is computed on K = k_cache * k_scale, V = v_cache * v_scale.  Any
 * decode KV type is accepted; with k_scale = v_scale = 1 it is
 * paged_attention_v3.  No reference counterpart: the reference has no FP8
 * cache (docs/REPORT.md:270 lists it as not done).  Scales must be finite
 * as float32, and so must scale * k_scale.  Workspace as for
 * paged_attention_v3 (same split plan). */
int paged_attention_v3_scaled(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                              const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                              const pa_tensor_t* context_lens, double scale, double k_scale, double v_scale,
                              int64_t num_splits, void* workspace, size_t workspace_bytes, void* stream);

/* paged_attention_v3 without a workspace and without any allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The split's partials go to a fixed device array of
 * PA_NOALLOC_SCRATCH_BYTES inside the library, one per GPU, held until the
 * process ends; a call whose split needs more (see
 * paged_attention_v3_workspace_size) fails with PA_ERR_WORKSPACE before any
 * device work.  Every call on a GPU shares that GPU's array: calls that
 * overlap on one GPU (different streams, or other threads) race, so
 * serialise them.  Same arguments, plan and results as paged_attention_v3. */
#define PA_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int paged_attention_v3_noalloc(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                               const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                               const pa_tensor_t* context_lens, double scale, int64_t num_splits,
                               void* stream);

/* paged_attention_prefill_wmma over a scaled cache (FP8 E4M3 pools written
 * by pa_write_kv_scaled): K holds k / k_scale and V holds v / v_scale, so
 * k_scale joins the softmax scale and v_scale multiplies the output rows.
 * No reference counterpart (the reference has no FP8 path,
 * docs/REPORT.md:270); the entry it extends is
 * kernels/paged_attn_wmma.h:13-15.  Scales must be finite as float32, and
 * so must scale * k_scale. */
int paged_attention_prefill_wmma_scaled(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                                        const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                                        const pa_tensor_t* context_lens, double scale, double k_scale,
                                        double v_scale, void* stream);

/* Variable-length (mixed decode + prefill) batches on the MFMA path.  The
 * reference's prefill takes q [B, S, H, D] with one S for every sequence
 * (kernels/paged_attn_prefill.cu:62-64 trailing-chunk semantics); here
 * sequence b brings q_len_b = cu_seqlens_q[b+1] - cu_seqlens_q[b] new tokens
 * (1 for a decode step, a chunk for prefill), packed in q/out [T, H, D]
 * from row cu_seqlens_q[b].  Row r of sequence b sits at position
 * context_lens[b] - q_len_b + r and attends keys [0, that position], as in
 * paged_attention_prefill_wmma.  cu_seqlens_q is int32 [B + 1] on the device;
 * max_q_len must bound every q_len_b (rows past it are not written).  A
 * sequence whose range is negative, decreasing or beyond T is skipped (its
 * rows are not written); nothing is read out of bounds.  Sequences of one
 * row are computed by the decode kernel and the others by the MFMA prefill
 * kernel: two launches on the stream, told apart on the device (no host
 * synchronisation). */
int paged_attention_prefill_varlen(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                                   const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                                   const pa_tensor_t* context_lens, const pa_tensor_t* cu_seqlens_q,
                                   int64_t max_q_len, double scale, void* stream);

/* paged_attention_prefill_varlen over a scaled cache (FP8 E4M3 pools written
 * by pa_write_kv_scaled): k_scale joins the softmax scale and v_scale
 * multiplies the output rows, in both kernels of the call.  No reference
 * counterpart (the reference has no FP8 path, docs/REPORT.md:270).  Scales
 * must be finite as float32, and so must scale * k_scale. */
int paged_attention_prefill_varlen_scaled(pa_tensor_t* out, const pa_tensor_t* q, const pa_tensor_t* k_cache,
                                          const pa_tensor_t* v_cache, const pa_tensor_t* block_tables,
                                          const pa_tensor_t* context_lens, const pa_tensor_t* cu_seqlens_q,
                                          int64_t max_q_len, double scale, double k_scale, double v_scale,
                                          void* stream);

/* KV-cache write ("reshape and cache"): token t's K and V rows, key[t] and
 * value[t] ([T, HKV, D], any non-negative token/head strides, 16-byte aligned
 * rows), go to block slot_mapping[t] / BS, row slot_mapping[t] % BS of
 * k_cache / v_cache ([NB, BS, HKV, D] views, as the attention entry points
 * take them), converted to the cache's type with round-to-nearest-even.
 * A negative slot (padding) or one >= NB * BS is skipped.  slot_mapping is
 * int32 or int64; key/value are float32, float16 or bfloat16, the caches
 * float32, float16, bfloat16 or float8_e4m3fn (see pa_write_kv_scaled).
 * Replaces the reference engine's TorchBlockAllocator.write_kv (external to
 * the reference; its call sites are harness/repro_crash.py:52-58 and
 * results/c001-20260901-223111/bench_b64_c2048.txt:16-22): one sequence's
 * [n_head, ctx, head_dim] layer slice is a strided [T, HKV, D] key with
 * slot_mapping[t] = block_ids[t / BS] * BS + t % BS. */
int pa_write_kv(pa_tensor_t* k_cache, pa_tensor_t* v_cache, const pa_tensor_t* key,
                const pa_tensor_t* value, const pa_tensor_t* slot_mapping, void* stream);

/* pa_write_kv into a scaled cache: the cache receives key / k_scale and
 * value / v_scale (fp32 division, correctly rounded, then the cache type's
 * rounding), the quantised form paged_attention_v3_scaled reads back.  With
 * an FP8 E4M3 cache (also accepted by pa_write_kv, scale 1) each value is
 * rounded to nearest even and saturated at +-448 (infinities too), NaN is
 * stored as 0x7f.  Scales must be finite and nonzero as float32.  The reference has no
 * FP8 path (docs/REPORT.md:270); the engine's write it extends is the one
 * pa_write_kv replaces (harness/repro_crash.py:52-58). */
int pa_write_kv_scaled(pa_tensor_t* k_cache, pa_tensor_t* v_cache, const pa_tensor_t* key,
                       const pa_tensor_t* value, const pa_tensor_t* slot_mapping, double k_scale,
                       double v_scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PAGEDATTN_H_ */
