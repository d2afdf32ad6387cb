/*
 * aicas_decode.h — C ABI of libaicas_decode.so: KV-cache append and q_len=1 GQA decode attention for
 * AMD Instinct MI355X (gfx950).
 *
 * Every entry point takes raw device pointers, element strides and an hipStream_t, and enqueues its work
 * on that stream without any host synchronisation or device allocation, so the calls can be captured in a
 * HIP graph. Return value: 0 on success, a nonzero AICAS_ERR_* code otherwise; aicas_last_error() then
 * returns a message for the calling thread.
 *
 * Reference interfaces these entry points replace (paths relative to the Frun1na/AICAS tree; the
 * transformers paths are transformers 5.15.0):
 *   aicas_kv_append         <- DynamicLayer.update, transformers/cache_utils.py:127-146 (torch.cat append),
 *                              called from Cache.update, transformers/cache_utils.py:1349-1381;
 *                              InplaceDecodeCacheLayer.update, dujunbaoV1/evaluation_wrapper.py:84-100;
 *                              GraphDecodeCacheLayer.update, dujunbaoV1/evaluation_wrapper.py:162-175;
 *                              _append_to_paged_kv_cache, new KV cache/evaluation_wrapper.py:143-195
 *                              (paged layout; fp8 e4m3 replaces the KIVI 2-bit codec).
 *   aicas_decode_attention  <- _gqa_decode_attention_forward / _gqa_decode_attention_fwd,
 *                              triton_qwen3vl/gqa_decode_attention.py:268-327 and :46-141;
 *                              decode_q1_gqa_forward, dujunbaoV1/native_cuda_ops/decode_q1_gqa.cpp:73-95;
 *                              _paged_kv_attention, new KV cache/evaluation_wrapper.py:248-265.
 *   aicas_kv_gather         <- _gather_paged_kv_cache, new KV cache/evaluation_wrapper.py:198-245 (the paged,
 *                              quantised cache dequantised into dense rows for a prefill's attention, called at
 *                              :428-453).
 *   aicas_decode_plan       <- the launch-configuration choice, triton_qwen3vl/gqa_decode_attention.py:287-292.
 *   aicas_last_error        <- the ValueError / TORCH_CHECK messages, gqa_decode_attention.py:282 and
 *                              decode_q1_gqa.cpp:65-92.
 */
#ifndef AICAS_DECODE_H
#define AICAS_DECODE_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AICAS_ABI_VERSION 7

/* Element types. */
#define AICAS_DTYPE_BF16 0
#define AICAS_DTYPE_FP16 1
#define AICAS_DTYPE_FP8_E4M3 2 /* OCP e4m3 ("e4m3fn"), one fp32 scale per (token, kv head) */

/* Return codes. */
#define AICAS_OK 0
#define AICAS_ERR_INVALID 1     /* null pointer, bad size, misaligned pointer or stride */
#define AICAS_ERR_UNSUPPORTED 2 /* head_dim / group size / dtype combination not built */
#define AICAS_ERR_WORKSPACE 3   /* workspace smaller than aicas_decode_plan asked for */
#define AICAS_ERR_LAUNCH 4      /* the HIP runtime rejected the launch */

/* Bits a kernel ORs into the optional device status word when it clamped instead of faulting. */
#define AICAS_STATUS_LEN_CLAMPED 1
#define AICAS_STATUS_BLOCK_OUT_OF_RANGE 2
#define AICAS_STATUS_APPEND_OVERFLOW 4
#define AICAS_STATUS_OUT_OF_BLOCKS 8
#define AICAS_STATUS_NONFINITE_ROW 16 /* an fp8 cache received a row holding NaN or +-Inf: stored poisoned */

/*
 * A KV cache. Two layouts share one description:
 *  - contiguous: K and V are [B, Hkv, capacity, D] (any element strides that keep rows 16-byte aligned,
 *    head_dim stride 1); block_table = NULL, page_size = capacity, num_blocks = B and stride_blk is the batch
 *    stride. HF's [B, Hkv, L, D] tensors and views into a preallocated buffer both fit.
 *  - paged: K and V are pools [num_blocks, Hkv, page_size, D]; block_table is [B, block_table_stride] int32
 *    physical block ids; token t of sequence b lives in block block_table[b][t / page_size], row
 *    t % page_size. page_size must be a power of two.
 * For AICAS_DTYPE_FP8_E4M3, k_scale / v_scale hold one fp32 per (block, head, row):
 * scale index = blk * scale_stride_blk + h * scale_stride_h + row. Dequantised value = code * scale.
 */
typedef struct aicas_kv_cache {
  void* k;
  void* v;
  float* k_scale;
  float* v_scale;
  const int32_t* block_table;
  int64_t block_table_stride;
  int64_t num_blocks;
  int64_t stride_blk;
  int64_t stride_h;
  int64_t stride_t;
  int64_t scale_stride_blk;
  int64_t scale_stride_h;
  int32_t page_size;
  int32_t kv_dtype;
} aicas_kv_cache_t;

/*
 * Append n_new tokens per sequence: rows k_src[b, h, j, :] / v_src[b, h, j, :] (src_dtype bf16 or fp16,
 * head_dim stride 1, strides in elements) go to token position positions[b] + j of sequence b. A 16-bit
 * cache must have kv_dtype == src_dtype and receives the rows bit for bit; an fp8 cache receives
 * e4m3(clamp(x / s, -448, 448)) with s = max|row| / 448 stored in k_scale / v_scale (s = 0 and all-zero
 * codes for an all-zero row; a row holding any NaN or +-Inf is stored poisoned, s = NaN and all-zero codes, so
 * that it dequantises to NaN, and AICAS_STATUS_NONFINITE_ROW is set). If seq_lens_out is not NULL,
 * seq_lens_out[b] = positions[b] + n_new is written after the rows; it may alias positions. A row whose
 * position falls outside the cache is dropped and AICAS_STATUS_APPEND_OVERFLOW is ORed into *status (status may
 * be NULL). batch <= 65535 and 2 * num_kv_heads * n_new < 2^31; the head and token strides of k_src / v_src and
 * the cache's stride_blk, stride_h, stride_t and scale strides must lie in [0, 2^32) elements (the batch strides
 * of k_src / v_src are unrestricted); otherwise AICAS_ERR_UNSUPPORTED. A decode step's append is one launch; a
 * prefill-sized one (a prompt written into the cache) spreads each sequence's rows over many workgroups and
 * bumps the lengths in a second, one-thread-per-sequence launch.
 * Replaces: transformers/cache_utils.py:127-146; dujunbaoV1/evaluation_wrapper.py:84-100, :162-175;
 * new KV cache/evaluation_wrapper.py:143-195.
 */
int aicas_kv_append(const aicas_kv_cache_t* cache, int32_t src_dtype, const void* k_src, int64_t k_stride_b,
                    int64_t k_stride_h, int64_t k_stride_t, const void* v_src, int64_t v_stride_b,
                    int64_t v_stride_h, int64_t v_stride_t, const int32_t* positions, int32_t* seq_lens_out,
                    int32_t* status, int32_t batch, int32_t num_kv_heads, int32_t head_dim, int32_t n_new,
                    hipStream_t stream);

/*
 * The first seq_lens[b] tokens of every (batch row b, kv head h) of the cache as dense rows: k_out[b, h, t, :] and
 * v_out[b, h, t, :] for t < out_len (element strides out_stride_b / _h / _t, head_dim stride 1; out_dtype bf16 or
 * fp16), rows at or past seq_lens[b] zero. A 16-bit cache is copied bit for bit (out_dtype must be its dtype); an
 * fp8 cache comes out as code * scale computed in fp32 and rounded to out_dtype once (nearest even; a poisoned
 * row, scale NaN, comes out NaN). Lengths beyond the cache are clamped (AICAS_STATUS_LEN_CLAMPED), invalid block
 * ids give zero rows (AICAS_STATUS_BLOCK_OUT_OF_RANGE); status may be NULL. The outputs may overlap neither each
 * other nor the cache. What a prefill's attention reads from a paged or fp8 cache: the rows the decode kernel
 * attends to, in the layout other attention backends take.
 * Replaces: _gather_paged_kv_cache, new KV cache/evaluation_wrapper.py:198-245.
 */
int aicas_kv_gather(const aicas_kv_cache_t* cache, const int32_t* seq_lens, int32_t batch, int32_t num_kv_heads,
                    int32_t head_dim, int32_t out_dtype, void* k_out, void* v_out, int64_t out_stride_b,
                    int64_t out_stride_h, int64_t out_stride_t, int32_t out_len, int32_t* status,
                    hipStream_t stream);

/*
 * Launch plan for aicas_decode_attention: the split size (tokens_per_split_hint, or 0 to choose automatically)
 * and split count — a sequence of L tokens is spread over min(num_splits, ceil(L / tokens_per_split)) splits —
 * and the workspace size in bytes. With few (batch row, kv head) pairs the automatic plan keeps its split count
 * whatever max_seq_len is, once sequences are long enough, so a launch sized for a loose bound (a graph captured
 * at the cache capacity) runs the grid a tight bound gives. A launch plans itself from the same arguments. The
 * workspace starts with 512 KiB of counters at fixed offsets, followed by the split partials; it must be
 * zero-filled once when first allocated, and the kernels leave the counters at zero after every launch, so
 * launches of any shapes may share one workspace in turn. Two launches that may run concurrently need two
 * workspaces. batch * num_kv_heads may not exceed 65536.
 * Replaces: triton_qwen3vl/gqa_decode_attention.py:287-292 (block size / warps choice).
 */
int aicas_decode_plan(int32_t kv_dtype, int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                      int32_t head_dim, int32_t max_seq_len, int32_t page_size, int32_t tokens_per_split_hint,
                      int32_t* tokens_per_split, int32_t* num_splits, size_t* workspace_bytes);

/*
 * out[b, hq, :] = softmax(q[b, hq, :] . K[b, hq / G, t, :] * sm_scale over t < L_b) . V[b, hq / G, t, :],
 * G = num_q_heads / num_kv_heads, L_b = seq_lens[b] (or uniform_len when seq_lens is NULL).
 * q and out are [B, Hq, D] with element strides (head_dim stride 1) in q_dtype (bf16 or fp16); a 16-bit
 * cache must have kv_dtype == q_dtype. max_seq_len sizes the launch (plan and workspace); a longer L_b is still
 * attended in full while the cache holds it (paged caches: up to the plan's per-split block-table limit, at least
 * max_seq_len), and clamped beyond that, with AICAS_STATUS_LEN_CLAMPED set. An empty sequence (L_b == 0) yields
 * zeros. head_dim in {16, 32, 64, 128},
 * G in {1, 2, 4, 8}. tokens_per_split as from aicas_decode_plan (0 = automatic). min_len is a lower bound on every
 * L_b that the caller may pass (0 if unknown): when it keeps every split of a contiguous cache busy, the launch
 * fetches its first rows before reading the lengths. Results never depend on it; a wrong bound costs bandwidth.
 * Replaces: triton_qwen3vl/gqa_decode_attention.py:46-141, :268-327; dujunbaoV1/native_cuda_ops/
 * decode_q1_gqa.cpp:73-95; new KV cache/evaluation_wrapper.py:248-265.
 */
int aicas_decode_attention(const aicas_kv_cache_t* cache, int32_t q_dtype, const void* q, int64_t q_stride_b,
                           int64_t q_stride_h, void* out, int64_t out_stride_b, int64_t out_stride_h,
                           const int32_t* seq_lens, int32_t uniform_len, int32_t min_len, int32_t max_seq_len,
                           int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                           float sm_scale, int32_t tokens_per_split, void* workspace, size_t workspace_bytes,
                           int32_t* status, hipStream_t stream);

/*
 * One decode step of append + attend in a single launch: for every sequence b the new rows
 * k_new[b, h, :] / v_new[b, h, :] ([B, Hkv, D], head_dim stride 1, dtype q_dtype) are written at token
 * positions[b] of the cache exactly as aicas_kv_append would write them (fp8 caches quantize on write), and
 * the attention runs over L_b = positions[b] + 1 tokens, the new one included, with the result
 * aicas_kv_append followed by aicas_decode_attention would give. If seq_lens_out is not NULL,
 * seq_lens_out[b] = positions[b] + 1 is stored once every workgroup has read positions[b]; it may be
 * positions itself, but no other overlap with positions is accepted (AICAS_ERR_INVALID). max_seq_len must bound positions[b] + 1; min_len (0 if unknown) is a lower bound on every
 * positions[b], used as by aicas_decode_attention. A token with no slot left in the cache is dropped and
 * AICAS_STATUS_APPEND_OVERFLOW is set. The workspace must come from aicas_decode_plan with the same shapes.
 * Replaces the pair Qwen3VLTextAttention.forward issues per layer and step
 * (transformers/models/qwen3_vl/modeling_qwen3_vl.py:487-503): past_key_values.update (cache_utils.py:127-146)
 * followed by the text attention function (triton_qwen3vl/backends.py:207-227).
 */
int aicas_decode_attention_append(const aicas_kv_cache_t* cache, int32_t q_dtype, const void* q,
                                  int64_t q_stride_b, int64_t q_stride_h, const void* k_new, int64_t k_stride_b,
                                  int64_t k_stride_h, const void* v_new, int64_t v_stride_b, int64_t v_stride_h,
                                  void* out, int64_t out_stride_b, int64_t out_stride_h, const int32_t* positions,
                                  int32_t* seq_lens_out, int32_t min_len, int32_t max_seq_len, int32_t batch,
                                  int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float sm_scale,
                                  int32_t tokens_per_split, void* workspace, size_t workspace_bytes, int32_t* status,
                                  hipStream_t stream);

/*
 * aicas_decode_attention_append without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. Same arguments, results and status bits as aicas_decode_attention_append; the split partials and
 * counters live in a 4 MiB static scratch array of the library, one per device, which each device holds until
 * the process ends. The entry point calls no allocator. A launch whose workspace (aicas_decode_plan's
 * workspace_bytes) exceeds 4 MiB is rejected with AICAS_ERR_WORKSPACE before anything is enqueued. Every call
 * on a device shares that device's scratch: calls that may overlap on one device (two streams, or two host
 * threads) race and must be serialised by the caller. The first call on a device also enqueues, on `stream`,
 * one small kernel that clears the scratch.
 */
int aicas_decode_attention_append_noalloc(const aicas_kv_cache_t* cache, int32_t q_dtype, const void* q,
                                          int64_t q_stride_b, int64_t q_stride_h, const void* k_new,
                                          int64_t k_stride_b, int64_t k_stride_h, const void* v_new,
                                          int64_t v_stride_b, int64_t v_stride_h, void* out, int64_t out_stride_b,
                                          int64_t out_stride_h, const int32_t* positions, int32_t* seq_lens_out,
                                          int32_t min_len, int32_t max_seq_len, int32_t batch, int32_t num_q_heads,
                                          int32_t num_kv_heads, int32_t head_dim, float sm_scale,
                                          int32_t tokens_per_split, int32_t* status, hipStream_t stream);

/*
 * The model's q/k preparation, fused into aicas_decode_attention_append_qk. Every pointer may be NULL (that
 * step is skipped); element types are q_dtype's, head_dim strides 1.
 *   q_norm_weight, k_norm_weight  [head_dim]: RMSNorm over head_dim of q and of the new K rows: x / sqrt(
 *                                 mean(x^2) + eps) in fp32, rounded to q_dtype, times the weight, rounded;
 *   cos, sin                      [B, head_dim] rows (strides cos_stride_b / sin_stride_b elements, multiples
 *                                 of 8): rotary embedding x * cos + rotate_half(x) * sin, rotate_half(x) =
 *                                 (-x[D/2:], x[:D/2]), each product and the sum rounded to q_dtype;
 *   q_out                         [B, Hq, head_dim] (strides in elements, multiples of 8): receives q as
 *                                 prepared, once every workgroup has read q; it may be q itself (same
 *                                 pointer and strides), but may not otherwise overlap q or k_new.
 * Pointers are 16-byte aligned.
 */
typedef struct aicas_qk_prologue {
  const void* q_norm_weight;
  const void* k_norm_weight;
  float eps;
  const void* cos;
  const void* sin;
  int64_t cos_stride_b;
  int64_t sin_stride_b;
  void* q_out;
  int64_t q_out_stride_b;
  int64_t q_out_stride_h;
} aicas_qk_prologue_t;

/*
 * aicas_decode_attention_append with the model's q/k preparation done in the same launch: q (the query
 * projection's output) and k_new (the key projection's output) are RMS-normalised and rotated as the
 * prologue says before the rows are written and attended to; v_new is written as given. One launch per layer
 * and decode step in place of the q/k norms, the rotary embedding, the cache update and the attention.
 * Replaces: transformers/models/qwen3_vl/modeling_qwen3_vl.py:481-488 (q_norm, k_norm,
 * apply_rotary_pos_emb, past_key_values.update) followed by the text attention function
 * (triton_qwen3vl/backends.py:207-227); the same fused step as dujunbaoV1/native_cuda_ops/
 * decode_q1_gqa_kernel.cu:376-480 plus the attention.
 */
int aicas_decode_attention_append_qk(const aicas_kv_cache_t* cache, const aicas_qk_prologue_t* prologue,
                                     int32_t q_dtype, const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                     const void* k_new, int64_t k_stride_b, int64_t k_stride_h, const void* v_new,
                                     int64_t v_stride_b, int64_t v_stride_h, void* out, int64_t out_stride_b,
                                     int64_t out_stride_h, const int32_t* positions, int32_t* seq_lens_out,
                                     int32_t min_len, int32_t max_seq_len, int32_t batch, int32_t num_q_heads,
                                     int32_t num_kv_heads, int32_t head_dim, float sm_scale, int32_t tokens_per_split,
                                     void* workspace, size_t workspace_bytes, int32_t* status, hipStream_t stream);

/* Message describing the last failure on the calling thread ("" if none). */
const char* aicas_last_error(void);

/*
 * Device block pool for paged caches: free block ids kept as a stack in device memory (free_blocks[0 ..
 * *free_count) are free, the top is the last), handed out to pages and taken back by kernels on the stream, so
 * that a decode step that needs a new page still involves no host synchronisation. The table is the int32
 * [batch, width] block table of aicas_kv_cache_t (-1: no block). Allocation and release run in sequence order
 * (sequence b's pages in page order), so the resulting table is reproducible.
 * Replaces: new KV cache/evaluation_wrapper.py:141-190 (the page table as a Python list of
 * {"logical_page_id", "block_id"} dicts, grown by list.append as pages fill), :198-232 (its walk) and
 * :502-521 (its reset).
 */
typedef struct aicas_block_pool {
  int32_t* free_blocks; /* [num_blocks] device */
  int32_t* free_count;  /* [1] device */
  int32_t num_blocks;
} aicas_block_pool_t;

/* Every block free: pops then hand out 0, 1, 2, ... */
int aicas_block_pool_init(const aicas_block_pool_t* pool, hipStream_t stream);

/*
 * Before appending n_new (>= 1) tokens at positions[b]: every page those tokens touch whose table entry is
 * negative gets the next free block. Pages past the row's width set AICAS_STATUS_APPEND_OVERFLOW; when the pool
 * runs out the entry stays -1 and AICAS_STATUS_OUT_OF_BLOCKS is set (the append then drops those rows).
 */
int aicas_block_alloc(const aicas_block_pool_t* pool, int32_t* block_table, int64_t block_table_stride,
                      int32_t table_width, const int32_t* positions, int32_t n_new, int32_t batch, int32_t page_size,
                      int32_t* status, hipStream_t stream);

/*
 * Every sequence with release[b] != 0 returns its blocks to the pool; its table row becomes -1 and, if seq_lens
 * is not NULL, seq_lens[b] = 0. Ids outside [0, num_blocks), and blocks that would overfill the pool (released
 * twice), are dropped and set AICAS_STATUS_BLOCK_OUT_OF_RANGE.
 */
int aicas_block_free(const aicas_block_pool_t* pool, int32_t* block_table, int64_t block_table_stride,
                     int32_t table_width, const int32_t* release, int32_t* seq_lens, int32_t batch, int32_t* status,
                     hipStream_t stream);

/* AICAS_ABI_VERSION of the loaded library. */
int32_t aicas_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* AICAS_DECODE_H */
