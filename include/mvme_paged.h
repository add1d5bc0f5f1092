/*
 * mvme_paged.h -- C ABI of the MI355X (gfx950) paged-attention library.
 *
 * One shared object, libmvme_paged.so, holds every hand-written HIP kernel of
 * the paged KV-cache hot path: the KV scatter (slot mapping, decode-batch and
 * contiguous-range variants), the block-table gather, GQA decode attention
 * with a split-K merge, and ragged chunked paged prefill on bf16/fp16 MFMA.
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers except where noted.  Tensors are
 *     contiguous row-major; the KV cache of one layer is
 *     [num_blocks, block_size, kv_heads, head_dim].
 *   - Metadata (tables, lengths, slots, offsets) is int64, matching the
 *     reference's contract.
 *   - `stream` is a hipStream_t passed as void* (0 = the null stream).
 *     Every kernel is launched on that stream; no entry point allocates,
 *     frees, synchronises or copies to the host, so calls are legal inside
 *     HIP graph capture.
 *   - Return value: MVME_OK, or an error code with a message readable through
 *     mvme_last_error() (thread-local, valid until the next failing call on
 *     the same thread).  Argument errors are detected before any launch.
 *   - Metadata *values* are not trusted blindly: out-of-range page ids and
 *     slots are treated as absent (skipped rows, -inf scores, zero output),
 *     never dereferenced.
 */
#ifndef MVME_PAGED_H
#define MVME_PAGED_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MVME_ABI_VERSION 2

/* Element types of the KV cache, queries and outputs (FP32: sampling logits only). */
enum mvme_dtype { MVME_FP16 = 0, MVME_BF16 = 1, MVME_FP32 = 2 };

/* Status codes. */
enum mvme_status { MVME_OK = 0, MVME_EINVAL = 1, MVME_ELAUNCH = 2, MVME_EWORKSPACE = 3 };

/* ABI version of the loaded library (MVME_ABI_VERSION at build time). */
int mvme_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* mvme_last_error(void);

/*
 * KV scatter through a slot mapping: for every t < tokens with
 * 0 <= slot_mapping[t] < num_blocks*block_size,
 *   key_cache row slot_mapping[t]   <- key row t
 *   value_cache row slot_mapping[t] <- value row t
 * where a row is kv_heads*head_dim elements.  Bit-exact byte copy.
 * key/value rows are `key_token_stride` / `value_token_stride` elements apart
 * (the [kv_heads, head_dim] part of each row must be contiguous).
 * Replaces: write_kv_cache_slots_cuda / kv_write_slots_kernel
 *   (mini_engine/kernels/csrc/data.cu:194-250), bound as
 *   extension.write_kv_cache_slots (csrc/bindings.cpp:220) and called from
 *   write_kv_cache_slots (mini_engine/kernels/data.py:84-130).
 */
int mvme_write_kv_cache_slots(void* key_cache, void* value_cache,
                              int64_t num_blocks, int64_t block_size,
                              int64_t kv_heads, int64_t head_dim,
                              const int64_t* slot_mapping,
                              const void* key, const void* value, int64_t tokens,
                              int64_t key_token_stride, int64_t value_token_stride,
                              int dtype, void* stream);

/*
 * Decode-step scatter of one token per sequence: for b < batch,
 *   pos = token_offsets[b]; page = block_tables[b, pos / block_size];
 *   slot = page*block_size + pos % block_size  (skipped if pos or page invalid)
 * Replaces: write_kv_cache_batch_cuda / kv_write_batch_kernel
 *   (mini_engine/kernels/csrc/data.cu:88-107, :175-192), bound as
 *   extension.write_kv_cache_batch (csrc/bindings.cpp:128-150, :215) and
 *   called from write_kv_cache_batch (mini_engine/kernels/data.py:67-81).
 */
int mvme_write_kv_cache_batch(void* key_cache, void* value_cache,
                              int64_t num_blocks, int64_t block_size,
                              int64_t kv_heads, int64_t head_dim,
                              const int64_t* block_tables, int64_t table_width,
                              const int64_t* token_offsets,
                              const void* key, const void* value, int64_t batch,
                              int dtype, void* stream);

/*
 * Contiguous-range write of one sequence: token t < tokens goes to logical
 * position token_offset + t through block_ids[num_ids].
 * Replaces: write_kv_cache_cuda / kv_write_kernel
 *   (mini_engine/kernels/csrc/data.cu:67-86, :165-173), bound as
 *   extension.write_kv_cache (csrc/bindings.cpp:98-126, :214) and called from
 *   write_kv_cache (mini_engine/kernels/data.py:39-64) and
 *   KVCachePool.write_cuda (mini_engine/cache/kv_cache.py:123-145).
 */
int mvme_write_kv_cache(void* key_cache, void* value_cache,
                        int64_t num_blocks, int64_t block_size,
                        int64_t kv_heads, int64_t head_dim,
                        const int64_t* block_ids, int64_t num_ids, int64_t token_offset,
                        const void* key, const void* value, int64_t tokens,
                        int dtype, void* stream);

/*
 * Block-table gather of the logical prefix [0, token_count) of one sequence
 * into dense [token_count, kv_heads, head_dim] outputs (rows whose page id is
 * out of range are zero-filled).  Bit-exact.
 * Replaces: KVCachePool.gather (mini_engine/cache/kv_cache.py:147-166), which
 * the reference implements with torch advanced indexing.
 */
int mvme_gather_kv_cache(void* key_out, void* value_out,
                         const void* key_cache, const void* value_cache,
                         int64_t num_blocks, int64_t block_size,
                         int64_t kv_heads, int64_t head_dim,
                         const int64_t* block_ids, int64_t num_ids, int64_t token_count,
                         int dtype, void* stream);

/*
 * Bytes of device workspace mvme_paged_attention needs for these shapes
 * (0 when no split-K merge is required).  Pure host function.
 * partition_tokens: 0 selects the library's plan; > 0 forces split-K
 * partitions of that many tokens; -1 forces the balanced walk when batch <=
 * 256 (every (sequence, kv head) unit laid end to end and cut into equal
 * shares of tokens, one per work-group, the units cut by a share boundary
 * merged from their pieces); larger batches, and other negative values,
 * take the library's plan.
 */
size_t mvme_paged_attention_workspace_size(int64_t batch, int64_t q_heads, int64_t kv_heads,
                                           int64_t head_dim, int64_t block_size,
                                           int64_t table_width, int64_t partition_tokens);

/*
 * GQA decode attention over block tables (one query token per sequence):
 *   out[b, h, :] = softmax(q[b,h,:] . K_b^T / sqrt(head_dim)) V_b
 * where K_b/V_b are the first context_lens[b] tokens of sequence b addressed
 * through block_tables[b, :] and kv head h / (q_heads / kv_heads).
 * Sequences with context_lens[b] <= 0 or beyond the table capacity produce
 * zeros; out-of-range pages are skipped.  fp32 accumulation, fp32 split-K
 * merge.  `workspace` must hold mvme_paged_attention_workspace_size(...)
 * bytes (may be NULL when that is 0), 16-byte aligned when the call takes
 * the balanced walk; partition_tokens as there.
 * Replaces: paged_attention_cuda, attention_vector128, attention_partition
 *   and merge_partitions (mini_engine/kernels/csrc/paged_attention.cu:52-280),
 *   bound as extension.paged_attention (csrc/bindings.cpp:152-184, :196-199)
 *   and called from paged_attention (mini_engine/kernels/paged.py:8-22).
 */
int mvme_paged_attention(void* out, const void* query,
                         const void* key_cache, const void* value_cache,
                         const int64_t* block_tables, const int64_t* context_lens,
                         int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                         int64_t num_blocks, int64_t block_size, int64_t table_width,
                         int64_t partition_tokens, int dtype,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * mvme_paged_attention without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Same arguments, kernels and results as mvme_paged_attention; the split-K
 * partials go to a fixed 8 MiB scratch array that the library holds on each
 * device until the process ends, so the call allocates nothing.  Calls whose
 * plan needs more scratch than 8 MiB (mvme_paged_attention_workspace_size
 * above 8388608) fail with MVME_EWORKSPACE before any launch.
 * The first call on a device resolves the scratch address there (make it
 * outside graph capture).  Every call on one device shares that device's
 * scratch: calls that may overlap on one GPU (different streams without an
 * ordering between them) race and must not be issued.
 */
int mvme_paged_attention_noalloc(void* out, const void* query,
                                 const void* key_cache, const void* value_cache,
                                 const int64_t* block_tables, const int64_t* context_lens,
                                 int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                 int64_t num_blocks, int64_t block_size, int64_t table_width,
                                 int64_t partition_tokens, int dtype, void* stream);

/*
 * The decode step's KV write and paged attention in one launch.  Before
 * attention, every sequence b's new token -- at position context_lens[b] - 1
 * -- is written into the cache:
 *   q_weight == NULL: key_cache / value_cache row = new_key / new_value row
 *     (the decode-batch KV write), and `query` is the attention query
 *     ([batch, q_heads, head_dim], contiguous);
 *   q_weight != NULL: the K row is rope(rmsnorm(new_key, k_weight), cos, sin)
 *     and the V row new_value, and the attention query is
 *     rope(rmsnorm(query, q_weight), cos, sin) of the raw query rows
 *     (query_token_stride elements apart); the rotated queries also go to
 *     q_out ([batch, q_heads, head_dim]) when it is not NULL; q_out must
 *     not overlap the raw query rows (MVME_EINVAL: every work-group reads
 *     them while the first writes q_out; rotate in place with
 *     mvme_qk_norm_rope_write_kv instead).  cos / sin are
 *     [batch, head_dim / 2] at each sequence's position; eps the RMSNorm eps.
 * Then attention over context_lens[b] tokens exactly as mvme_paged_attention
 * (same workspace).  Results equal the two-launch sequence
 * (mvme_write_kv_cache_batch, or mvme_qk_norm_rope_write_kv in decode mode,
 * then mvme_paged_attention) bit for bit: the norm/RoPE arithmetic is the
 * same code.  A new token whose page is absent or out of range is not
 * written.  new_key / new_value are [batch, kv_heads, head_dim] rows,
 * key_token_stride / value_token_stride elements apart.  head_dim 16, 32,
 * 64, 128 or 256; every row 16-byte aligned.
 * Fuses what the reference runs as separate launches in
 * Attention.forward_decode_batch (mini_engine/model/native_qwen3.py:179-197):
 * q/k RMSNorm (elementwise.cu norm kernel), RoPE (data.cu:29-65), the batch
 * KV write (data.cu:88-107) and paged_attention (paged_attention.cu:52-280).
 * No single counterpart in the reference.
 */
int mvme_paged_attention_decode_write(void* out, const void* query, void* key_cache, void* value_cache,
                                      const int64_t* block_tables, const int64_t* context_lens,
                                      int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                      int64_t num_blocks, int64_t block_size, int64_t table_width,
                                      int64_t partition_tokens, int dtype,
                                      const void* new_key, const void* new_value,
                                      int64_t key_token_stride, int64_t value_token_stride,
                                      const void* q_weight, const void* k_weight,
                                      const void* cos, const void* sin, float eps,
                                      int64_t query_token_stride, void* q_out,
                                      void* workspace, size_t workspace_bytes, void* stream);

/*
 * Bytes of device workspace mvme_paged_prefill_attention needs for these
 * shapes and element type (0 when no query block is split over key chunks).
 * Pure host function.  chunk_tokens: 0 selects the library's default key
 * chunking.  Layout: the key-chunk partial outputs (rows 128 wide for
 * head_dim <= 128, 256 wide for 256; 2-byte elements for MVME_BF16, 4-byte
 * for MVME_FP16), their fp32 (reference, sum) pairs, and one int per packed
 * token.
 */
size_t mvme_paged_prefill_workspace_size(int64_t num_seqs, int64_t total_tokens, int64_t q_heads,
                                         int64_t kv_heads, int64_t head_dim, int64_t block_size,
                                         int64_t table_width, int64_t chunk_tokens, int dtype);

/*
 * Ragged chunked paged prefill: packed queries q[total_tokens, q_heads,
 * head_dim]; sequence s owns rows [cu_seqlens_q[s], cu_seqlens_q[s+1]), whose
 * i-th row sits at absolute position query_starts[s] + i and attends keys
 * [0, query_starts[s] + i] of that sequence through block_tables[s, :]
 * (causal inside the chunk).  context_lens[s] = query_starts[s] + rows(s).
 * Rows whose position is inconsistent with the metadata produce zeros.
 * Long contexts are split over key chunks of `chunk_tokens` keys (0 = library
 * default) whose fp32 partials live in `workspace`, which must hold
 * mvme_paged_prefill_workspace_size(...) bytes (may be NULL when that is 0).
 * Replaces: paged_prefill_attention_cuda / paged_prefill_kernel
 *   (mini_engine/kernels/csrc/prefill.cu:106-240), bound as
 *   extension.paged_prefill_attention (csrc/bindings.cpp:219) and called from
 *   paged_prefill_attention (mini_engine/kernels/prefill.py:61-131).
 */
int mvme_paged_prefill_attention(void* out, const void* q,
                                 const void* key_cache, const void* value_cache,
                                 const int64_t* cu_seqlens_q, const int64_t* query_starts,
                                 const int64_t* block_tables, const int64_t* context_lens,
                                 int64_t num_seqs, int64_t total_tokens,
                                 int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                 int64_t num_blocks, int64_t block_size, int64_t table_width,
                                 int64_t chunk_tokens, int dtype,
                                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * Bytes of device workspace mvme_prefill_attention needs (0 when no query
 * block is split over key chunks); 0 also for shapes it rejects.  Pure host
 * function.  Same layout as mvme_paged_prefill_workspace_size.
 */
size_t mvme_prefill_attention_workspace_size(int64_t batch, int64_t q_tokens, int64_t q_heads,
                                             int64_t kv_heads, int64_t head_dim, int64_t query_start,
                                             int dtype);

/*
 * Dense causal suffix attention: q [batch, q_heads, q_tokens, head_dim], key /
 * value [batch, kv_heads, kv_tokens, head_dim] (the same strides), output
 * [batch, q_heads, q_tokens, head_dim].  Query row t of batch entry b and
 * head h attends keys [0, query_start + t] of entry b and kv head
 * h / (q_heads / kv_heads); 0 <= query_start, query_start + q_tokens <=
 * kv_tokens, query_start + q_tokens <= 1,048,576.  Strides are in elements
 * (batch, head, token; the head_dim dimension is dense), so views such as
 * the transposes of [tokens, heads, head_dim] tensors need no copy.  For
 * head dims that are multiples of 8 up to 256 (the MFMA path) every pointer
 * must be 16-byte aligned and every stride a multiple of 8 elements; other
 * head dims (up to 1024) need 2-byte alignment.  The output's elements must
 * be distinct (no stride 0 over more than one element, no interleaved
 * dimensions); inputs may overlap.  workspace: at least
 * mvme_prefill_attention_workspace_size(...) bytes (may be NULL when 0).
 * Runs the paged prefill kernels with each batch entry as one sequence whose
 * keys are a single page.
 * Replaces: causal_prefill_suffix_cuda / causal_prefill_kernel
 *   (mini_engine/kernels/csrc/prefill.cu:15-98), bound as
 *   extension.causal_prefill_suffix and causal_prefill
 *   (csrc/bindings.cpp:217-218) and called from prefill_attention
 *   (mini_engine/kernels/prefill.py:8-41, backend "cuda").
 */
int mvme_prefill_attention(void* out, const void* q, const void* key, const void* value,
                           int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t q_tokens,
                           int64_t kv_tokens, int64_t head_dim, int64_t query_start,
                           int64_t q_batch_stride, int64_t q_head_stride, int64_t q_token_stride,
                           int64_t kv_batch_stride, int64_t kv_head_stride, int64_t kv_token_stride,
                           int64_t out_batch_stride, int64_t out_head_stride, int64_t out_token_stride,
                           int dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Fused per-head q/k RMSNorm + rotary embedding + KV page write (the step
 * before paged attention).  For every token t:
 *   q_out[t, h]             = rope(rmsnorm(q[t, h], q_weight))  (h < q_heads)
 *   key_cache[slot(t), h]   = rope(rmsnorm(k[t, h], k_weight))  (h < kv_heads)
 *   value_cache[slot(t), h] = v[t, h]                           (bit-exact)
 * rmsnorm(x, w) = T(T(x / sqrt(mean(x^2) + eps)) * w); rope rotates the halves
 * [0, D/2) and [D/2, D) with cos[t, :], sin[t, :] ([tokens, head_dim/2]),
 * rounding each product to fp16/bf16 before the add/subtract (the eager
 * rounding the reference matches).  slot(t) = slot_mapping[t] when
 * slot_mapping is non-null (prefill), else page*block_size + pos%block_size
 * with pos = positions[t] and page = block_tables[t, pos/block_size]
 * (decode, one token per sequence).  Tokens with an invalid slot still get
 * q_out and skip the cache write.  q/k/v rows are `*_token_stride` elements
 * apart (slices of a fused QKV projection); their [heads, head_dim] part is
 * dense.  head_dim even and <= 512.
 * Replaces the sequence q_norm / k_norm (RMSNorm, mini_engine/kernels/
 *   elementwise.py:16-21 -> csrc/elementwise.cu norm_kernel, bindings.cpp:63-66),
 *   apply_rope (kernels/data.py:27-36 -> csrc/data.cu:29-65, bindings.cpp:96-108)
 *   and write_kv_cache_slots / write_kv_cache_batch (data.py:84-130, :67-81)
 *   that Attention._forward_prefill_batch and forward_decode_batch run
 *   (mini_engine/model/native_qwen3.py:150-157, :179-191): one launch instead
 *   of four.
 */
int mvme_qk_norm_rope_write_kv(void* q_out, void* key_cache, void* value_cache,
                               int64_t num_blocks, int64_t block_size,
                               int64_t kv_heads, int64_t head_dim,
                               const int64_t* slot_mapping,
                               const int64_t* block_tables, int64_t table_width,
                               const int64_t* positions,
                               const void* q, const void* k, const void* v,
                               int64_t q_token_stride, int64_t k_token_stride,
                               int64_t v_token_stride,
                               const void* q_weight, const void* k_weight,
                               const void* cos, const void* sin,
                               int64_t tokens, int64_t q_heads, float eps,
                               int dtype, void* stream);

/*
 * Bytes of device workspace mvme_greedy_argmax needs (0 when every row is
 * reduced by one work-group).  Pure host function.
 */
size_t mvme_greedy_argmax_workspace_size(int64_t batch, int64_t vocab);

/*
 * Greedy sampling: out[b] = argmax over v < vocab of logits[b * row_stride + v]
 * for b < batch (<= 65535), with torch.argmax's ranking (largest value; ties
 * and NaNs resolve to the lowest index, NaN above every number).  dtype:
 * MVME_FP16, MVME_BF16 or MVME_FP32.  `workspace` (8-byte aligned) holds
 * mvme_greedy_argmax_workspace_size(batch, vocab) bytes of per-slice partial
 * results.  batch = 0 is a no-op.
 * Replaces: greedy_argmax_cuda / partial_argmax + final_argmax
 *   (mini_engine/kernels/csrc/sampling.cu:1-68), bound as
 *   extension.greedy_argmax (csrc/bindings.cpp:186-193) and called from
 *   sample_next_token(..., backend="cuda") (mini_engine/sampling.py:4-17).
 */
int mvme_greedy_argmax(int64_t* out, const void* logits, int64_t batch, int64_t vocab,
                       int64_t row_stride, int dtype, void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * Linear layer for at most 64 rows (the decode batch): out[m, n] =
 * sum_k x[m * x_row_stride + k] * weight[n * in_features + k] (+ bias[n]),
 * weight in nn.Linear's [out_features, in_features] layout, fp32
 * accumulation, one rounding to dtype (MVME_FP16 / MVME_BF16).
 * in_features a multiple of 32, out_features a multiple of 16, x and weight
 * 16-byte aligned, out 8-byte aligned; rows = 0 is a no-op.  No workspace.
 * Replaces, for rows <= 64: CudaLinear.forward's torch.mm(x, weight.t())
 *   (mini_engine/kernels/linear.py:14-30), the attention output projection
 *   of the decode step (self.o_proj, mini_engine/model/native_qwen3.py:197).
 */
int mvme_linear_rows(void* out, const void* x, const void* weight, const void* bias, int64_t rows,
                     int64_t in_features, int64_t out_features, int64_t x_row_stride, int dtype,
                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MVME_PAGED_H */
