/*
 * C ABI of the MI355X (gfx950) paged-decode attention library.
 *
 * Every entry point takes plain device pointers, element strides and sizes, and
 * a HIP stream passed as `void*` (a hipStream_t; NULL means the default stream).
 * No function allocates device memory: split-K scratch is passed in by the
 * caller through `workspace`, sized by the matching *_workspace_bytes() call.
 * Every launch is asynchronous on the given stream; nothing synchronises the host.
 *
 * Workspace of pa_decode_batched_f16 / pa_decode_v2_f16: its first bytes hold
 * per-(sequence, kv-head group) arrival counters of the in-kernel merge of
 * split partitions. They must be zero before the first call that uses the
 * buffer (zero-fill it once after allocating); every call leaves them zero
 * again. Use one such buffer per stream (calls in flight on different streams
 * must not share one) and lend it to nothing else, pa_decode_v1_f16 included.
 *
 * Tensor layouts (element strides, fp16 = IEEE binary16):
 *   q        [num_seqs, num_q_heads, head_dim]            stride of head_dim must be 1
 *   k_cache  [num_blocks, block_size, num_kv_heads, head_dim]  (same for v_cache)
 *   block_tables [num_seqs, max_blocks_per_seq] int32, seq_lens [num_seqs] int32
 *   out      [num_seqs, num_q_heads, head_dim]
 * Query head h reads KV head h / (num_q_heads / num_kv_heads).
 *
 * Return value: PA_OK (0) on success, otherwise a PA_ERR_* code; the message is
 * available from pa_last_error() on the calling thread.
 */
#ifndef MI355X_PAGED_ATTENTION_H
#define MI355X_PAGED_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define PA_API __attribute__((visibility("default")))
#else
#define PA_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

enum {
  PA_OK = 0,
  PA_ERR_ARG = 1,          /* invalid argument: shapes, strides, alignment, null pointers */
  PA_ERR_UNSUPPORTED = 2,  /* valid but not compiled: head_dim / group size outside the built set */
  PA_ERR_WORKSPACE = 3,    /* workspace smaller than *_workspace_bytes() asked for */
  PA_ERR_HIP = 4           /* the HIP runtime reported an error at launch */
};

/* ABI revision of this header; bumps whenever a signature or a workspace
 * contract changes (2: zero-initialised decode workspace; 3: pa_rope_kv_write_f16;
 * 4: pa_prefill_attention_f16; 5: its workspace; 6: pa_rmsnorm_f16, pa_silu_mul_f16;
 * 7: residual input of pa_rmsnorm_f16, pa_top2_f16; 8: pa_linear_f16; 9: pa_linear_f16
 * removed, decode workspace sizes stated per current device; 10:
 * pa_decode_batched_noalloc_f16; 11: pa_decode_rope_batched_f16, decode workspace
 * with room for shared-prefix records; 12: pa_decode_batched_schedule; 13:
 * pa_decode_kv_write_batched_f16; 14: the decode workspace's head also holds the
 * schedule plan that pa_decode_kv_write_batched_f16's write launch leaves for its
 * attention launch, 8,448 bytes more). */
PA_API int pa_abi_version(void);

/* Message of the last failed call on this thread ("" after a success). */
PA_API const char* pa_last_error(void);

/*
 * The schedule pa_decode_batched_f16 picks for these sizes on the current
 * device, for a contiguous pool [num_blocks, block_size, num_kv_heads,
 * head_dim]; host only, no launch. No counterpart in the reference (its
 * Triton launch picks a tile size only, paged_attention.py:665-673); for
 * tests and tools that need to know which kernel path a shape takes.
 * info[0]: 0 stream-K ranges (decode_streamk_kernel), 1 one workgroup per
 * (sequence, kv-head group) pair (decode_pair_kernel), 2 fixed 512-token
 * splits (more than 1024 sequences); info[1]: kv heads per pair; info[2]:
 * workgroups of the launch; info[3]: 1 when the launch looks for shared
 * prefixes (prefix items), else 0.
 */
PA_API int pa_decode_batched_schedule(int num_seqs, int num_q_heads, int num_kv_heads,
                                      int head_dim, int block_size, int max_blocks_per_seq,
                                      int info[4]);

/*
 * Batched GQA paged decode attention, online softmax with split-K partitions.
 * Replaces paged_attention_decode_batched() and its Triton kernel,
 * engine/kernels/paged_attention.py:508-698 (argument meaning :634-663).
 * Tokens t < seq_lens[b] of sequence b are read from block
 * block_tables[b][t / block_size], row t % block_size. seq_lens[b] <= 0 gives
 * a zero output row; lengths beyond max_blocks_per_seq * block_size are clamped
 * to it, and block ids outside [0, num_blocks) are clamped into range, so a bad
 * table can give wrong numbers but never an out-of-bounds access.
 * out must not alias q, the caches or the workspace.
 */
PA_API int pa_decode_batched_f16(const void* q, const int64_t q_strides[3],
                          const void* k_cache, const int64_t k_strides[4],
                          const void* v_cache, const int64_t v_strides[4],
                          const int32_t* block_tables, const int64_t bt_strides[2],
                          const int32_t* seq_lens,
                          void* out, const int64_t out_strides[3],
                          int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                          int block_size, int num_blocks, int max_blocks_per_seq,
                          float scale, void* workspace, size_t workspace_bytes,
                          void* stream);

/*
 * The per-layer work of a decode step without the rotary embedding: the new
 * token's K/V write into its block followed by pa_decode_batched_f16. Replaces
 * the K/V write loop of paged_decode_attention_forward and the
 * paged_attention_decode_batched call after it
 * (engine/kernels/paged_attention_integration.py:148-161, :164-171). key and
 * value are [num_seqs, num_kv_heads, head_dim] rows with unit head_dim stride,
 * 8-element aligned strides and 16-byte aligned bases; row b is written to
 * position seq_lens[b] - 1 (block block_tables[b][(L-1) / block_size], row
 * (L-1) % block_size; skipped for L <= 0 or a slot outside the table or the
 * pool) and attended over with the other L - 1 tokens. The same results (the
 * same bits) as pa_kv_write_f16 followed by pa_decode_batched_f16 on the same
 * stream. One launch where the batch takes one workgroup per (sequence,
 * kv-head group) pair at head_dim 64 or 128 and block size 16 or 32 (the
 * decode step's shapes); otherwise those two launches, and where the batch
 * takes stream-K ranges at head_dim 64 or 128 and block size 16 or 32, the
 * write launch also derives the attention launch's schedule plan once (from
 * the same lengths and table rows) and leaves it in the workspace head, so
 * that no attention workgroup derives it again. Workspace: as for
 * pa_decode_batched_f16 (pa_decode_batched_workspace_bytes). As for every
 * fused write here, a slot whose block id lies outside the pool is not
 * written, and the one-launch form then attends over the new rows where the
 * two-launch form reads the clamped block's row (a malformed table either
 * way); no other sequence may read the written slot in the same call (the
 * reference refuses to write a block with more than one reference,
 * engine/kernels/paged_attention_integration.py:587-592).
 */
PA_API int pa_decode_kv_write_batched_f16(const void* q, const int64_t q_strides[3],
                                          const void* key, const int64_t key_strides[3],
                                          const void* value, const int64_t value_strides[3],
                                          void* k_cache, const int64_t k_strides[4],
                                          void* v_cache, const int64_t v_strides[4],
                                          const int32_t* block_tables,
                                          const int64_t bt_strides[2], const int32_t* seq_lens,
                                          void* out, const int64_t out_strides[3], int num_seqs,
                                          int num_q_heads, int num_kv_heads, int head_dim,
                                          int block_size, int num_blocks, int max_blocks_per_seq,
                                          float scale, void* workspace, size_t workspace_bytes,
                                          void* stream);

/* Workspace the call above needs for these sizes (0 is a valid answer), on the
 * current HIP device: the schedule, and so the size, depends on that device's
 * compute-unit count. Query it with the device of the call current. */
PA_API size_t pa_decode_batched_workspace_bytes(int num_seqs, int num_q_heads, int num_kv_heads,
                                         int head_dim, int block_size,
                                         int max_blocks_per_seq);

/*
 * Single-sequence online-softmax decode attention.
 * Replaces paged_attention_decode_v2(), engine/kernels/paged_attention.py:308-470.
 * q/out are [num_q_heads, head_dim]; block_table is a 1-D int32 array of
 * table_len entries with table_len >= ceil(seq_len / block_size)
 * (the reference asserts the same, :443-446). seq_len is a host integer.
 */
PA_API int pa_decode_v2_f16(const void* q, const int64_t q_strides[2],
                     const void* k_cache, const int64_t k_strides[4],
                     const void* v_cache, const int64_t v_strides[4],
                     const int32_t* block_table, int64_t bt_stride, int table_len,
                     int seq_len, void* out, const int64_t out_strides[2],
                     int num_q_heads, int num_kv_heads, int head_dim,
                     int block_size, int num_blocks, float scale,
                     void* workspace, size_t workspace_bytes, void* stream);

PA_API size_t pa_decode_v2_workspace_bytes(int num_q_heads, int num_kv_heads, int head_dim,
                                    int block_size, int table_len);

/*
 * Single-sequence two-pass decode attention: pass 1 the score maxima, a
 * denominator pass, pass 2 the normalised probability-weighted V sum.
 * Replaces paged_attention_decode_v1(), engine/kernels/paged_attention.py:102-305.
 * K is read once: scores are kept in the workspace between the passes.
 * Arguments as for pa_decode_v2_f16.
 */
PA_API int pa_decode_v1_f16(const void* q, const int64_t q_strides[2],
                     const void* k_cache, const int64_t k_strides[4],
                     const void* v_cache, const int64_t v_strides[4],
                     const int32_t* block_table, int64_t bt_stride, int table_len,
                     int seq_len, void* out, const int64_t out_strides[2],
                     int num_q_heads, int num_kv_heads, int head_dim,
                     int block_size, int num_blocks, float scale,
                     void* workspace, size_t workspace_bytes, void* stream);

PA_API size_t pa_decode_v1_workspace_bytes(int num_q_heads, int num_kv_heads, int head_dim,
                                    int block_size, int seq_len);

/*
 * Per-step K/V write: for each sequence b with L = seq_lens[b] (or
 * uniform_seq_len when seq_lens is NULL) and L >= 1, copies key[b, :, :] and
 * value[b, :, :] bit for bit into k_cache/v_cache at block
 * block_tables[b][(L-1) / block_size], row (L-1) % block_size, all kv heads.
 * Replaces the per-sequence index_put loop of paged_decode_attention_forward,
 * engine/kernels/paged_attention_integration.py:148-161 (single-sequence form
 * :120-133), which has no function of its own in the reference.
 * key/value are [num_seqs, num_kv_heads, head_dim] with any element strides.
 * Rows whose slot falls outside the table or whose block id is outside
 * [0, num_blocks) are skipped.
 */
PA_API int pa_kv_write_f16(const void* key, const int64_t key_strides[3],
                    const void* value, const int64_t value_strides[3],
                    void* k_cache, const int64_t k_strides[4],
                    void* v_cache, const int64_t v_strides[4],
                    const int32_t* block_tables, const int64_t bt_strides[2],
                    const int32_t* seq_lens, int uniform_seq_len,
                    int num_seqs, int num_kv_heads, int head_dim,
                    int block_size, int num_blocks, int max_blocks_per_seq,
                    void* stream);

/*
 * Prefill block copy: writes a prompt slice's K/V rows into whole cache blocks.
 * Source block j (slice tokens j*block_size .. j*block_size + block_size - 1)
 * goes to block block_ids[j]; rows at or past num_tokens are written as zeros.
 * Replaces the per-layer pad + index_copy_ of _copy_prefill_kv,
 * engine/kernels/paged_attention_integration.py:278-326. key/value are
 * [num_tokens, num_kv_heads, head_dim] with any element strides (the
 * permuted [Hkv, T, D] cache slice); block ids outside [0, num_blocks) are skipped.
 */
PA_API int pa_prefill_copy_f16(const void* key, const int64_t key_strides[3],
                        const void* value, const int64_t value_strides[3],
                        void* k_cache, const int64_t k_strides[4],
                        void* v_cache, const int64_t v_strides[4],
                        const int32_t* block_ids, int num_block_ids, int num_tokens,
                        int num_kv_heads, int head_dim, int block_size, int num_blocks,
                        void* stream);

/*
 * Fused rotary embedding and K/V write of one decode step. Replaces
 * transformers' apply_rotary_pos_emb on the new token's q and k (called by
 * paged_decode_attention_forward, engine/kernels/paged_attention_integration.py:108-109)
 * together with that function's K/V write loop (:148-161; single sequence :120-133).
 * q [num_seqs, num_q_heads, head_dim], key/value [num_seqs, num_kv_heads, head_dim]
 * (any element strides) and cos/sin [num_seqs, head_dim] (the per-sequence row
 * of the model's rotary table) are fp16. Writes
 *   q_out[b, h]        = rot(q[b, h])
 *   k_cache at slot    = rot(key[b, h]),  v_cache at slot = value[b, h]
 * where the slot of sequence b is block block_tables[b][(L-1) / block_size],
 * row (L-1) % block_size with L = seq_lens[b] (or uniform_seq_len when seq_lens
 * is NULL), and rot(x)[j] = x[j] cos[j] - x[j + D/2] sin[j],
 * rot(x)[j + D/2] = x[j + D/2] cos[j + D/2] + x[j] sin[j + D/2], every product and
 * sum rounded to fp16 as transformers computes it in fp16, so the results are
 * bit-identical to its apply_rotary_pos_emb. Rows whose slot is missing (L <= 0,
 * block outside the table or the pool) are not written.
 */
PA_API int pa_rope_kv_write_f16(const void* q, const int64_t q_strides[3], const void* key,
                                const int64_t key_strides[3], const void* value,
                                const int64_t value_strides[3], const void* cos,
                                const int64_t cos_strides[2], const void* sin,
                                const int64_t sin_strides[2], void* q_out,
                                const int64_t q_out_strides[3], void* k_cache,
                                const int64_t k_strides[4], void* v_cache,
                                const int64_t v_strides[4], const int32_t* block_tables,
                                const int64_t bt_strides[2], const int32_t* seq_lens,
                                int uniform_seq_len, int num_seqs, int num_q_heads,
                                int num_kv_heads, int head_dim, int block_size, int num_blocks,
                                int max_blocks_per_seq, void* stream);

/*
 * One decode step's attention block of a layer in one call: the rotary
 * embedding of the new token's q and key, the write of its rotated key and its
 * value into the pool, and batched decode attention over L_b tokens. Replaces
 * paged_decode_attention_forward's apply_rotary_pos_emb (engine/kernels/
 * paged_attention_integration.py:108-109), its K/V write loop (:148-161) and its
 * paged_attention_decode_batched call (:164-171). Results are the same bits as
 * pa_rope_kv_write_f16 (same arguments, its q_out) followed by
 * pa_decode_batched_f16 on the rotated queries; q, key, value, cos, sin, the
 * caches, tables and lengths are as for those two calls, out as for the second.
 * Batches that take one workgroup per (sequence, kv-head group) -- sequences x
 * kv heads within the GPU's compute units, short tables -- at head_dim 64 or
 * 128, block size 16 or 32, with 16-byte aligned unit-stride rows run as one
 * kernel launch (the new rows are written at the end of the launch; the
 * attention takes them from on-chip memory); all others as the two calls, with
 * the rotated queries in the workspace. Workspace: at least
 * pa_decode_rope_batched_workspace_bytes(), with the decode workspace's zeroed
 * counter region at its start (same contract as pa_decode_batched_f16).
 */
PA_API size_t pa_decode_rope_batched_workspace_bytes(int num_seqs, int num_q_heads,
                                                     int num_kv_heads, int head_dim,
                                                     int block_size, int max_blocks_per_seq);
PA_API int pa_decode_rope_batched_f16(const void* q, const int64_t q_strides[3], const void* key,
                                      const int64_t key_strides[3], const void* value,
                                      const int64_t value_strides[3], const void* cos,
                                      const int64_t cos_strides[2], const void* sin,
                                      const int64_t sin_strides[2], void* k_cache,
                                      const int64_t k_strides[4], void* v_cache,
                                      const int64_t v_strides[4], const int32_t* block_tables,
                                      const int64_t bt_strides[2], const int32_t* seq_lens,
                                      void* out, const int64_t out_strides[3], int num_seqs,
                                      int num_q_heads, int num_kv_heads, int head_dim,
                                      int block_size, int num_blocks, int max_blocks_per_seq,
                                      float scale, void* workspace, size_t workspace_bytes,
                                      void* stream);

/*
 * Paged prefill attention: the new tokens of each sequence attend causally over
 * the sequence's pool rows. Replaces the "full" prefix-cache prefill's
 * attention (engine/kernels/paged_attention_integration.py:459-482: the cached
 * prefix blocks gathered into a DynamicCache, :364-392, and the prompt suffix
 * forwarded through transformers' attention with a causal mask), reading the
 * prefix from the pool where it lies instead of copying it out.
 *   q     [num_tokens, num_q_heads, head_dim]; sequence b owns rows
 *         query_start_loc[b] .. query_start_loc[b + 1] - 1 (n_b rows; int32
 *         device array of num_seqs + 1 non-decreasing entries)
 *   seq_lens[b] = context length L_b after the new tokens; their K/V must
 *         already be in the pool at positions L_b - n_b .. L_b - 1
 *   out   [num_tokens, num_q_heads, head_dim]
 * Row i of sequence b (position p = L_b - n_b + i) gets
 * softmax(scale * q k^T) v over pool positions 0 .. p, query head h reading kv
 * head h / (num_q_heads / num_kv_heads). max_query_len must be at least every
 * n_b (rows past it are not computed); rows with p < 0 are written as zeros;
 * rows outside every sequence's range are not written. scale must be positive
 * and finite.
 *
 * Workspace: when the column blocks of the launch are too few to fill the GPU,
 * long key ranges are split over several workgroups, whose partial results
 * meet in the workspace; pa_prefill_attention_workspace_bytes() gives its size
 * (0: none needed). Like the decode workspace it starts with arrival counters
 * that must be zero before the buffer's first use and that every call leaves
 * zero; use one buffer per stream and lend it to nothing else.
 */
PA_API size_t pa_prefill_attention_workspace_bytes(int num_seqs, int num_q_heads,
                                                   int num_kv_heads, int head_dim,
                                                   int block_size, int max_blocks_per_seq,
                                                   int max_query_len);
PA_API int pa_prefill_attention_f16(const void* q, const int64_t q_strides[3],
                                    const void* k_cache, const int64_t k_strides[4],
                                    const void* v_cache, const int64_t v_strides[4],
                                    const int32_t* block_tables, const int64_t bt_strides[2],
                                    const int32_t* seq_lens, const int32_t* query_start_loc,
                                    int max_query_len, void* out, const int64_t out_strides[3],
                                    int num_seqs, int num_tokens, int num_q_heads,
                                    int num_kv_heads, int head_dim, int block_size,
                                    int num_blocks, int max_blocks_per_seq, float scale,
                                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * Fused elementwise chains of the decode step. None has a counterpart in the
 * reference, whose decode step runs them as transformers' separate ops
 * (paged_attention_integration.py:620-634 calls the model) and its greedy
 * selection as torch arg-max / top-k (:636-651); each replaces one chain with
 * one launch and the same roundings.
 *
 * pa_rmsnorm_f16: y[r] = fp16(w * fp16(s[r] * rsqrt(mean(s[r]^2) + eps))), mean
 * and product in fp32 -- transformers' Qwen2RMSNorm.forward -- where s = x, or,
 * when residual is not NULL, s = fp16(x + residual) (the decoder layer's
 * residual add), which is also written to sum. All fp16 with unit element
 * stride; rows are row_stride elements apart.
 *
 * pa_silu_mul_f16: out[r, i] = fp16(fp16(silu(g)) * u) with g = gate_up[r, i],
 * u = gate_up[r, inter + i], silu in fp32 -- Qwen2MLP.forward's
 * act_fn(gate_proj(x)) * up_proj(x) when gate and up come from one merged
 * projection.
 *
 * pa_top2_f16: per row of fp16 logits, index[r] = the first position of the
 * maximum (torch.argmax) and top[2r], top[2r+1] = the two largest values
 * (torch.topk(row, 2).values, a repeated maximum counted twice), as fp32.
 * NaN logits are skipped (torch would rank them first); a one-entry row gives
 * top[2r+1] = -inf.
 */
PA_API int pa_rmsnorm_f16(const void* x, int64_t x_row_stride, const void* residual,
                          int64_t residual_row_stride, void* sum, int64_t sum_row_stride,
                          const void* weight, void* y, int64_t y_row_stride, int rows, int hidden,
                          float eps, void* stream);
PA_API int pa_silu_mul_f16(const void* gate_up, int64_t gate_up_row_stride, void* out,
                           int64_t out_row_stride, int rows, int inter, void* stream);
PA_API int pa_top2_f16(const void* logits, int64_t row_stride, int rows, int vocab,
                       int64_t* index, float* top, void* stream);

/*
 * Batched decode attention that allocates nothing. No counterpart in the
 * reference; it is for callers that cannot allocate device memory or hand
 * over a workspace: code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation. Same arguments, kernels and results (the
 * same bits) as pa_decode_batched_f16, without the workspace: the split-K
 * scratch lives in a fixed array of PA_NOALLOC_SCRATCH_BYTES that the library
 * holds on each GPU it runs on until the process ends. One exception: where
 * the shared-prefix records of a stream-K launch would not fit the array
 * (head_dim 64: from 465 sequences at 2 kv heads, 117 at 8; in general
 * 262144 + 2 x 256 x 4 x R + 2 x num_seqs x num_kv_heads x R > 16 MiB with R =
 * (32 + 16 x head_dim) x 4 bytes), the call reads shared prefixes once per
 * sequence instead: results within the attention tolerance of
 * pa_decode_batched_f16 but not the same bits (the sums run in another order).
 * Calls whose scratch need still exceeds the array, and batches beyond the
 * stream-K plan (more than 1024 sequences or 65536 sequence x kv-head-group
 * pairs), are refused with PA_ERR_UNSUPPORTED before any launch. Every call on one GPU uses that GPU's
 * one array: calls that overlap in time on one GPU (concurrent streams or
 * threads) race and must not be made; calls ordered on one stream are fine.
 * The first call on a device also launches a small fill kernel, on the call's
 * stream, that clears the array's counters.
 */
#define PA_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
PA_API int pa_decode_batched_noalloc_f16(const void* q, const int64_t q_strides[3],
                                         const void* k_cache, const int64_t k_strides[4],
                                         const void* v_cache, const int64_t v_strides[4],
                                         const int32_t* block_tables, const int64_t bt_strides[2],
                                         const int32_t* seq_lens, void* out,
                                         const int64_t out_strides[3], int num_seqs,
                                         int num_q_heads, int num_kv_heads, int head_dim,
                                         int block_size, int num_blocks, int max_blocks_per_seq,
                                         float scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MI355X_PAGED_ATTENTION_H */
