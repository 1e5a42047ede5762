/*
 * mvattn.h — C ABI of the MI355X (gfx950) paged-attention decode step.
 *
 * Two kernels sit behind this ABI, called once per transformer layer per
 * engine step by the mini_vllm attention backend:
 *   - the KV-cache write (scatter of new K/V rows by slot index into the
 *     paged block pool), and
 *   - the paged decode attention (block-table gather of K/V, scaled QK^T,
 *     softmax, GQA grouping, PV accumulate), split over context partitions
 *     with a cross-partition log-sum-exp reduce.
 * Two helpers validate per-step metadata on the device (slots; lengths and
 * block tables, plus the decode work list) so that the per-layer calls
 * need no host synchronisation.
 *
 * Conventions
 *   - All pointers are device pointers unless stated otherwise.
 *   - Strides are in ELEMENTS; the innermost (head_dim) dimension of every
 *     tensor is contiguous.
 *   - KV pool layout (per layer, K and V separately):
 *       [num_blocks, num_kv_heads, block_size, head_dim], contiguous.
 *     Physical slot s lives at block s / block_size, offset s % block_size.
 *   - `stream` is a hipStream_t passed as void* (0 = null stream).
 *     Every call only enqueues work on that stream; none synchronises.
 *   - Return value: MV_OK (0) or a negative MV_ERR_* code; the message of
 *     the last error on the calling thread is returned by mv_last_error().
 *     No entry point aborts the process.
 *   - No entry point allocates device memory: buffers beyond the inputs
 *     and outputs (workspaces, status words) are the caller's. The library
 *     keeps the thread-local error string, a per-device cache of one
 *     device address (looked up once, never changed), and one static
 *     device array of MV_DECODE_SCRATCH_BYTES per GPU that only
 *     mv_paged_decode_noalloc uses (see there).
 */
#ifndef MVATTN_H
#define MVATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MVATTN_ABI_VERSION 7

/* Element types of query / key / value / cache / output. */
#define MV_DTYPE_F32 0
#define MV_DTYPE_F16 1
#define MV_DTYPE_BF16 2

/* Return codes. */
#define MV_OK 0
#define MV_ERR_INVALID_ARGUMENT (-1) /* shape / pointer / alignment problem */
#define MV_ERR_UNSUPPORTED (-2)      /* head_dim, block_size, GQA ratio, dtype */
#define MV_ERR_HIP (-3)              /* a HIP runtime call failed */

/* Status words written by mv_kv_slots_check (int32[2], device memory). */
#define MV_SLOTS_OUT_OF_RANGE 0 /* # slots < -1 or >= num_blocks*block_size */
#define MV_SLOTS_DUPLICATES 1   /* # (i < j) pairs with slot[i] == slot[j] >= 0 */

/* Status words written by mv_decode_write_check (int32[2], device memory). */
#define MV_WRITE_CHECK_OWN_SLOT 0 /* # slots not at their own sequence's kv_len - 1 */
#define MV_WRITE_CHECK_SHARED 1   /* # table entries of the batch reading a slot written */
#define MV_WRITE_CHECK_MAX_SEQS 4096

/* Status words written by mv_decode_step_check (int32[MV_STEP_WORDS], device). */
#define MV_STEP_SLOTS_OUT_OF_RANGE 0 /* as MV_SLOTS_OUT_OF_RANGE, over the decode slots */
#define MV_STEP_SLOTS_DUPLICATES 1   /* as MV_SLOTS_DUPLICATES */
#define MV_STEP_WRITE_OWN_SLOT 2     /* as MV_WRITE_CHECK_OWN_SLOT */
#define MV_STEP_WRITE_SHARED 3       /* as MV_WRITE_CHECK_SHARED */
#define MV_STEP_POSITIONS 4          /* # positions outside [0, max_positions) */
#define MV_STEP_WORDS 8

/* Status words written by mv_decode_plan (int32[8], device memory). */
#define MV_PLAN_NUM_ITEMS 0     /* number of work groups (launch grid) */
#define MV_PLAN_BAD_KV_LEN 1    /* # sequences with kv_len < 1 */
#define MV_PLAN_INSUFFICIENT 2  /* # sequences whose table row cannot cover kv_len */
#define MV_PLAN_BAD_BLOCK 3     /* # table entries used by kv_len outside [0, num_blocks) */
#define MV_PLAN_MAX_PARTS 4     /* max pieces of any sequence */
#define MV_PLAN_MIN_KV_LEN 5    /* min kv_len (clamped to int32) */
#define MV_PLAN_PARTITION_TOKENS 6 /* piece bound P chosen for this step */
#define MV_PLAN_IDS_PER_ITEM 7  /* block ids stored per work group (-1: capacity exceeded) */
#define MV_PLAN_WORDS 8

/* Version of this ABI (MVATTN_ABI_VERSION of the built library). */
int mv_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* mv_last_error(void);

/*
 * Capture id of `stream`: *capture_id = the id of the graph capture the
 * stream is in (nonzero), or 0 when it is not being captured. No
 * counterpart in the reference (which has no graph capture): the host side
 * keys its per-capture caches and deferred checks by it, so that a second
 * capture over the same metadata tensors records its own plan and checks.
 */
int mv_stream_capture_id(void* stream, uint64_t* capture_id);

/* Tokens one decode work group iteration covers for (head_dim, dtype):
 * partitions are multiples of it (0 for an unsupported pair). */
int mv_decode_chunk_tokens(int32_t head_dim, int32_t dtype);

/* Decode work groups one compute unit holds at once for (head_dim, dtype)
 * (LDS-limited); times the CU count it is the work-group count that runs in
 * a single dispatch round (the groups_per_cu of mv_decode_plan). */
int mv_decode_groups_per_cu(int32_t head_dim, int32_t dtype);

/*
 * KV-cache write.
 * Replaces the launch of `_cache_write_kernel` in `triton_cache_write`
 * (mini_vllm/attention/paged_attention_gpu.py:90-154, kernel :33-87) and
 * follows `write_to_paged_cache` (mini_vllm/cache/cache_write.py:25-74):
 *   for t in [0, num_tokens): s = slot_mapping[t]; s == -1 skips;
 *     key_cache[s / block_size, h, s % block_size, :] = key[t, h, :]
 *     value_cache[... same ...]                        = value[t, h, :]
 * The copy is bitwise. Unlike the Triton kernel it reads strided key/value
 * (e.g. V as a column view of a fused QKV projection) without a staging
 * copy. Slots outside [0, num_blocks*block_size) are skipped, never
 * written; mv_kv_slots_check reports them (and duplicates) beforehand.
 * Duplicate slots must be rejected by the caller: parallel writes to one
 * slot have no defined winner.
 */
int mv_kv_cache_write(const void* key, int64_t key_stride_tok, int64_t key_stride_head,
                      const void* value, int64_t value_stride_tok, int64_t value_stride_head,
                      void* key_cache, void* value_cache, const int64_t* slot_mapping,
                      int64_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                      int32_t block_size, int64_t num_blocks, int32_t dtype, void* stream);

/*
 * Slot validation for mv_kv_cache_write.
 * Replaces the host-side duplicate check of `triton_cache_write`
 * (paged_attention_gpu.py:126-135, `slot_mapping.unique()`, O(T log T)
 * with a host sync) and the range check of `write_to_paged_cache`
 * (cache_write.py:61-66). Writes status[MV_SLOTS_OUT_OF_RANGE] and
 * status[MV_SLOTS_DUPLICATES] (int32[2], device; the pair count saturates
 * at INT32_MAX) in O(T) expected work: every slot is counted into a hash
 * table. Up to 4096 tokens one work group does it in LDS and `workspace`
 * may be null; above, `workspace` (device, 8-byte aligned) must hold
 * mv_kv_slots_check_workspace_bytes(num_tokens) bytes, which the call
 * clears itself (two launches). num_tokens < 2^20 and total_slots < 2^44,
 * else MV_ERR_UNSUPPORTED. The caller reads the two words back.
 */
size_t mv_kv_slots_check_workspace_bytes(int64_t num_tokens);
int mv_kv_slots_check(const int64_t* slot_mapping, int64_t num_tokens, int64_t total_slots,
                      int32_t* status, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Precondition check of mv_paged_decode_write (the fused decode + KV write;
 * no counterpart in the reference, whose runner makes the two calls
 * write_kv_cache then decode_attention, qwen_runner.py:168-190). Writes two
 * int32 status words (device):
 *   status[MV_WRITE_CHECK_OWN_SLOT] = number of sequences b whose
 *     slot_mapping[b] is neither -1 nor the table position of b's token
 *     kv_len[b] - 1, i.e. block_table[b, (kv_len[b]-1) / block_size] *
 *     block_size + (kv_len[b]-1) % block_size (a sequence whose kv_len or
 *     table entry cannot address that position counts too);
 *   status[MV_WRITE_CHECK_SHARED] = number of table entries (c, j) that a
 *     sequence c attends (j < ceil(kv_len[c] / block_size)) and that name a
 *     block holding a slot written by this call at an offset c reads
 *     through that entry (below kv_len[c] - j * block_size), other than c's
 *     own slot at its own position kv_len[c] - 1. Counted only among the
 *     writers that pass the first check. Such a batch arises when blocks
 *     are shared without copy-on-write (the reference's prefix cache shares
 *     a prompt's partial last block: mini_vllm/cache/manager.py:140-172).
 * When both are 0 the fused call is bit-identical to mv_kv_cache_write
 * followed by mv_paged_decode; otherwise a work group could read a pool row
 * another one rewrites. The block table and kv_len may each be int32 or
 * int64. `workspace` (device, 8-byte aligned) holds
 * mv_decode_write_check_workspace_bytes(num_seqs) bytes (a hash table of
 * the writers, rebuilt by every call). num_seqs <= MV_WRITE_CHECK_MAX_SEQS
 * and block_size <= 2^20, else MV_ERR_UNSUPPORTED (make the two calls).
 * Two launches: one work group, then a (sequence, 256 table entries) grid.
 */
size_t mv_decode_write_check_workspace_bytes(int32_t num_seqs);
int mv_decode_write_check(const int64_t* slot_mapping, const void* block_table, int32_t bt_is_i64,
                          int64_t bt_stride, const void* kv_len, int32_t kv_len_is_i64,
                          int32_t num_seqs, int32_t max_blocks, int32_t block_size,
                          int32_t* status, void* workspace, size_t workspace_bytes, void* stream);

/*
 * The per-step checks of the fused decode layer call (mv_paged_decode_write,
 * with or without its RoPE) in two launches, for one host read-back per
 * step: over the step's num_seqs decode rows it writes status[MV_STEP_*]
 * (int32[MV_STEP_WORDS], device; words 5-7 unused):
 *   - the slot check of mv_kv_slots_check (out-of-range slots, duplicate
 *     pairs) -- the reference's `slot_mapping.unique()` check of
 *     `triton_cache_write` (paged_attention_gpu.py:126-135) and the range
 *     check of `write_to_paged_cache` (cache_write.py:61-66);
 *   - both counts of mv_decode_write_check (fused write precondition);
 *   - with positions (int64 [num_seqs], else null: word 4 is 0 and no rows
 *     are written): the positions check of mv_positions_check (the
 *     reference's rotary table lookup, mini_vllm/model/rotary.py:64-65),
 *     and cos_rows / sin_rows [num_seqs][head_dim] (contiguous, 16-byte
 *     aligned) = the tables' rows (row stride table_stride elements,
 *     16-byte aligned) at each position, clamped into [0, max_positions):
 *     the rope_cos_rows / rope_sin_rows of mv_paged_decode_write.
 * num_seqs <= MV_WRITE_CHECK_MAX_SEQS, block_size <= 2^20 and
 * num_blocks * block_size < 2^44, else MV_ERR_UNSUPPORTED. `workspace` as
 * for mv_decode_write_check (mv_decode_write_check_workspace_bytes).
 */
int mv_decode_step_check(const int64_t* slot_mapping, const void* block_table, int32_t bt_is_i64,
                         int64_t bt_stride, const void* kv_len, int32_t kv_len_is_i64,
                         int32_t num_seqs, int32_t max_blocks, int32_t block_size,
                         int64_t num_blocks, const int64_t* positions, const void* cos_table,
                         const void* sin_table, int64_t table_stride, int64_t max_positions,
                         int32_t head_dim, int32_t dtype, void* cos_rows, void* sin_rows,
                         int32_t* status, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Per-step decode metadata: validation, work split, work list.
 * Replaces the per-layer `kv_len_after.clone().to(int32)` of
 * `AttentionBackendGPU.decode_attention` (paged_attention_gpu.py:560-562)
 * and the `(kv_len_after < 1).any()` check of `triton_decode_attention`
 * (:294-300); adds the table-coverage check of `gather_paged_kv`
 * (mini_vllm/cache/cache_read.py:60-67).
 *   kv_len      [num_seqs] int64 (kv_len_is_i64=1) or int32
 *   block_table [num_seqs, max_blocks] (row stride bt_stride), int64
 *               (bt_is_i64=1) or int32, -1 padded
 * Cuts every sequence into pieces of equal 16-token tile counts, at most P
 * tokens each, P the smallest multiple of 16 that keeps the (sequence, kv
 * head, piece) work groups within groups_per_cu * cu_count
 * (mv_decode_groups_per_cu: one dispatch round) -- unless that takes
 * pieces over twice the slots' fair share, then about the fair share in
 * several rounds -- aiming at no more than 128 pieces per sequence and
 * spanning at most 511 table entries. When the groups fit one round they
 * are dealt to launch slots by size so the compute units carry near-equal
 * bytes. Outputs:
 *   work_items  per work group (launch slot), int32[8]: (seq, kv head,
 *               piece, pieces of the sequence, first token, end token, 0,
 *               0); 32-byte aligned, capacity work_capacity groups
 *               (num_seqs * num_kv_heads * ceil(max_blocks * block_size /
 *               16) always suffices);
 *   block_ids   for slot s, int32 [s * n, (s + 1) * n) with
 *               n = status[MV_PLAN_IDS_PER_ITEM]: the pool blocks of the
 *               table entries its tokens lie in (-1 for one outside the
 *               pool), then -1 to a multiple of 4 entries; the rest of
 *               the n entries is left unwritten (no launch reads it);
 *               16-byte aligned, block_ids_capacity >=
 *               mv_decode_block_ids_capacity(num_seqs, max_blocks,
 *               num_kv_heads, work_capacity) ints;
 *   counters    [num_seqs * num_kv_heads] set to zero;
 *   status      [MV_PLAN_WORDS] (MV_PLAN_NUM_ITEMS = work groups to launch,
 *               MV_PLAN_PARTITION_TOKENS = P, MV_PLAN_MAX_PARTS = most pieces
 *               of one sequence).
 * fixed_partition_tokens = 0 sizes the id lists for this step's P (the
 * host reads the status back before launching the decode). A value > 0
 * (from mv_decode_graph_bounds) is for a launch of fixed size that never
 * reads the status on the host, e.g. inside a captured HIP graph: the
 * lists take that bound's stride, and the work_items slots from
 * status[MV_PLAN_NUM_ITEMS] up to work_capacity get sequence -1, which the
 * decode kernel skips. Enqueues the plan and the block-id lists: one
 * launch when num_seqs <= 64 and num_seqs * max_blocks <= 8192, else a
 * plan launch (one work group) and an id-list launch (many work groups);
 * never synchronises.
 */
int mv_decode_plan(const void* kv_len, int32_t kv_len_is_i64, const void* block_table,
                   int32_t bt_is_i64, int64_t bt_stride, int32_t num_seqs, int32_t max_blocks,
                   int32_t block_size, int64_t num_blocks, int32_t num_kv_heads,
                   int32_t groups_per_cu, int32_t cu_count, int32_t fixed_partition_tokens,
                   int32_t* work_items, int64_t work_capacity, int32_t* block_ids,
                   int64_t block_ids_capacity, int32_t* counters, int32_t* status, void* stream);

/*
 * mv_decode_plan and mv_decode_step_check of one fused decode step
 * (mv_paged_decode_write), enqueued together: the arguments of the first
 * (kv_len ... status, the plan's words) and then those of the second that
 * the first does not already give (slot_mapping, positions ... status as
 * step_status, workspace as check_workspace), with the same meaning and
 * the same results, errors and outputs as the two calls in that order.
 * It replaces what those two replace in the reference: the metadata
 * checks of `triton_decode_attention` (paged_attention_gpu.py:294-300) and
 * `gather_paged_kv` (cache_read.py:60-67), and the slot checks of
 * `triton_cache_write` (:126-135). With at most 64 sequences over a table
 * of at most 8192 entries the plan, its block-id lists and the step check
 * are one launch (and the shared-read scan a second); otherwise it is the
 * launches of the two calls. Never synchronises.
 */
int mv_decode_plan_step_check(const void* kv_len, int32_t kv_len_is_i64, const void* block_table,
                              int32_t bt_is_i64, int64_t bt_stride, int32_t num_seqs,
                              int32_t max_blocks, int32_t block_size, int64_t num_blocks,
                              int32_t num_kv_heads, int32_t groups_per_cu, int32_t cu_count,
                              int32_t fixed_partition_tokens, int32_t* work_items,
                              int64_t work_capacity, int32_t* block_ids, int64_t block_ids_capacity,
                              int32_t* counters, int32_t* status, const int64_t* slot_mapping,
                              const int64_t* positions, const void* cos_table, const void* sin_table,
                              int64_t table_stride, int64_t max_positions, int32_t head_dim,
                              int32_t dtype, void* cos_rows, void* sin_rows, int32_t* step_status,
                              void* check_workspace, size_t check_workspace_bytes, void* stream);

/*
 * Sizes of a decode launch of fixed size, for batches of at most num_seqs
 * sequences and max_blocks table entries each (no counterpart in the
 * reference: it lets a caller launch the decode without reading the plan's
 * status back, as a captured graph must). out[0] = work groups to launch
 * (the plan never makes more; unused slots are marked and exit at once),
 * out[1] = fixed_partition_tokens for mv_decode_plan and partition_tokens
 * for mv_paged_decode, out[2] = max_partitions for mv_paged_decode and
 * its workspace.
 */
int mv_decode_graph_bounds(int32_t num_seqs, int32_t max_blocks, int32_t block_size,
                           int32_t num_kv_heads, int32_t groups_per_cu, int32_t cu_count,
                           int64_t* out);

/* Ints of block_ids storage mv_decode_plan needs (an upper bound for any
 * kv_len and piece size). */
int64_t mv_decode_block_ids_capacity(int32_t num_seqs, int32_t max_blocks, int32_t num_kv_heads,
                                     int64_t work_capacity);

/* Bytes of fp32 workspace mv_paged_decode needs for `max_partitions`
 * partitions per sequence (0 when max_partitions <= 1). */
size_t mv_paged_decode_workspace_bytes(int32_t num_seqs, int32_t num_q_heads, int32_t head_dim,
                                       int32_t max_partitions);

/*
 * Paged decode attention (one kernel launch).
 * Replaces the launch of `_paged_decode_kernel` in `triton_decode_attention`
 * (paged_attention_gpu.py:252-321, kernel :163-249); the math is that of
 * `AttentionBackendRef.decode_attention`
 * (mini_vllm/attention/paged_attention_ref.py:102-161):
 *   out[b, hq, :] = softmax(scale * q[b, hq] . K_b[hk]^T) V_b[hk],
 *   hk = hq / (num_q_heads / num_kv_heads), over kv_len[b] tokens whose
 *   token j lives at block block_table[b, j / block_size], offset
 *   j % block_size.
 * The sequences, token ranges and blocks come from mv_decode_plan on the
 * same metadata: work_items, block_ids, counters, num_work_groups =
 * status[MV_PLAN_NUM_ITEMS] (one work group each), partition_tokens =
 * status[MV_PLAN_PARTITION_TOKENS], max_partitions =
 * status[MV_PLAN_MAX_PARTS]; the block table itself is not read.
 * Sequences split into several partitions are merged inside the same
 * launch (log-sum-exp over partials in `workspace`: normalised O rows in
 * the data type for F16 / BF16, fp32 for F32, and fp32 (max, sum) pairs;
 * mv_paged_decode_workspace_bytes sizes the rows as fp32 for every dtype); calls sharing one plan's counters or
 * one workspace must be ordered on one stream. Output rows of sequences the
 * plan rejected are left untouched. Supported: head_dim 64 or 128,
 * block_size a power of two, num_q_heads / num_kv_heads in [1, 16], dtype
 * F32 / F16 / BF16 (query, caches and output share it); query rows and
 * strides, caches, work_items and block_ids 16-byte aligned.
 */
int mv_paged_decode(const void* query, int64_t q_stride_tok, int64_t q_stride_head,
                    const void* key_cache, const void* value_cache, const int32_t* work_items,
                    const int32_t* block_ids, int64_t block_ids_capacity, int32_t num_work_groups,
                    int32_t partition_tokens, int32_t max_partitions, int32_t* counters, void* out,
                    int64_t out_stride_tok, int64_t out_stride_head, float scale,
                    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                    int32_t head_dim, int32_t block_size, int64_t num_blocks, int32_t dtype,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of the static scratch buffer of mv_paged_decode_noalloc (per GPU). */
#define MV_DECODE_SCRATCH_BYTES (16 << 20)

/*
 * mv_paged_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under graph capture, serving loops that
 * forbid allocation). No counterpart in the reference. The split-K partials
 * live in a static device array of MV_DECODE_SCRATCH_BYTES per GPU, shared
 * by every call on that GPU: calls that overlap on one GPU race, so order
 * them on one stream. The call allocates nothing (no hipMalloc / hipFree,
 * no allocating library routine); its first call on a device looks the
 * array's address up once. Batches whose merge needs more
 * (mv_paged_decode_workspace_bytes > MV_DECODE_SCRATCH_BYTES) are rejected
 * with MV_ERR_INVALID_ARGUMENT; so is a stream of another device than the
 * current one. Otherwise identical to mv_paged_decode (same kernels, same
 * results).
 */
int mv_paged_decode_noalloc(const void* query, int64_t q_stride_tok, int64_t q_stride_head,
                            const void* key_cache, const void* value_cache,
                            const int32_t* work_items, const int32_t* block_ids,
                            int64_t block_ids_capacity, int32_t num_work_groups,
                            int32_t partition_tokens, int32_t max_partitions, int32_t* counters,
                            void* out, int64_t out_stride_tok, int64_t out_stride_head,
                            float scale, int32_t num_seqs, int32_t num_q_heads,
                            int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                            int64_t num_blocks, int32_t dtype, void* stream);

/*
 * Prefix gather (prefill support).
 * Replaces the launch of `_gather_prefix_kv_kernel` in `gather_prefix_kv`
 * (mini_vllm/attention/paged_attention_gpu.py:391-446, kernel :330-388),
 * semantics of `gather_paged_kv` (mini_vllm/cache/cache_read.py:19-84):
 *   out[cu_tokens[i] + p, h, :] = cache[bt[seq_rows[i], p / bs], h, p % bs, :]
 *   for p < cu_tokens[i+1] - cu_tokens[i], i < num_seqs.
 * seq_rows [num_seqs] and cu_tokens [num_seqs + 1] are int64 device arrays;
 * the caller guarantees every table entry read is a pool block (entries
 * outside [0, num_blocks) produce zero rows). head_dim * element bytes must
 * be a multiple of 16.
 */
int mv_gather_paged_kv(const void* key_cache, const void* value_cache, const void* block_table,
                       int32_t bt_is_i64, int64_t bt_stride, const int64_t* seq_rows,
                       const int64_t* cu_tokens, int32_t num_seqs, int64_t total_tokens,
                       void* out_key, void* out_value, int32_t num_kv_heads, int32_t head_dim,
                       int32_t block_size, int64_t num_blocks, int32_t dtype, void* stream);

/*
 * Fused rotary embedding + KV-cache write of one step's new tokens.
 * Replaces, in `QwenModelRunner.execute_model`
 * (mini_vllm/model_runner/qwen_runner.py:164-170), the three calls
 *   q = rope(q, positions); k = rope(k, positions);
 *   write_kv_cache(layer, k, v, slot_mapping)
 * with `RotaryEmbedding.__call__` / `_rotate_half`
 * (mini_vllm/model/rotary.py:44-82):
 *   x_rot = x * cos[pos] + [-x[D/2:], x[:D/2]] * sin[pos]
 * for every query head (-> query_out; may equal query) and key head
 * (-> key_cache at slot_mapping[t], as mv_kv_cache_write; also -> key_out
 * when key_out is not null), and the bitwise copy of value into
 * value_cache. Each product and the sum are rounded to the storage dtype,
 * as the reference's eager ops do: the results are bit-identical.
 *   cos_table, sin_table  [max_positions, >= head_dim] rows of
 *                         table_stride elements, the tensors' dtype
 *   positions             [num_tokens] int64, checked by mv_positions_check
 * key_cache == NULL skips the cache write (value, value_cache and
 * slot_mapping are then ignored): a plain rotary on query / key.
 * Pointers and strides (in elements) must give 16-byte aligned rows, and
 * head_dim must be a multiple of 32 bytes' worth of elements.
 */
int mv_rope_kv_cache_write(const void* query, int64_t q_stride_tok, int64_t q_stride_head,
                           void* query_out, int64_t qo_stride_tok, int64_t qo_stride_head,
                           const void* key, int64_t k_stride_tok, int64_t k_stride_head,
                           void* key_out, int64_t ko_stride_tok, int64_t ko_stride_head,
                           const void* value, int64_t v_stride_tok, int64_t v_stride_head,
                           void* key_cache, void* value_cache, const int64_t* slot_mapping,
                           const int64_t* positions, const void* cos_table, const void* sin_table,
                           int64_t table_stride, int64_t max_positions, int64_t num_tokens,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                           int32_t block_size, int64_t num_blocks, int32_t dtype, void* stream);

/*
 * Position validation for mv_rope_kv_cache_write: status[0] (int32,
 * device) = number of positions outside [0, max_positions). Replaces the
 * bounds check of the reference's table lookup `self._cos[positions]`
 * (mini_vllm/model/rotary.py:64-65), which raises IndexError.
 */
int mv_positions_check(const int64_t* positions, int64_t num_tokens, int64_t max_positions,
                       int32_t* status, void* stream);

/*
 * Decode layer call with the step's KV write fused in (no counterpart
 * function in the reference: it does `triton_cache_write` of the decode
 * tokens (paged_attention_gpu.py:90-154) and `triton_decode_attention`
 * (:252-321) in one launch). Arguments as mv_paged_decode, plus the new
 * rows new_key / new_value [num_seqs, num_kv_heads, head_dim] (strides in
 * elements, 16-byte aligned rows) and slot_mapping [num_seqs] int64:
 * row b is stored bitwise into pool slot slot_mapping[b] (-1 skips; slots
 * outside the pool are skipped -- mv_kv_slots_check reports them and
 * duplicates first). Sequence b's last token (kv_len - 1) is taken from
 * the new rows when its slot is that token's table position, which is
 * what the block manager produces; otherwise it is read from the pool.
 * Precondition (the block manager's layout): every slot is -1 or its
 * sequence's position kv_len - 1, and no other table entry of the batch
 * reads it (mv_decode_write_check counts both; the caller makes the two
 * calls when either count is nonzero). The output and the pool are then
 * bit-identical to mv_kv_cache_write followed by mv_paged_decode.
 *
 * With rope_cos_rows / rope_sin_rows ([num_seqs][head_dim] rows of the
 * rotary cos / sin tables at each sequence's position, query dtype,
 * contiguous, 16-byte aligned; both or neither), the launch also applies
 * the rotary embedding to the query and to new_key before using and
 * storing them: `RotaryEmbedding.__call__` (mini_vllm/model/rotary.py:
 * 44-82) with the reference's rounding, so output and pool are
 * bit-identical to mv_rope_kv_cache_write followed by mv_paged_decode on
 * the rotated query. This replaces the runner's rope(q), rope(k),
 * write_kv_cache and decode_attention for the decode rows
 * (qwen_runner.py:164-190) with one launch.
 */
int mv_paged_decode_write(const void* query, int64_t q_stride_tok, int64_t q_stride_head,
                          const void* new_key, int64_t nk_stride_tok, int64_t nk_stride_head,
                          const void* new_value, int64_t nv_stride_tok, int64_t nv_stride_head,
                          const int64_t* slot_mapping, const void* rope_cos_rows,
                          const void* rope_sin_rows, void* key_cache, void* value_cache,
                          const int32_t* work_items, const int32_t* block_ids,
                          int64_t block_ids_capacity, int32_t num_work_groups,
                          int32_t partition_tokens, int32_t max_partitions, int32_t* counters,
                          void* out, int64_t out_stride_tok, int64_t out_stride_head, float scale,
                          int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads,
                          int32_t head_dim, int32_t block_size, int64_t num_blocks, int32_t dtype,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Query tokens one mv_paged_prefill work group covers for this head shape
 * and dtype (0: unsupported; at most 16 query heads per kv head). */
int mv_prefill_tokens_per_group(int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                int32_t dtype);

/*
 * Chunked-prefill attention over the paged pool.
 * Replaces `AttentionBackendGPU.prefill_attention`
 * (mini_vllm/attention/paged_attention_gpu.py:577-661): its per-sequence
 * gather of the cached prefix (`gather_prefix_kv` / `_gather_prefix_kv_kernel`
 * :330-446), `cat` with the chunk, `repeat_interleave` and masked SDPA,
 * with one launch and no gathered copy. For sequence i,
 *   seqs[4i .. 4i+3] = (table row, cached tokens, first chunk row, chunk tokens)  int64
 * and chunk token t (row first + t of query / key / value / out) attends
 * keys 0 .. cached + t: prefix keys from the pool through block_table row
 * (int64 or int32, row stride bt_stride; every entry a prefix needs must
 * be a pool block -- the caller checks), chunk keys from key / value.
 *   work_items  int32[4] per work group: (sequence, kv head, first chunk
 *               token, tokens <= mv_prefill_tokens_per_group); the caller
 *               lists every (sequence, kv head, token block) once, in any
 *               order (longest first balances best); an item whose
 *               sequence is -1 is an unused slot and does nothing;
 *   out         [rows, num_q_heads, head_dim], query dtype.
 * head_dim 64 or 128, power-of-two block_size, 16-byte aligned rows.
 */
int mv_paged_prefill(const void* query, int64_t q_stride_tok, int64_t q_stride_head,
                     const void* key, int64_t k_stride_tok, int64_t k_stride_head,
                     const void* value, int64_t v_stride_tok, int64_t v_stride_head,
                     const void* key_cache, const void* value_cache, const void* block_table,
                     int32_t bt_is_i64, int64_t bt_stride, const int64_t* seqs, int32_t num_seqs,
                     const int32_t* work_items, int32_t num_work_groups, void* out,
                     int64_t out_stride_tok, int64_t out_stride_head, float scale,
                     int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                     int32_t block_size, int64_t num_blocks, int32_t dtype, void* stream);

/*
 * Bytes of the workspace mv_paged_prefill_parts needs for num_units units
 * cut into at most max_parts parts (0 when max_parts <= 1 or the head
 * shape is unsupported). Its first 64 KiB are the units' counters and must
 * be zero before the first call; every call leaves them zero again.
 */
size_t mv_paged_prefill_workspace_bytes(int32_t num_units, int32_t max_parts,
                                        int32_t num_q_heads, int32_t num_kv_heads,
                                        int32_t head_dim, int32_t dtype);

/*
 * mv_paged_prefill with the keys of a unit (one (sequence, kv head, token
 * block) of mv_paged_prefill's work list) cut into parts, one work group
 * each, for launches with fewer units than the device has CUs (one long
 * sequence's chunk: 64 units at 512 tokens). No counterpart in the
 * reference, whose prefill runs one SDPA per sequence; the result is that
 * of mv_paged_prefill on the same units within fp32 rounding of the
 * log-sum-exp merge, and it does not depend on which part finishes last.
 *   work_items  int32[8] per work group: the 4 of mv_paged_prefill, then
 *               (first key, end key, unit, part | parts << 8 |
 *               max_parts << 16): the part's keys [first key, min(end key,
 *               cached + first token + tokens)), first key a multiple of
 *               256 and the parts of a unit contiguous from key 0, units
 *               numbered 0 .. num_units-1 (at most 16384), parts 0 ..
 *               parts-1 (parts <= max_parts <= 8); every part of a unit
 *               in the same launch;
 *   workspace   mv_paged_prefill_workspace_bytes(num_units, max_parts, ..)
 *               bytes, 256-byte aligned, counters zero (see there); calls
 *               sharing one workspace must be ordered on one stream.
 * The part that completes a unit's count folds the parts in part order and
 * writes the unit's rows of out.
 */
int mv_paged_prefill_parts(const void* query, int64_t q_stride_tok, int64_t q_stride_head,
                           const void* key, int64_t k_stride_tok, int64_t k_stride_head,
                           const void* value, int64_t v_stride_tok, int64_t v_stride_head,
                           const void* key_cache, const void* value_cache, const void* block_table,
                           int32_t bt_is_i64, int64_t bt_stride, const int64_t* seqs,
                           int32_t num_seqs, const int32_t* work_items, int32_t num_work_groups,
                           int32_t num_units, int32_t max_parts, void* out,
                           int64_t out_stride_tok, int64_t out_stride_head, float scale,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                           int32_t block_size, int64_t num_blocks, int32_t dtype, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * Device-side plan of mv_paged_prefill for a launch of fixed size, e.g.
 * inside a captured graph where the step's lengths cannot be read back (no
 * counterpart in the reference: its prefill plans on the host). Inputs are
 * device int64 arrays of num_seqs entries: seq_rows (block-table row of each
 * sequence), cached_len and query_len (chunk tokens; the chunks' rows follow
 * each other in the query / key / value tensors, total_query_rows of them).
 * Writes seqs [num_seqs][4] int64 (row, cached, first chunk row, chunk
 * tokens) and work_items [work_capacity][4] int32 in sequence order
 * (ceil(query_len / tokens_per_group) work groups per sequence and kv head;
 * slots past the last one marked unused, which mv_paged_prefill skips);
 * launch mv_paged_prefill with num_work_groups = work_capacity.
 * status (int32[2], device): [0] = sequences whose row, lengths or prefix
 * table entries (the first ceil(cached_len / block_size) of the row) are
 * invalid; [1] = work groups, or -1 when the chunks exceed total_query_rows
 * or the work groups the capacity. Any error leaves every slot unused.
 */
int mv_prefill_plan(const int64_t* seq_rows, const int64_t* cached_len, const int64_t* query_len,
                    int32_t num_seqs, int64_t total_query_rows, const void* block_table,
                    int32_t bt_is_i64, int64_t bt_stride, int32_t bt_rows, int32_t max_blocks,
                    int32_t block_size, int64_t num_blocks, int32_t tokens_per_group,
                    int32_t num_kv_heads, int64_t* seqs, int32_t* work_items,
                    int32_t work_capacity, int32_t* status, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MVATTN_H */
