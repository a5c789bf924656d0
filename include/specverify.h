/*
 * specverify.h -- C ABI of the gfx950 paged-KV speculative-verify library
 * (libspecverify.so).
 *
 * Every pointer argument is a DEVICE pointer unless stated otherwise. The
 * library allocates nothing: pools, tables, counters, outputs and workspaces
 * belong to the caller. All work is enqueued on `stream` (a hipStream_t, NULL =
 * the default stream) and the functions return without synchronising.
 * Return value: SPV_OK (0) or a negative SPV_ERR_* code for invalid arguments
 * or a failed launch; nothing is enqueued when an argument check fails.
 * Thread-compatible: one caller per stream; calls on one pool must be ordered.
 *
 * Data layout in HBM (fixed by this library):
 *   K pool  [num_layers][capacity][num_kv_heads][block_size][head_dim]
 *   V pool  [num_layers][capacity][num_kv_heads][head_dim][block_size]
 *   block_tables [max_seqs][max_blocks_per_seq] int32, num_blocks[max_seqs],
 *   seq_lens[max_seqs], free_stack[capacity] (bottom..top), free_flag[capacity]
 *   (1 = on the free list), ctr[SPV_CTR_WORDS]: [0] free count, [1] 1 + batch
 *   index whose allocation exhausted the pool (last allocation), [2] slow-path
 *   rewinds, [3] blocks pushed by the last rewind, [4] last single alloc, [5]
 *   arrival count (zero between calls), [6] sticky 1 + batch index whose
 *   allocation the table width (max_blocks_per_seq) capped, [7] sticky 1 +
 *   batch index of a forbidden attention read (see spv_verify_attn), [8] sticky
 *   1 + batch index whose draft cache was shorter than the round's start (see
 *   spv_kv_draft_align); [9..15] zero.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   engine/kv.py, engine/attention.py, engine/spec_scheduler.py,
 *   specdec/sampler.py -- cited per entry point below.
 */
#ifndef SPECVERIFY_H
#define SPECVERIFY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPV_OK 0
#define SPV_ERR_ARG (-1)
#define SPV_ERR_LAUNCH (-2)
#define SPV_ERR_WORKSPACE (-3)
#define SPV_ERR_UNSUPPORTED (-4)

#define SPV_CTR_WORDS 16

/* element types */
#define SPV_F32 0
#define SPV_BF16 1
#define SPV_F16 2
#define SPV_FP8E4M3 3

/* Library version string (host pointer). */
const char* spv_version(void);

/* ------------------------------------------------------------------ pool */

/* BlockAllocator.__init__ free list [0..cap-1] (engine/kv.py:48-55) and
 * PagedKVCache.reset of the free list (engine/kv.py:173-183). */
int spv_pool_init(int32_t* free_stack, int32_t* free_flag, int32_t* ctr,
                  int32_t capacity, void* stream);

/* BlockAllocator.alloc (engine/kv.py:61-70): pops the stack top. The id (or -1
 * when the pool is exhausted) is written to *out_block (device int32). */
int spv_pool_alloc_one(int32_t* free_stack, int32_t* free_flag, int32_t* ctr,
                       int32_t capacity, int32_t* out_block, void* stream);

/* BlockAllocator.free (engine/kv.py:72-76): pushes `block` unless it is already
 * free; *out_pushed (device int32) receives 1 if pushed, 0 if ignored. */
int spv_pool_free_one(int32_t* free_stack, int32_t* free_flag, int32_t* ctr,
                      int32_t capacity, int32_t block, int32_t* out_pushed,
                      void* stream);

/* PagedKVCache.write (engine/kv.py:119-147) for a whole verify/extend block,
 * i.e. the loop `for b in batch: for j < C: write(layer, sid_b, start_b + j)`
 * of engine/model.py:184-187 in one launch. k_new/v_new are (B, C, Hkv, d) in
 * kv_dtype (fp8 not accepted here). With may_alloc != 0 the missing blocks are
 * first popped in batch order, each sequence's in logical order (one
 * workgroup, exclusive scan). On exhaustion the sequences before the failing
 * one get all their blocks, the failing one gets what is left, and ctr[1] is
 * set to 1 + its batch index. `write_limit_b` (the failing batch index, or B)
 * restricts the token writes exactly as the reference's raise would: sequences
 * after it write nothing, and it writes only tokens whose block exists.
 * write_limit_b = -1 takes that index from ctr[1] as the last allocation on
 * this pool set it: with may_alloc, this call's own; with may_alloc = 0, the
 * allocation of an earlier call for the same chunk (the later layers of one
 * verify round, whose blocks the first layer's call allocated), so a caller
 * need not know the index in advance.
 * seq_lens[sid] = max(seq_lens[sid], last written position + 1). seq_ids must
 * be distinct within one call. k_new = v_new = NULL allocates only
 * (PagedKVCache._ensure_blocks_up_to, kv.py:119-122): no copy, no length change.
 * A table holds at most max_blocks_per_seq blocks (the reference's list has no
 * bound): a sequence whose chunk needs more gets only the blocks that fit, its
 * tokens beyond them are not written, and ctr[6] is set to 1 + its batch index
 * (sticky). Callers keep start + C <= max_blocks_per_seq * block_size. */
int spv_kv_append(void* k_pool, void* v_pool, int kv_dtype,
                  const void* k_new, const void* v_new,
                  int32_t* block_tables, int32_t max_blocks_per_seq,
                  int32_t* num_blocks, int32_t* seq_lens,
                  int32_t* free_stack, int32_t* free_flag, int32_t* ctr,
                  const int32_t* seq_ids, const int32_t* start_pos,
                  int32_t B, int32_t C, int32_t layer, int32_t capacity,
                  int32_t block_size, int32_t num_kv_heads, int32_t head_dim,
                  int32_t may_alloc, int32_t write_limit_b, void* stream);

/* spv_kv_append that also records the round's write plan: write_plan (B x C
 * int32, device) receives for chunk token j of entry b the pool row
 * phys * block_size + (start_b + j) % block_size it was written to, or -1 where
 * nothing was written (the write limit, the entry's blocks, an out-of-pool id).
 * The plan then serves the same chunk's appends into the round's later layers
 * (spv_kv_write_planned): the loop of engine/model.py:184-187 runs once per
 * layer over the same positions, and only its first layer allocates
 * (kv.py:119-147). No reference counterpart for the plan itself.
 * Requires capacity * block_size < 2^31. */
int spv_kv_append_plan(void* k_pool, void* v_pool, int kv_dtype,
                       const void* k_new, const void* v_new,
                       int32_t* block_tables, int32_t max_blocks_per_seq,
                       int32_t* num_blocks, int32_t* seq_lens,
                       int32_t* free_stack, int32_t* free_flag, int32_t* ctr,
                       const int32_t* seq_ids, const int32_t* start_pos,
                       int32_t B, int32_t C, int32_t layer, int32_t capacity,
                       int32_t block_size, int32_t num_kv_heads, int32_t head_dim,
                       int32_t may_alloc, int32_t write_limit_b, int32_t* write_plan,
                       void* stream);

/* PagedKVCache.write (engine/kv.py:125-147) of a chunk into a later layer of
 * its round by the write plan of the round's first layer (spv_kv_append_plan):
 * k_new/v_new (B, C, Hkv, d) in kv_dtype (not fp8) go to the planned rows of
 * `layer`; no table, block count, length or counter is read or written, so the
 * result equals spv_kv_append with may_alloc = 0 and write_limit_b = -1 on the
 * state the plan was made from. C <= 64, head_dim * element size a multiple
 * of 16 bytes and C * head_dim * element size <= 16 KB. */
int spv_kv_write_planned(void* k_pool, void* v_pool, int kv_dtype,
                         const void* k_new, const void* v_new, const int32_t* write_plan,
                         int32_t B, int32_t C, int32_t layer, int32_t capacity,
                         int32_t block_size, int32_t num_kv_heads, int32_t head_dim,
                         void* stream);

/* spv_kv_append for an fp8 (OCP e4m3, SPV_FP8E4M3) pool with one fp32 scale
 * per (layer, block, K | V): kv_scales is [num_layers][capacity][2] (K, V), a
 * stored code q meaning q * scale. The reference pool has no fp8 storage
 * (engine/kv.py:99-101 allocates the model dtype); this entry point keeps
 * spv_kv_append's allocation, exhaustion, write-limit and length semantics and
 * replaces the copy by a quantisation. Blocks the allocation hands out get zero
 * scales in every layer. For each block the chunk writes, separately for K
 * and V: a = max |x| over the chunk's rows in the block (all heads and dims),
 * scale' = max(scale, a / 448); if scale' > scale every other row of the block
 * is re-encoded as e4m3((q * scale) / scale'); the chunk's rows are stored as
 * e4m3(x / scale') (0 when scale' = 0). e4m3 rounds to nearest even and
 * saturates at +-448; every product and quotient is a correctly rounded fp32
 * operation. k_new/v_new are (B, C, Hkv, d) in new_dtype (f32, bf16 or f16);
 * k_new = v_new = NULL allocates only. */
int spv_kv_append_fp8(void* k_pool, void* v_pool, float* kv_scales, int new_dtype,
                      const void* k_new, const void* v_new,
                      int32_t* block_tables, int32_t max_blocks_per_seq,
                      int32_t* num_blocks, int32_t* seq_lens,
                      int32_t* free_stack, int32_t* free_flag, int32_t* ctr,
                      const int32_t* seq_ids, const int32_t* start_pos,
                      int32_t B, int32_t C, int32_t layer, int32_t num_layers,
                      int32_t capacity, int32_t block_size, int32_t num_kv_heads,
                      int32_t head_dim, int32_t may_alloc, int32_t write_limit_b,
                      void* stream);

/* Rewind of a spec round (engine/spec_scheduler.py:302-307, 320-322) built
 * from PagedKVCache.truncate (engine/kv.py:150-162) and .clear (kv.py:164-171),
 * applied per entry in order: if new_len[i] >= 0 (and, with shrink_only, only
 * when seq_lens > new_len) truncate -- free the table tail tail-first, set
 * seq_len = max(0, new_len); then if finished[i] != 0 clear -- free the rest in
 * forward order, seq_len = 0. new_len/finished may be NULL (= -1 / 0). One
 * workgroup; pushes are placed by an exclusive scan in entry order; a block
 * already free is detected and the whole call then replays sequentially with
 * the reference's ignore-if-free rule. ctr[3] = blocks pushed. seq_ids must be
 * distinct within one call. Also serves PagedKVCache.reset (kv.py:173-183):
 * every sequence, new_len NULL, finished = 1. */
int spv_kv_rewind(int32_t* block_tables, int32_t max_blocks_per_seq,
                  int32_t* num_blocks, int32_t* seq_lens,
                  int32_t* free_stack, int32_t* free_flag, int32_t* ctr,
                  const int32_t* seq_ids, const int32_t* new_len,
                  const int32_t* finished, int32_t n, int32_t capacity,
                  int32_t block_size, int32_t shrink_only, void* stream);

/* One round's commit and the next round's append of the same batch in one
 * launch: exactly spv_kv_rewind(seq_ids, new_len, finished, B, shrink_only =
 * 0) followed by spv_kv_append_plan(k_new, v_new at start_pos, may_alloc = 1,
 * write_limit_b = -1, write_plan) -- PagedKVCache.truncate / clear of the
 * commit loop (engine/spec_scheduler.py:296-322, engine/kv.py:150-171) then
 * the next round's per-token writes (engine/model.py:184-187, engine/kv.py:
 * 119-147), with nothing between them (no admission). Block tables, lengths,
 * the free stack (bottom to top), flags, counters, stored K/V and the write
 * plan (B x C int32, or NULL) equal the two calls' results in every case,
 * including exhaustion, table-width overflow, finished sequences and blocks
 * already free. One launch for 16-byte-multiple K rows, B <= 256, chunks of
 * at most 1024 K/V elements per head touching at most 8 blocks; otherwise the
 * two calls are enqueued. new_len / finished may be NULL (no truncation /
 * none finished). Not for fp8 pools (SPV_ERR_ARG). No reference counterpart
 * for the fusion itself. */
int spv_kv_rewind_append(void* k_pool, void* v_pool, int kv_dtype,
                         const void* k_new, const void* v_new,
                         int32_t* block_tables, int32_t max_blocks_per_seq,
                         int32_t* num_blocks, int32_t* seq_lens,
                         int32_t* free_stack, int32_t* free_flag, int32_t* ctr,
                         const int32_t* seq_ids, const int32_t* new_len,
                         const int32_t* finished, const int32_t* start_pos,
                         int32_t B, int32_t C, int32_t layer, int32_t capacity,
                         int32_t block_size, int32_t num_kv_heads, int32_t head_dim,
                         int32_t* write_plan, void* stream);

/* Draft-cache alignment after a verify round (engine/spec_scheduler.py:296-322:
 * the draft truncate / catch-up / clear of the commit loop, on the draft pool).
 * Entry i: sequence seq_ids[i] started the round at start_pos[i] = L and
 * committed n_commit[i] = k tokens, so the target keeps keep = L + k. If k > 0
 * and the draft cache holds d > keep tokens it is truncated to keep
 * (PagedKVCache.truncate, engine/kv.py:150-162); if d < keep, positions
 * d .. keep-1 are caught up: their blocks are allocated as the reference's
 * draft decode writes would allocate them (engine/kv.py:119-122) and the
 * length becomes keep; catch_n[i] = keep - d, catch_pos[i] = d and
 * catch_tok[i][j] = chunk_tokens[i][d - L + j] (the round's chunk row: the
 * pending token, then the proposals) name the tokens the caller's draft model
 * must decode there, without allocating (the rest of catch_tok[i] is -1). A
 * finished sequence (finished[i] != 0) is then cleared (engine/kv.py:164-171)
 * and gets catch_n = 0. Pops and frees follow the reference's per-sequence
 * order exactly. d < L (tokens from before the round needed) skips the
 * catch-up and sets ctr[8] = 1 + i; an exhausted pool sets ctr[1] = 1 + i
 * and leaves later entries untouched, as the reference's exception does; a
 * table too narrow sets ctr[6]. kv_scales (fp8 pools, NULL otherwise) get
 * zero scales for allocated blocks in all num_layers layers. chunk_tokens,
 * catch_tok: (n, C) int32. 1 <= n <= 1024, seq_ids distinct. One workgroup. */
int spv_kv_draft_align(int32_t* block_tables, int32_t max_blocks_per_seq,
                       int32_t* num_blocks, int32_t* seq_lens,
                       int32_t* free_stack, int32_t* free_flag, int32_t* ctr,
                       float* kv_scales, int32_t num_layers,
                       const int32_t* seq_ids, const int32_t* start_pos,
                       const int32_t* n_commit, const int32_t* finished,
                       const int32_t* chunk_tokens, int32_t C,
                       int32_t* catch_n, int32_t* catch_pos, int32_t* catch_tok,
                       int32_t n, int32_t capacity, int32_t block_size,
                       void* stream);

/* One round's record of the scheduler metrics (engine/spec_scheduler.py:200-205
 * over PagedKVCache.num_allocated_blocks / logical_tokens / kv_stats,
 * engine/kv.py:186-224), computed on the device so the round needs no host
 * read: record[0] allocated blocks (capacity - ctr[0]), [1] logical tokens (sum
 * of seq_lens[0..rows)), [2] longest sequence, [3] B, [4] sum of n_commit[0..B),
 * [5] count of finished[0..B) != 0 (n_commit / finished may be NULL: 0);
 * peak (NULL to skip) = max(peak, allocated blocks), i.e. kv_peak_blocks.
 * record: 6 int64, peak: 1 int64. */
int spv_pool_metrics(const int32_t* ctr, const int32_t* seq_lens, int32_t rows,
                     int32_t capacity, const int32_t* n_commit,
                     const int32_t* finished, int32_t B, int64_t* record,
                     int64_t* peak, void* stream);

/* gather_ctx (engine/attention.py:41-63): out = (2, length, Hkv, d) in kv_dtype
 * (fp8 pools are dequantised to fp32 with kv_scales, see spv_verify_attn). */
int spv_kv_gather(const void* k_pool, const void* v_pool, int kv_dtype,
                  const float* kv_scales, const int32_t* block_tables,
                  int32_t max_blocks_per_seq, int32_t seq_id, int32_t length,
                  int32_t layer, int32_t capacity, int32_t block_size,
                  int32_t num_kv_heads, int32_t head_dim, void* out, void* stream);

/* PagedKVCache.key_map / value_map (engine/kv.py:208-213): out = (n, bs, Hkv, d)
 * in kv_dtype for the physical ids phys[0..n) of `layer`. */
int spv_kv_read_blocks(const void* pool, int is_value, int kv_dtype,
                       const int32_t* phys, int32_t n, int32_t layer,
                       int32_t capacity, int32_t block_size,
                       int32_t num_kv_heads, int32_t head_dim, void* out,
                       void* stream);

/* ------------------------------------------------------------- attention */

/* Bytes at the head of the attention workspace that hold per-segment arrival
 * counters. They must be zero when a workspace is first used (allocate it
 * zero-filled); every call leaves them zero again. Calls that share one
 * workspace must be ordered (one stream), as they also share its partials. */
#define SPV_ATTN_COUNTER_BYTES (1 << 18)

/* Workspace needed by spv_verify_attn for contexts up to max_ctx tokens
 * (0 when the call needs none). */
size_t spv_verify_attn_workspace_bytes(int32_t B, int32_t C, int32_t num_q_heads,
                                       int32_t num_kv_heads, int32_t head_dim,
                                       int32_t block_size, int32_t max_ctx);

/* paged_attention_extend (engine/attention.py:170-216): for sequence b, row j,
 * q head h: out = softmax(scale * q . K[0..start_b+j]) V[0..start_b+j] using kv
 * head h / (Hq/Hkv) (attention.py:32-38). q/out are (B, C, Hq, d) in q_dtype
 * (f32/bf16/f16); the pool holds kv_dtype. For SPV_FP8E4M3 pools kv_scales is
 * [layers][capacity][2] fp32 (K, V scale of each block). max_ctx must be >=
 * start_b + C for every b. bf16 queries over bf16 or fp8 pools, and fp16
 * queries over fp16 pools, with head_dim 128 or 64, block_size 16 and
 * B <= 2048 take the MFMA path (any (Hq/Hkv)*C); everything else (including
 * larger batches and mixed bf16 / fp16 operands) the VALU path.
 * seq_lens / ctr (the pool's, both may be NULL): a read the contract forbids
 * -- a table entry outside [0, capacity), start_b + C > seq_lens[seq_ids[b]]
 * (keys not written yet), start_b < 0 or start_b + C > max_ctx -- sets
 * ctr[7] = 1 + b (sticky; the caller clears it). Such a page reads block 0
 * instead, so the call never faults, and the rows of b are meaningless. */
int spv_verify_attn(void* out, const void* q, int q_dtype,
                    const void* k_pool, const void* v_pool, int kv_dtype,
                    const float* kv_scales, const int32_t* block_tables,
                    int32_t max_blocks_per_seq, const int32_t* seq_ids,
                    const int32_t* start_pos, const int32_t* seq_lens,
                    int32_t* ctr, int32_t B, int32_t C,
                    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                    int32_t block_size, int32_t layer, int32_t capacity,
                    int32_t max_ctx, float scale, void* workspace,
                    size_t workspace_bytes, void* stream);

/* The plan of a round's paged_attention_extend calls. The reference calls it
 * once per layer with the same seq_ids / start_positions
 * (engine/model.py:182-190 under spec_scheduler.py:255-259); what those calls
 * share -- the split of the batch over the persistent grid and the block id
 * of each workgroup's first pages -- is computed here once, after the round's
 * blocks are allocated, into `plan` (spv_verify_attn_plan_bytes(B) bytes,
 * caller-owned). The sequence-length check of spv_verify_attn (ctr[7]) is made
 * here, once. The plan is made for the MFMA path's query type of kv_dtype
 * (fp16 for fp16 pools, else bf16). Shapes off the MFMA path need no plan:
 * the call then does nothing. */
size_t spv_verify_attn_plan_bytes(int32_t B);
int spv_verify_attn_plan(const int32_t* block_tables, int32_t max_blocks_per_seq,
                         const int32_t* seq_ids, const int32_t* start_pos,
                         const int32_t* seq_lens, int32_t* ctr, int32_t B,
                         int32_t C, int32_t num_q_heads, int32_t num_kv_heads,
                         int32_t head_dim, int32_t block_size, int32_t kv_dtype,
                         int32_t capacity, int32_t max_ctx, void* plan,
                         size_t plan_bytes, void* stream);

/* spv_verify_attn reading a plan made by spv_verify_attn_plan with the same
 * block_tables contents, seq_ids, start_pos, B, C, heads, head_dim,
 * block_size, kv_dtype, capacity and max_ctx (any layer): the MFMA path skips
 * its prologue and starts the page walk one round trip after launch. Same
 * results as spv_verify_attn; other shapes run spv_verify_attn. */
int spv_verify_attn_planned(void* out, const void* q, int q_dtype,
                            const void* k_pool, const void* v_pool, int kv_dtype,
                            const float* kv_scales, const int32_t* block_tables,
                            int32_t max_blocks_per_seq, const int32_t* seq_ids,
                            const int32_t* start_pos, const int32_t* seq_lens,
                            int32_t* ctr, int32_t B, int32_t C,
                            int32_t num_q_heads, int32_t num_kv_heads,
                            int32_t head_dim, int32_t block_size, int32_t layer,
                            int32_t capacity, int32_t max_ctx, float scale,
                            const void* plan, void* workspace,
                            size_t workspace_bytes, void* stream);

/* spv_verify_attn with no allocation and no caller workspace. No counterpart
 * in the reference: it serves callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The kernels keep their counters and partials in the library's
 * own static device array of spv_verify_attn_static_max_bytes() bytes (24 MiB;
 * one per GPU, held until the process ends); a call that needs more (see
 * spv_verify_attn_workspace_bytes: the VALU path with long split contexts) is
 * rejected with SPV_ERR_WORKSPACE before anything is enqueued. Every call on
 * one GPU shares that array: calls that overlap on a GPU (other streams,
 * other host threads) race and give wrong results; order them. Arguments and
 * results are spv_verify_attn's. */
size_t spv_verify_attn_static_max_bytes(void);
int spv_verify_attn_static(void* out, const void* q, int q_dtype,
                           const void* k_pool, const void* v_pool, int kv_dtype,
                           const float* kv_scales, const int32_t* block_tables,
                           int32_t max_blocks_per_seq, const int32_t* seq_ids,
                           const int32_t* start_pos, const int32_t* seq_lens,
                           int32_t* ctr, int32_t B, int32_t C,
                           int32_t num_q_heads, int32_t num_kv_heads,
                           int32_t head_dim, int32_t block_size, int32_t layer,
                           int32_t capacity, int32_t max_ctx, float scale,
                           void* stream);

/* Kernel timing hook (no counterpart in the reference; for measurement): the
 * next spv_verify_attn / spv_verify_attn_static call made on this host thread
 * records the start of its first kernel into start_event and the end of its
 * last kernel into stop_event (hipEvent_t handles the caller created), from
 * the kernels' own dispatch timestamps -- the interval a profiler reports,
 * without the queue gaps around it. The arming ends with that call. */
int spv_time_next_attention(void* start_event, void* stop_event);

/* paged_attention_prefill_chunk (engine/attention.py:121-167): causal
 * attention of a freshly prefilled prompt chunk over itself. q (B, Lc, Hq, d),
 * k / v (B, Lc, Hkv, d) and out (B, Lc, Hq, d) are dense, in dtype (f32, bf16
 * or f16); lengths (device int32, B entries) holds the valid positions of each
 * row (clamped to [0, Lc]). Position j < lengths[b], q head h attends keys
 * 0 .. j of kv head h / (Hq/Hkv) with softmax(scale * q.k); positions >=
 * lengths[b] are written as zeros and none of them enters a result (the
 * padding may hold anything). bf16 or f16 with head_dim 64 or 128, a finite
 * positive scale and Hq/Hkv <= 256 take the MFMA path (within its 32-bit
 * offsets: Lc*Hkv*d*2 < 2^32, B*Hkv*Lc < 2^31), other cases an fp32 VALU
 * path. No workspace. */
int spv_prefill_attn(void* out, const void* q, const void* k, const void* v,
                     int dtype, const int32_t* lengths, int32_t B, int32_t Lc,
                     int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                     float scale, void* stream);

/* -------------------------------------------------------------- sampling */

/* Workspace needed by spv_verify_sample. Its first SPV_SAMPLE_COUNTER_BYTES
 * hold per-sequence arrival counters (two per sequence, B <= 65535): they must
 * be zero when a workspace is first used (allocate it zero-filled); every call
 * leaves them zero again, whatever its B. Calls that share one workspace must
 * be ordered (one stream); the attention and sampling entry points each need
 * a workspace of their own. */
#define SPV_SAMPLE_COUNTER_BYTES (1 << 19)
size_t spv_verify_sample_workspace_bytes(int32_t B, int32_t gamma, int32_t V);

/* Bits of a sequence's flag word (spv_verify_sample, spv_draft_sample). Given
 * logits, this library forms p and q with its own fp32 softmax, which sits
 * within a few 1e-6 of torch's; a flag marks a result that the reference,
 * computing its own softmax, may have decided the other way. Unflagged
 * results are the reference's. Given probabilities nothing but the draw's
 * rounding is left (a re-raced draw within a few ulp of another key). */
#define SPV_FLAG_ACCEPT_BAND 1 /* an examined u lay inside the error band of min(1, p/q) */
#define SPV_FLAG_DRAW_BAND 2   /* the drawn token's key is within the keys' error bound of another key's */
#define SPV_FLAG_TOP_P_BAND 4  /* (host) a filtered row's nucleus boundary is within rounding */

/* One fused verify-sampling step: logits_to_probs (specdec/sampler.py:19-36)
 * on every row, then batch_accept (engine/spec_scheduler.py:46-88) with
 * acceptance_probability (specdec/sampler.py:86-92), residual_distribution
 * (specdec/sampler.py:72-83) and sample_token (specdec/sampler.py:59-69) drawn
 * as argmax(probs / E), then the commit cut of engine/spec_scheduler.py:274-303.
 *   target (B, gamma+1, V) fp32, draft (B, gamma, V) fp32: logits, or already
 *     probabilities when is_probs != 0 (batch_accept's own inputs);
 *   temperature <= 0 -> greedy one-hot rows, else softmax(z / max(T, 1e-12));
 *   proposals (B, gamma) int32; u_accept (B, gamma) fp32 uniforms: position j
 *     is accepted iff (double)u < acceptance probability; exp_noise (B, V) fp32
 *     Exp(1) variates for the one race per sequence (read only when sampling;
 *     must be finite and > 0);
 *   draft_stats (B, gamma) float2 or NULL (logits only): the draft rows'
 *     statistics as spv_draft_sample wrote them at the same temperature (the
 *     draft loop keeps q's normaliser, spec_scheduler.py:243-252); the draft
 *     rows are then read only at the proposals and at the raced row;
 *   start_pos / remaining (B) int32 or NULL, eos_id (-1 = none): commit cut.
 * Outputs (device, may be NULL except accept_len/out_tokens):
 *   accept_len[B] drafts accepted, out_tokens[B][gamma+1] (-1 padded),
 *   n_commit[B], finished[B] (budget or eos; 1 also when n_commit == 0),
 *   new_len[B] = start + n_commit, or -1 when n_commit == 0 (no truncate),
 *   accept_prob[B][gamma] float64 acceptance probabilities,
 *   flags[B] SPV_FLAG_* words.
 * decide_only != 0 stops after accept_prob (no noise read, no outputs but
 * accept_prob and flags). */
int spv_verify_sample(const float* target, const float* draft, int is_probs,
                      float temperature, const int32_t* proposals,
                      const float* u_accept, const float* exp_noise,
                      const float* draft_stats, const int32_t* start_pos,
                      const int32_t* remaining, int32_t eos_id, int32_t B,
                      int32_t gamma, int32_t V, int32_t* accept_len,
                      int32_t* out_tokens, int32_t* n_commit, int32_t* finished,
                      int32_t* new_len, double* accept_prob, int32_t* flags,
                      int32_t decide_only, void* workspace,
                      size_t workspace_bytes, void* stream);

/* One draft step of the draft loop (engine/spec_scheduler.py:243-252): for
 * every row b of the draft logits (row b at logits + b * row_stride, V fp32
 * entries), out_tokens[b * out_stride] = sample_token(logits_to_probs(row))
 * (specdec/sampler.py:19-36, 59-69): argmax over i of q_i / exp_noise[b][i]
 * (q = softmax(z / max(T, 1e-12)), caller-supplied Exp(1) rows, lowest index
 * on ties), or, for temperature <= 0, the first-index argmax of the logits
 * (exp_noise not read). row_stats (may be NULL): row b's softmax statistics
 * (max, sum exp(x - max)) as a float2 at row_stats + 2 * b * out_stride, or
 * (unused, argmax index) when greedy -- what spv_verify_sample takes as
 * draft_stats. flags (may be NULL): row b's SPV_FLAG_* word at
 * flags[b * out_stride]. One launch for the batch; the workspace's first
 * SPV_SAMPLE_COUNTER_BYTES hold arrival counters that must be zero when it is
 * first used and are zero after every call. V <= 3,145,728. */
size_t spv_draft_sample_workspace_bytes(int32_t B, int32_t V);
int spv_draft_sample(const float* logits, int64_t row_stride, float temperature,
                     const float* exp_noise, int32_t B, int32_t V,
                     int32_t* out_tokens, int32_t out_stride, float* row_stats,
                     int32_t* flags, void* workspace, size_t workspace_bytes,
                     void* stream);

/* The top-k / top-p part of logits_to_probs (specdec/sampler.py:19-56) for
 * `rows` rows of V fp32 logits (row r at logits + r * in_stride, written at
 * out + r * out_stride): x = z / max(T, 1e-12), then apply_top_k (values below
 * the k-th largest become -inf, ties at it stay; 0 < top_k < V, else off),
 * then apply_top_p on what remains (descending order, a value stays while the
 * softmax mass before it is below top_p; 0 < top_p < 1, else off). out holds
 * x where it stays and -inf elsewhere: softmax(out) is logits_to_probs, and
 * out is what spv_verify_sample / spv_draft_sample take at temperature 1.
 * Masses are summed in fp64; equal values at the nucleus boundary stay in
 * ascending index order. The reference decides the nucleus edge on torch's
 * fp32 softmax, so values whose exact preceding mass lies within 5e-5 W of
 * top_p W (W: the kept mass) can fall either way there: ambiguous (may be
 * NULL) receives, per row, the count of such values (0 without top_p).
 * temperature must be > 0 (greedy rows are not filtered). One workgroup per
 * row; out may equal logits (same strides). */
int spv_filter_logits(const float* logits, int64_t in_stride, float* out,
                      int64_t out_stride, int32_t rows, int32_t V,
                      float temperature, int32_t top_k, float top_p,
                      int32_t* ambiguous, void* stream);

/* logits_to_probs (specdec/sampler.py:19-36) on `rows` rows of V fp32 logits. */
int spv_logits_to_probs(const float* logits, float* probs, int32_t rows, int32_t V,
                        float temperature, void* stream);

/* residual_distribution (specdec/sampler.py:72-83) of one row pair. */
int spv_residual(const float* p, const float* q, float* out, int32_t V,
                 void* stream);

/* sample_token (specdec/sampler.py:59-69) given its Exp(1) row:
 * *out_index = argmax(probs / noise), lowest index on ties, NaN wins. */
int spv_race_argmax(const float* probs, const float* noise, int32_t V,
                    int32_t* out_index, void* stream);

/* acceptance_probability (specdec/sampler.py:86-92): *out = a (float64). */
int spv_accept_prob(const float* p, const float* q, int32_t token_id, double* out,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPECVERIFY_H */
