/*
 * rvkv.h - C ABI of the MI355X (gfx950) paged KV-cache hot path.
 *
 * Drop-in boundary for rvllm's KV storage + attention read path. Every entry
 * point takes plain pointers and sizes; device pointers are caller-owned
 * (hipMalloc'd, torch-allocated, anything addressable by the pool's device).
 * A Rust `-sys` crate binds this header 1:1 (see the binding stubs shipped
 * with the integration notes).
 *
 * Conventions (mirroring rvllm's CUDA backend, src/cuda/ops.rs:325-352 and
 * src/cuda/kv_storage.rs:65-164):
 *  - every call validates its scalar arguments BEFORE launching anything and
 *    returns 0 or a negative RVKV_E* code; the reason is then readable from
 *    rvkv_last_error() as "<op>: <reason>" (thread-local string);
 *  - every call enqueues on the pool's stream and never synchronises; the
 *    caller synchronises (rvllm: stream.synchronize() in
 *    src/cuda/engine.rs:374);
 *  - a pool is driven from one thread at a time (rvllm's single engine
 *    thread, src/server/worker.rs:1-5);
 *  - block ids and slot offsets found in device arrays are bounds-checked by
 *    the kernels: an out-of-range id makes the kernel skip that row (append,
 *    copy) or read zeros (gather, decode) instead of faulting.
 *
 * Cache layout (physical, per layer, per K/V tensor): f16
 *   [num_blocks][n_kv_heads][block_size][head_dim]
 * i.e. head-major inside a block, so one (block, head) tile is one contiguous
 * block_size*head_dim*2-byte run. The LOGICAL contents are rvllm's
 * [num_blocks, block_size, n_kv_heads, head_dim] (src/kv_storage.rs:7-13);
 * rvkv_read_blocks / rvkv_gather expose the logical view.
 */
#ifndef RVKV_H
#define RVKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct rvkv_pool rvkv_pool;

/* A hipStream_t, passed as an opaque pointer so this header needs no HIP
 * include. NULL is the device's null stream. */
typedef void *rvkv_stream;

typedef enum {
  RVKV_F16 = 1, /* IEEE binary16 */
  RVKV_F32 = 2  /* IEEE binary32 */
} rvkv_dtype;

enum {
  RVKV_OK = 0,
  RVKV_EINVAL = -1,      /* bad argument (message says which) */
  RVKV_EHIP = -2,        /* a HIP runtime call failed */
  RVKV_ENOMEM = -3,      /* device allocation failed */
  RVKV_EUNSUPPORTED = -4 /* valid but not implemented shape */
};

/* Thread-local "<op>: <reason>" of the last failing call on this thread
 * ("" if none). Replaces the Box<dyn Error> strings of src/cuda/ops.rs. */
const char *rvkv_last_error(void);

/* ---- pool ------------------------------------------------------------
 * Replaces CudaKvStorage::new (src/cuda/kv_storage.rs:77-100) /
 * KvStorage::new (src/kv_storage.rs:84-104): zeroed K and V storage for
 * n_layers attention layers. One device allocation for all layers; 64-bit
 * offsets throughout. cache_dtype RVKV_F16 (the fast path) or RVKV_F32
 * (the reference's own cell type): an f32 pool supports append (f32 rows
 * copied, f16 rows widened exactly), gather into F32 only, copy_blocks,
 * read_blocks, block_checksums, attn_prep, paged decode and paged prefill.
 * The pool binds to the current HIP device and to `stream`. */
int rvkv_pool_create(uint32_t n_layers, uint32_t num_blocks,
                     uint32_t block_size, uint32_t n_kv_heads,
                     uint32_t head_dim, rvkv_dtype cache_dtype,
                     rvkv_stream stream, rvkv_pool **out);
void rvkv_pool_destroy(rvkv_pool *pool);
/* Bytes of device memory the pool holds (K+V, all layers). */
size_t rvkv_pool_bytes(const rvkv_pool *pool);
/* Rebinds the pool to another stream on the same device. */
int rvkv_pool_set_stream(rvkv_pool *pool, rvkv_stream stream);

/* ---- KV append -------------------------------------------------------
 * Replaces CudaKvStorage::write_tokens (src/cuda/kv_storage.rs:105-126) ->
 * kv_write_wrapper (src/cuda/ops.rs:313-373) -> kv_write.cu, and the CPU
 * KvStorage::write_tokens (src/kv_storage.rs:116-150).
 * k, v: device [n_tokens, n_kv_heads, head_dim], src_dtype F32 (rounded to
 * f16 round-to-nearest-even) or F16 (copied bit for bit).
 * slot_block, slot_off: device u32[n_tokens], token i -> (block, offset).
 * Slots must be distinct within one call (the reference's precondition,
 * src/cuda/kernels/kv_write.cu:33). n_tokens == 0 is an error, as in
 * kv_write_wrapper. */
int rvkv_append(rvkv_pool *pool, uint32_t layer, const void *k, const void *v,
                rvkv_dtype src_dtype, const uint32_t *slot_block,
                const uint32_t *slot_off, uint32_t n_tokens);

/* n_layers calls of rvkv_append with the same slots, layers layer0 ..
 * layer0+n_layers-1, in one launch: the batched form of the per-layer
 * KvStorage::write_tokens (src/kv_storage.rs:116-150) that a prefill makes
 * for every layer with one slot list (write_positions, src/engine.rs:365-388).
 * Layer l's rows are k/v + l*src_layer_stride elements of src_dtype
 * (src_layer_stride >= n_tokens*n_kv_heads*head_dim when n_layers > 1).
 * Same rounding, validation and out-of-range slot rule as rvkv_append; the
 * cache afterwards is bit-identical to the per-layer calls. f32 pools and
 * head_dim % 8 != 0 run one append per layer. */
int rvkv_append_layers(rvkv_pool *pool, uint32_t layer0, uint32_t n_layers,
                       const void *k, const void *v, rvkv_dtype src_dtype,
                       uint64_t src_layer_stride, const uint32_t *slot_block,
                       const uint32_t *slot_off, uint32_t n_tokens);

/* ---- block-table gather ---------------------------------------------
 * Replaces CudaKvStorage::gather (src/cuda/kv_storage.rs:132-164) ->
 * kv_gather_wrapper (src/cuda/ops.rs:381-445) -> kv_gather.cu, and
 * KvStorage::gather (src/kv_storage.rs:157-173).
 * block_idx: device u32[batch*max_blocks], each sequence's block table padded
 * to max_blocks (rvllm's GatherPlan convention, src/kv_storage.rs:59-67).
 * out_k, out_v: device [batch, n_kv_heads, ctx_len, head_dim] of out_dtype
 * (F32 = the reference's output type; F16 = raw cache bits, f16 pools
 * only: an f32 pool gathers into F32, bit for bit).
 * ctx_len must not exceed max_blocks*block_size. */
int rvkv_gather(const rvkv_pool *pool, uint32_t layer,
                const uint32_t *block_idx, uint32_t batch, uint32_t max_blocks,
                uint32_t ctx_len, void *out_k, void *out_v,
                rvkv_dtype out_dtype);

/* ---- paged GQA decode attention ---------------------------------
 * Replaces, for q_len == 1, the chain kv_gather x2 -> attention_scores ->
 * mask_add_broadcast -> softmax -> attention_apply
 * (src/cuda/model.rs:528-569) and the CPU gather + batch_mask +
 * gqa_attention (src/model.rs:346-415, 628-644).
 * q: device f32 [batch, n_heads, head_dim]; out: device f32, same shape.
 * block_tables: device u32 [batch, max_blocks]; ctx_lens: device u32[batch],
 * the real context length of each sequence INCLUDING the token appended this
 * step (rvllm's read_num_tokens). Each ctx_len must be <= max_ctx_len and
 * <= max_blocks*block_size (larger values are clamped).
 * Query head h reads KV head h / (n_heads / n_kv_heads).
 * scale multiplies q.k (rvllm: 1/sqrt(head_dim)).
 * window > 0 keeps only the last `window` keys (rvllm's sliding-window mask
 * j + window <= offset, src/model.rs:361, with offset = ctx_len - 1);
 * window <= 0 means no window.
 * ws: device scratch of at least rvkv_decode_workspace_bytes(...) bytes,
 * 256-byte aligned; contents need no initialisation.
 * A sequence with ctx_len 0 gets an all-zero output row.
 * Supported: head_dim <= 1024, any block_size, n_heads a multiple of
 * n_kv_heads. The tuned kernels take head_dim <= 256 (32, 64, 128 and 256
 * at full speed; other values read rows element by element) with block_size
 * a power of two >= 512/HD, HD being head_dim rounded up to 32, 64, 128 or
 * 256 (an f32 pool: head_dim exactly 32, 64, 128 or 256); every other shape
 * runs a generic kernel (f32 arithmetic, no workspace, slower). */
int rvkv_paged_decode(const rvkv_pool *pool, uint32_t layer, const float *q,
                      const uint32_t *block_tables, const uint32_t *ctx_lens,
                      uint32_t batch, uint32_t max_blocks, uint32_t n_heads,
                      uint32_t max_ctx_len, float scale, int32_t window,
                      float *out, void *ws, size_t ws_bytes);

/* rvkv_paged_decode without a workspace argument and without any device
 * allocation. No counterpart in the reference: it is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). The split-sequence partials go to a static 8 MiB
 * array of device memory that each GPU holds for the life of the process;
 * a shape whose rvkv_decode_workspace_bytes exceeds 8 MiB is rejected with
 * RVKV_EUNSUPPORTED (only reachable at head_dim 256 with > 4 query heads per
 * KV head). Every call on one GPU shares that GPU's array and finds the
 * last call's contents in it. Calls on one stream are ordered by the
 * stream; a call on another stream of the same GPU first waits (on the
 * device, via an event created once per GPU) for the last call that used
 * the array, and calls from several host threads take it one at a time.
 * Not ordered: a stream under graph capture, so a captured graph's replays
 * race with calls on other streams of that GPU. Same arguments, rules and
 * results as rvkv_paged_decode otherwise. */
int rvkv_paged_decode_noalloc(const rvkv_pool *pool, uint32_t layer,
                              const float *q, const uint32_t *block_tables,
                              const uint32_t *ctx_lens, uint32_t batch,
                              uint32_t max_blocks, uint32_t n_heads,
                              uint32_t max_ctx_len, float scale,
                              int32_t window, float *out);

/* Workspace bytes rvkv_paged_decode needs for this batch shape. */
size_t rvkv_decode_workspace_bytes(const rvkv_pool *pool, uint32_t batch,
                                   uint32_t n_heads, uint32_t max_ctx_len);

/* Tokens per context partition rvkv_paged_decode will use for this shape
 * (each partition is one workgroup per (sequence, KV head)). */
uint32_t rvkv_decode_partition_tokens(const rvkv_pool *pool, uint32_t batch,
                                      uint32_t n_heads, uint32_t max_ctx_len);

/* ---- planned paged decode (ragged batches) ------------------
 * The counterpart of GatherPlan::new / CudaGatherPlan::new
 * (src/kv_storage.rs:50-75, src/cuda/kv_storage.rs:26-54): built once per
 * forward from the host-side read_num_tokens (BatchItem::read_num_tokens,
 * src/model.rs:430-433) and shared by every layer. It splits each
 * sequence's visible context into work items of at most part_tokens tokens,
 * orders them longest first so ragged batches balance across the GPU, sends
 * single-item sequences straight to the output and reduces only the split
 * ones. Creating a plan allocates device and pinned host memory for the
 * item list and uploads it on the pool's stream.
 * The device ctx_lens given to rvkv_paged_decode_planned must equal the
 * host ones the plan was built from (larger values are clamped to them). */
typedef struct rvkv_decode_plan rvkv_decode_plan;

int rvkv_decode_plan_create(const rvkv_pool *pool,
                            const uint32_t *ctx_lens_host, uint32_t batch,
                            uint32_t n_heads, int32_t window,
                            rvkv_decode_plan **out);
/* Rebuilds the plan in place for this step's context lengths (same n_heads
 * and window; batch may change), reusing its device and pinned buffers
 * unless the work list outgrows them. Waits only for the plan's own upload
 * three updates back (its pinned staging is used in turn), so a host loop
 * can build up to three steps ahead of the device. The plan keeps a pointer
 * to the pool: destroy it first. */
int rvkv_decode_plan_update(rvkv_decode_plan *plan,
                            const uint32_t *ctx_lens_host, uint32_t batch);
/* rvkv_decode_plan_update with the host copy of this step's padded block
 * tables ([batch, max_blocks], what GatherPlan::new takes besides the read
 * counts, src/kv_storage.rs:50-75): items of sequences that share prefix
 * blocks are then ordered back to back, so those blocks are read from HBM
 * about once per XCD instead of once per sharer. On the matrix-core decode
 * (head_dim 64, 5-16 query heads per KV head, no window) the blocks that up
 * to 32 / group sharers hold alike, below each one's last position, become
 * group items: one workgroup reads them once for all those sharers, whose
 * partials the reduction merges with their own ranges' (results then match
 * the lengths-only plan to within the decode tolerance, not bit for bit).
 * tables_host must hold the same block ids as the device tables the decode
 * calls pass (a group reads its first member's table for every member).
 * tables_host NULL is rvkv_decode_plan_update. */
int rvkv_decode_plan_update_tables(rvkv_decode_plan *plan,
                                   const uint32_t *ctx_lens_host,
                                   const uint32_t *tables_host,
                                   uint32_t max_blocks, uint32_t batch);
/* Waits for the pool's stream (queued decodes may read the plan), frees. */
void rvkv_decode_plan_destroy(rvkv_decode_plan *plan);
/* Device scratch rvkv_paged_decode_planned needs (0 if nothing is split). */
size_t rvkv_decode_plan_workspace_bytes(const rvkv_decode_plan *plan);
/* Work items (workgroups per KV head) of the plan. */
uint32_t rvkv_decode_plan_items(const rvkv_decode_plan *plan);
/* Same contract as rvkv_paged_decode, with batch, n_heads, window and the
 * context bound taken from the plan. */
int rvkv_paged_decode_planned(const rvkv_pool *pool,
                              const rvkv_decode_plan *plan, uint32_t layer,
                              const float *q, const uint32_t *block_tables,
                              const uint32_t *ctx_lens, uint32_t max_blocks,
                              float scale, float *out, void *ws,
                              size_t ws_bytes);

/* ---- one layer of a decode step ----------------------
 * The per-layer order of src/model.rs:628-644 (write_tokens, then attend
 * over the context including the new token) in ONE launch: row b of k/v
 * ([batch, n_kv_heads, head_dim], F32 rounded to f16 nearest-even or F16) is
 * sequence b's token at position ctx_lens[b]-1 and is stored at
 * (slot_block[b], slot_off[b]); the workgroup that attends over that
 * position uses the same f16 values, so the cache afterwards and the output
 * equal rvkv_append followed by rvkv_paged_decode (or _planned). Precondition
 * (as in the engine, src/engine.rs:446-451): the slot is the block-table slot
 * of position ctx_lens[b]-1. plan may be NULL (uniform partitioning, same
 * workspace as rvkv_paged_decode) or a plan built for this batch (then
 * batch/n_heads/window must match it and max_ctx_len is ignored). On an f32
 * pool the rows are stored as f32 (F32 copied, F16 widened exactly), also in
 * one launch; shapes that run the generic kernel take an append launch and
 * then the decode. */
int rvkv_decode_step(rvkv_pool *pool, const rvkv_decode_plan *plan,
                     uint32_t layer, const void *k, const void *v,
                     rvkv_dtype src_dtype, const uint32_t *slot_block,
                     const uint32_t *slot_off, const float *q,
                     const uint32_t *block_tables, const uint32_t *ctx_lens,
                     uint32_t batch, uint32_t max_blocks, uint32_t n_heads,
                     uint32_t max_ctx_len, float scale, int32_t window,
                     float *out, void *ws, size_t ws_bytes);

/* ---- attention prep fused with the append -----------------
 * Everything between the QKV projection and attention for `rows` tokens,
 * as src/model.rs:600-639 computes it (the reference's own fused form is
 * the Metal attn_prep, src/metal/kernels/attention.metal:8-88):
 *   q, k: + bias (optional) -> per-head RMS norm (optional, q_norm/k_norm
 *         [head_dim], eps) -> rotate-half RoPE with this row's cos/sin;
 *   v:    + bias (optional).
 * q_in [rows, n_heads, hd], k_in/v_in [rows, n_kv_heads, hd] f32 (device);
 * biases [heads*hd] or NULL; cos/sin [rows, hd/2] f32 (rope_cos_sin of each
 * row's position, src/model.rs:224-250, built once per forward).
 * The rotated q goes to q_out [rows, n_heads, hd] f32; k and v are rounded
 * to f16 (nearest-even; stored as they are in an f32 pool) and written to
 * (slot_block[i], slot_off[i]) of `layer`, as rvkv_append would. head_dim
 * even and <= 1024 (32, 64, 128 and 256 on the tuned kernel, others and f32
 * pools on a generic one); every float buffer 16-byte aligned (RVKV_EINVAL
 * otherwise). Rows whose slot is
 * out of range still produce q_out but write no k/v. */
int rvkv_attn_prep(rvkv_pool *pool, uint32_t layer, const float *q_in,
                   const float *k_in, const float *v_in, uint32_t rows,
                   uint32_t n_heads, const float *q_bias, const float *k_bias,
                   const float *v_bias, const float *q_norm,
                   const float *k_norm, float eps, const float *cos_t,
                   const float *sin_t, const uint32_t *slot_block,
                   const uint32_t *slot_off, float *q_out);

/* ---- paged prefill / chunked-prefill attention ------------
 * Attention for q_len >= 1 query rows per sequence straight over the paged
 * cache: what rvllm's prefill computes with kv_gather + batch_mask +
 * gqa_attention (src/model.rs:346-415 called at :628-644; CUDA:
 * src/cuda/model.rs:528-569; the Metal attn_decode with q_len > 1,
 * src/metal/ops.rs:680-685). Row i of sequence b is at position
 * pos_offset[b] + i and sees key j iff j < read_num_tokens[b], j <= its
 * position and, with window > 0, j + window > its position. q and out are
 * token-major [batch * q_len, n_heads, head_dim] f32, 16-byte aligned;
 * block_tables [batch, max_blocks] u32; pos_offset, read_num_tokens [batch]
 * u32 (all device). Table entries >= num_blocks mark keys unreadable (they
 * get probability 0); a row that sees no key gets zeros. With an f16 pool,
 * head_dim in {32, 64, 128, 256} and block_size a power of two >= 8 it is
 * computed on the matrix cores in f16 with f32 accumulation; any other
 * head_dim <= 1024, block size or an f32 pool runs a generic kernel in f32
 * arithmetic. Allocates nothing. */
int rvkv_paged_prefill(rvkv_pool *pool, uint32_t layer, const float *q,
                       const uint32_t *block_tables,
                       const uint32_t *pos_offset,
                       const uint32_t *read_num_tokens, uint32_t batch,
                       uint32_t q_len, uint32_t max_blocks, uint32_t n_heads,
                       float scale, int32_t window, float *out);

/* The same step over one fused [rows, (n_heads + 2 n_kv_heads) * head_dim]
 * QKV buffer (Q heads, then K, then V) with one fused bias [that width] or
 * NULL: the interface of the reference's fused attn_prep (Metal,
 * src/metal/ops.rs:357-420, kernel src/metal/kernels/attention.metal:8-88),
 * so the projection's output is consumed in place. Same rules otherwise. */
int rvkv_attn_prep_qkv(rvkv_pool *pool, uint32_t layer, const float *qkv,
                       uint32_t rows, uint32_t n_heads, const float *bias,
                       const float *q_norm, const float *k_norm, float eps,
                       const float *cos_t, const float *sin_t,
                       const uint32_t *block_ids, const uint32_t *offsets,
                       float *q_out);

/* ---- prefix-cache copy-on-write -------------------------------------
 * No counterpart in the reference (rvllm never mutates a shared block; its
 * only copy is the whole-cache KvStorage::clone, src/kv_storage.rs:15-33).
 * Copies block src[i] -> dst[i] for every layer, K and V, bit for bit.
 * src, dst: device u32[n]. dst blocks must be distinct and not among src. */
int rvkv_copy_blocks(rvkv_pool *pool, const uint32_t *src,
                     const uint32_t *dst, uint32_t n);

/* ---- inspection (test and integration support) --------------------------
 * Logical view of whole blocks: out is device [n, block_size, n_kv_heads,
 * head_dim] of the pool's cell type for blocks block_ids[0..n) of (layer, which: 0 = K, 1 = V).
 * The raw-cache view rvllm's tests read (src/cuda/ops.rs:1104-1114). */
int rvkv_read_blocks(const rvkv_pool *pool, uint32_t layer, uint32_t which,
                     const uint32_t *block_ids, uint32_t n, void *out);

/* 64-bit FNV-1a over the logical little-endian f16 bytes of each listed
 * block of (layer, which): out device u64[n]. Lets a host compare full-size
 * caches against a CPU model block by block. */
int rvkv_block_checksums(const rvkv_pool *pool, uint32_t layer,
                         uint32_t which, const uint32_t *block_ids, uint32_t n,
                         uint64_t *out);

/* ---- host side: block manager -----------------------------------
 * Host-only (no device memory). Stands in for the external
 * kv-cache-scheduler 0.2.0 crate as rvllm's engine uses it
 * (src/engine.rs:351-539): a block pool with a free list, per-sequence block
 * tables, logical_to_physical slot mapping, refcounted prefix sharing and the
 * copy-on-write decision before an append. */
typedef struct rvkv_bm rvkv_bm;

rvkv_bm *rvkv_bm_create(uint32_t num_blocks, uint32_t block_size);
void rvkv_bm_destroy(rvkv_bm *bm);
/* Free blocks (kv-cache-scheduler's pool.available()). */
uint32_t rvkv_bm_available(const rvkv_bm *bm);
/* Shuffles the free list with a seeded Fisher-Yates (fragmented pools). */
void rvkv_bm_shuffle_free(rvkv_bm *bm, uint64_t seed);
/* Adds a sequence holding n_tokens, allocating ceil(n_tokens/bs) blocks.
 * Returns the new sequence id (>= 0) or a negative code (pool full). */
int64_t rvkv_bm_add_seq(rvkv_bm *bm, uint32_t n_tokens);
/* Adds a sequence whose first n_shared tokens reuse `parent`'s blocks
 * (refcount + 1 each; a partially filled shared last block is shared too),
 * then allocates private blocks up to n_tokens. */
int64_t rvkv_bm_fork_seq(rvkv_bm *bm, int64_t parent, uint32_t n_shared,
                         uint32_t n_tokens);
/* Drops a sequence; blocks whose refcount reaches 0 return to the free list.
 */
int rvkv_bm_free_seq(rvkv_bm *bm, int64_t seq);
/* Reserves the slot for the sequence's next token (position num_tokens):
 * allocates a block at a block boundary; if the target block is shared
 * (refcount > 1) it is replaced by a fresh private block and the pair
 * (old, new) is reported in *cow_src / *cow_dst (else both UINT32_MAX) so
 * the caller can enqueue rvkv_copy_blocks before the append. Writes the
 * slot to *block, *offset. */
int rvkv_bm_append_slot(rvkv_bm *bm, int64_t seq, uint32_t *block,
                        uint32_t *offset, uint32_t *cow_src,
                        uint32_t *cow_dst);
/* Batch forms of free_seq / add_seq (an engine step's finishes and
 * admissions). add_seqs is all-or-nothing: RVKV_ENOMEM if the pool cannot
 * hold every prompt; ids[i] receives the new sequence ids. */
int rvkv_bm_free_seqs(rvkv_bm *bm, const int64_t *seqs, uint32_t n);
int rvkv_bm_add_seqs(rvkv_bm *bm, const uint32_t *n_tokens, uint32_t n,
                     int64_t *ids);
/* rvkv_bm_append_slot for seqs[0..n) in order (one decode step's writes,
 * rvllm's DecodeRow.write, src/engine.rs:446-451): slot i -> blocks[i],
 * offsets[i]; the copy-on-write pairs go to cow_src/cow_dst[0..*n_cow)
 * (capacity n). Stops at the first failure (its code is returned). */
int rvkv_bm_append_slots(rvkv_bm *bm, const int64_t *seqs, uint32_t n,
                         uint32_t *blocks, uint32_t *offsets,
                         uint32_t *cow_src, uint32_t *cow_dst,
                         uint32_t *n_cow);
/* The padded block tables and token counts of seqs[0..n): tables is
 * [n, max_blocks], each row padded with its last block (GatherPlan's rule,
 * src/kv_storage.rs:59-67); ctx_lens[i] = num_tokens. */
int rvkv_bm_fill_tables(const rvkv_bm *bm, const int64_t *seqs, uint32_t n,
                        uint32_t max_blocks, uint32_t *tables,
                        uint32_t *ctx_lens);
/* logical_to_physical(pos) of rvllm's BlockTable. */
int rvkv_bm_slot(const rvkv_bm *bm, int64_t seq, uint32_t pos,
                 uint32_t *block, uint32_t *offset);
uint32_t rvkv_bm_num_tokens(const rvkv_bm *bm, int64_t seq);
uint32_t rvkv_bm_num_blocks(const rvkv_bm *bm, int64_t seq);
uint32_t rvkv_bm_refcount(const rvkv_bm *bm, uint32_t block);
/* Copies the sequence's block table into table[0..cap); returns its length
 * or a negative code. */
int rvkv_bm_table(const rvkv_bm *bm, int64_t seq, uint32_t *table,
                  uint32_t cap);

/* ---- greedy token pick on the GPU --------------------------
 * out[r] = index of the maximum of logits[r * row_len ...] (f32, device):
 * ties go to the lowest index, NaN is ignored, a row with nothing above
 * -inf gives 0 - the greedy scan of Sampler::sample_slice
 * (src/sampler.rs:64-75) that rvllm's CUDA argmax kernel reproduces
 * (argmax_wrapper, src/cuda/ops.rs:516-550). Asynchronous on `stream`. */
int rvkv_argmax(const float *logits, uint32_t rows, uint32_t row_len,
                uint32_t *out, rvkv_stream stream);

/* ---- continuous-batching scheduler with prefix cache -----
 * The contract rvllm's engine uses from the kv-cache-scheduler crate (0.2.0,
 * not vendored; used at src/engine.rs:351-539): a refcounted block pool
 * (pool.available(), pool.total_allocs), FIFO `waiting` and `running`
 * lists, sequences holding token_ids and a block table, prefix_cache.
 * match_prefix, prefill(seq), step() (one more slot for every running
 * sequence, preempting from the back of `running` when the pool is empty),
 * finish_sequence(seq) and the prefix_hits / prefix_total metrics. Host
 * only; ids are int64, blocks u32. Full blocks whose tokens are final are
 * kept matchable in a prefix cache (also after release, until evicted, LRU);
 * the block of a sequence's last prompt token is never matched. Errors: -1
 * (RVKV_EINVAL) or RVKV_ENOMEM, message in rvkv_sched_last_error(). */
typedef struct rvkv_sched rvkv_sched;

const char *rvkv_sched_last_error(void);
/* Scheduler::new(num_blocks, block_size), src/engine.rs:226 */
rvkv_sched *rvkv_sched_create(uint32_t num_blocks, uint32_t block_size);
void rvkv_sched_destroy(rvkv_sched *s);
/* scheduler.add_request(tokens), src/engine.rs:314-316: queued at the back
 * of waiting; returns the sequence id. */
int64_t rvkv_sched_add_request(rvkv_sched *s, const int32_t *tokens,
                               uint32_t n);
/* pool.available() / pool.total_allocs, src/engine.rs:361, 626 */
uint32_t rvkv_sched_available(const rvkv_sched *s);
uint64_t rvkv_sched_total_allocs(const rvkv_sched *s);
/* metrics.prefix_hits / prefix_total (src/engine.rs:624-625) and the
 * number of preemptions so far; any pointer may be NULL. */
void rvkv_sched_metrics(const rvkv_sched *s, uint64_t *prefix_hits,
                        uint64_t *prefix_total, uint64_t *preemptions);
/* waiting.len() / running.len() and their contents in order (copies at
 * most cap ids, returns the length), src/engine.rs:272-282, 353-357 */
uint32_t rvkv_sched_num_waiting(const rvkv_sched *s);
uint32_t rvkv_sched_num_running(const rvkv_sched *s);
uint32_t rvkv_sched_waiting(const rvkv_sched *s, int64_t *out, uint32_t cap);
uint32_t rvkv_sched_running(const rvkv_sched *s, int64_t *out, uint32_t cap);
int rvkv_sched_has_seq(const rvkv_sched *s, int64_t id);
/* prefix_cache.match_prefix(tokens).1, src/engine.rs:365-367: the cached
 * blocks of the longest matching run of full leading blocks (copies at most
 * cap, returns the count); no side effects. */
uint32_t rvkv_sched_match_prefix(const rvkv_sched *s, const int32_t *tokens,
                                 uint32_t n, uint32_t *blocks, uint32_t cap);
/* scheduler.prefill(seq), src/engine.rs:371: gives the sequence's token_ids
 * a block table (matched prefix blocks shared, the rest allocated) and moves
 * it from waiting to running; all-or-nothing (RVKV_ENOMEM). */
int rvkv_sched_prefill(rvkv_sched *s, int64_t id, uint32_t *matched_blocks);
/* scheduler.step(), src/engine.rs:418: every running sequence gets one more
 * slot and a placeholder token; sequences are preempted from the back of
 * running (blocks released, back to the front of waiting) while the pool is
 * empty. */
int rvkv_sched_step(rvkv_sched *s, uint32_t *n_preempted);
/* Copy-on-write pairs created by step() since the last call (no
 * counterpart in the reference, which never shares a written block): if n
 * > cap nothing is copied and n is returned; run rvkv_copy_blocks on them
 * before the forward that writes the new slots. */
uint32_t rvkv_sched_take_cow(rvkv_sched *s, uint32_t *src, uint32_t *dst,
                             uint32_t cap);
/* scheduler.finish_sequence(seq) (src/engine.rs:510) and
 * sequences.remove(seq) (src/engine.rs:513); remove also finishes. */
int rvkv_sched_finish(rvkv_sched *s, int64_t id);
int rvkv_sched_remove(rvkv_sched *s, int64_t id);
/* A sequence sharing all of `parent`'s blocks (parallel sampling); a write
 * into a shared last block copies it first (see take_cow). No counterpart
 * in the reference engine. */
int64_t rvkv_sched_fork(rvkv_sched *s, int64_t parent);
/* block_table.num_tokens() / blocks() / logical_to_physical(pos) and
 * token_ids, src/engine.rs:372-382, 426-447 */
uint32_t rvkv_sched_num_tokens(const rvkv_sched *s, int64_t id);
uint32_t rvkv_sched_num_blocks(const rvkv_sched *s, int64_t id);
uint32_t rvkv_sched_table(const rvkv_sched *s, int64_t id, uint32_t *out,
                          uint32_t cap);
int rvkv_sched_slot(const rvkv_sched *s, int64_t id, uint32_t pos,
                    uint32_t *block, uint32_t *offset);
uint32_t rvkv_sched_tokens(const rvkv_sched *s, int64_t id, int32_t *out,
                           uint32_t cap);
/* Replaces token_ids (the engine's fix-ups, src/engine.rs:424-437); tokens
 * that already hold K/V must stay as they are. */
int rvkv_sched_set_tokens(rvkv_sched *s, int64_t id, const int32_t *tokens,
                          uint32_t n);
uint32_t rvkv_sched_refcount(const rvkv_sched *s, uint32_t block);

#ifdef __cplusplus
}
#endif

#endif /* RVKV_H */
