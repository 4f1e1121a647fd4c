/*
 * it_kv.h -- C ABI of the MI355X (gfx950) KV-cache hot path.
 *
 * This is the drop-in boundary for InferTrain's KV-cache path.  Every entry
 * point is `extern "C"`, takes plain pointers, sizes and a HIP stream passed
 * as `void*`, and returns a status code that mirrors the reference's OpError
 * (src/types.rs:227-231).  No call aborts: conditions the reference asserts
 * on (src/backend/arm/flash_attn.rs:16-19, quant.rs:150) return
 * IT_INVALID_INPUT, and it_last_error() holds a thread-local message.
 *
 * Memory: every tensor argument of a device entry point (it_kv_*, it_paged_*,
 * it_flash_attention) is DEVICE memory owned by the caller; work is enqueued
 * on `stream` and returns without synchronising.  Host-side objects
 * (it_block_pool, it_kv_manager) take host memory.  Device-side checks that
 * cannot be made before launch (a slot or block id out of range in a device
 * array) never fault: the access is skipped or clamped, and the condition is
 * latched in the cache and reported by it_kv_cache_check().
 *
 * dtype codes are the ggml QuantType ids of src/types.rs:106-144.
 */
#ifndef IT_KV_H
#define IT_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: OpError (src/types.rs:227-231) ----------------------- */
#define IT_OK 0
#define IT_NOT_IMPLEMENTED 1 /* OpError::NotImplemented */
#define IT_INVALID_INPUT 2   /* OpError::InvalidInput  */
#define IT_DEVICE_ERROR 3    /* OpError::DeviceError   */

/* ---- dtype codes: QuantType (src/types.rs:106-144) ---------------------- */
#define IT_F32 0
#define IT_F16 1
#define IT_Q4_0 2
#define IT_Q4_1 3
#define IT_Q5_0 6
#define IT_Q5_1 7
#define IT_Q8_0 8
#define IT_BF16 30

#define IT_BLOCK_SIZE 16        /* src/memory/paged.rs:9, default page size */
#define IT_QK8_0 32             /* src/types.rs:11 */
#define IT_BLOCK_Q8_0_BYTES 34  /* sizeof(BlockQ8_0), src/types.rs:34-41,250 */
#define IT_QK4_0 32             /* src/types.rs:7 */
#define IT_BLOCK_Q4_0_BYTES 18  /* sizeof(BlockQ4_0), src/types.rs:15-22 */
#define IT_QK4_1 32             /* src/types.rs:8 */
#define IT_BLOCK_Q4_1_BYTES 20  /* sizeof(BlockQ4_1), src/types.rs:24-32,249 */
#define IT_QK5_0 32             /* src/types.rs:9 */
#define IT_BLOCK_Q5_0_BYTES 22  /* ggml block_q5_0 {u16 d; u8 qh[4]; u8 qs[16]}: the reference has the
                                   type id (types.rs:116) and no struct */
#define IT_QK5_1 32             /* src/types.rs:10 */
#define IT_BLOCK_Q5_1_BYTES 24  /* ggml block_q5_1 {u16 d; u16 m; u8 qh[4]; u8 qs[16]} (types.rs:117) */

/* ---- operator ids for it_supports (Backend::supports_op/_quant,
 *      src/backend.rs:184-186) ------------------------------------------- */
#define IT_OP_KV_APPEND 1
#define IT_OP_KV_GATHER 2
#define IT_OP_KV_EVICT 3
#define IT_OP_PAGED_DECODE 4
#define IT_OP_PAGED_PREFILL 5
#define IT_OP_FLASH_ATTENTION 6 /* CoreOperator::FlashAttention, src/types.rs:202-208 */
#define IT_OP_KV_COPY_BLOCKS 7

/* Thread-local message for the last non-OK status on this thread. */
const char* it_last_error(void);
int32_t it_abi_version(void);
/* 1 if (op, dtype) is implemented, else 0.  dtype is the cache dtype. */
int32_t it_supports(int32_t op, int32_t dtype);

/* ======================================================================== */
/* Host: block allocator.  Replaces memory::paged::BlockPool                */
/* (src/memory/paged.rs:21-58).                                              */
/* ======================================================================== */
typedef struct it_block_pool it_block_pool;

/* BlockPool::new (paged.rs:28-34): free list 0..capacity, refcounts 0. */
int32_t it_block_pool_new(int64_t capacity, int32_t quant_type, it_block_pool** out);
/* As new, but the free list is `order` (a permutation of 0..capacity-1),
 * bottom to top, so the first allocate returns order[capacity-1]. */
int32_t it_block_pool_new_ordered(const int64_t* order, int64_t capacity, int32_t quant_type,
                                  it_block_pool** out);
void it_block_pool_destroy(it_block_pool* pool);
/* BlockPool::allocate (paged.rs:36-42): LIFO pop, refcount 1; -1 = None. */
int64_t it_block_pool_allocate(it_block_pool* pool);
/* BlockPool::share (paged.rs:44-46), with one departure: the reference
 * increments the refcount of any block, a free one included, which leaves
 * that block on the free list and referenced at once (the next allocate
 * would hand out a live block).  Here sharing a free block (refcount 0) is
 * IT_INVALID_INPUT and changes nothing. */
int32_t it_block_pool_share(it_block_pool* pool, int64_t id);
/* BlockPool::free (paged.rs:48-53); a free at refcount 0 (a u32 underflow
 * in the reference) is IT_INVALID_INPUT. */
int32_t it_block_pool_free(it_block_pool* pool, int64_t id);
/* BlockPool::quant_type (paged.rs:55-57). */
int32_t it_block_pool_quant_type(const it_block_pool* pool);
int64_t it_block_pool_num_free(const it_block_pool* pool);
int64_t it_block_pool_capacity(const it_block_pool* pool);
/* Refcount of `id`, -1 if out of range. */
int64_t it_block_pool_ref_count(const it_block_pool* pool, int64_t id);

/* ======================================================================== */
/* Host: slot mapping, block tables and sliding-window eviction.  The        */
/* reference batcher (src/batcher/continuous.rs:28-74) only admits requests; */
/* this is the per-step state it lacks.                                      */
/*   slot(pos) = table[pos / block_size] * block_size + pos % block_size     */
/*   a block is allocated from the pool when pos % block_size == 0           */
/*   window W > 0: before the token at position p, every held block whose    */
/*   last position is < p - W + 1 is released with BlockPool::free, oldest   */
/*   first; sequences are processed in the order the caller lists them.      */
/* Block tables are indexed by absolute logical block (pos / block_size).    */
/* ======================================================================== */
typedef struct it_kv_manager it_kv_manager;

/* The manager borrows `pool`; the pool must outlive it. window 0 = none. */
int32_t it_kv_manager_new(it_block_pool* pool, int32_t block_size, int32_t max_seqs,
                          int32_t max_blocks_per_seq, int32_t window, it_kv_manager** out);
void it_kv_manager_destroy(it_kv_manager* mgr);
/* Make sequence `seq` hold `blocks` (already allocated from the pool) as
 * logical blocks first_block.., with the next token at position `pos`. */
int32_t it_kv_manager_seed_seq(it_kv_manager* mgr, int32_t seq, int64_t pos, int64_t first_block,
                               const int32_t* blocks, int32_t n_blocks);
/* One step's plan, filled by it_kv_manager_step.  The caller owns every
 * array; a NULL pointer marks an output it does not want.
 * Blocks "released" by a sequence drop that sequence's reference
 * (BlockPool::free, paged.rs:48-53); only those whose refcount reaches 0
 * return to the pool.  `evicted` lists exactly those, in free order: the
 * pages to clear with it_kv_evict.  A block that another (forked) sequence
 * still holds is released but not listed, and its pages stay intact.
 * Returned blocks go back on the pool's free list when the step ends, in
 * free order, so within one step no block is both freed and handed out
 * again.  A token whose block the window returns later in the same step
 * (a step that appends more tokens than the window holds) gets slot -1:
 * it is never written.
 * Device order of a step: it_kv_copy_blocks(cow_src, cow_dst), then
 * it_kv_evict(evicted), then the append, then it_kv_sync_tables; a copy
 * source the same step returns to the pool is read before it is cleared. */
typedef struct {
  int64_t* slots;      /* [tokens_cap] slot of every new token, in list order */
  int32_t* token_seq;  /* [tokens_cap] its sequence, or NULL (it_kv_sync_tables' seq) */
  int32_t* token_pos;  /* [tokens_cap] its position, or NULL (it_kv_sync_tables' pos) */
  int32_t tokens_cap;
  int32_t n_tokens;    /* out: sum(n_tokens) */
  int32_t* evicted;    /* [evicted_cap] blocks returned to the pool by the window */
  int32_t evicted_cap;
  int32_t n_evicted;   /* out */
  int32_t* cow_src;    /* [cow_cap] copy-on-write pairs (page copies to make  */
  int32_t* cow_dst;    /*   before the append); cow_src NULL = no copy-on-write */
  int32_t cow_cap;
  int32_t n_cow;       /* out */
  int32_t* ctx_lens;   /* [max_seqs] after the step (next position), or NULL */
  int32_t* start_pos;  /* [max_seqs] after the step (window start, else 0), or NULL */
} it_kv_step_plan;

/* Append n_tokens[i] tokens to seqs[i], in list order (a sequence may be
 * listed more than once), and fill `plan`.  Sequence ids, counts and
 * tokens_cap are checked before any state changes; a later error (pool
 * exhausted, a capacity exceeded) leaves the manager state unspecified.
 * No counterpart in the reference: its batcher (continuous.rs:28-74)
 * admits requests but builds no slot mapping; this is that step. */
int32_t it_kv_manager_step(it_kv_manager* mgr, const int32_t* seqs, const int32_t* n_tokens,
                           int32_t n, it_kv_step_plan* plan);
/* it_kv_manager_step with slots (sized sum(n_tokens)) and the evicted list
 * only. */
int32_t it_kv_manager_append(it_kv_manager* mgr, const int32_t* seqs, const int32_t* n_tokens,
                             int32_t n, int64_t* slots_out, int32_t* evicted_out,
                             int32_t evicted_cap, int32_t* n_evicted);
/* Release every block of `seq` (BlockPool::free, lowest logical block
 * first) and reset it to position 0.  The blocks that return to the pool
 * (refcount 0) go to evicted_out; evicted_cap must cover every block the
 * sequence holds, else IT_INVALID_INPUT and nothing changes. */
int32_t it_kv_manager_release_seq(it_kv_manager* mgr, int32_t seq, int32_t* evicted_out,
                                  int32_t evicted_cap, int32_t* n_evicted);
/* Prefix sharing: dst takes src's blocks and position; each block gets
 * BlockPool::share (paged.rs:44-46).  dst must be empty.  The first append
 * to a shared partial block copies it (copy-on-write): the manager
 * allocates a fresh block and reports the (src, dst) pair in cow_out. */
int32_t it_kv_manager_fork(it_kv_manager* mgr, int32_t src_seq, int32_t dst_seq);
/* it_kv_manager_step with copy-on-write, slots, evicted and cow lists. */
int32_t it_kv_manager_append_cow(it_kv_manager* mgr, const int32_t* seqs, const int32_t* n_tokens,
                                 int32_t n, int64_t* slots_out, int32_t* evicted_out,
                                 int32_t evicted_cap, int32_t* n_evicted, int32_t* cow_src,
                                 int32_t* cow_dst, int32_t cow_cap, int32_t* n_cow);
/* Export tables [max_seqs][max_blocks] (-1 = not held), ctx_lens[max_seqs]
 * (= next position) and start_pos[max_seqs] (window start, else 0).  Any
 * output pointer may be NULL. */
int32_t it_kv_manager_tables(const it_kv_manager* mgr, int32_t* tables, int32_t max_blocks,
                             int32_t* ctx_lens, int32_t* start_pos);

/* ======================================================================== */
/* Device: the paged cache.  Replaces ForwardExecutor's contiguous           */
/* kv_cache_k/kv_cache_v (src/inference/forward.rs:16-19, 31-37).            */
/* Layout per pool (one for K, one for V), HBM:                              */
/*   [num_blocks][n_kv_heads] pages; a page holds block_size token rows.     */
/*   F32/F16/BF16 page: [block_size][head_dim] elements.                     */
/*   Q8_0 page: int8 qs[block_size][head_dim], then fp16 d[block_size]       */
/*   [head_dim/32] (structure of arrays of BlockQ8_0, src/types.rs:34-41).   */
/*   Q4_0 page: u8 qs[block_size][head_dim/2] (each 32-group's 16 bytes as   */
/*   in BlockQ4_0: low nibble = element j, high = element j+16), then fp16   */
/*   d[block_size][head_dim/32] (src/types.rs:15-22).                        */
/*   Q4_1 page: the Q4_0 nibble plane, then fp16 (d, m) pairs                */
/*   [block_size][head_dim/32] (BlockQ4_1, src/types.rs:24-32).              */
/*   Q5_0 / Q5_1 page: the Q4_0 nibble plane (the low four bits of each      */
/*   5-bit value), then per token a side row: head_dim/32 u32 qh words (bit  */
/*   e = bit 4 of element e, as ggml's block_q5_*), then head_dim/32 fp16 d  */
/*   (Q5_0) or (d, m) pairs (Q5_1).                                          */
/* ======================================================================== */
typedef struct it_kv_cache it_kv_cache;

typedef struct {
  void* k_pool;        /* device */
  void* v_pool;        /* device */
  int64_t num_blocks;
  int64_t page_bytes;  /* bytes of one (block, head) page */
  int32_t block_size;  /* power of two */
  int32_t n_kv_heads;
  int32_t head_dim;
  int32_t dtype;
  int32_t device;
  int32_t owns_memory;
  int32_t n_layers;    /* layers in each pool (1 for a layer view) */
} it_kv_cache_desc;

int64_t it_kv_page_bytes(int32_t block_size, int32_t head_dim, int32_t dtype);
/* Allocates both pools on `device` (hipMalloc) and zero-fills them. */
int32_t it_kv_cache_new(int32_t device, int64_t num_blocks, int32_t block_size,
                        int32_t n_kv_heads, int32_t head_dim, int32_t dtype, it_kv_cache** out);
/* Wraps caller-owned pools (num_blocks * n_kv_heads * page_bytes each,
 * 16-byte aligned).  The cache never frees them. */
int32_t it_kv_cache_wrap(int32_t device, void* k_pool, void* v_pool, int64_t num_blocks,
                         int32_t block_size, int32_t n_kv_heads, int32_t head_dim, int32_t dtype,
                         it_kv_cache** out);
/* Every layer of a model in one cache: the reference's per-layer
 * kv_cache_k/kv_cache_v (forward.rs:17-18, 36-37, indexed by layer_idx at
 * :224-228).  Each pool holds n_layers (1..4096) layers one after another,
 * [n_layers][num_blocks][n_kv_heads] pages, so one block id (one manager,
 * one block table) names the same pages in every layer.  it_kv_evict and
 * it_kv_copy_blocks on a multi-layer cache act on every layer in one
 * launch; it_kv_sync_tables and it_kv_cache_check take it as it is.  The
 * per-layer entry points (append, append_rope, gather, decode, prefill)
 * take a layer's view from it_kv_cache_layer and return IT_INVALID_INPUT
 * for a multi-layer handle. */
int32_t it_kv_cache_new_layers(int32_t device, int32_t n_layers, int64_t num_blocks, int32_t block_size,
                               int32_t n_kv_heads, int32_t head_dim, int32_t dtype, it_kv_cache** out);
/* Wraps caller-owned pools of n_layers * num_blocks * n_kv_heads * page_bytes
 * bytes each. */
int32_t it_kv_cache_wrap_layers(int32_t device, int32_t n_layers, void* k_pool, void* v_pool,
                                int64_t num_blocks, int32_t block_size, int32_t n_kv_heads,
                                int32_t head_dim, int32_t dtype, it_kv_cache** out);
/* A one-layer view of layer `layer` (no allocation on the device: the
 * view's pools point into the parent's, and it shares the parent's
 * latched-error word).  Destroy views before their parent. */
int32_t it_kv_cache_layer(const it_kv_cache* cache, int32_t layer, it_kv_cache** out);
int32_t it_kv_cache_destroy(it_kv_cache* cache);
int32_t it_kv_cache_describe(const it_kv_cache* cache, it_kv_cache_desc* out);
/* Synchronises `stream`, then reports (and clears) a latched device-side
 * error: a slot, block id or block-table entry out of range seen by an
 * earlier kernel on this cache.  IT_OK if none. */
int32_t it_kv_cache_check(it_kv_cache* cache, void* stream);

/* KV append: k_cache[slot/bs][h][slot%bs][:] = k[t][h][:], likewise v
 * (forward.rs:219-229 with seq_pos generalised to a slot mapping).
 *   k, v: [n_tokens][n_kv_heads][head_dim] of src_dtype, device.
 *   slot_mapping: int64[n_tokens], device; slot < 0 = padding, skipped.
 * F32/F16/BF16 caches take src_dtype == cache dtype (bit copy).  A Q8_0
 * cache takes F32 and quantises each 32-group exactly as
 * quantize_row_q8_0 (src/backend/arm/quant.rs:149-183).  A Q4_0 cache takes
 * F32 and quantises as ggml's quantize_row_q4_0_ref (the reference has the
 * block and its dequantisation, vec_dot.rs:425-440, but no quantiser).  A
 * Q4_1 cache takes F32 and quantises as ggml's quantize_row_q4_1_ref (the
 * reference has only the block).  Q5_0 / Q5_1 caches take F32 and quantise
 * as ggml's quantize_row_q5_0_ref / quantize_row_q5_1_ref (the reference has
 * only the type ids, types.rs:116-117). */
int32_t it_kv_append(it_kv_cache* cache, const void* k, const void* v, int32_t src_dtype,
                     const int64_t* slot_mapping, int32_t n_tokens, void* stream);

/* RoPE then append (forward.rs:195-229): rope_f32 (src/backend/arm/rope.rs:
 * 6-44) of every q and k head row at its token's position, then the rotated
 * k and the unrotated v into the cache as it_kv_append stores them.
 * The rotation's cos/sin come from `rope`, a table built once on the host
 * with the C library's float32 powf/cosf/sinf in rope_f32's order
 * (theta = (float)pos * powf(freq_base, -(float)i / n_dims) for each even
 * i < n_dims), so device results equal rope_f32's bit for bit.  Elements
 * past n_dims are not rotated (forward.rs passes n_dims = head_dim).
 *   q: F32 [n_tokens][n_heads][head_dim]; k, v: F32 [n_tokens][n_kv_heads][head_dim]
 *   positions: int32[n_tokens] in [0, max_pos) (else latched; the token writes nothing)
 *   slot_mapping: as it_kv_append (slot < 0 = padding: q still rotated)
 *   q_out: [n_tokens][n_heads][head_dim] of q_out_dtype: F32, or the cache
 *          dtype for BF16/F16 caches (round to nearest even)
 * F32 caches store the rotated fp32 values; BF16/F16 caches round them to
 * nearest even; Q8_0 / Q4_0 / Q4_1 / Q5_0 / Q5_1 caches quantise them as
 * it_kv_append does. */
typedef struct it_rope_table it_rope_table;
/* n_dims: a multiple of 4 up to 4096; positions [0, max_pos); device memory
 * max_pos * n_dims * 4 bytes. */
int32_t it_rope_table_new(int32_t device, int32_t n_dims, float freq_base, int32_t max_pos,
                          it_rope_table** out);
int32_t it_rope_table_destroy(it_rope_table* rope);
int32_t it_kv_append_rope(it_kv_cache* cache, const it_rope_table* rope, const float* q, int32_t n_heads,
                          const float* k, const float* v, const int64_t* slot_mapping,
                          const int32_t* positions, int32_t n_tokens, void* q_out, int32_t q_out_dtype,
                          void* stream);

/* Block-table gather: materialise the contiguous slices that
 * forward.rs:233-243 reads, through a block table.
 *   block_tables: int32[n_seqs][max_blocks] (absolute logical block index)
 *   ctx_lens: int32[n_seqs]; start_pos: int32[n_seqs] or NULL (all 0)
 *   cu_out: int64[n_seqs] output token offset of each sequence
 *   max_tokens: upper bound of ctx_lens[b] - start_pos[b] (sizes the grid)
 * Output for sequence b: [n_kv_heads][ctx_b - start_b][head_dim] at token
 * offset cu_out[b] (element offset cu_out[b]*n_kv_heads*head_dim).  A Q8_0
 * cache writes packed 34-byte BlockQ8_0 records, head_dim/32 per row; a Q4_0
 * cache 18-byte BlockQ4_0 records, a Q4_1 cache 20-byte BlockQ4_1 ones, Q5_0
 * and Q5_1 caches 22- and 24-byte ggml block_q5_0 / block_q5_1 records. */
int32_t it_kv_gather(const it_kv_cache* cache, const int32_t* block_tables, int32_t max_blocks,
                     const int32_t* ctx_lens, const int32_t* start_pos, const int64_t* cu_out,
                     int32_t n_seqs, int32_t max_tokens, void* k_out, void* v_out, void* stream);

/* Evict: zero every page (all heads, K and V, every layer) of the given
 * blocks, so a recycled block starts clean.  blocks: int32[n], device. */
int32_t it_kv_evict(it_kv_cache* cache, const int32_t* blocks, int32_t n, void* stream);

/* Keep a device block table in step with the slot mapping: for each token
 * i with slots[i] >= 0, tables[seq[i]][pos[i] / block_size] :=
 * slots[i] / block_size (every token of a block writes the same id).
 * tables: int32[n_seqs][max_blocks]; seq, pos: int32[n]; slots:
 * int64[n]; all device.  Out-of-range entries are skipped and latched
 * (it_kv_cache_check). */
int32_t it_kv_sync_tables(it_kv_cache* cache, int32_t* tables, int32_t max_blocks, int32_t n_seqs,
                          const int32_t* seq, const int32_t* pos, const int64_t* slots, int32_t n,
                          void* stream);

/* Copy-on-write page copy: block dst[i] := block src[i] (all heads, K, V,
 * every layer). */
int32_t it_kv_copy_blocks(it_kv_cache* cache, const int32_t* src, const int32_t* dst, int32_t n,
                          void* stream);

/* ======================================================================== */
/* Device: attention over the cache.                                         */
/* ======================================================================== */
/* Workspace bytes it_paged_decode needs (fp32 partial (m, l, O) for every
 * (sequence, head, partition)). */
size_t it_paged_decode_workspace(int32_t n_seqs, int32_t n_heads, int32_t head_dim,
                                 int32_t max_tokens, int32_t partition);

/* Partition (tokens per split) for it_paged_decode over contexts the caller
 * knows on the host, as a batcher does: the smallest multiple of 64 in
 * [64, 2048] whose non-empty (sequence, KV head, partition) units run in the
 * fewest rounds of four resident workgroups per compute unit.  Short
 * partitions keep each workgroup's chain of dependent page loads short;
 * units beyond the resident slots would run a second round.  A batch that
 * needs more than two rounds at any size takes the longest partition that
 * keeps two workgroups per compute unit instead (fewest partials).
 *   ctx_lens, start_pos: host int32[n_seqs] (start_pos may be NULL)
 *   n_cu: compute units of the device (0 = ask the current HIP device)
 * No counterpart in the reference: flash_attn_f32 (flash_attn.rs:6-72) does
 * not split keys.  Its caller is the batcher's step (continuous.rs:28-74),
 * which holds the lengths. */
int32_t it_paged_decode_partition(int32_t dtype, int32_t head_dim, int32_t block_size, int32_t n_heads,
                                  int32_t n_kv_heads, const int32_t* ctx_lens, const int32_t* start_pos,
                                  int32_t n_seqs, int32_t n_cu, int32_t* partition);

/* Paged split-K flash-decode, one query per sequence.  For each sequence b
 * and query head h the result equals flash_attn_f32 (flash_attn.rs:6-72)
 * over keys start_b..ctx_b-1 of KV head h*Hkv/Hq (forward.rs:231-254),
 * within fp32 tolerance.
 *   q: [n_seqs][n_heads][head_dim]; q_dtype F32 (F32 and quantised caches),
 *      BF16 (BF16 cache) or F16 (F16 cache); 16-byte aligned
 *   block_tables/ctx_lens/start_pos: as it_kv_gather
 *   max_tokens: upper bound of ctx_b - start_b
 *   partition: tokens per split, a multiple of 64 in [64, 2048]
 *              (it_paged_decode_partition picks one for a batch)
 *   ws: it_paged_decode_workspace(...) bytes, device, 256-byte aligned
 *   out: [n_seqs][n_heads][head_dim] of out_dtype (F32 or q_dtype); 8-byte
 *        aligned for F32, 4-byte for 16-bit types
 * Two kernels: the split pass writes (m, l, O) per partition, the combine
 * pass merges them.  n_heads must be a multiple of n_kv_heads. */
int32_t it_paged_decode(const it_kv_cache* cache, const void* q, int32_t q_dtype, int32_t n_heads,
                        const int32_t* block_tables, int32_t max_blocks, const int32_t* ctx_lens,
                        const int32_t* start_pos, int32_t n_seqs, int32_t max_tokens, float scale,
                        int32_t partition, void* ws, size_t ws_bytes, void* out,
                        int32_t out_dtype, void* stream);

/* The two passes of it_paged_decode as separate launches, same arguments:
 * it_paged_decode_split then it_paged_decode_combine on one stream equals
 * it_paged_decode (lets a caller time or schedule the passes apart). */
int32_t it_paged_decode_split(const it_kv_cache* cache, const void* q, int32_t q_dtype, int32_t n_heads,
                              const int32_t* block_tables, int32_t max_blocks, const int32_t* ctx_lens,
                              const int32_t* start_pos, int32_t n_seqs, int32_t max_tokens, float scale,
                              int32_t partition, void* ws, size_t ws_bytes, void* out, int32_t out_dtype,
                              void* stream);
int32_t it_paged_decode_combine(const it_kv_cache* cache, const void* q, int32_t q_dtype, int32_t n_heads,
                                const int32_t* block_tables, int32_t max_blocks, const int32_t* ctx_lens,
                                const int32_t* start_pos, int32_t n_seqs, int32_t max_tokens, float scale,
                                int32_t partition, void* ws, size_t ws_bytes, void* out, int32_t out_dtype,
                                void* stream);

/* it_paged_decode without a workspace argument.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * partials live in a 32 MiB device array of the library (one per GPU, held
 * until the process ends); a call that needs more than that
 * (it_paged_decode_workspace > 32 MiB) is IT_INVALID_INPUT.  It allocates
 * nothing: the array's device address is looked up once per device, on the
 * first call there.  Calls on one GPU share the array, so calls that
 * overlap in time on one GPU (different streams) race.  Other arguments and
 * results as it_paged_decode. */
int32_t it_paged_decode_noalloc(const it_kv_cache* cache, const void* q, int32_t q_dtype, int32_t n_heads,
                                const int32_t* block_tables, int32_t max_blocks, const int32_t* ctx_lens,
                                const int32_t* start_pos, int32_t n_seqs, int32_t max_tokens, float scale,
                                int32_t partition, void* out, int32_t out_dtype, void* stream);

/* Chunked prefill attention over the cache (the chunk's K/V already
 * appended).  Sequence b has q_len_b = cu_q[b+1]-cu_q[b] query rows at
 * positions ctx_b - q_len_b + i; with causal != 0 row i attends keys
 * 0..ctx_b - q_len_b + i, else all ctx_b keys.
 *   q/out: [cu_q[n_seqs]][n_heads][head_dim], BF16 q; out F32 or BF16
 *   cu_q: int32[n_seqs+1], device; max_q_len bounds q_len_b. */
int32_t it_paged_prefill(const it_kv_cache* cache, const void* q, int32_t q_dtype, int32_t n_heads,
                         const int32_t* cu_q, int32_t max_q_len, const int32_t* block_tables,
                         int32_t max_blocks, const int32_t* ctx_lens, int32_t n_seqs, float scale,
                         int32_t causal, void* out, int32_t out_dtype, void* stream);

/* CoreOperator::FlashAttention as ArmCpuBackend executes it
 * (src/backend/arm.rs:304-370): every one of n_heads query heads attends
 * the same K/V [n_kv][head_dim] with scale 1/sqrtf(head_dim) and an
 * optional additive mask [n_kv] (NULL = none; -inf skips the key).
 *   q/out: [n_heads][head_dim] F32; k, v: [n_kv][head_dim] F32; device.
 *   ws: it_flash_attention_workspace(...) bytes, device. */
size_t it_flash_attention_workspace(int32_t n_heads, int32_t head_dim, int32_t n_kv);
int32_t it_flash_attention(const float* q, const float* k, const float* v, const float* mask,
                           float* out, int32_t n_heads, int32_t head_dim, int32_t n_kv, void* ws,
                           size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* IT_KV_H */
