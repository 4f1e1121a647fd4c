/*
 * it_oracle.h -- CPU oracle for the KV-cache hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * crate's CPU arithmetic (OpenMachineware/infer_train, Rust).  It is the
 * checker that the HIP library is compared against and the CPU baseline that
 * bench.py times.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library (libit_kv.so) never
 * links, loads or calls it.
 *
 * Every function names the reference file:line it follows.  Functions that
 * restate behaviour the reference does not have (slot mapping, paged reads,
 * window eviction, chunked prefill) are defined here as compositions of the
 * reference functions and say so.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math), because
 * Rust never contracts a*b+c into an FMA.
 */
#ifndef IT_ORACLE_H
#define IT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes, same values as the product ABI (OpError, types.rs:227-231). */
#define ORC_OK 0
#define ORC_NOT_IMPLEMENTED 1
#define ORC_INVALID_INPUT 2

/* dtype codes = ggml QuantType ids (types.rs:106-144). */
#define ORC_F32 0
#define ORC_F16 1
#define ORC_Q4_0 2
#define ORC_Q4_1 3
#define ORC_Q5_0 6
#define ORC_Q5_1 7
#define ORC_Q8_0 8
#define ORC_BF16 30

#define ORC_QK8_0 32          /* types.rs:11 */
#define ORC_BLOCK_Q8_0_BYTES 34 /* types.rs:34-41: repr(C) {u16 d; i8 qs[32]} */
#define ORC_QK4_0 32          /* types.rs:7 */
#define ORC_BLOCK_Q4_0_BYTES 18 /* types.rs:15-22: repr(C) {u16 d; u8 qs[16]} */
#define ORC_QK4_1 32          /* types.rs:8 */
#define ORC_BLOCK_Q4_1_BYTES 20 /* types.rs:24-32, size asserted at :249: {u16 d; u16 m; u8 qs[16]} */
#define ORC_QK5_0 32          /* types.rs:9 */
#define ORC_BLOCK_Q5_0_BYTES 22 /* ggml block_q5_0: {u16 d; u8 qh[4]; u8 qs[16]} (no struct in the reference) */
#define ORC_QK5_1 32          /* types.rs:10 */
#define ORC_BLOCK_Q5_1_BYTES 24 /* ggml block_q5_1: {u16 d; u16 m; u8 qh[4]; u8 qs[16]} */

/* ---- seeded synthetic inputs (not a reference function: test plumbing) -- */
uint64_t orc_splitmix64(uint64_t* state);
/* N(0,1) via Box-Muller in double, rounded to f32. */
void orc_fill_normal_f32(uint64_t seed, float* out, size_t n);
/* Uniform integers in [lo, hi] (inclusive). */
void orc_fill_uniform_i32(uint64_t seed, int32_t lo, int32_t hi, int32_t* out, size_t n);
/* Fisher-Yates permutation of 0..n-1. */
void orc_permutation_i64(uint64_t seed, int64_t* out, size_t n);

/* ---- scalar conversions ------------------------------------------------- */
/* fp32 -> fp16 round-to-nearest-even (half 2.7.1 f16::from_f32, called by
 * fp32_to_fp16, types.rs:237-240). */
uint16_t orc_f32_to_f16(float f);
/* fp16 -> fp32, exact (types.rs:233-235). */
float orc_f16_to_f32(uint16_t h);
/* fp32 -> bf16 round-to-nearest-even (NaN kept quiet). */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_bf16_array(const float* in, uint16_t* out, size_t n);
void orc_bf16_to_f32_array(const uint16_t* in, float* out, size_t n);
void orc_f32_to_f16_array(const float* in, uint16_t* out, size_t n);
void orc_f16_to_f32_array(const uint16_t* in, float* out, size_t n);

/* ---- BlockPool (src/memory/paged.rs:21-58) ------------------------------ */
typedef struct orc_block_pool orc_block_pool;
/* paged.rs:28-34: free_list = 0..capacity, all refcounts 0. */
orc_block_pool* orc_pool_new(int64_t capacity, int32_t quant_type);
/* Same pool, but the free list holds `order` (a permutation of 0..cap-1), so
 * allocate() pops order[cap-1] first.  Used for the configs' "seeded random
 * permutation of the pool". */
orc_block_pool* orc_pool_new_ordered(const int64_t* order, int64_t capacity, int32_t quant_type);
void orc_pool_destroy(orc_block_pool* p);
/* paged.rs:36-42: LIFO pop, refcount := 1.  Returns -1 for None. */
int64_t orc_pool_allocate(orc_block_pool* p);
/* paged.rs:44-46: refcount += 1.  ORC_INVALID_INPUT on a bad id or ref 0. */
int orc_pool_share(orc_block_pool* p, int64_t id);
/* paged.rs:48-53: refcount -= 1, push on 0.  The reference underflows a u32
 * on ref 0; here that is ORC_INVALID_INPUT. */
int orc_pool_free(orc_block_pool* p, int64_t id);
int32_t orc_pool_quant_type(const orc_block_pool* p); /* paged.rs:55-57 */
int64_t orc_pool_num_free(const orc_block_pool* p);
int64_t orc_pool_ref_count(const orc_block_pool* p, int64_t id);
/* Copies the free list bottom..top into out (n = num_free). */
void orc_pool_free_list(const orc_block_pool* p, int64_t* out);

/* ---- Q8_0 (src/backend/arm/quant.rs:149-183, x86 scalar path) ----------- */
/* x: n floats (n % 32 == 0); y: n/32 packed 34-byte BlockQ8_0 records. */
int orc_quantize_row_q8_0(const float* x, size_t n, uint8_t* y);
/* Dequant semantics fp16_to_fp32(d) * q (gemv.rs:48-59, 151-160). */
void orc_dequantize_row_q8_0(const uint8_t* y, size_t n, float* x);

/* ---- Q4_0 ---------------------------------------------------------------- */
/* The reference fixes the block (types.rs:15-22) and its dequantisation
 * (vec_dot.rs:425-440): element j of a group is the low nibble of qs[j],
 * element j + 16 the high nibble, value fp16_to_fp32(d) * (nibble - 8).  It
 * has no Q4_0 quantiser; orc_quantize_row_q4_0 restates ggml's
 * quantize_row_q4_0_ref (ggml-quants.c, the library whose block_q4_0 the
 * reference's BlockQ4_0 mirrors; not vendored): max = the first element of
 * largest magnitude, d = max / -8, id = d ? 1/d : 0, nibble =
 * min(15, (int8_t)(x * id + 8.5f)), d stored as fp16 (RNE). */
int orc_quantize_row_q4_0(const float* x, size_t n, uint8_t* y);
void orc_dequantize_row_q4_0(const uint8_t* y, size_t n, float* x);

/* ---- Q4_1 ---------------------------------------------------------------- */
/* The reference fixes only the block (types.rs:24-32, 20 bytes, :249); no
 * code in it reads or writes one.  Restated from ggml (ggml-quants.c, not
 * vendored): quantize_row_q4_1_ref -- min / max of the group (NaN never
 * wins), d = (max - min) / 15, id = d ? 1/d : 0, nibble = min(15,
 * (int8_t)((x - min) * id + 0.5f)), d and m = min stored as fp16 (RNE), the
 * nibble order of Q4_0; dequantize_row_q4_1 -- value = f32(d) * nibble +
 * f32(m), product and sum rounded separately. */
int orc_quantize_row_q4_1(const float* x, size_t n, uint8_t* y);
void orc_dequantize_row_q4_1(const uint8_t* y, size_t n, float* x);

/* ---- Q5_0 / Q5_1 ----------------------------------------------------------- */
/* The reference names the types (QuantType::Q5_0 = 6, Q5_1 = 7, types.rs:
 * 116-117; KV cache formats in tools/bench.rs:66-68, 188-203) and their
 * group size (types.rs:9-10) but has no block struct and no code for them.
 * Restated from ggml (ggml-quants.c, not vendored).  A 5-bit value of
 * element e of a group is its nibble (low nibble of qs[e] for e < 16, high
 * nibble of qs[e - 16] otherwise) plus 16 x bit e of the little-endian u32
 * qh.  quantize_row_q5_0_ref: max = the first element of largest magnitude,
 * d = max / -16, id = d ? 1/d : 0, q = min(31, (int8_t)(x * id + 16.5f)),
 * value f32(d) * (q - 16).  quantize_row_q5_1_ref: min / max (strict
 * compares), d = (max - min) / 31, id = d ? 1/d : 0, q = (uint8_t)((x -
 * min) * id + 0.5f) (no clamp), value f32(d) * q + f32(m), product and sum
 * rounded separately.  d and m = min stored as fp16 (RNE). */
int orc_quantize_row_q5_0(const float* x, size_t n, uint8_t* y);
void orc_dequantize_row_q5_0(const uint8_t* y, size_t n, float* x);
int orc_quantize_row_q5_1(const float* x, size_t n, uint8_t* y);
void orc_dequantize_row_q5_1(const uint8_t* y, size_t n, float* x);

/* ---- RoPE (src/backend/arm/rope.rs:6-44) -------------------------------- */
/* out = x rotated pairwise: for each head row of head_dim floats and each
 * even i < n_dims, theta = (float)pos * powf(freq_base, -(float)i / n_dims),
 * (x[i], x[i+1]) -> (x0 cos - x1 sin, x0 sin + x1 cos), float32 throughout,
 * cosf/sinf/powf of the C library, no FMA.  Elements past n_dims are
 * copied.  n = number of floats (a multiple of head_dim). */
int orc_rope_f32(const float* x, float* out, size_t n, int64_t pos, int32_t n_dims, int32_t head_dim,
                 float freq_base);

/* ---- attention ---------------------------------------------------------- */
/* src/backend/arm/flash_attn.rs:6-72, same operation order. mask may be NULL. */
void orc_flash_attn_f32(const float* q, const float* k, const float* v, const float* mask,
                        float* out, int32_t head_dim, int32_t n_kv, float scale);

/* ArmCpuBackend FlashAttention arm (src/backend/arm.rs:304-370): all n_heads
 * share one K/V [n_kv][head_dim]; optional mask [n_kv]; scale 1/sqrtf(D). */
int orc_backend_flash_attention(const float* q, const float* k, const float* v,
                                const float* mask, float* out, int32_t n_heads,
                                int32_t head_dim, int32_t n_kv);

/* ---- paged cache restatement ------------------------------------------- */
/* Pool layout: [num_blocks][n_kv_heads][block_size][head_dim] elements of
 * elem_bytes each, one pool for K and one for V.  For Q8_0 each
 * (block, head) page holds block_size*head_dim int8 values followed by
 * block_size*head_dim/32 fp16 scales (slot-major).  Q4_0 likewise:
 * block_size*head_dim/2 bytes of nibbles (each 32-group's 16 bytes in
 * BlockQ4_0 order), then block_size*head_dim/32 fp16 scales.  Q4_1: the
 * nibbles, then per token and group the fp16 pair (d, m).  Q5_0 / Q5_1:
 * the nibbles, then per token a side row of head_dim/32 u32 qh words
 * followed by head_dim/32 fp16 d (Q5_0) or (d, m) pairs (Q5_1). */
typedef struct {
  int64_t num_blocks;
  int32_t block_size;
  int32_t n_kv_heads;
  int32_t head_dim;
  int32_t dtype;
} orc_cache_desc;

size_t orc_page_bytes(const orc_cache_desc* c);

/* KV append (forward.rs:219-229 generalised from `seq_pos` to a slot):
 * k_cache[slot/bs][h][slot%bs][:] = k[t][h][:].  Negative slots are skipped.
 * F32/F16/BF16: bit copy (src dtype == cache dtype).  Q8_0 / Q4_0: src is
 * f32 and each 32-group is quantised with orc_quantize_row_q8_0 / _q4_0. */
int orc_kv_append(const orc_cache_desc* c, uint8_t* k_pool, uint8_t* v_pool,
                  const void* k, const void* v, const int64_t* slots, int32_t n_tokens);

/* Block-table gather: the contiguous slice k_cache[kv][start..ctx] of
 * forward.rs:233-243 read through a block table.  Output per sequence b is
 * [n_kv_heads][ctx_b - start_b][head_dim] at token offset cu_out[b].  Q8_0
 * outputs packed 34-byte BlockQ8_0 records, Q4_0 18-byte BlockQ4_0 ones. */
int orc_kv_gather(const orc_cache_desc* c, const uint8_t* k_pool, const uint8_t* v_pool,
                  const int32_t* block_tables, int32_t max_blocks, const int32_t* ctx_lens,
                  const int32_t* start_pos, const int64_t* cu_out, int32_t n_seqs,
                  void* k_out, void* v_out);

/* Evict: zero the pages of the given blocks (all heads, K and V). */
int orc_kv_evict(const orc_cache_desc* c, uint8_t* k_pool, uint8_t* v_pool,
                 const int32_t* blocks, int32_t n);

/* Paged decode: for each seq b and q-head h, flash_attn_f32 over the
 * widened (bf16/f16 -> f32, Q8_0 -> f32(d)*q, Q4_0 -> f32(d)*(n-8)) keys
 * start_b..ctx_b-1 of KV
 * head h*Hkv/Hq (forward.rs:231-254).  q: [n_seqs][n_heads][D] f32,
 * out: [n_seqs][n_heads][D] f32.  start_pos may be NULL (all zero). */
int orc_paged_decode(const orc_cache_desc* c, const uint8_t* k_pool, const uint8_t* v_pool,
                     const float* q, int32_t n_heads, const int32_t* block_tables,
                     int32_t max_blocks, const int32_t* ctx_lens, const int32_t* start_pos,
                     int32_t n_seqs, float scale, float* out);

/* The same results as orc_paged_decode, computed on n_threads host threads
 * (OpenMP over the (sequence, KV head) pairs; each pair's query heads run
 * flash_attn_f32 exactly as above).  For the all-cores CPU baseline: the
 * reference itself is single-threaded. */
int orc_paged_decode_mt(const orc_cache_desc* c, const uint8_t* k_pool, const uint8_t* v_pool,
                        const float* q, int32_t n_heads, const int32_t* block_tables,
                        int32_t max_blocks, const int32_t* ctx_lens, const int32_t* start_pos,
                        int32_t n_seqs, float scale, float* out, int32_t n_threads);

/* Chunked prefill, causal: query row i of sequence b sits at position
 * ctx_b - q_len_b + i and runs flash_attn_f32 over keys 0..that position
 * (n_kv = cached + i + 1).  q/out: [total_q][n_heads][D] f32, rows of seq b
 * at cu_q[b]..cu_q[b+1]. causal=0 attends all ctx_b keys. */
int orc_paged_prefill(const orc_cache_desc* c, const uint8_t* k_pool, const uint8_t* v_pool,
                      const float* q, int32_t n_heads, const int32_t* cu_q,
                      const int32_t* block_tables, int32_t max_blocks, const int32_t* ctx_lens,
                      int32_t n_seqs, float scale, int32_t causal, float* out);
/* Same, only rows [row_begin,row_end) of sequence `seq` (CPU baseline sample). */
int orc_paged_prefill_rows(const orc_cache_desc* c, const uint8_t* k_pool, const uint8_t* v_pool,
                           const float* q, int32_t n_heads, const int32_t* cu_q,
                           const int32_t* block_tables, int32_t max_blocks,
                           const int32_t* ctx_lens, int32_t seq, int32_t row_begin,
                           int32_t row_end, float scale, int32_t causal, float* out);
/* orc_paged_prefill_rows on n_threads host threads (OpenMP over the rows of
 * each KV head); same results. */
int orc_paged_prefill_rows_mt(const orc_cache_desc* c, const uint8_t* k_pool, const uint8_t* v_pool,
                              const float* q, int32_t n_heads, const int32_t* cu_q,
                              const int32_t* block_tables, int32_t max_blocks,
                              const int32_t* ctx_lens, int32_t seq, int32_t row_begin,
                              int32_t row_end, float scale, int32_t causal, float* out,
                              int32_t n_threads);

/* ---- sequence / window manager (restated on BlockPool) ----------------- */
/* Slot rule: slot = table[pos / bs] * bs + pos % bs; a new block is taken
 * from the pool (paged.rs:36-42) when pos % bs == 0.  With window W > 0,
 * before each token at position p every block whose last position is
 * < p - W + 1 is released with BlockPool::free (paged.rs:48-53), oldest
 * first.  Sequences of one step are processed in the order given. */
typedef struct orc_kv_manager orc_kv_manager;
orc_kv_manager* orc_mgr_new(orc_block_pool* pool, int32_t block_size, int32_t max_seqs,
                            int32_t max_blocks_per_seq, int32_t window);
void orc_mgr_destroy(orc_kv_manager* m);
/* Start sequence s at position `pos` holding the blocks `blocks` for logical
 * blocks first_block..first_block+n-1 (already allocated by the caller). */
int orc_mgr_seed_seq(orc_kv_manager* m, int32_t s, int64_t pos, int64_t first_block,
                     const int32_t* blocks, int32_t n);
/* Append n_tokens[i] tokens to sequence seqs[i], i = 0..n-1 in order.
 * Writes sum(n_tokens) slots and, in free order, the ids of the blocks the
 * window returned to the pool (refcount 0); a released block that another
 * sequence still holds is not listed.  Returned blocks go back on the free
 * list when the step ends (none is freed and handed out again within one
 * step), and the step's tokens inside them get slot -1 (dead). */
int orc_mgr_append(orc_kv_manager* m, const int32_t* seqs, const int32_t* n_tokens, int32_t n,
                   int64_t* slots_out, int32_t* evicted_out, int32_t evicted_cap,
                   int32_t* n_evicted);
/* As orc_mgr_append; with cow != 0 a token written into a partial block
 * whose refcount is > 1 first moves its sequence to a fresh block and lists
 * the (shared, fresh) pair in cow_src/cow_dst (the page copy to make). */
int orc_mgr_append_cow(orc_kv_manager* m, const int32_t* seqs, const int32_t* n_tokens, int32_t n,
                       int32_t cow, int64_t* slots_out, int32_t* evicted_out, int32_t evicted_cap,
                       int32_t* n_evicted, int32_t* cow_src, int32_t* cow_dst, int32_t cow_cap,
                       int32_t* n_cow);
/* Prefix sharing: empty sequence dst takes src's blocks (BlockPool::share,
 * paged.rs:44-46) and position. */
int orc_mgr_fork(orc_kv_manager* m, int32_t src, int32_t dst);
/* Sequence s drops every block (BlockPool::free, lowest logical block
 * first) and restarts at position 0; the blocks returned to the pool are
 * listed. */
int orc_mgr_release(orc_kv_manager* m, int32_t s, int32_t* evicted_out, int32_t evicted_cap,
                    int32_t* n_evicted);
/* Export block tables (absolute logical index, -1 = not held), positions
 * (ctx lens) and window starts. */
int orc_mgr_tables(const orc_kv_manager* m, int32_t* tables, int32_t max_blocks,
                   int32_t* ctx_lens, int32_t* start_pos);

#ifdef __cplusplus
}
#endif
#endif
