// it_host.cpp -- host side of the KV-cache path: block allocator, slot
// mapping / block tables / sliding-window eviction, and the thread-local
// error channel of the C ABI.  No device code here.
//
// Objects are not internally locked: like `&mut self` in the Rust reference,
// concurrent mutation of one pool or manager is the caller's to serialise.
#include <cstdarg>
#include <climits>
#include <cstdio>
#include <algorithm>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "it_kv.h"
#include "it_internal.hpp"

namespace {
thread_local std::string g_last_error;
}

namespace itkv {
int32_t fail(int32_t code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}
}  // namespace itkv

using itkv::fail;

extern "C" const char* it_last_error(void) { return g_last_error.c_str(); }
extern "C" int32_t it_abi_version(void) { return 1; }

// ---------------------------------------------------------------------------
// BlockPool -- src/memory/paged.rs:21-58
// ---------------------------------------------------------------------------
struct it_block_pool {
  std::vector<int64_t> free_list;   // Vec<usize>: top of the stack is back()
  std::vector<uint32_t> ref_counts; // Vec<u32>
  int32_t quant_type;
};

extern "C" int32_t it_block_pool_new(int64_t capacity, int32_t quant_type, it_block_pool** out) {
  if (!out) return fail(IT_INVALID_INPUT, "it_block_pool_new: out is NULL");
  *out = nullptr;
  if (capacity < 0 || capacity > (int64_t(1) << 31))
    return fail(IT_INVALID_INPUT, "it_block_pool_new: capacity %lld out of range", (long long)capacity);
  auto* p = new (std::nothrow) it_block_pool;
  if (!p) return fail(IT_DEVICE_ERROR, "it_block_pool_new: out of host memory");
  // paged.rs:28-34: free_list = (0..capacity).collect(), ref_counts = 0.
  p->free_list.resize(size_t(capacity));
  for (int64_t i = 0; i < capacity; ++i) p->free_list[size_t(i)] = i;
  p->ref_counts.assign(size_t(capacity), 0u);
  p->quant_type = quant_type;
  *out = p;
  return IT_OK;
}

extern "C" int32_t it_block_pool_new_ordered(const int64_t* order, int64_t capacity,
                                             int32_t quant_type, it_block_pool** out) {
  if (!order && capacity > 0) return fail(IT_INVALID_INPUT, "it_block_pool_new_ordered: order is NULL");
  int32_t rc = it_block_pool_new(capacity, quant_type, out);
  if (rc) return rc;
  std::vector<char> seen(size_t(capacity), 0);
  for (int64_t i = 0; i < capacity; ++i) {
    int64_t id = order[i];
    if (id < 0 || id >= capacity || seen[size_t(id)]) {
      delete *out;
      *out = nullptr;
      return fail(IT_INVALID_INPUT, "it_block_pool_new_ordered: order is not a permutation (index %lld)",
                  (long long)i);
    }
    seen[size_t(id)] = 1;
    (*out)->free_list[size_t(i)] = id;
  }
  return IT_OK;
}

extern "C" void it_block_pool_destroy(it_block_pool* pool) { delete pool; }

extern "C" int64_t it_block_pool_allocate(it_block_pool* pool) {
  // paged.rs:36-42: Vec::pop (the LAST element), refcount := 1; None -> -1.
  if (!pool || pool->free_list.empty()) return -1;
  int64_t id = pool->free_list.back();
  pool->free_list.pop_back();
  pool->ref_counts[size_t(id)] = 1;
  return id;
}

extern "C" int32_t it_block_pool_share(it_block_pool* pool, int64_t id) {
  // paged.rs:44-46
  if (!pool) return fail(IT_INVALID_INPUT, "it_block_pool_share: pool is NULL");
  if (id < 0 || id >= int64_t(pool->ref_counts.size()))
    return fail(IT_INVALID_INPUT, "it_block_pool_share: block %lld out of range", (long long)id);
  if (pool->ref_counts[size_t(id)] == 0)
    return fail(IT_INVALID_INPUT, "it_block_pool_share: block %lld is free", (long long)id);
  pool->ref_counts[size_t(id)] += 1;
  return IT_OK;
}

extern "C" int32_t it_block_pool_free(it_block_pool* pool, int64_t id) {
  // paged.rs:48-53; the reference's u32 underflow at refcount 0 is an error.
  if (!pool) return fail(IT_INVALID_INPUT, "it_block_pool_free: pool is NULL");
  if (id < 0 || id >= int64_t(pool->ref_counts.size()))
    return fail(IT_INVALID_INPUT, "it_block_pool_free: block %lld out of range", (long long)id);
  uint32_t& rc = pool->ref_counts[size_t(id)];
  if (rc == 0) return fail(IT_INVALID_INPUT, "it_block_pool_free: block %lld already free", (long long)id);
  rc -= 1;
  if (rc == 0) pool->free_list.push_back(id);
  return IT_OK;
}

namespace {
// The manager's step holds back the free-list push of the blocks it
// returns until the step ends: it_block_pool_free pushed `id` last, so it
// is the top of the stack.
void it_block_pool_unpush(it_block_pool* pool, int64_t id) {
  if (!pool->free_list.empty() && pool->free_list.back() == id) pool->free_list.pop_back();
}
void it_block_pool_push(it_block_pool* pool, int64_t id) { pool->free_list.push_back(id); }
}  // namespace

extern "C" int32_t it_block_pool_quant_type(const it_block_pool* pool) {
  return pool ? pool->quant_type : -1;  // paged.rs:55-57
}
extern "C" int64_t it_block_pool_num_free(const it_block_pool* pool) {
  return pool ? int64_t(pool->free_list.size()) : -1;
}
extern "C" int64_t it_block_pool_capacity(const it_block_pool* pool) {
  return pool ? int64_t(pool->ref_counts.size()) : -1;
}
extern "C" int64_t it_block_pool_ref_count(const it_block_pool* pool, int64_t id) {
  if (!pool || id < 0 || id >= int64_t(pool->ref_counts.size())) return -1;
  return int64_t(pool->ref_counts[size_t(id)]);
}

// ---------------------------------------------------------------------------
// Slot mapping, block tables, sliding window, prefix sharing.
// ---------------------------------------------------------------------------
struct it_kv_manager {
  it_block_pool* pool;
  int32_t bs, max_seqs, max_blocks, window;
  std::vector<int32_t> table;  // [max_seqs][max_blocks], -1 = not held
  std::vector<int64_t> pos;    // next position of each sequence (= ctx len)
  std::vector<int64_t> first;  // lowest logical block still held
  // Scratch of one step, reused across steps.
  std::vector<int32_t> pending;    // blocks the step returned to the pool, in free order
  std::vector<uint32_t> blk_step;  // [pool capacity] step number of a block's first write...
  std::vector<int32_t> blk_first;  // ...and the output index of that write
  uint32_t step = 0;
};

extern "C" int32_t it_kv_manager_new(it_block_pool* pool, int32_t block_size, int32_t max_seqs,
                                     int32_t max_blocks_per_seq, int32_t window,
                                     it_kv_manager** out) {
  if (!out) return fail(IT_INVALID_INPUT, "it_kv_manager_new: out is NULL");
  *out = nullptr;
  if (!pool) return fail(IT_INVALID_INPUT, "it_kv_manager_new: pool is NULL");
  if (block_size <= 0 || max_seqs <= 0 || max_blocks_per_seq <= 0 || window < 0)
    return fail(IT_INVALID_INPUT, "it_kv_manager_new: bad shape (bs=%d seqs=%d blocks=%d window=%d)",
                block_size, max_seqs, max_blocks_per_seq, window);
  auto* m = new (std::nothrow) it_kv_manager;
  if (!m) return fail(IT_DEVICE_ERROR, "it_kv_manager_new: out of host memory");
  m->pool = pool;
  m->bs = block_size;
  m->max_seqs = max_seqs;
  m->max_blocks = max_blocks_per_seq;
  m->window = window;
  m->table.assign(size_t(max_seqs) * size_t(max_blocks_per_seq), -1);
  m->pos.assign(size_t(max_seqs), 0);
  m->first.assign(size_t(max_seqs), 0);
  m->blk_step.assign(size_t(it_block_pool_capacity(pool)), 0u);
  m->blk_first.assign(size_t(it_block_pool_capacity(pool)), 0);
  *out = m;
  return IT_OK;
}

extern "C" void it_kv_manager_destroy(it_kv_manager* mgr) { delete mgr; }

extern "C" int32_t it_kv_manager_seed_seq(it_kv_manager* m, int32_t seq, int64_t pos,
                                          int64_t first_block, const int32_t* blocks,
                                          int32_t n_blocks) {
  if (!m) return fail(IT_INVALID_INPUT, "it_kv_manager_seed_seq: manager is NULL");
  if (seq < 0 || seq >= m->max_seqs || first_block < 0 || n_blocks < 0 ||
      first_block + n_blocks > m->max_blocks || pos < 0)
    return fail(IT_INVALID_INPUT, "it_kv_manager_seed_seq: seq %d / blocks [%lld, +%d) out of range", seq,
                (long long)first_block, n_blocks);
  int32_t* row = &m->table[size_t(seq) * size_t(m->max_blocks)];
  for (int32_t j = 0; j < m->max_blocks; ++j) row[j] = -1;
  for (int32_t j = 0; j < n_blocks; ++j) row[first_block + j] = blocks[j];
  m->pos[size_t(seq)] = pos;
  m->first[size_t(seq)] = first_block;
  return IT_OK;
}

namespace {
// Exports ctx_lens / start_pos of every sequence slot (either may be NULL).
void export_lengths(const it_kv_manager* m, int32_t* ctx_lens, int32_t* start_pos) {
  for (int32_t s = 0; s < m->max_seqs; ++s) {
    if (ctx_lens) ctx_lens[s] = int32_t(m->pos[size_t(s)]);
    if (start_pos) {
      const int64_t st = m->window > 0 ? m->pos[size_t(s)] - m->window : 0;
      start_pos[s] = int32_t(st > 0 ? st : 0);
    }
  }
}

// BlockPool::free (paged.rs:48-53) without the push: the refcount drops,
// and a block that reaches 0 goes back on the free list when the step ends
// (end_step).  Returns the refcount left, or -1 for a free block.
int64_t drop_ref(it_block_pool* p, int64_t id) {
  if (it_block_pool_ref_count(p, id) <= 0) {
    fail(IT_INVALID_INPUT, "block %lld is already free", (long long)id);
    return -1;
  }
  // A block held more than once only loses a reference; the last reference
  // is taken by the pool's own free, whose push end_step undoes and redoes
  // in free order.
  if (it_block_pool_ref_count(p, id) > 1) return it_block_pool_free(p, id) == IT_OK ? 1 : -1;
  if (it_block_pool_free(p, id) != IT_OK) return -1;
  it_block_pool_unpush(p, id);
  return 0;
}

// The step's tokens written into block `id` are dead: the window returned
// that block to the pool later in the same step.  Their slots become -1
// (padding: never written), so a page the step clears stays clear.  The
// scan starts at the block's first write of this step.
void kill_tokens(it_kv_manager* m, it_kv_step_plan* pl, int32_t id, int32_t t) {
  if (m->blk_step[size_t(id)] != m->step) return;
  for (int32_t u = m->blk_first[size_t(id)]; u < t; ++u)
    if (pl->slots[u] >= 0 && pl->slots[u] / m->bs == id) pl->slots[u] = -1;
}

// Ends a step: the blocks it returned go back on the free list, in free
// order; returns rc.
int32_t end_step(it_kv_manager* m, int32_t rc) {
  for (int32_t id : m->pending) it_block_pool_push(m->pool, id);
  m->pending.clear();
  return rc;
}

int32_t step_impl(it_kv_manager* m, const int32_t* seqs, const int32_t* n_tokens, int32_t n,
                  it_kv_step_plan* pl, const char* who) {
  if (!m || !pl || (n > 0 && (!seqs || !n_tokens)))
    return fail(IT_INVALID_INPUT, "%s: NULL argument", who);
  if (n < 0) return fail(IT_INVALID_INPUT, "%s: n = %d", who, n);
  pl->n_tokens = pl->n_evicted = pl->n_cow = 0;
  // Checks that need no state change come first: sequence ids, counts and
  // the token capacity.
  int64_t total = 0;
  for (int32_t i = 0; i < n; ++i) {
    if (seqs[i] < 0 || seqs[i] >= m->max_seqs || n_tokens[i] < 0)
      return fail(IT_INVALID_INPUT, "%s: seq %d / n_tokens %d invalid", who, seqs[i], n_tokens[i]);
    total += n_tokens[i];
  }
  if (total > 0 && !pl->slots) return fail(IT_INVALID_INPUT, "%s: slots is NULL", who);
  if (total > pl->tokens_cap)
    return fail(IT_INVALID_INPUT, "%s: %lld tokens exceed tokens_cap %d", who, (long long)total, pl->tokens_cap);
  const bool cow = pl->cow_src != nullptr;
  if (cow && !pl->cow_dst) return fail(IT_INVALID_INPUT, "%s: cow_dst is NULL", who);
  m->pending.clear();
  if (++m->step == 0) {  // wrapped: no stale stamp may match
    std::fill(m->blk_step.begin(), m->blk_step.end(), 0u);
    m->step = 1;
  }
  int32_t nc = 0;
  int32_t t = 0;
  for (int32_t i = 0; i < n; ++i) {
    const int32_t s = seqs[i];
    int32_t* row = &m->table[size_t(s) * size_t(m->max_blocks)];
    for (int32_t k = 0; k < n_tokens[i]; ++k) {
      const int64_t p = m->pos[size_t(s)];
      if (m->window > 0) {
        // Blocks wholly below the window [p - W + 1, p] drop this
        // sequence's reference, oldest first.  Only a block whose refcount
        // reaches 0 returns to the pool (at the end of the step) and is
        // listed for clearing; one a forked sequence still holds keeps its
        // pages.
        while (m->first[size_t(s)] * m->bs + m->bs - 1 < p - m->window + 1) {
          const int64_t j = m->first[size_t(s)];
          if (j >= m->max_blocks) break;
          if (row[j] >= 0) {
            const int32_t id = row[j];
            const bool last_ref = it_block_pool_ref_count(m->pool, id) == 1;
            // Capacity first: a block is released only together with
            // clearing its table entry, so an error leaves no table naming
            // a freed block.
            if (last_ref && (!pl->evicted || int32_t(m->pending.size()) >= pl->evicted_cap))
              return end_step(m, fail(IT_INVALID_INPUT, "%s: evicted capacity %d exceeded", who, pl->evicted_cap));
            if (drop_ref(m->pool, id) < 0) return end_step(m, IT_INVALID_INPUT);
            if (last_ref) {
              m->pending.push_back(id);
              kill_tokens(m, pl, id, t);
            }
            row[j] = -1;
          }
          m->first[size_t(s)] = j + 1;
        }
      }
      const int64_t lb = p / m->bs;
      if (lb >= m->max_blocks || p > INT32_MAX)
        return end_step(m, fail(IT_INVALID_INPUT, "%s: seq %d position %lld exceeds %d blocks", who, s,
                                (long long)p, m->max_blocks));
      if (p % m->bs == 0) {
        const int64_t id = it_block_pool_allocate(m->pool);
        if (id < 0) return end_step(m, fail(IT_INVALID_INPUT, "%s: block pool exhausted", who));
        row[lb] = int32_t(id);
      } else if (row[lb] < 0) {
        return end_step(m, fail(IT_INVALID_INPUT, "%s: seq %d holds no block for position %lld", who, s,
                                (long long)p));
      } else if (cow && it_block_pool_ref_count(m->pool, row[lb]) > 1) {
        // Copy-on-write: a shared partial block is about to be written.
        // Capacity before allocating, so an error leaks no block.
        if (nc >= pl->cow_cap)
          return end_step(m, fail(IT_INVALID_INPUT, "%s: cow capacity %d exceeded", who, pl->cow_cap));
        const int64_t id = it_block_pool_allocate(m->pool);
        if (id < 0) return end_step(m, fail(IT_INVALID_INPUT, "%s: block pool exhausted (copy-on-write)", who));
        pl->cow_src[nc] = row[lb];
        pl->cow_dst[nc] = int32_t(id);
        ++nc;
        if (drop_ref(m->pool, row[lb]) < 0) return end_step(m, IT_INVALID_INPUT);  // refcount > 1: stays held
        row[lb] = int32_t(id);
      }
      const int32_t id = row[lb];
      if (m->blk_step[size_t(id)] != m->step) {
        m->blk_step[size_t(id)] = m->step;
        m->blk_first[size_t(id)] = t;
      }
      pl->slots[t] = int64_t(id) * m->bs + p % m->bs;
      if (pl->token_seq) pl->token_seq[t] = s;
      if (pl->token_pos) pl->token_pos[t] = int32_t(p);
      ++t;
      m->pos[size_t(s)] = p + 1;
    }
  }
  const int32_t ne = int32_t(m->pending.size());
  for (int32_t i = 0; i < ne; ++i) pl->evicted[i] = m->pending[size_t(i)];
  pl->n_tokens = t;
  pl->n_evicted = ne;
  pl->n_cow = nc;
  export_lengths(m, pl->ctx_lens, pl->start_pos);
  return end_step(m, IT_OK);
}
}  // namespace

extern "C" int32_t it_kv_manager_step(it_kv_manager* m, const int32_t* seqs, const int32_t* n_tokens,
                                      int32_t n, it_kv_step_plan* plan) {
  return step_impl(m, seqs, n_tokens, n, plan, "it_kv_manager_step");
}

extern "C" int32_t it_kv_manager_append(it_kv_manager* m, const int32_t* seqs,
                                        const int32_t* n_tokens, int32_t n, int64_t* slots_out,
                                        int32_t* evicted_out, int32_t evicted_cap,
                                        int32_t* n_evicted) {
  if (!n_evicted) return fail(IT_INVALID_INPUT, "it_kv_manager_append: n_evicted is NULL");
  it_kv_step_plan pl{};
  pl.slots = slots_out;
  pl.tokens_cap = INT32_MAX;  // the caller sized slots_out to sum(n_tokens)
  pl.evicted = evicted_out;
  pl.evicted_cap = evicted_cap;
  const int32_t rc = step_impl(m, seqs, n_tokens, n, &pl, "it_kv_manager_append");
  if (rc == IT_OK) *n_evicted = pl.n_evicted;
  return rc;
}

extern "C" int32_t it_kv_manager_append_cow(it_kv_manager* m, const int32_t* seqs,
                                            const int32_t* n_tokens, int32_t n, int64_t* slots_out,
                                            int32_t* evicted_out, int32_t evicted_cap,
                                            int32_t* n_evicted, int32_t* cow_src, int32_t* cow_dst,
                                            int32_t cow_cap, int32_t* n_cow) {
  if (!cow_src || !cow_dst || !n_cow) return fail(IT_INVALID_INPUT, "it_kv_manager_append_cow: NULL cow output");
  if (!n_evicted) return fail(IT_INVALID_INPUT, "it_kv_manager_append_cow: n_evicted is NULL");
  it_kv_step_plan pl{};
  pl.slots = slots_out;
  pl.tokens_cap = INT32_MAX;
  pl.evicted = evicted_out;
  pl.evicted_cap = evicted_cap;
  pl.cow_src = cow_src;
  pl.cow_dst = cow_dst;
  pl.cow_cap = cow_cap;
  const int32_t rc = step_impl(m, seqs, n_tokens, n, &pl, "it_kv_manager_append_cow");
  if (rc == IT_OK) {
    *n_evicted = pl.n_evicted;
    *n_cow = pl.n_cow;
  }
  return rc;
}

extern "C" int32_t it_kv_manager_release_seq(it_kv_manager* m, int32_t seq, int32_t* evicted_out,
                                             int32_t evicted_cap, int32_t* n_evicted) {
  if (!m || !n_evicted) return fail(IT_INVALID_INPUT, "it_kv_manager_release_seq: NULL argument");
  if (seq < 0 || seq >= m->max_seqs) return fail(IT_INVALID_INPUT, "it_kv_manager_release_seq: seq %d", seq);
  int32_t* row = &m->table[size_t(seq) * size_t(m->max_blocks)];
  // Capacity before any free: room for every block the sequence holds
  // (the most that can return to the pool), so an error changes nothing.
  int32_t held = 0;
  for (int32_t j = 0; j < m->max_blocks; ++j) held += row[j] >= 0;
  if (held > 0 && (!evicted_out || held > evicted_cap))
    return fail(IT_INVALID_INPUT, "it_kv_manager_release_seq: evicted capacity %d < %d held blocks", evicted_cap,
                held);
  int32_t ne = 0;
  for (int32_t j = 0; j < m->max_blocks; ++j) {
    if (row[j] < 0) continue;
    const int32_t id = row[j];
    if (it_block_pool_free(m->pool, id) != IT_OK) return IT_INVALID_INPUT;
    // Only blocks no other sequence holds go back to the pool (and are
    // listed for clearing); shared ones keep their pages.
    if (it_block_pool_ref_count(m->pool, id) == 0) evicted_out[ne++] = id;
    row[j] = -1;
  }
  m->pos[size_t(seq)] = 0;
  m->first[size_t(seq)] = 0;
  *n_evicted = ne;
  return IT_OK;
}

extern "C" int32_t it_kv_manager_fork(it_kv_manager* m, int32_t src, int32_t dst) {
  if (!m) return fail(IT_INVALID_INPUT, "it_kv_manager_fork: manager is NULL");
  if (src < 0 || src >= m->max_seqs || dst < 0 || dst >= m->max_seqs || src == dst)
    return fail(IT_INVALID_INPUT, "it_kv_manager_fork: bad seqs %d -> %d", src, dst);
  int32_t* drow = &m->table[size_t(dst) * size_t(m->max_blocks)];
  const int32_t* srow = &m->table[size_t(src) * size_t(m->max_blocks)];
  for (int32_t j = 0; j < m->max_blocks; ++j)
    if (drow[j] >= 0) return fail(IT_INVALID_INPUT, "it_kv_manager_fork: destination seq %d not empty", dst);
  for (int32_t j = 0; j < m->max_blocks; ++j) {
    if (srow[j] < 0) continue;
    if (it_block_pool_share(m->pool, srow[j]) != IT_OK) return IT_INVALID_INPUT;
    drow[j] = srow[j];
  }
  m->pos[size_t(dst)] = m->pos[size_t(src)];
  m->first[size_t(dst)] = m->first[size_t(src)];
  return IT_OK;
}

extern "C" int32_t it_kv_manager_tables(const it_kv_manager* m, int32_t* tables, int32_t max_blocks,
                                        int32_t* ctx_lens, int32_t* start_pos) {
  if (!m) return fail(IT_INVALID_INPUT, "it_kv_manager_tables: manager is NULL");
  if (tables && max_blocks < m->max_blocks)
    return fail(IT_INVALID_INPUT, "it_kv_manager_tables: max_blocks %d < %d", max_blocks, m->max_blocks);
  if (tables)
    for (int32_t s = 0; s < m->max_seqs; ++s)
      for (int32_t j = 0; j < max_blocks; ++j)
        tables[size_t(s) * size_t(max_blocks) + size_t(j)] =
            j < m->max_blocks ? m->table[size_t(s) * size_t(m->max_blocks) + size_t(j)] : -1;
  export_lengths(m, ctx_lens, start_pos);
  return IT_OK;
}
