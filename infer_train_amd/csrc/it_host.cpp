// it_host.cpp -- host side of the KV-cache path: block allocator, slot
// mapping / block tables / sliding-window eviction, and the thread-local
// error channel of the C ABI.  No device code here.
//
// Objects are not internally locked: like `&mut self` in the Rust reference,
// concurrent mutation of one pool or manager is the caller's to serialise.
#include <cstdarg>
#include <cstdio>
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
int32_t append_impl(it_kv_manager* m, const int32_t* seqs, const int32_t* n_tokens, int32_t n,
                    int64_t* slots_out, int32_t* evicted_out, int32_t evicted_cap,
                    int32_t* n_evicted, int32_t* cow_src, int32_t* cow_dst, int32_t cow_cap,
                    int32_t* n_cow) {
  if (!m || (n > 0 && (!seqs || !n_tokens || !slots_out)) || !n_evicted)
    return fail(IT_INVALID_INPUT, "it_kv_manager_append: NULL argument");
  int32_t ne = 0, nc = 0;
  size_t t = 0;
  for (int32_t i = 0; i < n; ++i) {
    const int32_t s = seqs[i];
    if (s < 0 || s >= m->max_seqs || n_tokens[i] < 0)
      return fail(IT_INVALID_INPUT, "it_kv_manager_append: seq %d / n_tokens %d invalid", s, n_tokens[i]);
    int32_t* row = &m->table[size_t(s) * size_t(m->max_blocks)];
    for (int32_t k = 0; k < n_tokens[i]; ++k) {
      const int64_t p = m->pos[size_t(s)];
      if (m->window > 0) {
        // Release blocks wholly below the window [p - W + 1, p], oldest first.
        while (m->first[size_t(s)] * m->bs + m->bs - 1 < p - m->window + 1) {
          const int64_t j = m->first[size_t(s)];
          if (j >= m->max_blocks) break;
          if (row[j] >= 0) {
            // Capacity first: a block is freed only together with clearing
            // its table entry, so an error leaves no table naming a freed
            // block.
            if (!evicted_out || ne >= evicted_cap)
              return fail(IT_INVALID_INPUT, "it_kv_manager_append: evicted_out capacity %d exceeded", evicted_cap);
            if (it_block_pool_free(m->pool, row[j]) != IT_OK) return IT_INVALID_INPUT;
            evicted_out[ne++] = row[j];
            row[j] = -1;
          }
          m->first[size_t(s)] = j + 1;
        }
      }
      const int64_t lb = p / m->bs;
      if (lb >= m->max_blocks)
        return fail(IT_INVALID_INPUT, "it_kv_manager_append: seq %d position %lld exceeds %d blocks", s,
                    (long long)p, m->max_blocks);
      if (p % m->bs == 0) {
        const int64_t id = it_block_pool_allocate(m->pool);
        if (id < 0) return fail(IT_INVALID_INPUT, "it_kv_manager_append: block pool exhausted");
        row[lb] = int32_t(id);
      } else if (row[lb] < 0) {
        return fail(IT_INVALID_INPUT, "it_kv_manager_append: seq %d holds no block for position %lld", s,
                    (long long)p);
      } else if (cow_src && it_block_pool_ref_count(m->pool, row[lb]) > 1) {
        // Copy-on-write: a shared partial block is about to be written.
        // Capacity before allocating, so an error leaks no block.
        if (nc >= cow_cap) return fail(IT_INVALID_INPUT, "it_kv_manager_append: cow capacity %d exceeded", cow_cap);
        const int64_t id = it_block_pool_allocate(m->pool);
        if (id < 0) return fail(IT_INVALID_INPUT, "it_kv_manager_append: block pool exhausted (CoW)");
        cow_src[nc] = row[lb];
        cow_dst[nc] = int32_t(id);
        ++nc;
        if (it_block_pool_free(m->pool, row[lb]) != IT_OK) return IT_INVALID_INPUT;
        row[lb] = int32_t(id);
      }
      slots_out[t++] = int64_t(row[lb]) * m->bs + p % m->bs;
      m->pos[size_t(s)] = p + 1;
    }
  }
  *n_evicted = ne;
  if (n_cow) *n_cow = nc;
  return IT_OK;
}
}  // namespace

extern "C" int32_t it_kv_manager_append(it_kv_manager* m, const int32_t* seqs,
                                        const int32_t* n_tokens, int32_t n, int64_t* slots_out,
                                        int32_t* evicted_out, int32_t evicted_cap,
                                        int32_t* n_evicted) {
  return append_impl(m, seqs, n_tokens, n, slots_out, evicted_out, evicted_cap, n_evicted, nullptr,
                     nullptr, 0, nullptr);
}

extern "C" int32_t it_kv_manager_append_cow(it_kv_manager* m, const int32_t* seqs,
                                            const int32_t* n_tokens, int32_t n, int64_t* slots_out,
                                            int32_t* evicted_out, int32_t evicted_cap,
                                            int32_t* n_evicted, int32_t* cow_src, int32_t* cow_dst,
                                            int32_t cow_cap, int32_t* n_cow) {
  if (!cow_src || !cow_dst || !n_cow) return fail(IT_INVALID_INPUT, "it_kv_manager_append_cow: NULL cow output");
  return append_impl(m, seqs, n_tokens, n, slots_out, evicted_out, evicted_cap, n_evicted, cow_src,
                     cow_dst, cow_cap, n_cow);
}

extern "C" int32_t it_kv_manager_release_seq(it_kv_manager* m, int32_t seq, int32_t* evicted_out,
                                             int32_t evicted_cap, int32_t* n_evicted) {
  if (!m || !n_evicted) return fail(IT_INVALID_INPUT, "it_kv_manager_release_seq: NULL argument");
  if (seq < 0 || seq >= m->max_seqs) return fail(IT_INVALID_INPUT, "it_kv_manager_release_seq: seq %d", seq);
  int32_t* row = &m->table[size_t(seq) * size_t(m->max_blocks)];
  int32_t ne = 0;
  for (int32_t j = 0; j < m->max_blocks; ++j) {
    if (row[j] < 0) continue;
    if (it_block_pool_free(m->pool, row[j]) != IT_OK) return IT_INVALID_INPUT;
    if (ne < evicted_cap && evicted_out) evicted_out[ne] = row[j];
    ++ne;
    row[j] = -1;
  }
  if (ne > evicted_cap) return fail(IT_INVALID_INPUT, "it_kv_manager_release_seq: evicted capacity %d < %d", evicted_cap, ne);
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
  for (int32_t s = 0; s < m->max_seqs; ++s) {
    if (tables)
      for (int32_t j = 0; j < max_blocks; ++j)
        tables[size_t(s) * size_t(max_blocks) + size_t(j)] =
            j < m->max_blocks ? m->table[size_t(s) * size_t(m->max_blocks) + size_t(j)] : -1;
    if (ctx_lens) ctx_lens[s] = int32_t(m->pos[size_t(s)]);
    if (start_pos) {
      const int64_t st = m->window > 0 ? m->pos[size_t(s)] - m->window : 0;
      start_pos[s] = int32_t(st > 0 ? st : 0);
    }
  }
  return IT_OK;
}
