// it_internal.hpp -- shared declarations of the libit_kv implementation.
#pragma once
#include <cstdint>

#include "it_kv.h"

namespace itkv {
// Sets the thread-local message and returns `code`.
int32_t fail(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Bits latched in it_kv_cache::err_flag by kernels (reported by
// it_kv_cache_check).
enum : uint32_t {
  kErrSlot = 1u,        // slot_mapping entry >= num_blocks * block_size
  kErrBlock = 2u,       // block id (table, evict or copy list) out of range
  kErrTable = 4u,       // logical block beyond max_blocks
  kErrCtx = 8u,         // context longer than the max_tokens bound
  kErrPos = 16u,        // RoPE position outside the table
  kErrStart = 32u,      // negative start position (the sequence is skipped)
};

// Quantised KV formats (32-element groups, F32 source rows).
inline bool is_quant(int32_t dt) {
  return dt == IT_Q8_0 || dt == IT_Q4_0 || dt == IT_Q4_1 || dt == IT_Q5_0 || dt == IT_Q5_1;
}

inline bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }
inline int ilog2(int64_t x) {
  int r = 0;
  while ((int64_t(1) << r) < x) ++r;
  return r;
}
inline int64_t dtype_bytes(int32_t dt) {
  switch (dt) {
    case IT_F32: return 4;
    case IT_F16: return 2;
    case IT_BF16: return 2;
    default: return 0;
  }
}
}  // namespace itkv

struct it_kv_cache {
  void* k_pool;        // layer 0 of the K pool
  void* v_pool;        // layer 0 of the V pool
  uint32_t* err_flag;  // device word (a layer view shares its parent's)
  int64_t num_blocks;
  int64_t page_bytes;
  int64_t layer_bytes;  // bytes of one layer of one pool: num_blocks * n_kv_heads * page_bytes
  int32_t n_layers;     // layers in each pool (a layer view: 1)
  int32_t block_size;
  int32_t log2_bs;
  int32_t n_kv_heads;
  int32_t head_dim;
  int32_t dtype;
  int32_t device;
  int32_t owns_memory;
  int32_t owns_flag;    // 0 for a layer view
};

namespace itkv {
// Entry points that read or write one layer's pages take a one-layer cache
// (a single-layer cache or a view from it_kv_cache_layer).
inline int32_t one_layer(const it_kv_cache* c, const char* who) {
  if (c && c->n_layers != 1)
    return fail(IT_INVALID_INPUT, "%s: the cache holds %d layers; pass the layer's view (it_kv_cache_layer)", who,
                c->n_layers);
  return IT_OK;
}
// Looks up the device address of the no-allocation decode's array on the
// current device (done once per device; it_kv_cache_new/_wrap call it so
// that the first no-allocation decode does no lookup).
int32_t noalloc_prepare(int device);
}  // namespace itkv
