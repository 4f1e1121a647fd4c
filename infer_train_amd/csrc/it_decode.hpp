// it_decode.hpp -- shared pieces of the paged split-K flash-decode for gfx950:
// the kernel argument block, direct global->LDS loads, and the combine pass
// that merges the partitions' (m, l, O) partials.  The split kernel itself is
// in it_decode_split.hpp.
#pragma once
#include <hip/hip_runtime.h>

#include "it_device.hpp"
#include "it_internal.hpp"
#include "it_kv.h"

namespace itkv {
struct DecodeArgs {
  const void* q;            // [n_seqs][n_heads][D]
  const char* k_pool;
  const char* v_pool;
  const int32_t* bt;        // [n_seqs][max_blocks], NULL = identity
  const int32_t* ctx_lens;  // NULL = ctx_const for every sequence
  const int32_t* start_pos; // NULL = 0
  const float* mask;        // additive mask by position, NULL = none
  float* ws_o;              // [n_seqs][n_heads][max_parts][D]
  float* ws_ml;             // [n_seqs][n_heads][max_parts][2]
  uint32_t* err;
  int64_t page_bytes;
  int64_t num_blocks;
  float scale_log2;         // softmax scale * log2(e)
  float scale;              // softmax scale (mask path)
  int ctx_const;
  int max_blocks;
  int n_heads;
  int n_kv_heads;
  int group;                // n_heads / n_kv_heads
  int chunks;               // head chunks per KV head (group / GC)
  int log2_bs;
  int partition;            // tokens per split, multiple of 64
  int max_parts;
  int max_pages;            // page-list entries per partition: (partition >> log2_bs) + 2
  int compact;              // 1: workgroup L runs the L-th non-empty unit (needs ctx_lens)
};

constexpr float kLog2e = 1.4426950408889634f;

// ---- LDS DMA and counted waits --------------------------------------------
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  // Generic -> LDS address-space cast (a C-style cast is the only spelling
  // clang accepts), then the 32-bit LDS byte offset.
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}
// 64 lanes x 16 B from per-lane global addresses into LDS [m0, m0 + 1 KiB).
// One wait state between the SALU write of M0 and the LDS-DMA read of it.
// The loads carry the non-temporal hint: cache pages are streamed once per
// step, and with `nt` the paged read pattern of config 2 runs at 6.65 TB/s
// instead of 5.9 TB/s (measured with a DMA-only kernel of the same pattern).
__device__ __forceinline__ void dma_b128(const void* g, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt" ::"s"(m0), "v"(g) : "memory", "m0");
}
// Active lanes x 4 B into LDS [m0 + 4 lane], non-temporal like dma_b128.
__device__ __forceinline__ void dma_b32(const void* g, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off nt" ::"s"(m0), "v"(g) : "memory", "m0");
}
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One merged output element in the caller's dtype.  The value is o / l when
// l > 0, else zero (flash_attn.rs:66-71: multiply by 1/s when s > 0).
__device__ __forceinline__ void store_combined(void* out, int out_dtype, int64_t idx, float v) {
  if (out_dtype == IT_F32) static_cast<float*>(out)[idx] = v;
  else if (out_dtype == IT_BF16) static_cast<uint16_t*>(out)[idx] = uint16_t(f32_to_bf16_bits(v));
  else static_cast<uint16_t*>(out)[idx] = uint16_t(f32_to_f16_bits(v));
}

// Merge the partitions of one (sequence, head) over a 64-dim slice (grid z):
// M = max m_p, L = sum l_p 2^(m_p - M), O = sum O_p 2^(m_p - M) / L (the
// split-K form of flash_attn_f32's rescaling, flash_attn.rs:42-71).  Lane d
// owns one output dim.  The partials are read in chunks of kChunk partitions
// whose loads are all in flight together; every lane reads the chunk's
// (m, l) pairs itself, so no cross-lane step sits between them and the O
// loads.  With more than one chunk, M comes from a first pass over the
// (m, l) pairs.
template <int D>
__global__ __launch_bounds__(64) void paged_decode_combine(const float* __restrict__ ws_o,
                                                           const float* __restrict__ ws_ml,
                                                           const int32_t* __restrict__ ctx_lens,
                                                           const int32_t* __restrict__ start_pos,
                                                           int ctx_const, int n_heads, int partition,
                                                           int max_parts, void* out, int out_dtype) {
  // Partitions beyond max_parts were never computed (the split pass latched
  // the error); only the computed ones are merged.
  constexpr int kChunk = 16;
  const int h = blockIdx.x, b = blockIdx.y, d = 64 * blockIdx.z + threadIdx.x, lane = threadIdx.x;
  const int64_t row = int64_t(b) * n_heads + h;
  const float2* ml = reinterpret_cast<const float2*>(ws_ml) + row * max_parts;
  const float* op = ws_o + row * max_parts * D + d;
  // With at most kChunk partitions the loads of all max_parts slots go out
  // before the context length arrives (the addresses do not depend on it);
  // slots past this sequence's count hold stale bytes and are replaced by
  // (-inf, 0) and 0 once the count is known.
  float2 pre_ml[kChunk];
  float pre_o[kChunk];
  if (max_parts <= kChunk) {
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      if (c < max_parts) {
        pre_ml[c] = ml[c];
        pre_o[c] = op[int64_t(c) * D];
      }
    }
  }
  const int ctx = ctx_lens ? ctx_lens[b] : ctx_const;
  const int st = start_pos ? start_pos[b] : 0;
  const int n = ctx - st;
  // A negative start position was skipped by the split pass (and latched):
  // no partitions, zeros.
  const int np = (n > 0 && st >= 0) ? min((n + partition - 1) / partition, max_parts) : 0;
  float mx = -INFINITY;
  if (max_parts <= kChunk) {
    float l = 0.0f, o = 0.0f;
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      if (c < np) mx = fmaxf(mx, pre_ml[c].x);
    }
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      if (c < np) {
        const float w = (pre_ml[c].x == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(pre_ml[c].x - mx);
        l = fmaf(pre_ml[c].y, w, l);
        o = fmaf(pre_o[c], w, o);
      }
    }
    store_combined(out, out_dtype, row * D + d, l > 0.0f ? o * (1.0f / l) : 0.0f);
    return;
  }
  if (np > kChunk) {
    for (int p = lane; p < np; p += 64) mx = fmaxf(mx, ml[p].x);
    mx = group_max<64>(mx);
  }
  float l = 0.0f, o = 0.0f;
  for (int p0 = 0; p0 < np; p0 += kChunk) {
    float2 mlc[kChunk];
    float oc[kChunk];
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      const bool in = p0 + c < np;
      mlc[c] = in ? ml[p0 + c] : make_float2(-INFINITY, 0.0f);
      oc[c] = in ? op[int64_t(p0 + c) * D] : 0.0f;
    }
    if (np <= kChunk) {
#pragma unroll
      for (int c = 0; c < kChunk; ++c) mx = fmaxf(mx, mlc[c].x);
    }
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      const float w = (mlc[c].x == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mlc[c].x - mx);
      l = fmaf(mlc[c].y, w, l);
      o = fmaf(oc[c], w, o);
    }
  }
  store_combined(out, out_dtype, row * D + d, l > 0.0f ? o * (1.0f / l) : 0.0f);
}

}  // namespace itkv
