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
  int compact;              // 1: one-dimensional grid over the non-empty units (needs ctx_lens)
  int n_seqs;
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
// dma_b128 from a wave-uniform base (an SGPR pair) plus a per-lane 32-bit
// byte offset: the address costs no vector instructions.
__device__ __forceinline__ void dma_b128_s(const void* base, uint32_t off, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt" ::"s"(m0), "v"(off), "s"(base)
               : "memory", "m0");
}
// dma_b32 from a wave-uniform base plus a per-lane 32-bit byte offset.
__device__ __forceinline__ void dma_b32_s(const void* base, uint32_t off, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2 nt" ::"s"(m0), "v"(off), "s"(base)
               : "memory", "m0");
}
// Active lanes x 4 B into LDS [m0 + 4 lane], non-temporal like dma_b128.
__device__ __forceinline__ void dma_b32(const void* g, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off nt" ::"s"(m0), "v"(g) : "memory", "m0");
}
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Lane `l`'s value of x (v_readlane_b32 on the bits; l uniform).
__device__ __forceinline__ float lane_f32(float x, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}

// Where a combine workgroup's row sits.  The split pass deals its units to
// the XCDs in contiguous ranges of q8 = ceil(T / 8) units (T = n_seqs * hc *
// max_parts when every sequence fills max_parts partitions); head row r =
// b * n_heads + h belongs to unit row u = r / gc, whose first unit is
// u * max_parts.  So XCD x wrote the rows [first_row(x), first_row(x + 1)),
// and combine workgroup L (on XCD L % 8, dealt round-robin) takes row
// first_row(L % 8) + L / 8 of that range: it reads the partials from the L2
// they were written to (measured on config 2 at 4k: 0.24 us per decode).
// For unequal contexts the split's ranges move and some rows are read from
// another XCD; the mapping is a bijection onto the rows either way.
struct CombineMap {
  int64_t q8;      // units per XCD range under equal contexts
  int64_t n_rows;  // n_seqs * n_heads
  int gc;          // heads per unit row
  int max_parts;
  __host__ __device__ int64_t first_row(int64_t x) const {
    const int64_t u = (x * q8 + max_parts - 1) / max_parts;
    return u * gc < n_rows ? u * gc : n_rows;
  }
};

// Merge the partitions of one (sequence, head) row over a 128-dim slice
// (grid z): M = max m_p, L = sum l_p 2^(m_p - M), O = sum O_p 2^(m_p - M) / L
// (the split-K form of flash_attn_f32's rescaling, flash_attn.rs:42-71).
// One wave (four for long rows, below) per row slice, two adjacent dims per lane (8-byte partial loads
// and one packed store: half the workgroups and load instructions of one dim
// per lane, 0.9 us less per config-2 decode).  Lane c also holds the (m, l)
// pairs of partitions c and 64 + c, so M and L are wave reductions and
// partition p's weight comes from its lane (readlane).  The pairs and the
// first kBatch partitions' outputs are all loaded before the context length
// arrives (their addresses do not depend on it; slots past this sequence's
// count hold stale bytes and get weight 0 once the count is known): one
// memory round trip up to kBatch partitions.  Partitions beyond 128 read
// their pairs directly.
// The leading scalar arguments (the map's fields, the workspace and the
// length pointers: 16 dwords) are preloaded into SGPRs at wave launch
// (kernarg preloading, gfx950), so the first loads do not wait for a
// kernel-argument fetch.
// NW waves per workgroup (1, or 4 for rows of more than kBatch partitions):
// wave w takes partitions w, w + NW, ... and the waves' sums meet in LDS in
// a fixed order, so a row of up to NW kBatch partitions costs one round trip.
template <int D, int NW>
__global__ __launch_bounds__(64 * NW) void paged_decode_combine(const float* __restrict__ ws_o,
                                                                const float* __restrict__ ws_ml, int64_t q8,
                                                                int64_t n_rows, int gc, int max_parts, int n_heads,
                                                                const int32_t* __restrict__ ctx_lens,
                                                                const int32_t* __restrict__ start_pos, int ctx_const,
                                                                int partition, void* out, int out_dtype) {
  // Partitions beyond max_parts were never computed (the split pass latched
  // the error); only the computed ones are merged.
  constexpr int kBatch = 32;
  CombineMap map;
  map.q8 = q8;
  map.n_rows = n_rows;
  map.gc = gc;
  map.max_parts = max_parts;
  const int x = int(blockIdx.x & 7);
  const int64_t row = map.first_row(x) + (blockIdx.x >> 3);
  if (row >= map.first_row(x + 1)) return;  // uniform for the workgroup
  const int lane = int(threadIdx.x & 63), wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int b = int(row / n_heads), d = 2 * (64 * int(blockIdx.z) + lane);
  const float2* ml = reinterpret_cast<const float2*>(ws_ml) + row * max_parts;
  const float* op = ws_o + row * max_parts * D + d;
  const float2 none = make_float2(-INFINITY, 0.0f);
  float2 m0 = lane < max_parts ? ml[lane] : none;
  float2 m1 = 64 + lane < max_parts ? ml[64 + lane] : none;
  float2 ob[kBatch];
#pragma unroll
  for (int c = 0; c < kBatch; ++c)
    if (wave + NW * c < max_parts) ob[c] = *reinterpret_cast<const float2*>(op + int64_t(wave + NW * c) * D);
  const int ctx = ctx_lens ? ctx_lens[b] : ctx_const;
  const int st = start_pos ? start_pos[b] : 0;
  const int n = ctx - st;
  // A negative start position was skipped by the split pass (and latched):
  // no partitions, zeros.
  const int np = (n > 0 && st >= 0) ? min((n + partition - 1) / partition, max_parts) : 0;
  if (lane >= np) m0 = none;
  if (64 + lane >= np) m1 = none;
  float mx = fmaxf(m0.x, m1.x);
  for (int p = 128 + lane; p < np; p += 64) mx = fmaxf(mx, ml[p].x);
  mx = group_max<64>(mx);
  float o0 = 0.0f, o1 = 0.0f, l = 0.0f;
  if (mx != -INFINITY) {  // else no partition, or every key skipped: zeros (flash_attn.rs:66-71)
    const float w0 = m0.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m0.x - mx);
    const float w1 = m1.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1.x - mx);
    l = fmaf(m0.y, w0, m1.y * w1);
    for (int p = 128 + lane; p < np; p += 64) {
      const float2 v = ml[p];
      if (v.x != -INFINITY) l = fmaf(v.y, __builtin_amdgcn_exp2f(v.x - mx), l);
    }
    l = group_sum<64>(l);
    // Partition p's weight (p uniform): from its lane's pair, or read.
    auto weight = [&](int p) {
      if (p < 64) return lane_f32(w0, p);
      if (p < 128) return lane_f32(w1, p - 64);
      const float2 v = ml[p];
      return v.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(v.x - mx);
    };
    for (int c0 = 0; wave + NW * c0 < np; c0 += kBatch) {
      if (c0 > 0) {
#pragma unroll
        for (int c = 0; c < kBatch; ++c)
          if (wave + NW * (c0 + c) < np) ob[c] = *reinterpret_cast<const float2*>(op + int64_t(wave + NW * (c0 + c)) * D);
      }
#pragma unroll
      for (int c = 0; c < kBatch; ++c) {
        const int p = wave + NW * (c0 + c);
        if (p < np) {
          const float w = weight(p);
          o0 = fmaf(ob[c].x, w, o0);
          o1 = fmaf(ob[c].y, w, o1);
        }
      }
    }
  }
  if constexpr (NW > 1) {
    __shared__ float2 red[NW][64];
    red[wave][lane] = make_float2(o0, o1);
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 1; w < NW; ++w) {
      const float2 t = red[w][lane];
      o0 += t.x;
      o1 += t.y;
    }
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  const float r0 = l > 0.0f ? o0 * inv : 0.0f, r1 = l > 0.0f ? o1 * inv : 0.0f;
  const int64_t oi = row * D + d;
  if (out_dtype == IT_F32) {
    *reinterpret_cast<float2*>(static_cast<float*>(out) + oi) = make_float2(r0, r1);
  } else {
    const uint32_t lo = out_dtype == IT_BF16 ? f32_to_bf16_bits(r0) : f32_to_f16_bits(r0);
    const uint32_t hi = out_dtype == IT_BF16 ? f32_to_bf16_bits(r1) : f32_to_f16_bits(r1);
    *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(out) + oi) = lo | (hi << 16);
  }
}

}  // namespace itkv
