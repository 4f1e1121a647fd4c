// it_cache.hip -- the paged KV cache on gfx950: pool allocation, slot-mapped
// append (bit copy, or quantise to Q8_0 / Q4_0 / Q4_1 / Q5_0 / Q5_1), block-table gather, evict (page clear)
// and copy-on-write page copy.
//
// All of these are HBM-bound data movement.  Each lane moves one 16-byte
// vector (global_load_dwordx4 / global_store_dwordx4) and consecutive lanes
// cover consecutive bytes of a token row, so a wavefront touches whole
// 128-byte lines of both source and destination.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>

#include "it_device.hpp"
#include "it_internal.hpp"
#include "it_quant.hpp"

using namespace itkv;

#define IT_HIP(call, what)                                                          \
  do {                                                                              \
    hipError_t e_ = (call);                                                         \
    if (e_ != hipSuccess) return fail(IT_DEVICE_ERROR, "%s: %s", what, hipGetErrorString(e_)); \
  } while (0)

namespace {
constexpr int kThreads = 256;
constexpr int32_t kMaxLayers = 4096;

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// Append, bit copy (F32 / F16 / BF16).  A wave moves kVecsPerLane x 64
// 16-byte vectors, and every instruction covers one KiB: TPG = 64 / row_vecs
// consecutive tokens of one KV head (row_vecs = head_dim * elem / 16 = 16,
// 32 or 64 vectors per row).  Vectors are numbered (token group of TPG,
// head, token in group, vector in row): consecutive tokens at consecutive
// positions are consecutive rows of one page, so each store instruction
// writes one contiguous KiB, and the sources are TPG row-sized runs (config
// 3's chunk append: 6.07 -> 5.58 us against (token, head, vector) order,
// whose instructions scatter TPG head pages).  All loads are issued before
// the first store.  The sources are read once: non-temporal loads.
// ---------------------------------------------------------------------------
constexpr int kVecsPerLane = 4;

__global__ __launch_bounds__(kThreads) void kv_append_copy(
    const uint4* __restrict__ k, const uint4* __restrict__ v, char* __restrict__ kpool,
    char* __restrict__ vpool, const int64_t* __restrict__ slots, int32_t n_tok, int hkv,
    int log2_row_vecs, int log2_bs, int64_t page_bytes, int64_t n_slots, uint32_t* err) {
  const int32_t wave_base = (int32_t(blockIdx.x) * kThreads + int32_t(threadIdx.x & ~63u)) * kVecsPerLane;
  const int lane = int(threadIdx.x & 63u);
  const int log2_tpg = log2_row_vecs < 6 ? 6 - log2_row_vecs : 0;  // tokens per instruction
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  u4 kv[kVecsPerLane], vv[kVecsPerLane];
  int64_t slot[kVecsPerLane];
  int32_t tok[kVecsPerLane];
  int head[kVecsPerLane], vec[kVecsPerLane];
  // Loads are unconditional (past the last token a lane re-reads the last
  // token's row), so they all go out before any wait; only the stores are
  // predicated.
#pragma unroll
  for (int j = 0; j < kVecsPerLane; ++j) {
    const int32_t ip = wave_base + 64 * j + lane;
    const int c = ip & ((1 << log2_row_vecs) - 1);
    const int tg_in = (ip >> log2_row_vecs) & ((1 << log2_tpg) - 1);
    const int32_t rest = ip >> (log2_row_vecs + log2_tpg);
    const int32_t group = rest / hkv;
    const int h = rest - group * hkv;
    const int32_t t = (group << log2_tpg) + tg_in;
    tok[j] = t;
    head[j] = h;
    vec[j] = c;
    const int32_t tc = min(t, n_tok - 1);
    const int32_t i = ((tc * hkv + h) << log2_row_vecs) + c;  // source [token][head][vector]
    kv[j] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(k) + i);
    vv[j] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(v) + i);
    slot[j] = slots[tc];
  }
#pragma unroll
  for (int j = 0; j < kVecsPerLane; ++j) {
    if (tok[j] >= n_tok) continue;
    const int h = head[j];
    const int c = vec[j];
    const int64_t sl = slot[j];
    if (sl < 0) continue;  // padding token
    if (sl >= n_slots) {
      if (c == 0 && h == 0) atomicOr(err, kErrSlot);
      continue;
    }
    const int64_t blk = sl >> log2_bs;
    const int64_t off = sl & ((int64_t(1) << log2_bs) - 1);
    const int64_t dst = (blk * hkv + h) * page_bytes + ((off << log2_row_vecs) + c) * 16;
    __builtin_nontemporal_store(kv[j], reinterpret_cast<u4*>(kpool + dst));
    __builtin_nontemporal_store(vv[j], reinterpret_cast<u4*>(vpool + dst));
  }
}

// Append, bit copy, for rows that are not a power-of-two number of 16-byte
// vectors (e.g. BF16 head_dim 96 = 12 vectors): one vector per lane in
// (token, head, vector) order, indices by division.
__global__ __launch_bounds__(kThreads) void kv_append_copy_rows(
    const uint4* __restrict__ k, const uint4* __restrict__ v, char* __restrict__ kpool,
    char* __restrict__ vpool, const int64_t* __restrict__ slots, int64_t total, int hkv, int row_vecs,
    int log2_bs, int64_t page_bytes, int64_t n_slots, uint32_t* err) {
  const int64_t gid = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (gid >= total) return;
  const int c = int(gid % row_vecs);
  const int64_t th = gid / row_vecs;
  const int h = int(th % hkv);
  const int64_t t = th / hkv;
  const int64_t sl = slots[t];
  if (sl < 0) return;  // padding token
  if (sl >= n_slots) {
    if (c == 0 && h == 0) atomicOr(err, kErrSlot);
    return;
  }
  const int64_t blk = sl >> log2_bs;
  const int64_t off = sl & ((int64_t(1) << log2_bs) - 1);
  const int64_t dst = (blk * hkv + h) * page_bytes + (off * row_vecs + c) * 16;
  st16(kpool + dst, ld16_nt(k + gid));
  st16(vpool + dst, ld16_nt(v + gid));
}

// ---------------------------------------------------------------------------
// Append with quantisation (Q8_0, Q4_0, Q4_1, Q5_0, Q5_1: the quantisers of
// it_quant.hpp).  Eight lanes own one 32-element group, four floats each (one
// 16-byte load); blockIdx.y selects K (0) or V (1).
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(kThreads) void kv_append_quant(
    const float4* __restrict__ k, const float4* __restrict__ v, char* __restrict__ kpool,
    char* __restrict__ vpool, const int64_t* __restrict__ slots, int64_t total, int hkv, int d,
    int log2_bs, int64_t page_bytes, int64_t n_slots, uint32_t* err) {
  const int64_t gid = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  const bool is_v = blockIdx.y != 0;
  const bool live = gid < total;
  const float4 x = live ? (is_v ? v[gid] : k[gid]) : make_float4(0.f, 0.f, 0.f, 0.f);
  const QuantGroup q = quant_group<DT>(x, int(gid & 7));  // the 8 lanes of a group are lane-aligned
  if (!live) return;
  const int vecs_per_row = d >> 2;
  const int cv = int(gid % vecs_per_row);  // vector index in the row
  const int64_t th = gid / vecs_per_row;
  const int h = int(th % hkv);
  const int64_t t = th / hkv;
  const int64_t slot = slots[t];
  if (slot < 0) return;
  if (slot >= n_slots) {
    if (cv == 0 && h == 0) atomicOr(err, kErrSlot);
    return;
  }
  const int64_t blk = slot >> log2_bs;
  const int64_t off = slot & ((int64_t(1) << log2_bs) - 1);
  char* page = (is_v ? vpool : kpool) + (blk * hkv + h) * page_bytes;
  store_group<DT>(page, off, int64_t(1) << log2_bs, d, cv, q);
}

// Q8_0 quantise-append with 16-byte stores (head_dim D = 64, 128, 256).  A
// wave takes a "row group": 1024 consecutive source floats, RPW = 1024 / D
// whole (token, head) rows.
//  - Loads: instruction j reads floats 256 j .. 256 j + 255, lane l four of
//    them (16 bytes at 16 l): every load instruction is 1 KiB contiguous.
//    (Sixteen consecutive floats per lane, four 64-byte-strided loads,
//    took 11.2 us for 4096 config-5-shaped tokens with no arithmetic at
//    all: each such instruction touches 64 scattered pieces.)
//  - Quantise in that layout: eight lanes per 32-group (quant_group).
//  - The wave's 1024 int8 and 32 fp16 scales go through a wave-private
//    1088-byte LDS stage (same-wave LDS operations stay in order), and lane
//    L stores bytes 16 L .. 16 L + 15 of the group's int8, one 16-byte
//    vector (a 1 KiB store instruction); the first lane of each row stores
//    the row's D / 32 scales as one 4-, 8- or 16-byte word.
// blockIdx.y selects K (0) or V (1).
template <int D>
__global__ __launch_bounds__(kThreads) void kv_append_q8_wide(
    const float* __restrict__ k, const float* __restrict__ v, char* __restrict__ kpool, char* __restrict__ vpool,
    const int64_t* __restrict__ slots, int32_t n_rows, int32_t n_groups, int hkv, int log2_bs, int64_t page_bytes,
    int64_t n_slots, uint32_t* err) {
  constexpr int RPW = 1024 / D;  // rows per group
  constexpr int LPR = D / 16;    // store lanes per row
  __shared__ __attribute__((aligned(16))) char stage[kThreads / 64][1024 + 64];
  const bool is_v = blockIdx.y != 0;
  const int lane = int(threadIdx.x & 63u);
  char* const st = stage[threadIdx.x >> 6];
  const int32_t g0 = int32_t(blockIdx.x) * (kThreads / 64) + int32_t(threadIdx.x >> 6);
  const int log2_hkv = (hkv & (hkv - 1)) == 0 ? __builtin_ctz(unsigned(hkv)) : -1;  // uniform
  const float* const src = is_v ? v : k;
  char* const pool = is_v ? vpool : kpool;
  const int srow = lane / LPR, c = lane % LPR;  // the row and 16-byte piece this lane stores
  const int32_t stride = int32_t(gridDim.x) * (kThreads / 64);
  for (int32_t g = g0; g < n_groups; g += stride) {  // g and the stride are uniform
    const int32_t row = g * RPW + srow;
    const int32_t rs = row < n_rows ? row : n_rows - 1;
    const int64_t sl = slots[log2_hkv >= 0 ? rs >> log2_hkv : rs / hkv];
    const int64_t f0 = int64_t(g) * 1024 + 4 * lane;
    const int64_t last = int64_t(n_rows) * D - 4;
    typedef float f4 __attribute__((ext_vector_type(4)));
    float4 x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // Past the end (whole 32-groups only: n_rows * D is a multiple of
      // 32) a lane re-reads the last four floats; those rows are not stored.
      const int64_t f = min(f0 + 256 * j, last);
      const f4 t = __builtin_nontemporal_load(reinterpret_cast<const f4*>(src + f));
      x[j] = make_float4(t.x, t.y, t.z, t.w);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const QuantGroup q = quant_group<IT_Q8_0>(x[j], lane & 7);
      *reinterpret_cast<uint32_t*>(st + 256 * j + 4 * lane) = q.qs;
      if ((lane & 7) == 0) *reinterpret_cast<uint16_t*>(st + 1024 + 2 * (8 * j + (lane >> 3))) = uint16_t(q.meta);
    }
    const uint4 w = *reinterpret_cast<const uint4*>(st + 16 * lane);
    uint4 sw = make_uint4(0u, 0u, 0u, 0u);
    const char* const ss = st + 1024 + srow * (D / 16);  // the row's D / 32 scales
    if constexpr (LPR == 16) sw = *reinterpret_cast<const uint4*>(ss);
    else if constexpr (LPR == 8) sw.x = reinterpret_cast<const uint2*>(ss)->x, sw.y = reinterpret_cast<const uint2*>(ss)->y;
    else sw.x = *reinterpret_cast<const uint32_t*>(ss);
    if (row < n_rows && sl >= 0) {
      const int h = log2_hkv >= 0 ? row & (hkv - 1) : row % hkv;
      if (sl >= n_slots) {
        if (c == 0 && h == 0) atomicOr(err, kErrSlot);
      } else {
        const int64_t blk = sl >> log2_bs;
        const int64_t off = sl & ((int64_t(1) << log2_bs) - 1);
        char* const page = pool + (blk * hkv + h) * page_bytes;
        st16(page + off * D + 16 * c, w);
        if (c == 0) {
          char* const sp = page + (int64_t(1) << log2_bs) * D + off * (D / 16);
          if constexpr (LPR == 16) *reinterpret_cast<uint4*>(sp) = sw;
          else if constexpr (LPR == 8) *reinterpret_cast<uint2*>(sp) = make_uint2(sw.x, sw.y);
          else *reinterpret_cast<uint32_t*>(sp) = sw.x;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Gather.  grid.y = sequence; lane = one 16-byte vector of one output row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void kv_gather_vec(
    const char* __restrict__ kpool, const char* __restrict__ vpool, const int32_t* __restrict__ bt,
    int max_blocks, const int32_t* __restrict__ ctx_lens, const int32_t* __restrict__ start_pos,
    const int64_t* __restrict__ cu_out, int hkv, int row_vecs, int log2_bs, int64_t page_bytes,
    int64_t num_blocks, uint4* __restrict__ kout, uint4* __restrict__ vout, uint32_t* err) {
  const int b = blockIdx.y;
  const int st = start_pos ? start_pos[b] : 0;
  const int n = ctx_lens[b] - st;
  if (st < 0) {  // skipped and latched
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(err, kErrStart);
    return;
  }
  if (n <= 0) return;
  const int64_t gid = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (gid >= int64_t(hkv) * n * row_vecs) return;
  const int c = int(gid % row_vecs);
  const int64_t r = gid / row_vecs;
  const int i = int(r % n);
  const int h = int(r / n);
  const int pos = st + i;
  const int lb = pos >> log2_bs;
  if (lb >= max_blocks) {
    atomicOr(err, kErrTable);
    return;
  }
  const int blk = bt[int64_t(b) * max_blocks + lb];
  if (blk < 0 || blk >= num_blocks) {
    atomicOr(err, kErrBlock);
    return;
  }
  const int64_t src = (int64_t(blk) * hkv + h) * page_bytes +
                      (int64_t(pos & ((1 << log2_bs) - 1)) * row_vecs + c) * 16;
  const int64_t dst = (cu_out[b] * hkv + int64_t(h) * n + i) * row_vecs + c;
  st16(kout + dst, ld16_nt(kpool + src));
  st16(vout + dst, ld16_nt(vpool + src));
}

// Q8_0 gather: lane = one 32-element group, written as a packed 34-byte
// BlockQ8_0 record {u16 d; i8 qs[32]} (types.rs:34-41).
__global__ __launch_bounds__(kThreads) void kv_gather_q8_0(
    const char* __restrict__ kpool, const char* __restrict__ vpool, const int32_t* __restrict__ bt,
    int max_blocks, const int32_t* __restrict__ ctx_lens, const int32_t* __restrict__ start_pos,
    const int64_t* __restrict__ cu_out, int hkv, int d, int log2_bs, int64_t page_bytes,
    int64_t num_blocks, char* __restrict__ kout, char* __restrict__ vout, uint32_t* err) {
  const int b = blockIdx.y;
  const int st = start_pos ? start_pos[b] : 0;
  const int n = ctx_lens[b] - st;
  if (st < 0) {  // skipped and latched
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(err, kErrStart);
    return;
  }
  if (n <= 0) return;
  const int ng = d >> 5;
  const int64_t gid = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (gid >= int64_t(hkv) * n * ng) return;
  const int g = int(gid % ng);
  const int64_t r = gid / ng;
  const int i = int(r % n);
  const int h = int(r / n);
  const int pos = st + i;
  const int lb = pos >> log2_bs;
  if (lb >= max_blocks) {
    atomicOr(err, kErrTable);
    return;
  }
  const int blk = bt[int64_t(b) * max_blocks + lb];
  if (blk < 0 || blk >= num_blocks) {
    atomicOr(err, kErrBlock);
    return;
  }
  const int64_t bs = int64_t(1) << log2_bs;
  const int64_t off = pos & (bs - 1);
  const int64_t rec = ((cu_out[b] * hkv + int64_t(h) * n + i) * ng + g) * 34;
  for (int which = 0; which < 2; ++which) {
    const char* page = (which ? vpool : kpool) + (int64_t(blk) * hkv + h) * page_bytes;
    const uint4 q0 = ld16(page + off * d + g * 32);
    const uint4 q1 = ld16(page + off * d + g * 32 + 16);
    const uint16_t dd = *reinterpret_cast<const uint16_t*>(page + bs * d + (off * ng + g) * 2);
    uint16_t* o = reinterpret_cast<uint16_t*>((which ? vout : kout) + rec);  // 2-byte aligned
    o[0] = dd;
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      o[1 + 2 * j] = uint16_t(w[j] & 0xFFFFu);
      o[2 + 2 * j] = uint16_t(w[j] >> 16);
    }
  }
}

// Q4_0 / Q4_1 / Q5_0 / Q5_1 gather: lane = one 32-element group, written as
// a packed ggml record {meta; [qh;] qs[16]}: BlockQ4_0 {u16 d} (18 bytes,
// types.rs:15-22), BlockQ4_1 {u16 d; u16 m} (20, types.rs:24-32),
// block_q5_0 {u16 d; u8 qh[4]} (22) and block_q5_1 {u16 d; u16 m; u8
// qh[4]} (24).  Records of 18 and 22 bytes are 2-byte aligned, so the
// stores are 16-bit.
template <int DT>
__global__ __launch_bounds__(kThreads) void kv_gather_nib(
    const char* __restrict__ kpool, const char* __restrict__ vpool, const int32_t* __restrict__ bt,
    int max_blocks, const int32_t* __restrict__ ctx_lens, const int32_t* __restrict__ start_pos,
    const int64_t* __restrict__ cu_out, int hkv, int d, int log2_bs, int64_t page_bytes,
    int64_t num_blocks, char* __restrict__ kout, char* __restrict__ vout, uint32_t* err) {
  using N = NibFmt<DT>;
  const int b = blockIdx.y;
  const int st = start_pos ? start_pos[b] : 0;
  const int n = ctx_lens[b] - st;
  if (st < 0) {  // skipped and latched
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(err, kErrStart);
    return;
  }
  if (n <= 0) return;
  const int ng = d >> 5;
  const int64_t gid = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (gid >= int64_t(hkv) * n * ng) return;
  const int g = int(gid % ng);
  const int64_t r = gid / ng;
  const int i = int(r % n);
  const int h = int(r / n);
  const int pos = st + i;
  const int lb = pos >> log2_bs;
  if (lb >= max_blocks) {
    atomicOr(err, kErrTable);
    return;
  }
  const int blk = bt[int64_t(b) * max_blocks + lb];
  if (blk < 0 || blk >= num_blocks) {
    atomicOr(err, kErrBlock);
    return;
  }
  const int64_t bs = int64_t(1) << log2_bs;
  const int64_t off = pos & (bs - 1);
  const int64_t rec = ((cu_out[b] * hkv + int64_t(h) * n + i) * ng + g) * N::kRecord;
  for (int which = 0; which < 2; ++which) {
    const char* page = (which ? vpool : kpool) + (int64_t(blk) * hkv + h) * page_bytes;
    const uint4 q = ld16(page + off * (d >> 1) + g * 16);
    const char* side = page + bs * (d >> 1) + off * (ng * N::kSide);
    uint16_t w[N::kRecord / 2];
    int k = 0;
    if constexpr (N::kMin) {
      const uint32_t dm = *reinterpret_cast<const uint32_t*>(side + N::meta_off(ng) + 4 * g);
      w[k++] = uint16_t(dm & 0xFFFFu);
      w[k++] = uint16_t(dm >> 16);
    } else {
      w[k++] = *reinterpret_cast<const uint16_t*>(side + N::meta_off(ng) + 2 * g);
    }
    if constexpr (N::kQ5) {
      const uint32_t qh = *reinterpret_cast<const uint32_t*>(side + 4 * g);
      w[k++] = uint16_t(qh & 0xFFFFu);
      w[k++] = uint16_t(qh >> 16);
    }
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      w[k++] = uint16_t(qw[j] & 0xFFFFu);
      w[k++] = uint16_t(qw[j] >> 16);
    }
    uint16_t* o = reinterpret_cast<uint16_t*>((which ? vout : kout) + rec);
#pragma unroll
    for (int j = 0; j < N::kRecord / 2; ++j) o[j] = w[j];
  }
}

// ---------------------------------------------------------------------------
// Evict (zero pages) and copy-on-write page copy.  grid.y = list entry.
// ---------------------------------------------------------------------------
// grid.z = layer: a multi-layer cache clears (copies) the block in every
// layer in one launch.
__global__ __launch_bounds__(kThreads) void kv_clear_blocks(char* __restrict__ kpool,
                                                            char* __restrict__ vpool,
                                                            const int32_t* __restrict__ blocks,
                                                            int64_t block_vecs, int64_t num_blocks,
                                                            int64_t layer_bytes, uint32_t* err) {
  kpool += int64_t(blockIdx.z) * layer_bytes;
  vpool += int64_t(blockIdx.z) * layer_bytes;
  const int blk = blocks[blockIdx.y];
  if (blk < 0 || blk >= num_blocks) {
    if (blockIdx.x == 0 && blockIdx.z == 0 && threadIdx.x == 0) atomicOr(err, kErrBlock);
    return;
  }
  const uint4 z = make_uint4(0u, 0u, 0u, 0u);
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < block_vecs; i += int64_t(gridDim.x) * kThreads) {
    st16(kpool + (blk * block_vecs + i) * 16, z);
    st16(vpool + (blk * block_vecs + i) * 16, z);
  }
}

__global__ __launch_bounds__(kThreads) void kv_copy_blocks(char* __restrict__ kpool,
                                                           char* __restrict__ vpool,
                                                           const int32_t* __restrict__ src,
                                                           const int32_t* __restrict__ dst,
                                                           int64_t block_vecs, int64_t num_blocks,
                                                           int64_t layer_bytes, uint32_t* err) {
  kpool += int64_t(blockIdx.z) * layer_bytes;
  vpool += int64_t(blockIdx.z) * layer_bytes;
  const int s = src[blockIdx.y], d = dst[blockIdx.y];
  if (s < 0 || s >= num_blocks || d < 0 || d >= num_blocks) {
    if (blockIdx.x == 0 && blockIdx.z == 0 && threadIdx.x == 0) atomicOr(err, kErrBlock);
    return;
  }
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < block_vecs; i += int64_t(gridDim.x) * kThreads) {
    st16(kpool + (d * block_vecs + i) * 16, ld16_nt(kpool + (s * block_vecs + i) * 16));
    st16(vpool + (d * block_vecs + i) * 16, ld16_nt(vpool + (s * block_vecs + i) * 16));
  }
}

// ---------------------------------------------------------------------------
// Block-table sync: tables[seq][pos >> log2_bs] = slot >> log2_bs.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void kv_sync_tables(int32_t* __restrict__ tables, int max_blocks, int n_seqs,
                                                           const int32_t* __restrict__ seq,
                                                           const int32_t* __restrict__ pos,
                                                           const int64_t* __restrict__ slots, int n, int log2_bs,
                                                           int64_t num_blocks, uint32_t* err) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t slot = slots[i];
  if (slot < 0) return;  // padding token
  const int s = seq[i], p = pos[i];
  const int64_t blk = slot >> log2_bs;
  if (s < 0 || s >= n_seqs || p < 0 || (p >> log2_bs) >= max_blocks || blk >= num_blocks) {
    atomicOr(err, kErrTable);
    return;
  }
  tables[int64_t(s) * max_blocks + (p >> log2_bs)] = int32_t(blk);
}

// ---------------------------------------------------------------------------
// Cache set-up.
// ---------------------------------------------------------------------------
int32_t check_shape(int64_t num_blocks, int32_t block_size, int32_t n_kv_heads, int32_t head_dim,
                    int32_t dtype) {
  if (num_blocks <= 0 || n_kv_heads <= 0 || head_dim <= 0)
    return fail(IT_INVALID_INPUT, "kv cache: num_blocks=%lld n_kv_heads=%d head_dim=%d must be > 0",
                (long long)num_blocks, n_kv_heads, head_dim);
  if (!is_pow2(block_size) || block_size > 1024)
    return fail(IT_NOT_IMPLEMENTED, "kv cache: block_size %d must be a power of two <= 1024", block_size);
  if (is_quant(dtype)) {
    if (head_dim % 32) return fail(IT_INVALID_INPUT, "kv cache: quantised dtypes need head_dim %% 32 == 0");
    if (block_size < 8) return fail(IT_NOT_IMPLEMENTED, "kv cache: quantised dtypes need block_size >= 8");
  } else if (dtype_bytes(dtype) == 0) {
    return fail(IT_NOT_IMPLEMENTED,
                "kv cache: dtype %d not supported (F32=0, F16=1, Q4_0=2, Q4_1=3, Q5_0=6, Q5_1=7, Q8_0=8, BF16=30)",
                dtype);
  } else if ((head_dim * dtype_bytes(dtype)) % 16) {
    return fail(IT_NOT_IMPLEMENTED, "kv cache: head_dim*elem_bytes must be a multiple of 16");
  }
  return IT_OK;
}

int32_t make_cache(int32_t device, void* k, void* v, int32_t n_layers, int64_t num_blocks, int32_t block_size,
                   int32_t n_kv_heads, int32_t head_dim, int32_t dtype, int32_t owns, it_kv_cache** out) {
  auto* c = new (std::nothrow) it_kv_cache;
  if (!c) return fail(IT_DEVICE_ERROR, "kv cache: out of host memory");
  c->k_pool = k;
  c->v_pool = v;
  c->num_blocks = num_blocks;
  c->page_bytes = it_kv_page_bytes(block_size, head_dim, dtype);
  c->layer_bytes = num_blocks * n_kv_heads * c->page_bytes;
  c->n_layers = n_layers;
  c->owns_flag = 1;
  c->block_size = block_size;
  c->log2_bs = ilog2(block_size);
  c->n_kv_heads = n_kv_heads;
  c->head_dim = head_dim;
  c->dtype = dtype;
  c->device = device;
  c->owns_memory = owns;
  c->err_flag = nullptr;
  hipError_t e = hipMalloc(&c->err_flag, 256);
  if (e == hipSuccess) e = hipMemset(c->err_flag, 0, 256);
  if (e != hipSuccess) {
    delete c;
    return fail(IT_DEVICE_ERROR, "kv cache: error word allocation: %s", hipGetErrorString(e));
  }
  // A failed lookup here is retried (and reported) by the first
  // no-allocation decode.
  (void)noalloc_prepare(device);
  *out = c;
  return IT_OK;
}

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
}  // namespace

extern "C" int64_t it_kv_page_bytes(int32_t block_size, int32_t head_dim, int32_t dtype) {
  if (block_size <= 0 || head_dim <= 0) return -1;
  if (dtype == IT_Q8_0) return int64_t(block_size) * head_dim + int64_t(block_size) * (head_dim / IT_QK8_0) * 2;
  if (dtype == IT_Q4_0) return int64_t(block_size) * (head_dim / 2) + int64_t(block_size) * (head_dim / IT_QK4_0) * 2;
  if (dtype == IT_Q4_1) return int64_t(block_size) * (head_dim / 2) + int64_t(block_size) * (head_dim / IT_QK4_1) * 4;
  if (dtype == IT_Q5_0) return int64_t(block_size) * (head_dim / 2) + int64_t(block_size) * (head_dim / IT_QK5_0) * 6;
  if (dtype == IT_Q5_1) return int64_t(block_size) * (head_dim / 2) + int64_t(block_size) * (head_dim / IT_QK5_1) * 8;
  int64_t e = dtype_bytes(dtype);
  return e ? int64_t(block_size) * head_dim * e : -1;
}

extern "C" int32_t it_kv_cache_new_layers(int32_t device, int32_t n_layers, int64_t num_blocks,
                                          int32_t block_size, int32_t n_kv_heads, int32_t head_dim,
                                          int32_t dtype, it_kv_cache** out) {
  if (!out) return fail(IT_INVALID_INPUT, "it_kv_cache_new: out is NULL");
  *out = nullptr;
  if (n_layers <= 0 || n_layers > kMaxLayers)
    return fail(IT_INVALID_INPUT, "it_kv_cache_new: n_layers %d outside [1, %d]", n_layers, kMaxLayers);
  if (int32_t rc = check_shape(num_blocks, block_size, n_kv_heads, head_dim, dtype)) return rc;
  DeviceGuard g(device);
  const size_t bytes = size_t(n_layers) * size_t(num_blocks) * size_t(n_kv_heads) *
                       size_t(it_kv_page_bytes(block_size, head_dim, dtype));
  void *k = nullptr, *v = nullptr;
  hipError_t e = hipMalloc(&k, bytes);
  if (e == hipSuccess) e = hipMalloc(&v, bytes);
  if (e == hipSuccess) e = hipMemset(k, 0, bytes);
  if (e == hipSuccess) e = hipMemset(v, 0, bytes);
  if (e != hipSuccess) {
    if (k) (void)hipFree(k);
    if (v) (void)hipFree(v);
    return fail(IT_DEVICE_ERROR, "it_kv_cache_new: %zu bytes per pool: %s", bytes, hipGetErrorString(e));
  }
  int32_t rc = make_cache(device, k, v, n_layers, num_blocks, block_size, n_kv_heads, head_dim, dtype, 1, out);
  if (rc) {
    (void)hipFree(k);
    (void)hipFree(v);
  }
  return rc;
}

extern "C" int32_t it_kv_cache_new(int32_t device, int64_t num_blocks, int32_t block_size,
                                   int32_t n_kv_heads, int32_t head_dim, int32_t dtype,
                                   it_kv_cache** out) {
  return it_kv_cache_new_layers(device, 1, num_blocks, block_size, n_kv_heads, head_dim, dtype, out);
}

extern "C" int32_t it_kv_cache_wrap_layers(int32_t device, int32_t n_layers, void* k_pool, void* v_pool,
                                           int64_t num_blocks, int32_t block_size, int32_t n_kv_heads,
                                           int32_t head_dim, int32_t dtype, it_kv_cache** out) {
  if (!out) return fail(IT_INVALID_INPUT, "it_kv_cache_wrap: out is NULL");
  *out = nullptr;
  if (!k_pool || !v_pool) return fail(IT_INVALID_INPUT, "it_kv_cache_wrap: NULL pool");
  if (!aligned16(k_pool) || !aligned16(v_pool)) return fail(IT_INVALID_INPUT, "it_kv_cache_wrap: pools must be 16-byte aligned");
  if (n_layers <= 0 || n_layers > kMaxLayers)
    return fail(IT_INVALID_INPUT, "it_kv_cache_wrap: n_layers %d outside [1, %d]", n_layers, kMaxLayers);
  if (int32_t rc = check_shape(num_blocks, block_size, n_kv_heads, head_dim, dtype)) return rc;
  DeviceGuard g(device);
  return make_cache(device, k_pool, v_pool, n_layers, num_blocks, block_size, n_kv_heads, head_dim, dtype, 0, out);
}

extern "C" int32_t it_kv_cache_wrap(int32_t device, void* k_pool, void* v_pool, int64_t num_blocks,
                                    int32_t block_size, int32_t n_kv_heads, int32_t head_dim,
                                    int32_t dtype, it_kv_cache** out) {
  return it_kv_cache_wrap_layers(device, 1, k_pool, v_pool, num_blocks, block_size, n_kv_heads, head_dim, dtype,
                                 out);
}

extern "C" int32_t it_kv_cache_layer(const it_kv_cache* c, int32_t layer, it_kv_cache** out) {
  if (!out) return fail(IT_INVALID_INPUT, "it_kv_cache_layer: out is NULL");
  *out = nullptr;
  if (!c) return fail(IT_INVALID_INPUT, "it_kv_cache_layer: cache is NULL");
  if (layer < 0 || layer >= c->n_layers)
    return fail(IT_INVALID_INPUT, "it_kv_cache_layer: layer %d outside [0, %d)", layer, c->n_layers);
  auto* v = new (std::nothrow) it_kv_cache(*c);
  if (!v) return fail(IT_DEVICE_ERROR, "it_kv_cache_layer: out of host memory");
  v->k_pool = static_cast<char*>(c->k_pool) + int64_t(layer) * c->layer_bytes;
  v->v_pool = static_cast<char*>(c->v_pool) + int64_t(layer) * c->layer_bytes;
  v->n_layers = 1;
  v->owns_memory = 0;
  v->owns_flag = 0;
  *out = v;
  return IT_OK;
}

extern "C" int32_t it_kv_cache_destroy(it_kv_cache* c) {
  if (!c) return IT_OK;
  DeviceGuard g(c->device);
  if (c->owns_memory) {
    (void)hipFree(c->k_pool);
    (void)hipFree(c->v_pool);
  }
  if (c->owns_flag) (void)hipFree(c->err_flag);
  delete c;
  return IT_OK;
}

extern "C" int32_t it_kv_cache_describe(const it_kv_cache* c, it_kv_cache_desc* d) {
  if (!c || !d) return fail(IT_INVALID_INPUT, "it_kv_cache_describe: NULL argument");
  d->k_pool = c->k_pool;
  d->v_pool = c->v_pool;
  d->num_blocks = c->num_blocks;
  d->page_bytes = c->page_bytes;
  d->block_size = c->block_size;
  d->n_kv_heads = c->n_kv_heads;
  d->head_dim = c->head_dim;
  d->dtype = c->dtype;
  d->device = c->device;
  d->owns_memory = c->owns_memory;
  d->n_layers = c->n_layers;
  return IT_OK;
}

extern "C" int32_t it_kv_cache_check(it_kv_cache* c, void* stream) {
  if (!c) return fail(IT_INVALID_INPUT, "it_kv_cache_check: cache is NULL");
  DeviceGuard g(c->device);
  uint32_t flag = 0;
  IT_HIP(hipStreamSynchronize((hipStream_t)stream), "it_kv_cache_check: sync");
  IT_HIP(hipMemcpy(&flag, c->err_flag, 4, hipMemcpyDeviceToHost), "it_kv_cache_check: read flag");
  if (!flag) return IT_OK;
  IT_HIP(hipMemset(c->err_flag, 0, 4), "it_kv_cache_check: clear flag");
  return fail(IT_INVALID_INPUT, "kv cache: device-side range error (%s%s%s%s%s%s)", (flag & kErrSlot) ? "slot " : "",
              (flag & kErrBlock) ? "block-id " : "", (flag & kErrTable) ? "table-index " : "",
              (flag & kErrCtx) ? "ctx>max_tokens " : "", (flag & kErrPos) ? "rope-position " : "",
              (flag & kErrStart) ? "negative-start" : "");
}

extern "C" int32_t it_kv_append(it_kv_cache* c, const void* k, const void* v, int32_t src_dtype,
                                const int64_t* slots, int32_t n_tokens, void* stream) {
  if (!c) return fail(IT_INVALID_INPUT, "it_kv_append: cache is NULL");
  if (int32_t rc = one_layer(c, "it_kv_append")) return rc;
  if (n_tokens < 0) return fail(IT_INVALID_INPUT, "it_kv_append: n_tokens %d < 0", n_tokens);
  if (n_tokens == 0) return IT_OK;
  if (!k || !v || !slots) return fail(IT_INVALID_INPUT, "it_kv_append: NULL tensor");
  const bool quant = is_quant(c->dtype);
  const int32_t want = quant ? IT_F32 : c->dtype;
  if (src_dtype != want)
    return fail(IT_NOT_IMPLEMENTED, "it_kv_append: cache dtype %d takes source dtype %d, got %d", c->dtype, want, src_dtype);
  if (!aligned16(k) || !aligned16(v)) return fail(IT_INVALID_INPUT, "it_kv_append: k/v must be 16-byte aligned");
  DeviceGuard g(c->device);
  hipStream_t s = (hipStream_t)stream;
  const int64_t n_slots = c->num_blocks << c->log2_bs;
  const int64_t q8_rows = int64_t(n_tokens) * c->n_kv_heads;
  if (c->dtype == IT_Q8_0 && (c->head_dim == 64 || c->head_dim == 128 || c->head_dim == 256) &&
      q8_rows < (int64_t(1) << 30)) {
    // Row groups of 1 KiB of int8, one per wave, up to eight waves per SIMD
    // of a 256-CU device; larger appends loop.
    const int64_t groups = cdiv(q8_rows, 64 / (c->head_dim / 16));
    dim3 grid(unsigned(cdiv(std::min<int64_t>(groups, 8192), kThreads / 64)), 2);
    auto* kern = c->head_dim == 256 ? kv_append_q8_wide<256>
                 : c->head_dim == 128 ? kv_append_q8_wide<128>
                                      : kv_append_q8_wide<64>;
    hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, s, (const float*)k, (const float*)v, (char*)c->k_pool,
                       (char*)c->v_pool, slots, int32_t(q8_rows), int32_t(groups), c->n_kv_heads, c->log2_bs, c->page_bytes,
                       n_slots, c->err_flag);
  } else if (quant) {
    const int64_t total = int64_t(n_tokens) * c->n_kv_heads * (c->head_dim / 4);
    dim3 grid(unsigned(cdiv(total, kThreads)), 2);
    auto* kern = c->dtype == IT_Q8_0   ? kv_append_quant<IT_Q8_0>
                 : c->dtype == IT_Q4_0 ? kv_append_quant<IT_Q4_0>
                 : c->dtype == IT_Q4_1 ? kv_append_quant<IT_Q4_1>
                 : c->dtype == IT_Q5_0 ? kv_append_quant<IT_Q5_0>
                                       : kv_append_quant<IT_Q5_1>;
    hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, s,
                       (const float4*)k, (const float4*)v, (char*)c->k_pool, (char*)c->v_pool, slots, total,
                       c->n_kv_heads, c->head_dim, c->log2_bs, c->page_bytes, n_slots, c->err_flag);
  } else {
    const int row_vecs = int(c->head_dim * dtype_bytes(c->dtype) / 16);
    if (!is_pow2(row_vecs)) {
      const int64_t total = int64_t(n_tokens) * c->n_kv_heads * row_vecs;
      hipLaunchKernelGGL(kv_append_copy_rows, dim3(unsigned(cdiv(total, kThreads))), dim3(kThreads), 0, s,
                         (const uint4*)k, (const uint4*)v, (char*)c->k_pool, (char*)c->v_pool, slots, total,
                         c->n_kv_heads, row_vecs, c->log2_bs, c->page_bytes, n_slots, c->err_flag);
      IT_HIP(hipGetLastError(), "it_kv_append: launch");
      return IT_OK;
    }
    // Vectors in whole token groups of TPG = 64 / row_vecs tokens.
    const int64_t tpg = row_vecs < 64 ? 64 / row_vecs : 1;
    const int64_t total = cdiv(n_tokens, tpg) * tpg * c->n_kv_heads * row_vecs;
    if (total >= (int64_t(1) << 31) - int64_t(kThreads) * kVecsPerLane)
      return fail(IT_INVALID_INPUT, "it_kv_append: %lld vectors in one call (at most 2^31)", (long long)total);
    hipLaunchKernelGGL(kv_append_copy, dim3(unsigned(cdiv(total, int64_t(kThreads) * kVecsPerLane))), dim3(kThreads),
                       0, s, (const uint4*)k, (const uint4*)v, (char*)c->k_pool, (char*)c->v_pool, slots, n_tokens,
                       c->n_kv_heads, ilog2(row_vecs), c->log2_bs, c->page_bytes, n_slots, c->err_flag);
  }
  IT_HIP(hipGetLastError(), "it_kv_append: launch");
  return IT_OK;
}

extern "C" int32_t it_kv_gather(const it_kv_cache* c, const int32_t* bt, int32_t max_blocks,
                                const int32_t* ctx_lens, const int32_t* start_pos, const int64_t* cu_out,
                                int32_t n_seqs, int32_t max_tokens, void* k_out, void* v_out,
                                void* stream) {
  if (!c) return fail(IT_INVALID_INPUT, "it_kv_gather: cache is NULL");
  if (int32_t rc = one_layer(c, "it_kv_gather")) return rc;
  if (n_seqs < 0 || max_tokens < 0 || max_blocks <= 0)
    return fail(IT_INVALID_INPUT, "it_kv_gather: n_seqs=%d max_tokens=%d max_blocks=%d", n_seqs, max_tokens, max_blocks);
  if (n_seqs == 0 || max_tokens == 0) return IT_OK;
  if (!bt || !ctx_lens || !cu_out || !k_out || !v_out) return fail(IT_INVALID_INPUT, "it_kv_gather: NULL tensor");
  if (n_seqs > 65535) return fail(IT_NOT_IMPLEMENTED, "it_kv_gather: n_seqs %d > 65535", n_seqs);
  DeviceGuard g(c->device);
  hipStream_t s = (hipStream_t)stream;
  if (is_quant(c->dtype)) {
    const int64_t per_seq = int64_t(c->n_kv_heads) * max_tokens * (c->head_dim / 32);
    dim3 grid(unsigned(cdiv(per_seq, kThreads)), unsigned(n_seqs));
    auto* kern = c->dtype == IT_Q8_0   ? kv_gather_q8_0
                 : c->dtype == IT_Q4_0 ? kv_gather_nib<IT_Q4_0>
                 : c->dtype == IT_Q4_1 ? kv_gather_nib<IT_Q4_1>
                 : c->dtype == IT_Q5_0 ? kv_gather_nib<IT_Q5_0>
                                       : kv_gather_nib<IT_Q5_1>;
    hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, s,
                       (const char*)c->k_pool, (const char*)c->v_pool,
                       bt, max_blocks, ctx_lens, start_pos, cu_out, c->n_kv_heads, c->head_dim, c->log2_bs,
                       c->page_bytes, c->num_blocks, (char*)k_out, (char*)v_out, c->err_flag);
  } else {
    if (!aligned16(k_out) || !aligned16(v_out)) return fail(IT_INVALID_INPUT, "it_kv_gather: outputs must be 16-byte aligned");
    const int row_vecs = int(c->head_dim * dtype_bytes(c->dtype) / 16);
    const int64_t per_seq = int64_t(c->n_kv_heads) * max_tokens * row_vecs;
    dim3 grid(unsigned(cdiv(per_seq, kThreads)), unsigned(n_seqs));
    hipLaunchKernelGGL(kv_gather_vec, grid, dim3(kThreads), 0, s, (const char*)c->k_pool, (const char*)c->v_pool,
                       bt, max_blocks, ctx_lens, start_pos, cu_out, c->n_kv_heads, row_vecs, c->log2_bs,
                       c->page_bytes, c->num_blocks, (uint4*)k_out, (uint4*)v_out, c->err_flag);
  }
  IT_HIP(hipGetLastError(), "it_kv_gather: launch");
  return IT_OK;
}

extern "C" int32_t it_kv_evict(it_kv_cache* c, const int32_t* blocks, int32_t n, void* stream) {
  if (!c) return fail(IT_INVALID_INPUT, "it_kv_evict: cache is NULL");
  if (n < 0 || n > 65535) return fail(IT_INVALID_INPUT, "it_kv_evict: n=%d outside [0, 65535]", n);
  if (n == 0) return IT_OK;
  if (!blocks) return fail(IT_INVALID_INPUT, "it_kv_evict: blocks is NULL");
  DeviceGuard g(c->device);
  const int64_t block_vecs = c->page_bytes * c->n_kv_heads / 16;
  dim3 grid(unsigned(cdiv(block_vecs, kThreads) > 64 ? 64 : cdiv(block_vecs, kThreads)), unsigned(n),
            unsigned(c->n_layers));
  hipLaunchKernelGGL(kv_clear_blocks, grid, dim3(kThreads), 0, (hipStream_t)stream, (char*)c->k_pool,
                     (char*)c->v_pool, blocks, block_vecs, c->num_blocks, c->layer_bytes, c->err_flag);
  IT_HIP(hipGetLastError(), "it_kv_evict: launch");
  return IT_OK;
}

extern "C" int32_t it_kv_sync_tables(it_kv_cache* c, int32_t* tables, int32_t max_blocks, int32_t n_seqs,
                                     const int32_t* seq, const int32_t* pos, const int64_t* slots, int32_t n,
                                     void* stream) {
  if (!c) return fail(IT_INVALID_INPUT, "it_kv_sync_tables: cache is NULL");
  if (n < 0 || max_blocks <= 0 || n_seqs <= 0)
    return fail(IT_INVALID_INPUT, "it_kv_sync_tables: n=%d max_blocks=%d n_seqs=%d", n, max_blocks, n_seqs);
  if (n == 0) return IT_OK;
  if (!tables || !seq || !pos || !slots) return fail(IT_INVALID_INPUT, "it_kv_sync_tables: NULL tensor");
  DeviceGuard g(c->device);
  hipLaunchKernelGGL(kv_sync_tables, dim3(unsigned(cdiv(n, kThreads))), dim3(kThreads), 0, (hipStream_t)stream,
                     tables, max_blocks, n_seqs, seq, pos, slots, n, c->log2_bs, c->num_blocks, c->err_flag);
  IT_HIP(hipGetLastError(), "it_kv_sync_tables: launch");
  return IT_OK;
}

extern "C" int32_t it_kv_copy_blocks(it_kv_cache* c, const int32_t* src, const int32_t* dst, int32_t n,
                                     void* stream) {
  if (!c) return fail(IT_INVALID_INPUT, "it_kv_copy_blocks: cache is NULL");
  if (n < 0 || n > 65535) return fail(IT_INVALID_INPUT, "it_kv_copy_blocks: n=%d outside [0, 65535]", n);
  if (n == 0) return IT_OK;
  if (!src || !dst) return fail(IT_INVALID_INPUT, "it_kv_copy_blocks: NULL list");
  DeviceGuard g(c->device);
  const int64_t block_vecs = c->page_bytes * c->n_kv_heads / 16;
  dim3 grid(unsigned(cdiv(block_vecs, kThreads) > 64 ? 64 : cdiv(block_vecs, kThreads)), unsigned(n),
            unsigned(c->n_layers));
  hipLaunchKernelGGL(kv_copy_blocks, grid, dim3(kThreads), 0, (hipStream_t)stream, (char*)c->k_pool,
                     (char*)c->v_pool, src, dst, block_vecs, c->num_blocks, c->layer_bytes, c->err_flag);
  IT_HIP(hipGetLastError(), "it_kv_copy_blocks: launch");
  return IT_OK;
}

extern "C" int32_t it_supports(int32_t op, int32_t dtype) {
  const bool kv = dtype == IT_F32 || dtype == IT_F16 || dtype == IT_BF16 || is_quant(dtype);
  switch (op) {
    case IT_OP_KV_APPEND:
    case IT_OP_KV_GATHER:
    case IT_OP_KV_EVICT:
    case IT_OP_KV_COPY_BLOCKS:
    case IT_OP_PAGED_DECODE: return kv ? 1 : 0;
    case IT_OP_PAGED_PREFILL: return (dtype == IT_BF16 || dtype == IT_F16) ? 1 : 0;
    case IT_OP_FLASH_ATTENTION: return dtype == IT_F32 ? 1 : 0;
    default: return 0;
  }
}
