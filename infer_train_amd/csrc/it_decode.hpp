// it_decode.hpp -- paged split-K flash-decode for gfx950 (device code).
//
// One workgroup (8 wave64s) owns one (sequence, KV head, head chunk,
// partition of P tokens).  The GC query heads of the chunk share every K/V
// byte the workgroup reads, so each KV page is read from HBM once per
// partition.
//
// K/V staging.  The partition's K rows, then its V rows, stream through a
// ring of kRing 8 KiB LDS tiles filled by direct global->LDS loads
// (global_load_lds_dwordx4: 64 lanes x 16 B per instruction, no VGPR round
// trip).  Each wave moves 1 KiB of every tile; each lane supplies the
// address of its own 16 bytes, so one instruction gathers whole token rows
// from whatever pages the block table names.  In LDS a tile is [T tokens]
// [row bytes], and the 8 waves' loads of one tile cover 2 whole 4 KiB pages
// (bf16, D 128, 16-token blocks) at once, which keeps DRAM pages open.
// Before consuming tile s every wave waits for its own loads of tile s (an
// explicit vmcnt count) and meets the others at a barrier; the slot read at
// step s-1 is then free for the load of tile s+kRing-1.
//
// Occupancy is the design constraint.  Measured on MI355X, this read pattern
// reaches ~72% of HBM peak only with ~32 waves per CU each holding a few
// 1 KiB loads in flight (more loads per wave, fewer waves, is slower).  So
// a workgroup keeps <= 40 KiB of LDS (4 per CU) and a wave <= 64 VGPRs
// (8 per SIMD): q is held only during the QK phase, the PV accumulators only
// during the PV phase, 4 dims of each per lane.
//
// The loads are issued from inline asm on purpose: the compiler's wait
// insertion cannot tell which ring slot an LDS read touches and would drain
// every outstanding load (vmcnt(0)) before it, serialising the ring.  With
// the DMA hidden, the only vmcnt waits are the counted ones below, which
// cover every dependency on ring data by themselves.
//
// Three phases, as in flash_attn_f32 with the max taken over the partition
// first (src/backend/arm/flash_attn.rs:6-72):
//  1. QK over the K tiles.  A token row is split over LQ lanes (16 bytes
//     each); each lane forms GC partial dot products (v_dot2_f32_bf16 / _f16
//     on packed 16-bit data, fp32 FMA otherwise) and sums them across the LQ
//     lanes with DPP row operations.  Scaled scores (log2 domain) go to LDS.
//  2. Softmax statistics.  Per head, the partition max and the sum of
//     exp2(s - max) are wavefront reductions (DPP within rows, ds_swizzle
//     and a bpermute across rows); the probabilities replace the scores.
//     The first V tiles are already in flight meanwhile.
//  3. PV over the V tiles.  A value row is split over LV lanes (4 dims
//     each); each lane accumulates GC x 4 fp32 outputs; the partial sums are
//     reduced across lanes (bpermute) and across the 8 waves (LDS).
//
// The partition's (m, l, O) go to the workspace; a second kernel merges the
// partitions: M = max m_p, L = sum l_p 2^(m_p-M), O = sum O_p 2^(m_p-M) / L,
// the split-K form of flash_attn_f32's online rescaling
// (src/backend/arm/flash_attn.rs:42-63, final 1/s at :66-71).
#pragma once
#include <hip/hip_runtime.h>

#include <type_traits>

#include "it_device.hpp"
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
};

template <int DT> struct KvTraits;
template <> struct KvTraits<IT_BF16> { static constexpr int kElemBytes = 2; };
template <> struct KvTraits<IT_F16> { static constexpr int kElemBytes = 2; };
template <> struct KvTraits<IT_F32> { static constexpr int kElemBytes = 4; };
template <> struct KvTraits<IT_Q8_0> { static constexpr int kElemBytes = 1; };

constexpr int kDecodeWaves = 8;
constexpr int kDecodeThreads = 64 * kDecodeWaves;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kRing = 3;                        // LDS ring slots
constexpr int kTileBytes = 1024 * kDecodeWaves; // one slot: one 1 KiB load per wave
constexpr int kScaleTileBytes = 512;            // Q8_0 fp16 scales of one tile (64 B per wave)
constexpr size_t kDecodeLdsTarget = 40 * 1024;  // 4 workgroups (32 waves) per CU

// Tile geometry of a (dtype, head_dim) pair.  Every wave loads, and then
// computes on, its own kOwnRows rows of each tile.
template <int DT, int D>
struct DecodeGeo {
  static constexpr int kRowBytes = DT == IT_Q8_0 ? D : D * KvTraits<DT>::kElemBytes;  // main plane
  static constexpr int kTokens = kTileBytes / kRowBytes;  // tokens per tile
  static constexpr int kOwnRows = 1024 / kRowBytes;       // tokens per wave per tile
  static constexpr int kScaleBytes = DT == IT_Q8_0 ? D / 16 : 0;  // fp16 per 32 values, per token
  static constexpr int kLoadsPerTile = 1 + (DT == IT_Q8_0 ? 1 : 0);  // vmcnt units per wave per tile
  static constexpr int kScaleRing = DT == IT_Q8_0 ? kRing * kScaleTileBytes : 0;
  // QK: 16-bit caches give each lane 8 dims (16 B, packed pairs), F32 4 dims
  // (16 B), Q8_0 4 dims (4 B + the group's scale).  PV: 4 dims per lane.
  static constexpr int kQkDims = (DT == IT_BF16 || DT == IT_F16) ? 8 : 4;
  static constexpr int kPvDims = 4;
  static_assert(kRowBytes >= 16 && kRowBytes <= 1024, "row must fit one 1 KiB load");
  static_assert(DT != IT_Q8_0 || kOwnRows * kScaleBytes == kScaleTileBytes / kDecodeWaves, "scale tile");
};

// Dynamic LDS of one workgroup: ring, Q8_0 scale ring, the partition's
// scores ([P/4][GC][4] fp32), the page list.  The cross-wave reduction
// buffer [4][GC][D] fp32 (<= 32 KiB) reuses the same bytes at the end.
inline size_t decode_lds_bytes(int32_t dt, int gc, int d, int partition, int max_pages) {
  const size_t passes = size_t(kRing) * kTileBytes + (dt == IT_Q8_0 ? size_t(kRing) * kScaleTileBytes : 0) +
                        size_t(partition) * gc * 4 + size_t(max_pages) * 4;
  const size_t red = size_t(4) * gc * d * 4;
  return passes > red ? passes : red;
}

// ---- LDS DMA and counted waits --------------------------------------------
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  // Generic -> LDS address-space cast (a C-style cast is the only spelling
  // clang accepts), then the 32-bit LDS byte offset.
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}
// 64 lanes x 16 B from per-lane global addresses into LDS [m0, m0 + 1 KiB).
// One wait state between the SALU write of M0 and the LDS-DMA read of it.
__device__ __forceinline__ void dma_b128(const void* g, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(g) : "memory", "m0");
}
// Active lanes x 4 B into LDS [m0 + 4 lane].
__device__ __forceinline__ void dma_b32(const void* g, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(m0), "v"(g) : "memory", "m0");
}
// Wait until at most N of this wave's vector-memory ops are outstanding and
// its LDS ops are done, then meet the workgroup.
template <int N>
__device__ __forceinline__ void vm_wait_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ float i8f(uint32_t w, int j) { return float(int32_t(w << (24 - 8 * j)) >> 24); }

template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (DT == IT_BF16) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a), __builtin_bit_cast(bf2, b), c, false);
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
  }
}
// a.lo*b.lo + a.hi*b.hi with a zero accumulator, in the 3-operand VOP3P
// encoding (the builtin with 0.0f becomes v_mov 0 + v_dot2c).
template <int DT>
__device__ __forceinline__ float dot2_first(uint32_t a, uint32_t b) {
  float r;
  if constexpr (DT == IT_BF16) asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  else asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// fp32 -> the cache's 16-bit type (round to nearest even) and back.
template <int DT>
__device__ __forceinline__ uint32_t to16(float f) {
  if constexpr (DT == IT_BF16) return f32_to_bf16_bits(f);
  else return f32_to_f16_bits(f);
}
template <int DT>
__device__ __forceinline__ float from16(uint32_t h) {
  if constexpr (DT == IT_BF16) return __uint_as_float(h << 16);
  else return f16_bits_to_f32(h);
}

// Keep values in VGPRs as they are: an empty asm that "uses" them, so the
// compiler's wait for the loads that produced them lands here.
template <int N>
__device__ __forceinline__ void pin(uint32_t (&r)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(r[i]));
}

template <int DT, int D, int GC>
__global__ __launch_bounds__(kDecodeThreads) __attribute__((amdgpu_waves_per_eu(8, 8)))
void paged_decode_split(DecodeArgs a) {
  using G = DecodeGeo<DT, D>;
  constexpr int RB = G::kRowBytes;
  constexpr int TT = G::kTokens;   // tokens per tile
  constexpr int OR = G::kOwnRows;  // tokens per wave per tile
  constexpr int DPL = G::kQkDims;  // dims per lane, QK phase
  constexpr int LQ = D / DPL;      // lanes per token, QK phase
  constexpr int RQ = 64 / LQ;      // tokens per wave pass, QK phase
  constexpr int DPV = G::kPvDims;  // dims per lane, PV phase
  constexpr int LV = D / DPV;      // lanes per token (or token pair), PV phase
  constexpr int RV = 64 / LV;      // tokens (or token pairs) per wave pass, PV phase
  constexpr int LPT = G::kLoadsPerTile;
  constexpr bool k16 = DT == IT_BF16 || DT == IT_F16;
  constexpr int QW = k16 ? DPL / 2 : DPL;  // q registers per head
  // PV rows per pass: 16-bit caches take token pairs (v_dot2 over two tokens).
  constexpr int PVR = k16 ? 2 * RV : RV;
  static_assert(LQ >= 8 && LQ <= 64 && LV >= 16 && LV <= 64, "bad lane split");
  static_assert(OR % RQ == 0 && OR % PVR == 0, "own rows must fill whole wave passes");
  static_assert(GC <= kDecodeWaves && GC <= LQ, "stats give each head one wave; one writer lane per head");

  extern __shared__ __attribute__((aligned(16))) char smem[];
  char* const ring = smem;
  char* const sring = smem + size_t(kRing) * kTileBytes;
  // Scores, then probabilities, of the partition, [P/4][GC][4]: the GC
  // values of one token are 16 B apart (one address, immediate offsets in a
  // PV pass) and a head's consecutive tokens hit distinct banks.  A 16-bit
  // cache's probabilities are packed token pairs stored in the even slot.
  float* const s_sc = reinterpret_cast<float*>(sring + G::kScaleRing);
  int32_t* const s_pages = reinterpret_cast<int32_t*>(s_sc + a.partition * GC);
  auto sc_at = [&](int g, int i) -> float& { return s_sc[((i >> 2) * GC + g) * 4 + (i & 3)]; };

  const int part = blockIdx.x;
  const int kvh = blockIdx.y / a.chunks;
  const int chunk = blockIdx.y - kvh * a.chunks;
  const int b = blockIdx.z;
  const int head0 = kvh * a.group + chunk * GC;

  const int ctx = a.ctx_lens ? a.ctx_lens[b] : a.ctx_const;
  const int st = a.start_pos ? a.start_pos[b] : 0;
  const int n = ctx - st;
  const int P = a.partition;
  if (n <= 0 || part * P >= n) return;  // uniform for the workgroup
  if (part == a.max_parts - 1 && n > a.max_parts * P && threadIdx.x == 0)
    atomicOr(a.err, 8u);  // context longer than the caller's max_tokens: tail ignored
  const int tok0 = st + part * P;
  const int nt = min(P, n - part * P);
  // The wave index is uniform: readfirstlane keeps it, and everything
  // derived from it, in SGPRs (VGPRs are the occupancy budget).
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bs_mask = (1 << a.log2_bs) - 1;
  const int64_t bs = int64_t(bs_mask) + 1;

  // Page indices (block * n_kv_heads + kvh) of the partition, via LDS.
  const int lb0 = tok0 >> a.log2_bs;
  const int nlb = ((tok0 + nt - 1) >> a.log2_bs) - lb0 + 1;  // <= max_pages
  for (int i = tid; i < nlb; i += kDecodeThreads) {
    const int lb = lb0 + i;
    int blk = lb;
    if (a.bt) {
      if (lb >= a.max_blocks) {
        atomicOr(a.err, 4u);
        blk = 0;
      } else {
        blk = a.bt[int64_t(b) * a.max_blocks + lb];
      }
    }
    if (blk < 0 || blk >= a.num_blocks) {
      atomicOr(a.err, 2u);
      blk = 0;
    }
    s_pages[i] = blk * a.n_kv_heads + kvh;
  }

  // q of the chunk's GC heads, in the QK lane layout: lane li holds dims
  // [DPL li, DPL li + DPL) of every head.
  const int li_q = lane % LQ, tj_q = lane / LQ;
  const int64_t qrow = (int64_t(b) * a.n_heads + head0) * D;
  uint32_t qr[GC * QW];  // packed 16-bit pairs, or fp32 bits
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    const uint4 q4 = k16 ? ld16(static_cast<const uint16_t*>(a.q) + qrow + g * D + DPL * li_q)
                         : ld16(static_cast<const float*>(a.q) + qrow + g * D + DPL * li_q);
    qr[g * QW + 0] = q4.x;
    qr[g * QW + 1] = q4.y;
    qr[g * QW + 2] = q4.z;
    qr[g * QW + 3] = q4.w;
  }
  // Consume q (and the block-table loads) before any DMA is issued: the
  // compiler places its wait for those loads at their first use, and a wait
  // computed there would not know about the ring loads issued in between.
  pin(qr);
  __syncthreads();

  // The stream: the partition's K tiles, then its V tiles.
  const int nk = (nt + TT - 1) / TT;  // tiles per plane
  const int S = 2 * nk;
  const uint32_t ring_m0 = lds_offset(ring) + uint32_t(wave) * 1024u;
  const uint32_t sring_m0 = lds_offset(sring) + uint32_t(wave) * 64u;
  // This lane's 16-byte piece of its wave's 1 KiB load: tile row and column.
  const int dma_row = (wave * 1024 + lane * 16) / RB;
  const int dma_col = (wave * 1024 + lane * 16) % RB;
  const uint32_t page_bytes = uint32_t(a.page_bytes);

  // Issue this wave's loads of stream tile s into ring slot s % kRing: its
  // own rows [OR wave, OR wave + OR) of the tile (and their Q8_0 scales).
  auto issue = [&](int s) {
    const bool is_v = s >= nk;
    const int tt = is_v ? s - nk : s;
    const char* pool = is_v ? a.v_pool : a.k_pool;
    const int slot = s % kRing;
    {
      int tr = tt * TT + dma_row;
      if (tr >= nt) tr = 0;  // rows past the partition load a stand-in row (zeroed on arrival)
      const int t = tok0 + tr;
      const uint32_t page = uint32_t(s_pages[(t >> a.log2_bs) - lb0]);
      const char* g = pool + (uint64_t(page) * page_bytes + uint32_t((t & bs_mask) * RB + dma_col));
      dma_b128(g, __builtin_amdgcn_readfirstlane(ring_m0 + uint32_t(slot) * kTileBytes));
    }
    if constexpr (DT == IT_Q8_0) {
      if (lane < 16) {  // 16 lanes x 4 B = the scales of this wave's rows
        const int byte = wave * 64 + lane * 4;
        const int row = byte / G::kScaleBytes, col = byte % G::kScaleBytes;
        int tr = tt * TT + row;
        if (tr >= nt) tr = 0;
        const int t = tok0 + tr;
        const uint32_t page = uint32_t(s_pages[(t >> a.log2_bs) - lb0]);
        const char* g = pool + (uint64_t(page) * page_bytes +
                                uint32_t(bs * D + (t & bs_mask) * G::kScaleBytes + col));
        dma_b32(g, __builtin_amdgcn_readfirstlane(sring_m0 + uint32_t(slot) * kScaleTileBytes));
      }
    }
  };
  // Before consuming tile s: this wave's loads of tile s are done (at most
  // `later` tiles issued after it are outstanding), then the barrier, which
  // also frees the slot consumed at step s-1 for the load issued next.
  auto wait_tile = [&](int s) {
    if (s + kRing - 1 <= S) vm_wait_barrier<(kRing - 2) * LPT>();  // one tile issued after s
    else vm_wait_barrier<0>();
  };
  static_assert(kRing - 2 == 1, "wait_tile covers later = 0..1");
  // Rows of tile tt past the partition's end were loaded from a stand-in
  // row.  Once the tile has landed each lane zeroes its own 16 bytes (and
  // Q8_0 scale bytes) of such rows; a wave reads only rows it loaded, and
  // the LDS ops of one wave stay in order.
  auto zero_tail = [&](int slot, int tt) {
    if (tt * TT + dma_row >= nt)
      *reinterpret_cast<uint4*>(ring + slot * kTileBytes + wave * 1024 + lane * 16) = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (DT == IT_Q8_0) {
      if (lane < 16 && tt * TT + (wave * 64 + lane * 4) / G::kScaleBytes >= nt)
        *reinterpret_cast<uint32_t*>(sring + slot * kScaleTileBytes + wave * 64 + lane * 4) = 0u;
    }
  };

  // Prologue: the first kRing-1 tiles of the stream.
  for (int s = 0; s < kRing - 1 && s < S; ++s) issue(s);

  // ---------------- phase 1: raw q.k over the K tiles -----------------------
  // After the DPP reduction every lane of a token's LQ-lane row holds all GC
  // sums; lane li writes head li's (a select chain, one LDS write).
  for (int s = 0; s < nk; ++s) {
    wait_tile(s);
    if (s + kRing - 1 < S) issue(s + kRing - 1);
    const char* tile = ring + (s % kRing) * kTileBytes;
    const char* stile = sring + (s % kRing) * kScaleTileBytes;
    if ((s + 1) * TT > nt) zero_tail(s % kRing, s);
#pragma unroll 1
    for (int pass = 0; pass < OR / RQ; ++pass) {
      const int local = wave * OR + pass * RQ + tj_q;  // row in the tile
      const int tr = s * TT + local;                   // token in the partition
      const char* row = tile + local * RB;
      float sc[GC];
      if constexpr (k16) {
        const uint4 k4 = ld16(row + 16 * li_q);
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          float x = dot2_first<DT>(k4.x, qr[g * QW + 0]);
          x = dot2<DT>(k4.y, qr[g * QW + 1], x);
          x = dot2<DT>(k4.z, qr[g * QW + 2], x);
          x = dot2<DT>(k4.w, qr[g * QW + 3], x);
          sc[g] = group_sum<LQ>(x);
        }
      } else {
        float kf[4];
        float dsc = 1.0f;
        if constexpr (DT == IT_F32) {
          const float4 k4 = *reinterpret_cast<const float4*>(row + 16 * li_q);
          kf[0] = k4.x; kf[1] = k4.y; kf[2] = k4.z; kf[3] = k4.w;
        } else {
          const uint32_t w = *reinterpret_cast<const uint32_t*>(row + 4 * li_q);
#pragma unroll
          for (int j = 0; j < 4; ++j) kf[j] = i8f(w, j);
          dsc = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(stile + local * G::kScaleBytes + (li_q / 8) * 2));
        }
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          float x = __uint_as_float(qr[g * QW + 0]) * kf[0];
          x = fmaf(__uint_as_float(qr[g * QW + 1]), kf[1], x);
          x = fmaf(__uint_as_float(qr[g * QW + 2]), kf[2], x);
          x = fmaf(__uint_as_float(qr[g * QW + 3]), kf[3], x);
          if constexpr (DT == IT_Q8_0) x *= dsc;  // x = f32(d) * q (gemv.rs:151-160)
          sc[g] = group_sum<LQ>(x);
        }
      }
      float mine = sc[0];
#pragma unroll
      for (int g = 1; g < GC; ++g) mine = li_q == g ? sc[g] : mine;
      if (li_q < GC && tr < nt) sc_at(li_q, tr) = mine;
    }
  }
  lds_barrier();

  // ---------------- phase 2: softmax statistics ---------------------------
  // Scores become log2-domain: x * scale * log2(e), or with the Backend op's
  // additive mask (arm.rs:304-370) (x * scale + mask) * log2(e), where a
  // -inf mask skips the key (flash_attn.rs:35-40).  Probabilities
  // exp2(s - max) replace them; slots past the partition get 0.  16-bit
  // caches keep them as packed token pairs in the cache's type (the PV
  // products run on v_dot2, accumulating in fp32) and the sum adds the
  // rounded values, i.e. exactly the weights PV applies.
  const bool masked = a.mask != nullptr;
  const float mult = masked ? 1.0f : a.scale_log2;  // raw -> log2 domain (scale > 0 keeps the max)
  const int64_t part_row = (int64_t(b) * a.n_heads + head0) * a.max_parts + part;
  if (wave < GC) {
    const int g = wave;
    float mx = -INFINITY;
    if (masked) {
      for (int i = lane; i < nt; i += 64) {
        const float mk = a.mask[tok0 + i];
        const float x = (mk == -INFINITY) ? -INFINITY : (sc_at(g, i) * a.scale + mk) * kLog2e;
        sc_at(g, i) = x;
        mx = fmaxf(mx, x);
      }
    } else {
      for (int i = lane; i < nt; i += 64) mx = fmaxf(mx, sc_at(g, i));
    }
    mx = group_max<64>(mx);
    const bool none = mx == -INFINITY;  // every key skipped: zeros (flash_attn.rs:66-71)
    float sum = 0.0f;
    if constexpr (k16) {
      for (int j = lane; 2 * j < nk * TT; j += 64) {
        const int i0 = 2 * j, i1 = 2 * j + 1;
        const float p0 = (i0 < nt && !none) ? __builtin_amdgcn_exp2f((sc_at(g, i0) - mx) * mult) : 0.0f;
        const float p1 = (i1 < nt && !none) ? __builtin_amdgcn_exp2f((sc_at(g, i1) - mx) * mult) : 0.0f;
        const uint32_t h0 = to16<DT>(p0), h1 = to16<DT>(p1);
        sum += from16<DT>(h0) + from16<DT>(h1);
        reinterpret_cast<uint32_t&>(sc_at(g, i0)) = h0 | (h1 << 16);
      }
    } else {
      for (int i = lane; i < nk * TT; i += 64) {
        const float p = (i < nt && !none) ? __builtin_amdgcn_exp2f((sc_at(g, i) - mx) * mult) : 0.0f;
        sc_at(g, i) = p;
        sum += p;
      }
    }
    sum = group_sum<64>(sum);
    if (lane == 0) {
      float* ml = a.ws_ml + (part_row + int64_t(g) * a.max_parts) * 2;
      ml[0] = none ? mx : mx * mult;  // log2 domain for the combine
      ml[1] = sum;
    }
  }
  // (the barrier of the first V tile's wait orders these writes before PV)

  // ---------------- phase 3: P.V over the V tiles --------------------------
  float acc[GC][DPV];
#pragma unroll
  for (int g = 0; g < GC; ++g)
#pragma unroll
    for (int j = 0; j < DPV; ++j) acc[g][j] = 0.0f;
  const int li_v = lane % LV, tj_v = lane / LV;
  for (int s = nk; s < S; ++s) {
    wait_tile(s);
    if (s + kRing - 1 < S) issue(s + kRing - 1);
    const int i = s - nk;
    const char* tile = ring + (s % kRing) * kTileBytes;
    const char* stile = sring + (s % kRing) * kScaleTileBytes;
    if ((i + 1) * TT > nt) zero_tail(s % kRing, i);
#pragma unroll 1
    for (int pass = 0; pass < OR / PVR; ++pass) {
      if constexpr (k16) {
        // Lane li of pair slot tj: dims [4 li, 4 li + 4) of rows r and r+1;
        // v_perm builds (v_r[d], v_r+1[d]) pairs for v_dot2 against the
        // packed probability pair.
        const int local = wave * OR + pass * PVR + 2 * tj_v;
        const int tr = i * TT + local;
        const uint2 wa = *reinterpret_cast<const uint2*>(tile + local * RB + 8 * li_v);
        const uint2 wb = *reinterpret_cast<const uint2*>(tile + (local + 1) * RB + 8 * li_v);
        uint32_t vp[4];
        vp[0] = __builtin_amdgcn_perm(wb.x, wa.x, 0x05040100u);
        vp[1] = __builtin_amdgcn_perm(wb.x, wa.x, 0x07060302u);
        vp[2] = __builtin_amdgcn_perm(wb.y, wa.y, 0x05040100u);
        vp[3] = __builtin_amdgcn_perm(wb.y, wa.y, 0x07060302u);
        const uint32_t* pt = reinterpret_cast<const uint32_t*>(&sc_at(0, tr));
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          const uint32_t pp = pt[4 * g];
#pragma unroll
          for (int j = 0; j < DPV; ++j) acc[g][j] = dot2<DT>(vp[j], pp, acc[g][j]);
        }
      } else {
        const int local = wave * OR + pass * PVR + tj_v;
        const int tr = i * TT + local;
        const char* row = tile + local * RB;
        float vf[DPV];
        float dsc = 1.0f;
        if constexpr (DT == IT_F32) {
          const float4 v4 = *reinterpret_cast<const float4*>(row + 16 * li_v);
          vf[0] = v4.x; vf[1] = v4.y; vf[2] = v4.z; vf[3] = v4.w;
        } else {
          const uint32_t w = *reinterpret_cast<const uint32_t*>(row + 4 * li_v);
#pragma unroll
          for (int j = 0; j < 4; ++j) vf[j] = i8f(w, j);
          dsc = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(stile + local * G::kScaleBytes + (li_v / 8) * 2));
        }
        const float* pt = &sc_at(0, tr);
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          float p = pt[4 * g];
          if constexpr (DT == IT_Q8_0) p *= dsc;  // p * (d * q) = (p * d) * q
#pragma unroll
          for (int j = 0; j < DPV; ++j) acc[g][j] = fmaf(p, vf[j], acc[g][j]);
        }
      }
    }
  }

  // Reduce over the RV slots of the wave that share dims (lanes li, li + 32).
  // One head at a time: left alone the scheduler issues every bpermute
  // before the first add and the results need GC x DPV extra VGPRs.
  if constexpr (RV == 2) {
#pragma unroll
    for (int g = 0; g < GC; ++g) {
#pragma unroll
      for (int j = 0; j < DPV; ++j) acc[g][j] += swap_halves(acc[g][j]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // Across the 8 waves, in a fixed order: waves 4..7 park their sums, waves
  // 0..3 add theirs, then every thread sums the 4 slots of its outputs.
  lds_barrier();  // every wave is done with the ring
  float* s_red = reinterpret_cast<float*>(smem);  // [4][GC][D]
  const int slot = wave & 3;
  if (wave >= 4 && tj_v == 0) {
#pragma unroll
    for (int g = 0; g < GC; ++g)
      *reinterpret_cast<float4*>(&s_red[(slot * GC + g) * D + DPV * li_v]) =
          make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
  }
  lds_barrier();
  if (wave < 4 && tj_v == 0) {
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      float4* r = reinterpret_cast<float4*>(&s_red[(slot * GC + g) * D + DPV * li_v]);
      const float4 o = *r;
      *r = make_float4(acc[g][0] + o.x, acc[g][1] + o.y, acc[g][2] + o.z, acc[g][3] + o.w);
      __builtin_amdgcn_sched_barrier(0);  // one head in flight (else GC x 4 extra VGPRs)
    }
  }
  lds_barrier();
  for (int i = tid; i < GC * D; i += kDecodeThreads) {
    const float o = (s_red[i] + s_red[GC * D + i]) + (s_red[2 * GC * D + i] + s_red[3 * GC * D + i]);
    const int g = i / D, d = i - g * D;
    a.ws_o[(part_row + int64_t(g) * a.max_parts) * D + d] = o;
  }
}

// Merge the partitions of one (sequence, head).  64 lanes; lane owns D/64
// output dims.  M = max m_p, L = sum l_p 2^(m_p - M), O = sum O_p 2^(m_p - M)
// / L (the split-K form of flash_attn_f32's rescaling, flash_attn.rs:42-71).
// The partials are read in chunks of kChunk partitions whose loads are all in
// flight together (every lane reads the chunk's (m, l) pairs itself, so no
// cross-lane step sits between them and the O loads).  With more than one
// chunk, M comes from a first pass over the (m, l) pairs.
template <int D>
__global__ __launch_bounds__(64) void paged_decode_combine(const float* __restrict__ ws_o,
                                                           const float* __restrict__ ws_ml,
                                                           const int32_t* __restrict__ ctx_lens,
                                                           const int32_t* __restrict__ start_pos,
                                                           int ctx_const, int n_heads, int partition,
                                                           int max_parts, void* out, int out_dtype) {
  // Partitions beyond max_parts were never computed (the split pass latched
  // the error); only the computed ones are merged.
  constexpr int DL = D / 64;
  constexpr int kChunk = 8;
  const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int ctx = ctx_lens ? ctx_lens[b] : ctx_const;
  const int st = start_pos ? start_pos[b] : 0;
  const int n = ctx - st;
  const int np = n > 0 ? min((n + partition - 1) / partition, max_parts) : 0;
  const int64_t row = int64_t(b) * n_heads + h;
  const float2* ml = reinterpret_cast<const float2*>(ws_ml) + row * max_parts;
  const float* op = ws_o + row * max_parts * D + lane;
  float mx = -INFINITY;
  if (np > kChunk) {
    for (int p = lane; p < np; p += 64) mx = fmaxf(mx, ml[p].x);
    mx = group_max<64>(mx);
  }
  float l = 0.0f, o[DL];
#pragma unroll
  for (int j = 0; j < DL; ++j) o[j] = 0.0f;
  for (int p0 = 0; p0 < np; p0 += kChunk) {
    float2 mlc[kChunk];
    float oc[kChunk][DL];
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      const bool in = p0 + c < np;
      mlc[c] = in ? ml[p0 + c] : make_float2(-INFINITY, 0.0f);
#pragma unroll
      for (int j = 0; j < DL; ++j) oc[c][j] = in ? op[int64_t(p0 + c) * D + 64 * j] : 0.0f;
    }
    if (np <= kChunk) {
#pragma unroll
      for (int c = 0; c < kChunk; ++c) mx = fmaxf(mx, mlc[c].x);
    }
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      const float w = (mlc[c].x == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mlc[c].x - mx);
      l = fmaf(mlc[c].y, w, l);
#pragma unroll
      for (int j = 0; j < DL; ++j) o[j] = fmaf(oc[c][j], w, o[j]);
    }
  }
  // flash_attn.rs:66-71: multiply by 1/s when s > 0, else zeros.
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
  for (int j = 0; j < DL; ++j) {
    const float v = l > 0.0f ? o[j] * inv : 0.0f;
    const int64_t idx = row * D + lane + 64 * j;
    if (out_dtype == IT_F32) static_cast<float*>(out)[idx] = v;
    else if (out_dtype == IT_BF16) static_cast<uint16_t*>(out)[idx] = uint16_t(f32_to_bf16_bits(v));
    else static_cast<uint16_t*>(out)[idx] = uint16_t(f32_to_f16_bits(v));
  }
}

}  // namespace itkv
