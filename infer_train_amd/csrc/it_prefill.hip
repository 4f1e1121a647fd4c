// it_prefill.hip -- chunked-prefill attention over the paged cache, on MFMA.
//
// A chunk of q_len query rows per sequence, at positions ctx - q_len + i,
// attends (causally, or over the whole context) the keys in the paged cache
// (the chunk's own K/V already appended).  Per query row this is
// flash_attn_f32 (src/backend/arm/flash_attn.rs:6-72) over keys
// 0..ctx - q_len + i, with the GQA map of src/inference/forward.rs:231-254;
// the chunked prefill itself has no counterpart in the reference, whose
// generate loop feeds one token at a time (forward.rs:811).
//
// One workgroup = (sequence, KV head, block of 32 QT query positions) with
// W = G QT waves: wave w takes query head kvh G + w % G for the 32 positions
// of tile w / G.  All W waves share every K/V byte the workgroup stages, so
// a 64-key block is read from L2 once per 32 QT queries.  Per 64-key block:
//   S^T = K Q^T   v_mfma_f32_32x32x16 (keys are MFMA rows, queries columns),
//                 so each lane owns one query column: its row max and sum
//                 are in-lane plus one v_permlane32_swap with lane ^ 32;
//   O^T += V^T P^T the probabilities go back into MFMA operands straight
//                 from the S^T registers (bf16/f16 pairs, v_cvt_pk), and
//                 V^T comes from a transposed copy of the V block in LDS
//                 (made once per block by all waves, keys permuted into the
//                 order the S^T registers hold them), one ds_read_b128 per
//                 MFMA like the K operand.
// Ping-pong: the two waves sharing a SIMD alternate between a matrix phase
// (P.V of one block and S^T of the next: MFMA and LDS reads) and a softmax
// phase (VALU), separated by workgroup barriers, so the MFMA pipe and the
// VALU work at the same time.  Fully visible blocks (every key precedes
// every query of the workgroup and kend) run a loop without per-key masks;
// the blocks the causal diagonal or kend cut run a masked copy of it.
// Workgroups are placed so that the query blocks of one (sequence, KV head)
// share an XCD and its L2.
// K and V blocks (16 KiB each) are staged in LDS by direct global->LDS loads
// into rings of 3 K and 3 V slots, issued three blocks ahead; 16-byte chunks
// are XOR-swizzled by row so MFMA operand reads are conflict-free.  Each V
// block is transposed into one of 2 V^T slots the step before it is used.
// Page ids come from the workgroup's LDS copy of its block-table row, or
// through scalar loads when the row does not fit (they do not count against
// the vector-memory counter that orders the rings).  Online softmax in fp32
// (exp2 domain), accumulators fp32.
#include <hip/hip_runtime.h>

#include "it_device.hpp"
#include "it_internal.hpp"

using namespace itkv;

namespace {
constexpr int kD = 128;               // head_dim
constexpr int kQB = 32;               // query positions per wave tile
constexpr int kKB = 64;               // keys per block
constexpr int kRowB = kD * 2;         // bytes per K/V row
constexpr int kPlaneB = kKB * kRowB;  // 16 KiB
constexpr int kRingK = 3;             // K slots
constexpr int kRingV = 3;             // V slots (row-major, as loaded)
// V^T slots: row d holds dim d of the block's 64 keys, key k at position
// vt_pos(k); rows padded to 144 bytes so both the 16-byte operand reads (8
// consecutive rows per pass) and the 4-byte transpose stores are
// conflict-free.
constexpr int kVtRow = 144;
constexpr int kVtB = kD * kVtRow;     // 18 KiB
constexpr int kRingVt = 2;
constexpr int kLds = (kRingK + kRingV) * kPlaneB + kRingVt * kVtB;  // 132 KiB
constexpr int kMaxLds = 160 * 1024;                // per workgroup (one per CU)
constexpr int kMaxGroup = 8;          // query heads per KV head

typedef short v4s __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

struct PrefillArgs {
  const uint16_t* q;      // [total_q][n_heads][D]
  const char* k_pool;
  const char* v_pool;
  const int32_t* cu_q;    // [n_seqs + 1]
  const int32_t* bt;      // [n_seqs][max_blocks]
  const int32_t* ctx_lens;
  void* out;              // [total_q][n_heads][D]
  uint32_t* err;
  int64_t page_bytes;
  uint32_t num_blocks32;  // pool blocks (clamped to 2^31 - 1)
  float scale_log2;
  int n_heads, n_kv_heads, group, q_tiles, max_blocks, log2_bs, causal, out_f32;
  int n_qb;               // query blocks per (sequence, KV head)
};

// Query tiles per workgroup for a GQA group: up to 8 waves of work.
inline int prefill_q_tiles(int group) { return group >= kMaxGroup ? 1 : kMaxGroup / group; }

__device__ __forceinline__ uint32_t lds_off(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}
__device__ __forceinline__ void dma_b128(const void* g, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(g) : "memory", "m0");
}
// The 16 chunks of row r are XOR-permuted by sw(r) = ((r & 3) << 2) | ((r >> 2) & 3),
// a bijection of r mod 16: the A-operand reads (16 consecutive rows, one
// chunk each) hit 16 distinct bank groups, and the transposing V reads (4
// consecutive rows x 4 consecutive chunks per 32 lanes) hit 16 distinct ones.
__device__ __forceinline__ int sw(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
// Byte offset of 16-byte chunk c of row r in a swizzled tile.
__device__ __forceinline__ int swz(int r, int c) { return r * kRowB + ((c ^ sw(r)) << 4); }
// Position of key k (0..63) in a V^T row: bits 2 and 3 of k swapped.  The
// P.V k-step (n, t) takes, in lane half h, element e of its operand from key
// 32 n + 16 t + 8 (e / 4) + 4 h + e % 4, which sits at position
// 32 n + 16 t + 8 h + e: one 16-byte read per lane.
__device__ __forceinline__ int vt_pos(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

template <bool kBf16>
__device__ __forceinline__ v16f mfma(const uint4& a, const uint4& b, const v16f& c) {
  if constexpr (kBf16) {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  } else {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
}
// Two fp32 -> packed 16-bit pair (lo first), round to nearest even.
template <bool kBf16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (kBf16) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    bf2 p;
    p[0] = (__bf16)lo;  // v_cvt_pk_bf16_f32
    p[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, p);
  } else {
    return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
  }
}
// acc + lo + hi of a packed bf16 / f16 pair (v_dot2c_f32_*).
template <bool kBf16>
__device__ __forceinline__ float dot2_ones(uint32_t w, float acc) {
  if constexpr (kBf16) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, w), __builtin_bit_cast(bf2, 0x3f803f80u), acc, false);
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, w), __builtin_bit_cast(h2, 0x3c003c00u), acc, false);
  }
}
// max / sum of x over this lane and lane ^ 32 (v_permlane32_swap, no LDS).
__device__ __forceinline__ float max_halves(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// W: waves per workgroup (G query heads x QT query tiles).
// kTab: the block-table row is copied into LDS after the rings (it fits).
template <bool kBf16, int W, bool kTab>
__global__ __launch_bounds__(64 * W) void paged_prefill_kernel(PrefillArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];  // K ring, V ring, [table]
  constexpr int kDmaPerWave = (16 + W - 1) / W;  // 1 KiB loads per wave per plane (16 per plane)
  // Workgroup id -> (sequence, KV head, query block).  The dispatcher deals
  // ids to the 8 XCDs round-robin; the ids are remapped so that all query
  // blocks of one (sequence, KV head), which stream the same K/V pages, run
  // on one XCD and share its L2 (in id order each XCD would fetch every
  // sequence's pages).  In causal attention later query blocks see more
  // keys, so each XCD takes its units longest first: the k-th workgroup of
  // an XCD holding ppx whole (sequence, KV head) pairs takes query rank
  // k / ppx of pair k % ppx.  Workgroups start in id order on whichever CU
  // frees first, so a CU whose first workgroup was short takes the longest
  // one left (config 3, two workgroups per CU: 166 against 174 us with
  // query blocks in pair order).
  const int n_full = int(gridDim.x) & ~7;
  const int id = blockIdx.x;
  const int per_xcd = n_full >> 3;
  int k = id >> 3;
  if (per_xcd > 0 && per_xcd % a.n_qb == 0) {
    const int ppx = per_xcd / a.n_qb;
    k = (k % ppx) * a.n_qb + k / ppx;
  }
  const int unit = id < n_full ? (id & 7) * per_xcd + k : id;
  const int pair = unit / a.n_qb;
  const int qb = a.n_qb - 1 - (unit - pair * a.n_qb);
  const int kvh = pair % a.n_kv_heads, b = pair / a.n_kv_heads;
  const int q_begin = a.cu_q[b];
  const int q_len = a.cu_q[b + 1] - q_begin;
  const int ctx = a.ctx_lens[b];
  const int wg_q = kQB * a.q_tiles;  // query positions per workgroup
  if (qb * wg_q >= q_len) return;    // uniform
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = wave / a.group;
  const int head = kvh * a.group + (wave - tile * a.group);
  const int half = lane >> 5;  // 0 / 1
  const int col = lane & 31;   // this lane's query within the tile
  const int qi = qb * wg_q + tile * kQB + col;
  const bool q_ok = qi < q_len;
  const int q_pos = ctx - q_len + qi;  // absolute position of this lane's query
  // Keys this workgroup needs: up to its last valid query's position.
  const int last_q = min(q_len, (qb + 1) * wg_q) - 1;
  const int kend = a.causal ? min(ctx, ctx - q_len + last_q + 1) : ctx;
  const int nkb = (kend + kKB - 1) / kKB;
  const int first_pos = ctx - q_len + qb * wg_q;  // position of the workgroup's first query
  const int vis_end = a.causal ? min(kend, first_pos + 1) : kend;
  const int n_vis = max(vis_end, 0) / kKB;  // blocks every query of the workgroup sees whole

  // q: B operand of S^T = K Q^T, k-step ks holds dims 16 ks + 8 half + [0, 8).
  uint4 qv[kD / 16];
  {
    const uint16_t* qp = a.q + ((int64_t(q_begin) + (q_ok ? qi : 0)) * a.n_heads + head) * kD + 8 * half;
#pragma unroll
    for (int ks = 0; ks < kD / 16; ++ks) {
      qv[ks] = q_ok ? ld16(qp + 16 * ks) : make_uint4(0u, 0u, 0u, 0u);
      if (a.scale_log2 < 0.0f) {  // scale's sign into q (exact): the scaled max is the raw max
        qv[ks].x ^= 0x80008000u;
        qv[ks].y ^= 0x80008000u;
        qv[ks].z ^= 0x80008000u;
        qv[ks].w ^= 0x80008000u;
      }
      asm volatile("" : "+v"(qv[ks].x), "+v"(qv[ks].y), "+v"(qv[ks].z), "+v"(qv[ks].w));
    }
  }
  // The workgroup's block-table prefix into LDS (kTab), each entry checked
  // once: an id outside the pool becomes page 0 and is reported.
  int* const tab = reinterpret_cast<int*>(smem + kLds);
  const int n_ent = min((kend + (1 << a.log2_bs) - 1) >> a.log2_bs, a.max_blocks);  // entries read
  bool bad_tab = false;
  if constexpr (kTab) {
    bad_tab = kend > (a.max_blocks << a.log2_bs);  // keys past the table
    const int32_t* row = a.bt + int64_t(b) * a.max_blocks;
    bool lane_bad = false;
    for (int e = threadIdx.x; e < n_ent; e += 64 * W) {
      const int raw = row[e];
      const bool bad = uint32_t(raw) >= a.num_blocks32;
      lane_bad |= bad;
      tab[e] = bad ? 0 : raw;
    }
    bad_tab |= __builtin_amdgcn_ballot_w64(lane_bad) != 0;
  }
  // q (and the table) must be in registers / LDS before the first ring
  // load: the compiler's waits would not count the ring loads issued after.
  asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  const int bs_mask = (1 << a.log2_bs) - 1;
  // Block table row through scalar loads (constant address space).
  const __attribute__((address_space(4))) int32_t* bt =
      (const __attribute__((address_space(4))) int32_t*)(a.bt + int64_t(b) * a.max_blocks);
  char* const k_ring = smem;
  char* const v_ring = smem + kRingK * kPlaneB;
  char* const vt_ring = smem + (kRingK + kRingV) * kPlaneB;
  const uint32_t k_m0 = lds_off(k_ring), v_m0 = lds_off(v_ring);
  const int64_t page_stride = int64_t(a.n_kv_heads) * a.page_bytes;  // bytes per pool block
  const char* const k_head = a.k_pool + int64_t(kvh) * a.page_bytes;
  const char* const v_head = a.v_pool + int64_t(kvh) * a.page_bytes;
  // Loads of plane (K or V) of key block kb into LDS at m0: 16 1-KiB
  // instructions spread over the waves (instruction i covers tile rows
  // 4 i .. 4 i + 3; lane l row 4 i + l / 16 and, swizzled, global chunk
  // (l % 16) ^ sw(row)).  Waves past the 16th instruction repeat one (the
  // same bytes to the same place), so every wave issues kDmaPerWave.
  // Blocks past the last are replaced by the last: harmless refills of
  // slots no iteration reads again.  A page id outside the pool (or a
  // block past the table) is replaced by page 0 and reported once, after
  // the loop; no branch in the issue path.
  bool bad_page = false;
  // Pool block of each of this wave's instructions for key block kb: from
  // the LDS copy of the table row (kTab) or by scalar loads from the table.
  auto page_ids = [&](int kb, int (&blk)[kDmaPerWave]) __attribute__((always_inline)) {
    kb = min(kb, nkb - 1);
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) {
      const int i = (wave + W * j) & 15;
      const int lb = min(kb * kKB + 4 * i, kend - 1) >> a.log2_bs;  // one page for the 4 rows (block size >= 4)
      if constexpr (kTab) {
        blk[j] = tab[min(lb, n_ent - 1)];  // broadcast read; validated when the copy was made
      } else {
        const int raw = bt[min(lb, a.max_blocks - 1)];
        const bool bad = lb >= a.max_blocks || uint32_t(raw) >= a.num_blocks32;
        bad_page |= bad;
        blk[j] = bad ? 0 : raw;
      }
    }
  };
  auto dma_plane = [&](const char* head_base, int kb, uint32_t m0, const int (&blk)[kDmaPerWave])
      __attribute__((always_inline)) {
    kb = min(kb, nkb - 1);
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) {
      const int i = (wave + W * j) & 15;
      const int row = 4 * i + (lane >> 4);
      const int key = min(kb * kKB + row, kend - 1);
      const uint32_t off = uint32_t(key & bs_mask) * kRowB + uint32_t((lane & 15) ^ sw(row)) * 16u;
      const int pb = __builtin_amdgcn_readfirstlane(blk[j]);
      dma_b128(head_base + int64_t(pb) * page_stride + off, __builtin_amdgcn_readfirstlane(m0 + uint32_t(i) * 1024u));
    }
  };
  auto k_slot = [&](int kb) { return k_ring + (kb % kRingK) * kPlaneB; };
  auto v_slot = [&](int kb) { return v_ring + (kb % kRingV) * kPlaneB; };
  auto vt_slot = [&](int kb) { return vt_ring + (kb & 1) * kVtB; };
  // Iteration kb issues K(kb + 3) and V(kb + 3), needed two iterations
  // later (V is transposed the iteration before it is used), with page ids
  // fetched one iteration ahead: kblk holds block kb + 3's.
  int kblk[kDmaPerWave];
  auto issue_step = [&](int kb) __attribute__((always_inline)) {
    dma_plane(k_head, kb + 3, k_m0 + uint32_t((kb + 3) % kRingK) * kPlaneB, kblk);
    dma_plane(v_head, kb + 3, v_m0 + uint32_t((kb + 3) % kRingV) * kPlaneB, kblk);
    page_ids(kb + 4, kblk);
  };
  // V block kb (row-major slot) -> V^T slot kb & 1, in 8 units of 16 dims
  // spread over the waves (wave w takes units w, w + W, ...).  Lane l of a
  // unit u packs keys 2 kp and 2 kp + 1 (kp = l % 32) of dims
  // 8 dg .. 8 dg + 7 (dg = 2 u + l / 32) into 8 dwords, one per V^T row;
  // the two keys sit side by side there (vt_pos keeps bit 0).  Split into
  // the reads, issued before the softmax, and the stores after it.
  constexpr int kTu = (8 + W - 1) / W;  // units per wave
  const int tr_kp = lane & 31, tr_half = lane >> 5;
  auto transpose_read = [&](int kb, uint4 (&r)[kTu][2]) __attribute__((always_inline)) {
    const char* src = v_slot(kb);
#pragma unroll
    for (int j = 0; j < kTu; ++j) {
      const int dg = 2 * min(wave + W * j, 7) + tr_half;  // a unit past 7 repeats unit 7 (not stored)
      r[j][0] = *reinterpret_cast<const uint4*>(src + swz(2 * tr_kp, dg));
      r[j][1] = *reinterpret_cast<const uint4*>(src + swz(2 * tr_kp + 1, dg));
    }
  };
  auto transpose_store = [&](int kb, const uint4 (&r)[kTu][2]) __attribute__((always_inline)) {
    char* const dst = vt_slot(kb) + 2 * vt_pos(2 * tr_kp);
#pragma unroll
    for (int j = 0; j < kTu; ++j) {
      if (wave + W * j < 8) {  // uniform
        char* const d = dst + (16 * (wave + W * j) + 8 * tr_half) * kVtRow;
        const uint32_t a0[4] = {r[j][0].x, r[j][0].y, r[j][0].z, r[j][0].w};
        const uint32_t a1[4] = {r[j][1].x, r[j][1].y, r[j][1].z, r[j][1].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // dim 8 dg + 2 i: low halves of the two keys; dim 8 dg + 2 i + 1: high halves
          *reinterpret_cast<uint32_t*>(d + (2 * i) * kVtRow) = __builtin_amdgcn_perm(a1[i], a0[i], 0x05040100u);
          *reinterpret_cast<uint32_t*>(d + (2 * i + 1) * kVtRow) = __builtin_amdgcn_perm(a1[i], a0[i], 0x07060302u);
        }
      }
    }
  };

  // S^T of key block kb: two 32-key tiles; s[n][r] is key 64 kb + 32 n +
  // 8 (r / 4) + 4 half + r % 4 for query col.
  auto qk = [&](int kb, v16f (&s)[2]) __attribute__((always_inline)) {
    const char* kt = k_slot(kb);
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      s[n] = v16f{};
#pragma unroll
      for (int ks = 0; ks < kD / 16; ++ks) {
        // A: key row 32 n + col, dims 16 ks + 8 half + [0, 8) = chunk 2 ks + half.
        const uint4 kk = *reinterpret_cast<const uint4*>(kt + swz(32 * n + col, 2 * ks + half));
        s[n] = mfma<kBf16>(kk, qv[ks], s[n]);
      }
    }
  };

  v16f o[kD / 32];
#pragma unroll
  for (int d = 0; d < kD / 32; ++d) o[d] = v16f{};
  // Running max (log2 domain, of the scaled scores) and sum.  The max is
  // lazy: o and l are rescaled only when some lane's block max exceeds it
  // by more than kLazy, so probabilities stay below 2^kLazy.
  constexpr float kLazy = 8.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  const float exp_in = fabsf(a.scale_log2);  // q carries the scale's sign
  // Last visible key of this lane's query relative to block kb's first key
  // and to this lane's half (register c of a block holds key offset
  // 4 half + c, c = 32 n + 8 (r / 4) + r % 4).
  const int last_vis = min(kend - 1, a.causal ? q_pos : kend - 1) - 4 * half;
  auto lim_of = [&](int kb) { return last_vis - kb * kKB; };

  // Scaled max of block kb's visible scores over the lane's query (-inf if
  // none is visible); masked: keys past lim are not visible.
  auto block_max = [&](const v16f (&s)[2], bool masked, int lim, float bmax) __attribute__((always_inline)) {
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = 32 * n + 8 * (r >> 2) + (r & 3);
        bmax = fmaxf(bmax, (!masked || c <= lim) ? s[n][r] : -INFINITY);
      }
    bmax = max_halves(bmax);
    return bmax == -INFINITY ? bmax : bmax * exp_in;  // no 0 * -inf when the scale is 0
  };

  v16f s[2];     // S^T of the block the next softmax phase consumes
  uint4 pk[2][2];  // its probabilities, packed: [tile][k-step], 8 each

  // Softmax phase of key block kb (VALU only): block max, lazy rescale of
  // o and l, probabilities into pk, their sum into l.  masked: keys past
  // lim_of(kb) are not visible (blocks below n_vis are whole).
  // ninf: -inf, produced by the barrier the phase follows, so that the
  // compiler keeps the phase after that barrier.
  auto softmax_phase = [&](int kb, bool masked, float ninf) __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    const int lim = kb < n_vis ? kKB : lim_of(kb);
    const float bm = block_max(s, masked, lim, ninf);
    if (__builtin_amdgcn_ballot_w64(bm > m_run + kLazy) != 0) {  // uniform, rare after the first block
      const float m_new = fmaxf(m_run, bm);
      // 0 while m_run is -inf, 1 for a lane whose max stays -inf.
      const float alpha = m_new == m_run ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < kD / 32; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[d][r] *= alpha;
      m_run = m_new;
    }
    // A lane that has seen no visible key keeps m_run = -inf and all its p
    // are masked; any finite stand-in works in the exponent there.
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
    float bsum[2] = {0.0f, 0.0f};
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int c = 32 * n + 16 * t + 8 * (e >> 2) + (e & 3);
          p[e] = __builtin_amdgcn_exp2f(fmaf(s[n][8 * t + e], exp_in, -m_use));
          if (masked) p[e] = c <= lim ? p[e] : 0.0f;
        }
        uint32_t w[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          w[h] = pack2<kBf16>(p[2 * h], p[2 * h + 1]);
          // The sum is taken over the rounded probabilities the MFMA uses.
          bsum[h & 1] = dot2_ones<kBf16>(w[h], bsum[h & 1]);
        }
        pk[n][t] = make_uint4(w[0], w[1], w[2], w[3]);
      }
    l_run += bsum[0] + bsum[1];
    __builtin_amdgcn_sched_barrier(0);
  };

  // Matrix phase of key block kb (MFMA and LDS only): O^T += V^T P^T of
  // block kb, then S^T of block kb + 1 into s.
  auto matrix_phase = [&](int kb) __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    // k-step (n, t): lane L reads V^T row 32 dt + L % 32 at positions
    // 32 n + 16 t + 8 (L / 32) + [0, 8), the keys s[n][8 t + e] holds.
    const char* vt = vt_slot(kb) + col * kVtRow + 16 * half;
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int dt = 0; dt < kD / 32; ++dt) {
          const uint4 w = *reinterpret_cast<const uint4*>(vt + 32 * dt * kVtRow + 64 * n + 32 * t);
          o[dt] = mfma<kBf16>(w, pk[n][t], o[dt]);
        }
    qk(kb + 1, s);
    // Operand reads three MFMAs ahead, one per MFMA.
    __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
#pragma unroll
    for (int i = 0; i < 29; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
    __builtin_amdgcn_sched_barrier(0);
  };

  // Prologue: (K(0), V(0)), (K(1), V(1)), (K(2), V(2)); V(0) transposed;
  // S^T of block 0.  A workgroup with no keys (nkb uniform) skips straight
  // to the zero output.
  if (nkb > 0) {
  {
    int b0[kDmaPerWave], b1[kDmaPerWave];
    page_ids(0, b0);
    page_ids(1, b1);
    page_ids(2, kblk);
    dma_plane(k_head, 0, k_m0, b0);
    dma_plane(v_head, 0, v_m0, b0);
    dma_plane(k_head, 1, k_m0 + uint32_t(kPlaneB), b1);
    dma_plane(v_head, 1, v_m0 + uint32_t(kPlaneB), b1);
    dma_plane(k_head, 2, k_m0 + uint32_t(2 * kPlaneB), kblk);
    dma_plane(v_head, 2, v_m0 + uint32_t(2 * kPlaneB), kblk);
    page_ids(3, kblk);
  }
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(4 * kDmaPerWave) : "memory");
  {
    uint4 r[kTu][2];
    transpose_read(0, r);
    transpose_store(0, r);
  }
  qk(0, s);
  // Ping-pong: waves 0-3 (one per SIMD) run step kb as the matrix phase of
  // block kb, a workgroup barrier, then the softmax phase of block kb + 1;
  // waves 4-7 run the softmax phase of block kb, the barrier, then the
  // matrix phase of block kb.  So the two waves sharing a SIMD keep the MFMA
  // pipe and the VALU busy at the same time.  Waves 0-3 form block 0's
  // probabilities first, one half step ahead.  A step's softmax phases are
  // unmasked while blocks kb and kb + 1 are whole; the last step's block
  // nkb has no visible key.
  // At a step's start K(kb + 1), V(kb + 1) and V^T(kb) are in LDS (only
  // step kb - 1's loads may be outstanding) and every wave is done with the
  // slots step kb refills.
  // The phases use registers only, so the compiler may move them across a
  // barrier; each barrier therefore either consumes the probabilities the
  // phase before it made (so that phase stays before it) or produces the
  // -inf the phase after it starts from (so that phase stays after it).
  auto barrier_after_softmax = [&](bool step_start) __attribute__((always_inline)) {
    uint32_t* w = reinterpret_cast<uint32_t*>(&pk[0][0]);
    if (step_start) {
      asm volatile("s_waitcnt vmcnt(%16)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier"
                   : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]), "+v"(w[6]), "+v"(w[7]),
                     "+v"(w[8]), "+v"(w[9]), "+v"(w[10]), "+v"(w[11]), "+v"(w[12]), "+v"(w[13]), "+v"(w[14]), "+v"(w[15])
                   : "n"(2 * kDmaPerWave)
                   : "memory");
    } else {
      asm volatile("s_barrier"
                   : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]), "+v"(w[6]), "+v"(w[7]),
                     "+v"(w[8]), "+v"(w[9]), "+v"(w[10]), "+v"(w[11]), "+v"(w[12]), "+v"(w[13]), "+v"(w[14]), "+v"(w[15])
                   :
                   : "memory");
    }
  };
  auto barrier_before_softmax = [&](bool step_start) __attribute__((always_inline)) {
    float ninf;
    if (step_start)
      asm volatile("s_waitcnt vmcnt(%1)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier\n\tv_mov_b32 %0, 0xff800000"
                   : "=v"(ninf)
                   : "n"(2 * kDmaPerWave)
                   : "memory");
    else
      asm volatile("s_barrier\n\tv_mov_b32 %0, 0xff800000" : "=v"(ninf) : : "memory");
    return ninf;
  };
  // Every wave also transposes its share of V(kb + 1) during its softmax
  // phase of step kb: V(kb + 1) has landed at the step's start, and V^T slot
  // (kb + 1) & 1 was last read by the matrix phases of step kb - 1.  (The
  // last step transposes the refilled copy of the last block; no step reads
  // it.)
  const int u_end = max(n_vis - 1, 0);
  uint4 tr[kTu][2];
  if (wave < 4) {
    softmax_phase(0, true, -INFINITY);
#pragma nounroll
    for (int kb = 0; kb < u_end; ++kb) {
      barrier_after_softmax(true);
      issue_step(kb);
      matrix_phase(kb);
      const float ninf = barrier_before_softmax(false);
      transpose_read(kb + 1, tr);
      softmax_phase(kb + 1, false, ninf);
      transpose_store(kb + 1, tr);
    }
#pragma nounroll
    for (int kb = u_end; kb < nkb; ++kb) {
      barrier_after_softmax(true);
      issue_step(kb);
      matrix_phase(kb);
      const float ninf = barrier_before_softmax(false);
      transpose_read(kb + 1, tr);
      softmax_phase(kb + 1, true, ninf);
      transpose_store(kb + 1, tr);
    }
  } else {
#pragma nounroll
    for (int kb = 0; kb < u_end; ++kb) {
      const float ninf = barrier_before_softmax(true);
      issue_step(kb);
      transpose_read(kb + 1, tr);
      softmax_phase(kb, false, ninf);
      transpose_store(kb + 1, tr);
      barrier_after_softmax(false);
      matrix_phase(kb);
    }
#pragma nounroll
    for (int kb = u_end; kb < nkb; ++kb) {
      const float ninf = barrier_before_softmax(true);
      issue_step(kb);
      transpose_read(kb + 1, tr);
      softmax_phase(kb, true, ninf);
      transpose_store(kb + 1, tr);
      barrier_after_softmax(false);
      matrix_phase(kb);
    }
  }
  // No ring load may still be writing LDS when the workgroup ends.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if ((bad_page || bad_tab) && lane == 0) atomicOr(a.err, 2u);
  }

  // ---- normalise and store ------------------------------------------------
  // o[dt][r] is dim 32 dt + 8 (r / 4) + 4 half + r % 4 of query col.
  const float l_tot = sum_halves(l_run);
  if (!q_ok) return;
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;  // flash_attn.rs:66-71
  const int64_t orow = ((int64_t(q_begin) + qi) * a.n_heads + head) * kD;
#pragma unroll
  for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int dim = 32 * dt + 8 * g4 + 4 * half;
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = l_tot > 0.0f ? o[dt][4 * g4 + j] * inv : 0.0f;
      if (a.out_f32) {
        *reinterpret_cast<float4*>(static_cast<float*>(a.out) + orow + dim) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + orow + dim) =
            make_uint2(pack2<kBf16>(v[0], v[1]), pack2<kBf16>(v[2], v[3]));
      }
    }
}

template <bool kBf16, int W, bool kTab>
hipError_t launch_prefill_t(const PrefillArgs& a, dim3 grid, size_t smem, hipStream_t s) {
  static std::atomic<uint64_t> opted{0};
  const hipError_t e =
      opt_in_lds(reinterpret_cast<const void*>(&paged_prefill_kernel<kBf16, W, kTab>), kMaxLds, opted);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((paged_prefill_kernel<kBf16, W, kTab>), grid, dim3(64 * W), smem, s, a);
  return hipGetLastError();
}

template <bool kBf16, int W>
hipError_t launch_prefill_w(const PrefillArgs& a, dim3 grid, hipStream_t s) {
  // The table row fits beside the rings up to (160 - 132) KiB / 4 B entries.
  const size_t tab = (size_t(a.max_blocks) * 4 + 15) & ~size_t(15);
  if (kLds + tab <= size_t(kMaxLds)) return launch_prefill_t<kBf16, W, true>(a, grid, kLds + tab, s);
  return launch_prefill_t<kBf16, W, false>(a, grid, kLds, s);
}

template <bool kBf16>
hipError_t launch_prefill(const PrefillArgs& a, dim3 grid, hipStream_t s) {
  switch (a.group * a.q_tiles) {
    case 5: return launch_prefill_w<kBf16, 5>(a, grid, s);
    case 6: return launch_prefill_w<kBf16, 6>(a, grid, s);
    case 7: return launch_prefill_w<kBf16, 7>(a, grid, s);
    case 8: return launch_prefill_w<kBf16, 8>(a, grid, s);
    default: return hipErrorInvalidValue;
  }
}
}  // namespace

extern "C" int32_t it_paged_prefill(const it_kv_cache* c, const void* q, int32_t q_dtype, int32_t n_heads,
                                    const int32_t* cu_q, int32_t max_q_len, const int32_t* block_tables,
                                    int32_t max_blocks, const int32_t* ctx_lens, int32_t n_seqs, float scale,
                                    int32_t causal, void* out, int32_t out_dtype, void* stream) {
  const char* who = "it_paged_prefill";
  if (!c) return fail(IT_INVALID_INPUT, "%s: cache is NULL", who);
  if (int32_t rc = one_layer(c, who)) return rc;
  if (c->dtype != IT_BF16 && c->dtype != IT_F16)
    return fail(IT_NOT_IMPLEMENTED, "%s: cache dtype %d (BF16 or F16 supported)", who, c->dtype);
  if (q_dtype != c->dtype) return fail(IT_NOT_IMPLEMENTED, "%s: q dtype %d must equal the cache dtype", who, q_dtype);
  if (out_dtype != IT_F32 && out_dtype != q_dtype)
    return fail(IT_NOT_IMPLEMENTED, "%s: out dtype must be F32 or the q dtype", who);
  if (c->head_dim != kD) return fail(IT_NOT_IMPLEMENTED, "%s: head_dim %d (128 supported)", who, c->head_dim);
  if (n_heads <= 0 || n_heads % c->n_kv_heads)
    return fail(IT_INVALID_INPUT, "%s: n_heads %d must be a positive multiple of n_kv_heads %d", who, n_heads,
                c->n_kv_heads);
  const int group = n_heads / c->n_kv_heads;
  if (group > kMaxGroup) return fail(IT_NOT_IMPLEMENTED, "%s: %d query heads per KV head (max %d)", who, group, kMaxGroup);
  if (n_seqs < 0 || n_seqs > 65535 || max_q_len < 0 || max_blocks <= 0)
    return fail(IT_INVALID_INPUT, "%s: n_seqs %d, max_q_len %d, max_blocks %d", who, n_seqs, max_q_len, max_blocks);
  if (n_seqs == 0 || max_q_len == 0) return IT_OK;
  if (!q || !cu_q || !block_tables || !ctx_lens || !out) return fail(IT_INVALID_INPUT, "%s: NULL tensor", who);
  if ((reinterpret_cast<uintptr_t>(q) & 15u) || (reinterpret_cast<uintptr_t>(out) & 15u))
    return fail(IT_INVALID_INPUT, "%s: q and out must be 16-byte aligned", who);
  if (!(scale == scale)) return fail(IT_INVALID_INPUT, "%s: scale is NaN", who);
  PrefillArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k_pool = static_cast<const char*>(c->k_pool);
  a.v_pool = static_cast<const char*>(c->v_pool);
  a.cu_q = cu_q;
  a.bt = block_tables;
  a.ctx_lens = ctx_lens;
  a.out = out;
  a.err = c->err_flag;
  a.page_bytes = c->page_bytes;
  a.num_blocks32 = uint32_t(c->num_blocks < INT32_MAX ? c->num_blocks : INT32_MAX);
  a.scale_log2 = scale * 1.4426950408889634f;
  a.n_heads = n_heads;
  a.n_kv_heads = c->n_kv_heads;
  a.group = group;
  a.q_tiles = prefill_q_tiles(group);
  a.max_blocks = max_blocks;
  a.log2_bs = c->log2_bs;
  a.causal = causal ? 1 : 0;
  a.out_f32 = out_dtype == IT_F32;
  const int wg_q = kQB * a.q_tiles;
  a.n_qb = (max_q_len + wg_q - 1) / wg_q;
  const int64_t n_wg = int64_t(a.n_qb) * c->n_kv_heads * n_seqs;
  if (n_wg > INT32_MAX) return fail(IT_INVALID_INPUT, "%s: %lld workgroups (max 2^31 - 1)", who, (long long)n_wg);
  const dim3 grid(static_cast<unsigned>(n_wg), 1u, 1u);
  int dev = -1;
  (void)hipGetDevice(&dev);
  if (dev != c->device) (void)hipSetDevice(c->device);
  const hipError_t e = c->dtype == IT_BF16 ? launch_prefill<true>(a, grid, (hipStream_t)stream)
                                           : launch_prefill<false>(a, grid, (hipStream_t)stream);
  if (dev >= 0 && dev != c->device) (void)hipSetDevice(dev);
  if (e != hipSuccess) return fail(IT_DEVICE_ERROR, "%s: launch: %s", who, hipGetErrorString(e));
  return IT_OK;
}
