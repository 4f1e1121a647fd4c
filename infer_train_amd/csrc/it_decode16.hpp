// it_decode16.hpp -- paged split-K flash-decode for 16-bit (bf16 / f16) KV
// caches on gfx950 (device code).
//
// One workgroup (4 wave64s) owns one (sequence, KV head, head chunk,
// partition of P tokens); the GC query heads of the chunk share every K/V
// byte it reads.  The partition's tokens are cut into 16-token groups and
// group i belongs to wave i % 4: each wave streams its own groups' K rows,
// then their V rows, through a private ring of LDS slots filled by direct
// global->LDS loads (global_load_lds_dwordx4; 64 lanes x 16 B per
// instruction, each lane naming its own source, so the block table is
// applied per token).  A wave only reads what it loaded itself, so the ring
// needs no workgroup barrier; explicit vmcnt counts order it.
//
// The lane layouts are chosen so that no phase needs a per-token cross-lane
// reduction:
//  QK   lane (r, k) = (lane / 16, lane % 16) takes token k of the group and
//       quarter r of the head dimension.  q of head g over quarter r sits in
//       one VGPR per 128 dims, lane k of each row holding dword k, and each
//       v_dot2c_f32_{bf16,f16} reads its q dword straight from lane k of its
//       row through DPP row_newbcast:k.  The four quarter sums of every
//       head are then folded with v_permlane32_swap / v_permlane16_swap
//       (a transpose-reduce: 6 swaps and 6 adds for 8 heads and 16 tokens).
//       K rows are stored in LDS with their 16-byte pieces XOR-swizzled by
//       token, so the 16 lanes of a row read 16 distinct bank groups.
//  PV   lane l takes dims [D/64 l, D/64 (l+1)) of every token; a token
//       pair's probabilities (packed in the cache's 16-bit type) come from
//       lane j of the row through row_newbcast:j, and v_perm builds the
//       matching (v_t[d], v_t+1[d]) pairs for v_dot2c.
//
// Three phases, as in flash_attn_f32 with the max taken over the partition
// first (src/backend/arm/flash_attn.rs:6-72):
//  1. QK: scores in the log2 domain (x * scale * log2 e) go to LDS; each
//     lane tracks the running max of its heads (unmasked path).
//  2. Softmax over the partition by all 256 threads, one token pair each:
//     p = exp2(s - max), rounded to the cache's 16-bit type (the weights PV
//     applies), and l sums the rounded values, so the result is an exact
//     convex combination of V rows.  The Backend op's additive mask
//     (arm.rs:304-370) is applied here, where -inf skips the key
//     (flash_attn.rs:35-40).
//  3. PV over the V groups, then a fixed-order sum over the 4 waves.
// (m, l, O) of the partition go to the workspace; paged_decode_combine
// merges the partitions.
#pragma once
#include <hip/hip_runtime.h>

#include <type_traits>

#include "it_decode.hpp"

namespace itkv {

constexpr int kD16Tok = 16;  // tokens per group (one wave step)

template <int D>
struct D16Geo {
  static constexpr int kRowBytes = 2 * D;
  static constexpr int kGroupBytes = kD16Tok * kRowBytes;  // one group of one plane
  static constexpr int kDma = kGroupBytes / 1024;           // 1 KiB loads per group
  static constexpr int kQuarterPieces = D / 32;              // 16-byte pieces per lane in QK
  static constexpr int kQRegs = D / 128;                     // q VGPRs per head
  static constexpr int kPvDims = D / 64;                     // dims per lane in PV
  static_assert(D == 128 || D == 256, "head_dim 128 or 256");
};

// Dynamic LDS of a workgroup of NW waves: the rings (R slots per wave),
// scores [GC][P + 16] fp32, per-wave max and sum [NW][8] each, a 256-byte
// probability scratch per wave, the page list.  The final cross-wave buffer
// [NW][GC][D] fp32 reuses the rings.
inline size_t decode16_lds_bytes(int d, int gc, int partition, int max_pages, int nw, int ring_slots) {
  const size_t ring = size_t(nw) * ring_slots * kD16Tok * 2 * d;
  const size_t red = size_t(nw) * 8 * d * 4;
  return (ring > red ? ring : red) + size_t(gc) * (partition + 16) * 4 + 2 * size_t(nw) * 8 * 4 + size_t(nw) * 256 +
         size_t(max_pages + 1) * 4;
}

// Launch shape (waves per workgroup, ring slots per wave).  A grid of many
// workgroups wants four or more of them resident per CU (<= 40 KiB of LDS
// each), so that one workgroup's start, barrier and final reduction are
// covered by the others' loads: 2 waves with 2-slot rings (measured on
// config 2: as fast as 3 slots at 4k, 5% faster with ragged contexts).  A
// small grid is bound by each workgroup's own chain of dependent loads and
// takes 4 waves with a 4-slot ring.
struct Decode16Shape {
  int nw, ring;
};
inline Decode16Shape decode16_shape(int d, int gc, int partition, int max_pages, int64_t n_workgroups) {
  constexpr size_t kQuarterCu = 40 * 1024;
  if (n_workgroups >= 512 && decode16_lds_bytes(d, gc, partition, max_pages, 2, 2) <= kQuarterCu) return {2, 2};
  return {4, d == 128 ? 4 : 2};
}

// Compile-time loop: f(integral_constant<int, I>) for I in [B, E).
template <int B, int E>
struct Unroll {
  template <class F>
  __device__ __forceinline__ static void run(F&& f) {
    if constexpr (B < E) {
      f(std::integral_constant<int, B>{});
      Unroll<B + 1, E>::run(f);
    }
  }
};

// ---- v_dot2c with DPP row_newbcast, in asm blocks -------------------------
// A DPP instruction must not read a VGPR (any of its sources, the
// accumulator included) within 2 wait states of a VALU write to it, and the
// compiler cannot see DPP inside inline asm.  So the DPP dot products are
// emitted in blocks that begin with s_nop 1 (covering every VALU write before
// the block) and order their instructions so that an accumulator is read
// again only >= 2 instructions after it was written (heads interleaved;
// explicit nops when fewer than 3 heads).
#define IT_DOT2C(T, A, Q, K, L) "v_dot2c_f32_" T "_dpp %[" A "], %[" Q "], %[" K "] row_newbcast:%[" L "] row_mask:0xf bank_mask:0xf\n\t"
// QK: acc[g] += dot2(q[g] from lane l_j of the row, k_j), j = 0..3.
#define IT_QK1(T, j) IT_DOT2C(T, "a0", "q0", "k" #j, "l" #j)
#define IT_QK2(T, j) IT_QK1(T, j) IT_DOT2C(T, "a1", "q1", "k" #j, "l" #j)
#define IT_QK3(T, j) IT_QK2(T, j) IT_DOT2C(T, "a2", "q2", "k" #j, "l" #j)
#define IT_QK4(T, j) IT_QK3(T, j) IT_DOT2C(T, "a3", "q3", "k" #j, "l" #j)
#define IT_QK5(T, j) IT_QK4(T, j) IT_DOT2C(T, "a4", "q4", "k" #j, "l" #j)
#define IT_QK6(T, j) IT_QK5(T, j) IT_DOT2C(T, "a5", "q5", "k" #j, "l" #j)
#define IT_QK7(T, j) IT_QK6(T, j) IT_DOT2C(T, "a6", "q6", "k" #j, "l" #j)
#define IT_QK8(T, j) IT_QK7(T, j) IT_DOT2C(T, "a7", "q7", "k" #j, "l" #j)
#define IT_QK_BLOCK(T, G, NOP) "s_nop 1\n\t" G(T, 0) NOP G(T, 1) NOP G(T, 2) NOP G(T, 3)
#define IT_QK_OPS                                                                                       \
  : [a0] "+v"(acc[0]), [a1] "+v"(acc[1]), [a2] "+v"(acc[2]), [a3] "+v"(acc[3]), [a4] "+v"(acc[4]),       \
    [a5] "+v"(acc[5]), [a6] "+v"(acc[6]), [a7] "+v"(acc[7])                                              \
  : [q0] "v"(q[0]), [q1] "v"(q[1]), [q2] "v"(q[2]), [q3] "v"(q[3]), [q4] "v"(q[4]), [q5] "v"(q[5]),        \
    [q6] "v"(q[6]), [q7] "v"(q[7]), [k0] "v"(k.x), [k1] "v"(k.y), [k2] "v"(k.z), [k3] "v"(k.w),             \
    [l0] "n"(L0), [l1] "n"(L0 + 1), [l2] "n"(L0 + 2), [l3] "n"(L0 + 3)
#define IT_QK_CASES(T)                                                                   \
  if constexpr (GC == 1) asm(IT_QK_BLOCK(T, IT_QK1, "s_nop 1\n\t") IT_QK_OPS);          \
  else if constexpr (GC == 2) asm(IT_QK_BLOCK(T, IT_QK2, "s_nop 0\n\t") IT_QK_OPS);     \
  else if constexpr (GC == 3) asm(IT_QK_BLOCK(T, IT_QK3, "") IT_QK_OPS);                \
  else if constexpr (GC == 4) asm(IT_QK_BLOCK(T, IT_QK4, "") IT_QK_OPS);                \
  else if constexpr (GC == 5) asm(IT_QK_BLOCK(T, IT_QK5, "") IT_QK_OPS);                \
  else if constexpr (GC == 6) asm(IT_QK_BLOCK(T, IT_QK6, "") IT_QK_OPS);                \
  else if constexpr (GC == 7) asm(IT_QK_BLOCK(T, IT_QK7, "") IT_QK_OPS);                \
  else asm(IT_QK_BLOCK(T, IT_QK8, "") IT_QK_OPS);

// One 16-byte K piece k = dwords L0..L0+3 of the lane's quarter (mod 16):
// acc[g] += sum_j dot2(q[g] of lane L0 + j, k_j) for g < GC.
template <int DT, int GC, int L0>
__device__ __forceinline__ void qk_piece(float (&acc)[8], const uint32_t (&q)[8], uint4 k) {
  static_assert(L0 % 4 == 0 && L0 + 3 < 16, "piece lanes");
  if constexpr (DT == IT_BF16) {
    IT_QK_CASES("bf16")
  } else {
    IT_QK_CASES("f16")
  }
}

// PV: acc[g][x0], acc[g][x1] += dot2(p[g] from lane L of the row, v0 / v1).
// Each accumulator is written once per block; the leading s_nop covers the
// v_perm results the block reads.
#define IT_PV1(T) IT_DOT2C(T, "a00", "p0", "v0", "l") IT_DOT2C(T, "a01", "p0", "v1", "l")
#define IT_PV2(T) IT_PV1(T) IT_DOT2C(T, "a10", "p1", "v0", "l") IT_DOT2C(T, "a11", "p1", "v1", "l")
#define IT_PV3(T) IT_PV2(T) IT_DOT2C(T, "a20", "p2", "v0", "l") IT_DOT2C(T, "a21", "p2", "v1", "l")
#define IT_PV4(T) IT_PV3(T) IT_DOT2C(T, "a30", "p3", "v0", "l") IT_DOT2C(T, "a31", "p3", "v1", "l")
#define IT_PV5(T) IT_PV4(T) IT_DOT2C(T, "a40", "p4", "v0", "l") IT_DOT2C(T, "a41", "p4", "v1", "l")
#define IT_PV6(T) IT_PV5(T) IT_DOT2C(T, "a50", "p5", "v0", "l") IT_DOT2C(T, "a51", "p5", "v1", "l")
#define IT_PV7(T) IT_PV6(T) IT_DOT2C(T, "a60", "p6", "v0", "l") IT_DOT2C(T, "a61", "p6", "v1", "l")
#define IT_PV8(T) IT_PV7(T) IT_DOT2C(T, "a70", "p7", "v0", "l") IT_DOT2C(T, "a71", "p7", "v1", "l")
#define IT_PV_OPS                                                                                       \
  : [a00] "+v"(a0[0]), [a01] "+v"(a1[0]), [a10] "+v"(a0[1]), [a11] "+v"(a1[1]), [a20] "+v"(a0[2]),      \
    [a21] "+v"(a1[2]), [a30] "+v"(a0[3]), [a31] "+v"(a1[3]), [a40] "+v"(a0[4]), [a41] "+v"(a1[4]),       \
    [a50] "+v"(a0[5]), [a51] "+v"(a1[5]), [a60] "+v"(a0[6]), [a61] "+v"(a1[6]), [a70] "+v"(a0[7]),       \
    [a71] "+v"(a1[7])                                                                                   \
  : [p0] "v"(p[0]), [p1] "v"(p[1]), [p2] "v"(p[2]), [p3] "v"(p[3]), [p4] "v"(p[4]), [p5] "v"(p[5]),        \
    [p6] "v"(p[6]), [p7] "v"(p[7]), [v0] "v"(v0), [v1] "v"(v1), [l] "n"(L)
#define IT_PV_CASES(T)                                                                  \
  if constexpr (GC == 1) asm("s_nop 1\n\t" IT_PV1(T) IT_PV_OPS);                       \
  else if constexpr (GC == 2) asm("s_nop 1\n\t" IT_PV2(T) IT_PV_OPS);                  \
  else if constexpr (GC == 3) asm("s_nop 1\n\t" IT_PV3(T) IT_PV_OPS);                  \
  else if constexpr (GC == 4) asm("s_nop 1\n\t" IT_PV4(T) IT_PV_OPS);                  \
  else if constexpr (GC == 5) asm("s_nop 1\n\t" IT_PV5(T) IT_PV_OPS);                  \
  else if constexpr (GC == 6) asm("s_nop 1\n\t" IT_PV6(T) IT_PV_OPS);                  \
  else if constexpr (GC == 7) asm("s_nop 1\n\t" IT_PV7(T) IT_PV_OPS);                  \
  else asm("s_nop 1\n\t" IT_PV8(T) IT_PV_OPS);

// Token pair L of the group: a0[g] += dot2(p[g] of lane L, v0),
// a1[g] += dot2(p[g] of lane L, v1) for g < GC.
template <int DT, int GC, int L>
__device__ __forceinline__ void pv_pair(float (&a0)[8], float (&a1)[8], const uint32_t (&p)[8], uint32_t v0,
                                        uint32_t v1) {
  static_assert(L >= 0 && L < 16, "pair lane");
  if constexpr (DT == IT_BF16) {
    IT_PV_CASES("bf16")
  } else {
    IT_PV_CASES("f16")
  }
}

// Two fp32 -> packed 16-bit pair (lo = a), round to nearest even.
template <int DT>
__device__ __forceinline__ uint32_t pack16(float a, float b) {
  if constexpr (DT == IT_BF16) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    bf2 p;
    p[0] = (__bf16)a;  // v_cvt_pk_bf16_f32 (RNE)
    p[1] = (__bf16)b;
    return __builtin_bit_cast(uint32_t, p);
  } else {
    return f32_to_f16_bits(a) | (f32_to_f16_bits(b) << 16);
  }
}
template <int DT>
__device__ __forceinline__ float lo16(uint32_t w) {
  if constexpr (DT == IT_BF16) return __uint_as_float(w << 16);
  else return f16_bits_to_f32(w & 0xFFFFu);
}
template <int DT>
__device__ __forceinline__ float hi16(uint32_t w) {
  if constexpr (DT == IT_BF16) return __uint_as_float(w & 0xFFFF0000u);
  else return f16_bits_to_f32(w >> 16);
}

// (x, y) -> (x_lo + x_hi, y_lo + y_hi) across the two 32-lane halves:
// lanes 0-31 receive x's sum, lanes 32-63 y's.
__device__ __forceinline__ float fold32(float x, float y) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
// Rows (0,1) and (2,3) of x and y: row 0 <- x0 + x1, row 1 <- y0 + y1,
// row 2 <- x2 + x3, row 3 <- y2 + y3.
__device__ __forceinline__ float fold16(float x, float y) {
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// Reduce eight per-lane values over all 64 lanes without LDS: two permlane
// folds, then a DPP sum (or max) within each 16-lane row.  Row r of the
// first result holds value {0, 2, 1, 3}[r], of the second {4, 6, 5, 7}[r],
// in every lane of the row.
template <bool kMax>
__device__ __forceinline__ void fold8(const float (&x)[8], float& ra, float& rb) {
  auto f32 = [](float p, float q) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(p), __float_as_uint(q), false, false);
    return kMax ? fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1])) : __uint_as_float(s[0]) + __uint_as_float(s[1]);
  };
  auto f16 = [](float p, float q) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(p), __float_as_uint(q), false, false);
    return kMax ? fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1])) : __uint_as_float(s[0]) + __uint_as_float(s[1]);
  };
  ra = f16(f32(x[0], x[1]), f32(x[2], x[3]));
  rb = f16(f32(x[4], x[5]), f32(x[6], x[7]));
  if constexpr (kMax) {
    ra = group_max<16>(ra);
    rb = group_max<16>(rb);
  } else {
    ra = group_sum<16>(ra);
    rb = group_sum<16>(rb);
  }
}

template <int DT, int D, int GC, int NW, int R>
__global__ __launch_bounds__(64 * NW) void paged_decode_split16(DecodeArgs a) {
  using G = D16Geo<D>;
  constexpr int RB = G::kRowBytes, GB = G::kGroupBytes, NI = G::kDma;
  constexpr int PQ = G::kQuarterPieces, NQ = G::kQRegs, DPV = G::kPvDims;
  constexpr int NT = 64 * NW;  // threads
  static_assert(NW == 2 || NW == 4 || NW == 8, "2, 4 or 8 waves");
  static_assert(GC >= 1 && GC <= 8, "1..8 heads per workgroup");
  static_assert(R >= 2 && R <= 4, "ring wait covers R = 2..4");
  static_assert((R - 2) * NI < 64, "vmcnt is 6 bits");

  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr size_t kRingAll = size_t(NW) * R * GB;
  constexpr size_t kRed = size_t(NW) * 8 * D * 4;
  char* const ring = smem;
  float* const sc = reinterpret_cast<float*>(smem + (kRingAll > kRed ? kRingAll : kRed));
  const int SP = a.partition + 16;              // plane stride (staggers heads over the banks)
  float* const s_mx = sc + GC * SP;             // [NW][8] partition max per wave and head
  float* const s_l = s_mx + NW * 8;             // [NW][8] probability sums
  uint32_t* const s_pp = reinterpret_cast<uint32_t*>(s_l + NW * 8);  // [NW][8 heads][8 pairs]
  int32_t* const s_pages = reinterpret_cast<int32_t*>(s_pp + NW * 64);
  // Score of head h, token i (partition-relative): sc[h * SP + i].

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
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bs_mask = (1 << a.log2_bs) - 1;

  // Page indices (block * n_kv_heads + kvh) of the partition, via LDS.
  const int lb0 = tok0 >> a.log2_bs;
  const int nlb = ((tok0 + nt - 1) >> a.log2_bs) - lb0 + 1;  // <= max_pages
  for (int i = tid; i < nlb; i += NT) {
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

  // q in the QK layout: lane (r, k) holds, per head, dword k (and 16 + k for
  // D 256) of quarter r of the head dimension.
  const int qr_row = lane >> 4, qk_tok = lane & 15;
  uint32_t qv[GC][NQ];
  {
    const uint32_t* qp = reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.q) +
                                                           (int64_t(b) * a.n_heads + head0) * D + qr_row * (D / 4)) +
                         qk_tok;
#pragma unroll
    for (int g = 0; g < GC; ++g)
#pragma unroll
      for (int j = 0; j < NQ; ++j) qv[g][j] = qp[g * (D / 2) + 16 * j];
  }
  // Consume q and the block-table loads before any DMA is issued (the
  // compiler's wait for them would not know about the ring loads), and give
  // the DPP readers of q their wait states.
#pragma unroll
  for (int g = 0; g < GC; ++g)
#pragma unroll
    for (int j = 0; j < NQ; ++j) asm volatile("" : "+v"(qv[g][j]));
  asm volatile("s_waitcnt vmcnt(0)\n\ts_nop 4" ::: "memory");
  lds_barrier();

  // This wave's groups: w, w + NW, ...; the stream is their K rows, then
  // their V rows.
  const int n16 = (nt + kD16Tok - 1) / kD16Tok;
  const int ns = n16 > wave ? (n16 - 1 - wave) / NW + 1 : 0;
  const int S = 2 * ns;
  char* const my_ring = ring + size_t(wave) * R * GB;
  const uint32_t ring_m0 = lds_offset(my_ring);
  const uint32_t page_bytes = uint32_t(a.page_bytes);

  // Load stream item s (K or V group) into slot s % R: instruction j, lane i
  // moves bytes [1024 j + 16 i, +16) of the group, i.e. piece slot ps of
  // token row tt; K rows hold logical piece ps ^ tt there.  Rows past the
  // partition load the group's first row as a stand-in.
  int lane_row[NI], lane_off_k[NI], lane_off_v[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int o = 1024 * j + 16 * lane;
    const int tt = o / RB, ps = (o % RB) / 16;
    lane_row[j] = tt;
    lane_off_k[j] = tt * RB + ((ps ^ (tt & 15)) << 4);
    lane_off_v[j] = tt * RB + (ps << 4);
  }
  const int bs = bs_mask + 1;
  auto issue = [&](int s) {
    const bool is_v = s >= ns;
    const int gi = is_v ? s - ns : s;
    const int tb = (gi * NW + wave) * kD16Tok;  // partition-relative first token
    const int t0 = tok0 + tb;
    const char* pool = is_v ? a.v_pool : a.k_pool;
    const uint32_t m0 = ring_m0 + uint32_t(s % R) * GB;
    const int in_page = t0 & bs_mask;
    if (in_page + kD16Tok <= bs) {
      // The whole group lies in one page: one uniform base, one add per load.
      const uint32_t page = uint32_t(__builtin_amdgcn_readfirstlane(s_pages[(t0 >> a.log2_bs) - lb0]));
      const char* base = pool + (uint64_t(page) * page_bytes + uint32_t(in_page * RB));
      const bool full = tb + kD16Tok <= nt;
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        int off = is_v ? lane_off_v[j] : lane_off_k[j];
        if (!full && tb + lane_row[j] >= nt) off -= lane_row[j] * RB;
        dma_b128(base + off, __builtin_amdgcn_readfirstlane(m0 + 1024u * j));
      }
    } else {
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int tt = lane_row[j];
        int tr = tb + tt;
        int off = (is_v ? lane_off_v[j] : lane_off_k[j]) - tt * RB;  // piece offset within the row
        if (tr >= nt) tr = tb;
        const int t = tok0 + tr;
        const uint32_t page = uint32_t(s_pages[(t >> a.log2_bs) - lb0]);
        const char* g = pool + (uint64_t(page) * page_bytes + uint32_t((t & bs_mask) * RB + off));
        dma_b128(g, __builtin_amdgcn_readfirstlane(m0 + 1024u * j));
      }
    }
  };
  // Before consuming item s: its loads are done (at most the items issued
  // after it are outstanding) and this wave's LDS reads are done, so the
  // slot read at step s-1 may be refilled.
  auto wait_item = [&](int s) {
    const int later = min(R - 2, S - 1 - s);  // items issued after s
    if (R >= 4 && later >= 2) asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)" ::"n"(2 * NI) : "memory");
    else if (R >= 3 && later >= 1) asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)" ::"n"(NI) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)" ::: "memory");
  };
  for (int s = 0; s < R - 1 && s < S; ++s) issue(s);

  // ---------------- phase 1: scores -----------------------------------------
  const bool masked = a.mask != nullptr;
  const float qk_mult = masked ? 1.0f : a.scale_log2;
  // Head held by lane row r after the fold: {0, 2, 1, 3}[r] (+4 in hb).
  const int h_a = ((qr_row & 1) << 1) | (qr_row >> 1);
  float m_a = -INFINITY, m_b = -INFINITY;
  for (int s = 0; s < ns; ++s) {
    wait_item(s);
    if (s + R - 1 < S) issue(s + R - 1);
    const char* grp = my_ring + (s % R) * GB + qk_tok * RB;
    float acc[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) acc[g] = 0.0f;
    uint4 kk[PQ];
#pragma unroll
    for (int i = 0; i < PQ; ++i) kk[i] = ld16(grp + (((qr_row * PQ + i) ^ qk_tok) << 4));
    Unroll<0, PQ>::run([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      uint32_t qi[8];  // q VGPR of piece i: dwords 4i..4i+3 of the quarter live in VGPR i/4
#pragma unroll
      for (int g = 0; g < 8; ++g) qi[g] = qv[g < GC ? g : 0][i / 4];
      qk_piece<DT, GC, (4 * i) % 16>(acc, qi, kk[i]);
    });
    // v_permlane*_swap must not read the accumulators within a few wait
    // states of the asm that wrote them.
    asm volatile("s_nop 4" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(acc[4]), "+v"(acc[5]),
                 "+v"(acc[6]), "+v"(acc[7]));
    // Fold the four quarter sums: s_a rows hold heads {0,2,1,3}, s_b {4,6,5,7}.
    const float a01 = fold32(acc[0], acc[1]);
    const float a23 = GC > 2 ? fold32(acc[2], acc[3]) : 0.0f;
    float s_a = fold16(a01, a23) * qk_mult;
    float s_b = 0.0f;
    if constexpr (GC > 4) {
      const float a45 = fold32(acc[4], acc[5]);
      const float a67 = GC > 6 ? fold32(acc[6], acc[7]) : 0.0f;
      s_b = fold16(a45, a67) * qk_mult;
    }
    const int i_tok = (s * NW + wave) * kD16Tok + qk_tok;
    if (i_tok < nt) {
      if (h_a < GC) sc[h_a * SP + i_tok] = s_a;
      if (GC > 4 && 4 + h_a < GC) sc[(4 + h_a) * SP + i_tok] = s_b;
      m_a = fmaxf(m_a, s_a);
      m_b = fmaxf(m_b, s_b);
    }
  }
  m_a = group_max<16>(m_a);
  m_b = group_max<16>(m_b);
  if (qk_tok == 0) {
    s_mx[wave * 8 + h_a] = m_a;
    s_mx[wave * 8 + 4 + h_a] = m_b;
  }
  lds_barrier();

  // ---------------- the Backend op's additive mask ----------------------------
  // (arm.rs:304-370) Scores become (x * scale + mask) * log2 e, -inf where the
  // mask is -inf (flash_attn.rs:35-40), and the maxima are taken again.
  if (masked) {
    float mx[GC];
#pragma unroll
    for (int g = 0; g < GC; ++g) mx[g] = -INFINITY;
    for (int i = tid; i < nt; i += NT) {
      const float mk = a.mask[tok0 + i];
#pragma unroll
      for (int g = 0; g < GC; ++g) {
        float& x = sc[g * SP + i];
        const float y = (mk == -INFINITY) ? -INFINITY : (x * a.scale + mk) * kLog2e;
        x = y;
        mx[g] = fmaxf(mx[g], y);
      }
    }
    float x8[8], ra, rb;
#pragma unroll
    for (int g = 0; g < 8; ++g) x8[g] = g < GC ? mx[g] : -INFINITY;
    fold8<true>(x8, ra, rb);
    if (qk_tok == 0) {
      s_mx[wave * 8 + h_a] = ra;
      s_mx[wave * 8 + 4 + h_a] = rb;
    }
    lds_barrier();
  }

  // Softmax is folded into the PV loop: lane L computes the probability pair
  // (pair L % 8 of the group, head L / 8) from the partition max, rounds it to
  // the cache's 16-bit type (the weight PV applies) and adds the rounded
  // values to its running sum, so the output is an exact convex combination
  // of V rows (flash_attn.rs:42-71 with the max taken first).
  const int h_l = lane >> 3, k_l = lane & 7;
  float m_l = s_mx[h_l];
#pragma unroll
  for (int w = 1; w < NW; ++w) m_l = fmaxf(m_l, s_mx[w * 8 + h_l]);
  const bool none_l = m_l == -INFINITY;  // every key skipped: zeros (flash_attn.rs:66-71)
  const float* const sc_l = sc + (h_l < GC ? h_l : 0) * SP;
  uint32_t* const pp_w = s_pp + wave * 64;
  float lsum = 0.0f;

  // ---------------- phase 3: P.V over the V groups ---------------------------
  float acc2[DPV][8];  // [dim of the lane][head]; heads >= GC stay 0
#pragma unroll
  for (int x = 0; x < DPV; ++x)
#pragma unroll
    for (int g = 0; g < 8; ++g) acc2[x][g] = 0.0f;
  for (int s = ns; s < S; ++s) {
    wait_item(s);
    if (s + R - 1 < S) issue(s + R - 1);
    const int gi = s - ns;
    const int tb = (gi * NW + wave) * kD16Tok;
    char* const grp = my_ring + (s % R) * GB;
    if (tb + kD16Tok > nt) {
      // Rows past the partition hold a stand-in row: each lane zeroes the
      // bytes its own loads brought (this wave's LDS ops stay in order).
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int o = 1024 * j + 16 * lane;
        if (tb + o / RB >= nt) *reinterpret_cast<uint4*>(grp + o) = make_uint4(0u, 0u, 0u, 0u);
      }
    }
    // Probability pairs of the group: computed one (pair, head) per lane,
    // then read back with pair j in lane j of every row (same-wave LDS ops
    // stay in order).
    {
      const int i0 = tb + 2 * k_l;
      const float2 sv = *reinterpret_cast<const float2*>(sc_l + i0);
      const float p0 = (i0 < nt && !none_l) ? __builtin_amdgcn_exp2f(sv.x - m_l) : 0.0f;
      const float p1 = (i0 + 1 < nt && !none_l) ? __builtin_amdgcn_exp2f(sv.y - m_l) : 0.0f;
      const uint32_t pp = pack16<DT>(p0, p1);
      lsum += lo16<DT>(pp) + hi16<DT>(pp);
      pp_w[lane] = pp;
    }
    uint32_t ppv[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) ppv[g] = pp_w[(g < GC ? g : 0) * 8 + (qk_tok & 7)];
    Unroll<0, kD16Tok / 2>::run([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      if constexpr (DPV == 2) {
        const uint32_t w0 = *reinterpret_cast<const uint32_t*>(grp + (2 * j) * RB + 4 * lane);
        const uint32_t w1 = *reinterpret_cast<const uint32_t*>(grp + (2 * j + 1) * RB + 4 * lane);
        pv_pair<DT, GC, j>(acc2[0], acc2[1], ppv, __builtin_amdgcn_perm(w1, w0, 0x05040100u),
                           __builtin_amdgcn_perm(w1, w0, 0x07060302u));
      } else {
        const uint2 w0 = *reinterpret_cast<const uint2*>(grp + (2 * j) * RB + 8 * lane);
        const uint2 w1 = *reinterpret_cast<const uint2*>(grp + (2 * j + 1) * RB + 8 * lane);
        pv_pair<DT, GC, j>(acc2[0], acc2[1], ppv, __builtin_amdgcn_perm(w1.x, w0.x, 0x05040100u),
                           __builtin_amdgcn_perm(w1.x, w0.x, 0x07060302u));
        pv_pair<DT, GC, j>(acc2[2], acc2[3], ppv, __builtin_amdgcn_perm(w1.y, w0.y, 0x05040100u),
                           __builtin_amdgcn_perm(w1.y, w0.y, 0x07060302u));
      }
    });
  }

  // ---------------- across the waves, in a fixed order -----------------------
  lsum = group_sum<8>(lsum);  // the 8 pairs of head h_l
  if (k_l == 0) s_l[wave * 8 + h_l] = lsum;
  lds_barrier();  // every wave is done with its ring (its last wait was vmcnt(0))
  float* const red = reinterpret_cast<float*>(smem);  // [NW][GC][D]
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    float* dst = &red[(wave * GC + g) * D + DPV * lane];
    if constexpr (DPV == 2) *reinterpret_cast<float2*>(dst) = make_float2(acc2[0][g], acc2[1][g]);
    else *reinterpret_cast<float4*>(dst) = make_float4(acc2[0][g], acc2[1][g], acc2[2][g], acc2[3][g]);
  }
  lds_barrier();
  const int64_t part_row = (int64_t(b) * a.n_heads + head0) * a.max_parts + part;
  if (tid < GC) {
    float* ml = a.ws_ml + (part_row + int64_t(tid) * a.max_parts) * 2;
    float m = s_mx[tid], l = s_l[tid];
#pragma unroll
    for (int w = 1; w < NW; ++w) {
      m = fmaxf(m, s_mx[w * 8 + tid]);
      l += s_l[w * 8 + tid];
    }
    ml[0] = m;
    ml[1] = l;
  }
  for (int i = tid; i < GC * D; i += NT) {
    float o;
    if constexpr (NW == 2) o = red[i] + red[GC * D + i];
    else if constexpr (NW == 4) o = (red[i] + red[GC * D + i]) + (red[2 * GC * D + i] + red[3 * GC * D + i]);
    else
      o = ((red[i] + red[GC * D + i]) + (red[2 * GC * D + i] + red[3 * GC * D + i])) +
          ((red[4 * GC * D + i] + red[5 * GC * D + i]) + (red[6 * GC * D + i] + red[7 * GC * D + i]));
    const int g = i / D, d = i - g * D;
    a.ws_o[(part_row + int64_t(g) * a.max_parts) * D + d] = o;
  }
}

}  // namespace itkv
