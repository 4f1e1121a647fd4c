// it_decode_split.hpp -- the split pass of paged split-K flash-decode on
// gfx950, for BF16, F16, F32 and Q8_0 caches (device code).
//
// One workgroup (NW wave64s) owns one (sequence, KV head, head chunk,
// partition of P tokens); the GC query heads of the chunk share every K/V
// byte it reads.  The partition's tokens are cut into 16-token groups and
// group i belongs to wave i % NW: each wave streams its own groups' K rows,
// then their V rows, through a private ring of R LDS slots filled by direct
// global->LDS loads (global_load_lds_dwordx4: 64 lanes x 16 B per
// instruction, each lane naming its own source, so the block table is
// applied per token; Q8_0 scales ride along in global_load_lds_dword).  A
// wave only reads what it loaded itself, so the ring needs no workgroup
// barrier; explicit vmcnt counts order it.
//
// Lane layouts, chosen so that no per-token cross-lane reduction is left:
//  QK   lane (r, k) = (lane / 16, lane % 16) takes token k of the group and
//       quarter r of the head dimension.  q of head g over quarter r sits in
//       registers, lane k of each 16-lane row holding its k-th word, and every
//       multiply-add reads its q word straight from lane k of its row through
//       DPP row_newbcast:k (v_dot2c_f32_{bf16,f16} on packed 16-bit pairs,
//       v_fmac_f32 for F32).  The four quarter sums of every head are then
//       folded with v_permlane32_swap / v_permlane16_swap (6 swaps, 6 adds
//       for 8 heads).  K rows sit in LDS with their 16-byte pieces
//       XOR-swizzled by token, so a row of 16 lanes reads distinct bank
//       groups.
//  PV   lane l takes dims [D/64 l, D/64 (l+1)) of every token.  The
//       probability of token t (16-bit caches: of token pair t) comes from
//       lane t of the row through row_newbcast:t; 16-bit caches v_perm
//       (v_t[d], v_t+1[d]) pairs for v_dot2c.
//  The quantised formats run both products on v_mfma_f32_16x16x32_f16,
//       exactly: K values (int8, or nibbles n - 8) are exact in fp16, q
//       (scaled by a power of two per head) and the weights p 2^11 are split
//       into hi + lo fp16 parts, and B = d v of P.V into hi + lo parts, so
//       every product is exact and only the fp32 accumulation rounds.  QK:
//       two MFMAs per 32-group of the head dim, q heads x 16 tokens, then
//       f32(d) of the group scales the group's sum.  PV: two K = 32 MFMAs
//       per tile of 16 dims, heads x 16 tokens; items whose scales are too
//       large for fp16 products take a three-part bf16 form instead.
//
// The softmax follows flash_attn_f32 (src/backend/arm/flash_attn.rs:6-72)
// with the partition max taken first: phase 1 writes the scores (log2
// domain, x * scale * log2 e) to LDS and tracks the max; one barrier
// publishes the per-wave maxima; the PV loop turns each group's scores into
// probabilities (one (pair, head) per lane, 16-bit caches rounding them to
// the cache type, the weights PV applies) and sums them, so a 16-bit result
// is an exact convex combination of V rows.  The Backend op's additive mask
// (arm.rs:304-370) rewrites the scores between the two, a -inf key being
// skipped (flash_attn.rs:35-40).  The waves' partial outputs are summed in a
// fixed order; (m, l, O) of the partition go to the workspace and
// paged_decode_combine merges the partitions.
//
// Q8_0 (BlockQ8_0, src/types.rs:34-41): a page is int8 qs[bs][D] then fp16
// d[bs][D/32]; a key dot product is sum over 32-groups of f32(d) * sum q *
// qs, and a value element is f32(d) * qs, exact in fp32 (gemv.rs:151-160).
// Q4_0 (BlockQ4_0, src/types.rs:15-22): a page is u8 qs[bs][D/2], each
// group's 16 bytes holding element j in the low nibble of byte j and
// element j + 16 in the high nibble, then fp16 d[bs][D/32]; a value element
// is f32(d) * (nibble - 8) (vec_dot.rs:425-440), exact in fp32.  Q4_1
// (BlockQ4_1, src/types.rs:24-32): the same nibbles, then fp16 (d, m) pairs;
// a value is f32(d) * nibble + f32(m) (ggml), taken here as f32(d) (nibble -
// 8) + m' with m' = m + 8 d, the offset term a further small MFMA product.
// Q5_0 / Q5_1 (ggml block_q5_*, type ids types.rs:116-117): the nibble plane
// holds the low four bits of each 5-bit value q, and a token's side row its
// groups' u32 qh words (bit e = bit 4 of element e) and then their d (Q5_0)
// or (d, m) pairs (Q5_1); a value is f32(d) (q - 16), or f32(d) q + f32(m)
// taken as f32(d) (q - 16) + m' with m' = m + 16 d.
#pragma once
#include <hip/hip_runtime.h>

#include <cfloat>
#include <type_traits>

#include "it_decode.hpp"

namespace itkv {

constexpr int kGroupTok = 16;  // tokens per group (one wave step)
constexpr float kQPScale = 2048.0f;  // quantised P.V weights carry 2^11 (see the V loop)

// Geometry of a cache dtype at head_dim D.
template <int DT, int D>
struct SplitFmt {
  static constexpr bool k16 = DT == IT_BF16 || DT == IT_F16;
  static constexpr bool kQ8 = DT == IT_Q8_0;
  static constexpr bool kQ5 = DT == IT_Q5_0 || DT == IT_Q5_1;      // + a qh word per group
  static constexpr bool kOff = DT == IT_Q4_1 || DT == IT_Q5_1;     // (d, m) per group: an offset term
  static constexpr bool kNib = DT == IT_Q4_0 || DT == IT_Q4_1 || kQ5;  // nibble planes
  static constexpr bool kQuant = kQ8 || kNib;                       // MFMA products, fp16 group scales
  static constexpr int kElem = DT == IT_F32 ? 4 : (kQuant ? 1 : 2);  // bytes per main-plane element
  static constexpr int kRow = kNib ? D / 2 : D * kElem;            // main-plane bytes per token
  static constexpr int kGroup = kGroupTok * kRow;                 // main-plane bytes per group
  static constexpr int kDma = kGroup / 1024;                      // 16-byte-per-lane loads per group
  static constexpr int kMetaStride = kOff ? 4 : 2;                // bytes of a group's d or (d, m)
  static constexpr int kMetaOff = kQ5 ? D / 8 : 0;                // where the d words start in a side row
  static constexpr int kScaleRow = kQuant ? kMetaOff + D / 32 * kMetaStride : 0;  // side-row bytes per token
  static constexpr int kScaleGroup = kGroupTok * kScaleRow;       // 128..1024 B
  // B-operand factor of the bf16 P.V form: int8 8 (q - 16) for Q5, 16 (nibble - 8) for Q4.
  static constexpr float kBScale = kQ5 ? 0.125f : (kNib ? 0.0625f : 1.0f);
  static constexpr float kMid = kQ5 ? 16.0f : 8.0f;                // m' = m + kMid d
  static constexpr int kScaleLoads = (kScaleGroup + 255) / 256;   // dword loads (64 lanes x 4 B) per group
  static constexpr int kSlot = kGroup + kScaleGroup;
  static constexpr int kLoads = kDma + kScaleLoads;               // vmcnt units per group
  static constexpr int kPieces = D / 4 * kElem / 16;              // 16-byte pieces per lane in QK
  static constexpr int kRowPieces = kRow / 16;
  static constexpr int kSwz = (kRowPieces < 16 ? kRowPieces : 16) - 1;  // piece swizzle mask
  // V rows of quantised formats: the pieces of token row t are XOR-permuted
  // by kVQuad * ((t / 4) % 4), so that the P.V reads of the four token quads
  // (rows 4 kq + j, a multiple of 256 bytes apart) hit four different bank
  // sets: a group's 32 (Q8_0) or 16 (nibble) bytes move by kq group widths.
  static constexpr int kVQuad = kQ8 ? 2 : (kNib ? 1 : 0);
  static constexpr int kQRegs = (k16 ? D / 8 : D / 4) / 16;       // q VGPRs per head (16 words each)
  static constexpr int kDpv = D / 64;                             // PV dims per lane
  static constexpr int kScratch = k16 ? 256 : 512;                // probability scratch per wave (B)
  static_assert(D == 128 || D == 256, "head_dim 128 or 256");
  static_assert(kGroup % 1024 == 0 && kScaleGroup <= 1024, "group geometry");
};

template <int DT>
inline int split_slot_bytes(int d) {
  return d == 128 ? SplitFmt<DT, 128>::kSlot : SplitFmt<DT, 256>::kSlot;
}
inline int split_slot_bytes(int32_t dt, int d) {
  switch (dt) {
    case IT_BF16: return split_slot_bytes<IT_BF16>(d);
    case IT_F16: return split_slot_bytes<IT_F16>(d);
    case IT_F32: return split_slot_bytes<IT_F32>(d);
    case IT_Q4_0: return split_slot_bytes<IT_Q4_0>(d);
    case IT_Q4_1: return split_slot_bytes<IT_Q4_1>(d);
    case IT_Q5_0: return split_slot_bytes<IT_Q5_0>(d);
    case IT_Q5_1: return split_slot_bytes<IT_Q5_1>(d);
    default: return split_slot_bytes<IT_Q8_0>(d);
  }
}

// Dynamic LDS of a workgroup of NW waves: the rings (R slots per wave),
// scores [GC][P + 16] fp32, per-wave max and sum [NW][8] each, a probability
// scratch per wave, the page list.  The final cross-wave buffer [NW][GC][D]
// fp32 reuses the rings.
inline size_t split_lds_bytes(int32_t dt, int d, int gc, int partition, int max_pages, int nw, int ring) {
  const size_t rings = size_t(nw) * ring * split_slot_bytes(dt, d);
  const size_t red = size_t(nw) * 8 * d * 4;
  const size_t scratch = (dt == IT_BF16 || dt == IT_F16) ? 256 : 512;
  return (rings > red ? rings : red) + size_t(gc) * (partition + 16) * 4 + 2 * size_t(nw) * 8 * 4 + nw * scratch +
         size_t(max_pages + 1) * 4;
}

// Launch shape (waves per workgroup, ring slots per wave).  A grid of many
// workgroups wants four or more of them resident per CU (<= 40 KiB of LDS
// each), so that one workgroup's start, barrier and final reduction are
// covered by the others' loads: 2 waves with 2-slot rings (measured on
// config 2: as fast as 3 slots at 4k, 5% faster with ragged contexts); when
// that does not fit, 4 waves with 2-slot rings at two per CU.  A small grid
// is bound by each workgroup's own chain of dependent loads and takes 4
// waves with the deepest ring that fits.
struct SplitShape {
  int nw, ring;
};
inline SplitShape split_shape(int32_t dt, int d, int gc, int partition, int max_pages, int64_t n_workgroups) {
  constexpr size_t kQuarterCu = 40 * 1024, kHalfCu = 80 * 1024, kCu = 160 * 1024;
  if (n_workgroups >= 512) {
    if (split_lds_bytes(dt, d, gc, partition, max_pages, 2, 2) <= kQuarterCu) return {2, 2};
    if (split_lds_bytes(dt, d, gc, partition, max_pages, 4, 2) <= kHalfCu) return {4, 2};
  }
  for (int r = 4; r > 2; --r)
    if (split_lds_bytes(dt, d, gc, partition, max_pages, 4, r) <= kCu) return {4, r};
  return {4, 2};
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

// ---- multiply-adds with DPP row_newbcast, in asm blocks --------------------
// A DPP instruction must not read a VGPR (any of its sources, the
// accumulator included) within 2 wait states of a VALU write to it, and the
// compiler cannot see DPP inside inline asm.  So the DPP multiply-adds are
// emitted in blocks that begin with s_nop 1 (covering every VALU write before
// the block) and order their instructions so that an accumulator is read
// again only >= 2 instructions after it was written (heads interleaved;
// explicit nops when fewer than 3 heads).
#define IT_DPP(OP, A, Q, K, L) OP " %[" A "], %[" Q "], %[" K "] row_newbcast:%[" L "] row_mask:0xf bank_mask:0xf\n\t"
// QK: acc[g] += q[g] (lane l_j of the row) . k_j, j = 0..3.
#define IT_QK1(OP, j) IT_DPP(OP, "a0", "q0", "k" #j, "l" #j)
#define IT_QK2(OP, j) IT_QK1(OP, j) IT_DPP(OP, "a1", "q1", "k" #j, "l" #j)
#define IT_QK3(OP, j) IT_QK2(OP, j) IT_DPP(OP, "a2", "q2", "k" #j, "l" #j)
#define IT_QK4(OP, j) IT_QK3(OP, j) IT_DPP(OP, "a3", "q3", "k" #j, "l" #j)
#define IT_QK5(OP, j) IT_QK4(OP, j) IT_DPP(OP, "a4", "q4", "k" #j, "l" #j)
#define IT_QK6(OP, j) IT_QK5(OP, j) IT_DPP(OP, "a5", "q5", "k" #j, "l" #j)
#define IT_QK7(OP, j) IT_QK6(OP, j) IT_DPP(OP, "a6", "q6", "k" #j, "l" #j)
#define IT_QK8(OP, j) IT_QK7(OP, j) IT_DPP(OP, "a7", "q7", "k" #j, "l" #j)
#define IT_QK_BLOCK(OP, G, NOP) "s_nop 1\n\t" G(OP, 0) NOP G(OP, 1) NOP G(OP, 2) NOP G(OP, 3)
#define IT_QK_OPS                                                                                       \
  : [a0] "+v"(acc[0]), [a1] "+v"(acc[1]), [a2] "+v"(acc[2]), [a3] "+v"(acc[3]), [a4] "+v"(acc[4]),       \
    [a5] "+v"(acc[5]), [a6] "+v"(acc[6]), [a7] "+v"(acc[7])                                              \
  : [q0] "v"(q[0]), [q1] "v"(q[1]), [q2] "v"(q[2]), [q3] "v"(q[3]), [q4] "v"(q[4]), [q5] "v"(q[5]),        \
    [q6] "v"(q[6]), [q7] "v"(q[7]), [k0] "v"(k0), [k1] "v"(k1), [k2] "v"(k2), [k3] "v"(k3), [l0] "n"(L0),  \
    [l1] "n"(L0 + 1), [l2] "n"(L0 + 2), [l3] "n"(L0 + 3)
#define IT_QK_CASES(OP)                                                                  \
  if constexpr (GC == 1) asm(IT_QK_BLOCK(OP, IT_QK1, "s_nop 1\n\t") IT_QK_OPS);         \
  else if constexpr (GC == 2) asm(IT_QK_BLOCK(OP, IT_QK2, "s_nop 0\n\t") IT_QK_OPS);    \
  else if constexpr (GC == 3) asm(IT_QK_BLOCK(OP, IT_QK3, "") IT_QK_OPS);               \
  else if constexpr (GC == 4) asm(IT_QK_BLOCK(OP, IT_QK4, "") IT_QK_OPS);               \
  else if constexpr (GC == 5) asm(IT_QK_BLOCK(OP, IT_QK5, "") IT_QK_OPS);               \
  else if constexpr (GC == 6) asm(IT_QK_BLOCK(OP, IT_QK6, "") IT_QK_OPS);               \
  else if constexpr (GC == 7) asm(IT_QK_BLOCK(OP, IT_QK7, "") IT_QK_OPS);               \
  else asm(IT_QK_BLOCK(OP, IT_QK8, "") IT_QK_OPS);

// acc[g] += sum_j q[g] (of lane L0 + j of the row) . k_j for g < GC; the
// words are packed 16-bit pairs for BF16 / F16 (v_dot2c), fp32 otherwise.
template <int DT, int GC, int L0>
__device__ __forceinline__ void qk_words(float (&acc)[8], const uint32_t (&q)[8], uint32_t k0, uint32_t k1,
                                         uint32_t k2, uint32_t k3) {
  static_assert(L0 % 4 == 0 && L0 + 3 < 16, "word lanes");
  if constexpr (DT == IT_BF16) {
    IT_QK_CASES("v_dot2c_f32_bf16_dpp")
  } else if constexpr (DT == IT_F16) {
    IT_QK_CASES("v_dot2c_f32_f16_dpp")
  } else {
    IT_QK_CASES("v_fmac_f32_dpp")
  }
}

// PV: a0[g] += p[g] (lane L of the row) . v0, a1[g] += p[g] . v1.  Each
// accumulator is written once per block; the leading s_nop covers the
// converted / permuted values the block reads.
#define IT_PV1(OP) IT_DPP(OP, "a00", "p0", "v0", "l") IT_DPP(OP, "a01", "p0", "v1", "l")
#define IT_PV2(OP) IT_PV1(OP) IT_DPP(OP, "a10", "p1", "v0", "l") IT_DPP(OP, "a11", "p1", "v1", "l")
#define IT_PV3(OP) IT_PV2(OP) IT_DPP(OP, "a20", "p2", "v0", "l") IT_DPP(OP, "a21", "p2", "v1", "l")
#define IT_PV4(OP) IT_PV3(OP) IT_DPP(OP, "a30", "p3", "v0", "l") IT_DPP(OP, "a31", "p3", "v1", "l")
#define IT_PV5(OP) IT_PV4(OP) IT_DPP(OP, "a40", "p4", "v0", "l") IT_DPP(OP, "a41", "p4", "v1", "l")
#define IT_PV6(OP) IT_PV5(OP) IT_DPP(OP, "a50", "p5", "v0", "l") IT_DPP(OP, "a51", "p5", "v1", "l")
#define IT_PV7(OP) IT_PV6(OP) IT_DPP(OP, "a60", "p6", "v0", "l") IT_DPP(OP, "a61", "p6", "v1", "l")
#define IT_PV8(OP) IT_PV7(OP) IT_DPP(OP, "a70", "p7", "v0", "l") IT_DPP(OP, "a71", "p7", "v1", "l")
#define IT_PV_OPS                                                                                       \
  : [a00] "+v"(a0[0]), [a01] "+v"(a1[0]), [a10] "+v"(a0[1]), [a11] "+v"(a1[1]), [a20] "+v"(a0[2]),      \
    [a21] "+v"(a1[2]), [a30] "+v"(a0[3]), [a31] "+v"(a1[3]), [a40] "+v"(a0[4]), [a41] "+v"(a1[4]),       \
    [a50] "+v"(a0[5]), [a51] "+v"(a1[5]), [a60] "+v"(a0[6]), [a61] "+v"(a1[6]), [a70] "+v"(a0[7]),       \
    [a71] "+v"(a1[7])                                                                                   \
  : [p0] "v"(p[0]), [p1] "v"(p[1]), [p2] "v"(p[2]), [p3] "v"(p[3]), [p4] "v"(p[4]), [p5] "v"(p[5]),        \
    [p6] "v"(p[6]), [p7] "v"(p[7]), [v0] "v"(v0), [v1] "v"(v1), [l] "n"(L)
#define IT_PV_CASES(OP)                                                                 \
  if constexpr (GC == 1) asm("s_nop 1\n\t" IT_PV1(OP) IT_PV_OPS);                      \
  else if constexpr (GC == 2) asm("s_nop 1\n\t" IT_PV2(OP) IT_PV_OPS);                 \
  else if constexpr (GC == 3) asm("s_nop 1\n\t" IT_PV3(OP) IT_PV_OPS);                 \
  else if constexpr (GC == 4) asm("s_nop 1\n\t" IT_PV4(OP) IT_PV_OPS);                 \
  else if constexpr (GC == 5) asm("s_nop 1\n\t" IT_PV5(OP) IT_PV_OPS);                 \
  else if constexpr (GC == 6) asm("s_nop 1\n\t" IT_PV6(OP) IT_PV_OPS);                 \
  else if constexpr (GC == 7) asm("s_nop 1\n\t" IT_PV7(OP) IT_PV_OPS);                 \
  else asm("s_nop 1\n\t" IT_PV8(OP) IT_PV_OPS);

template <int DT, int GC, int L>
__device__ __forceinline__ void pv_words(float (&a0)[8], float (&a1)[8], const uint32_t (&p)[8], uint32_t v0,
                                         uint32_t v1) {
  static_assert(L >= 0 && L < 16, "probability lane");
  if constexpr (DT == IT_BF16) {
    IT_PV_CASES("v_dot2c_f32_bf16_dpp")
  } else if constexpr (DT == IT_F16) {
    IT_PV_CASES("v_dot2c_f32_f16_dpp")
  } else {
    IT_PV_CASES("v_fmac_f32_dpp")
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
// Signed byte J of w as fp32 (v_cvt_f32_i32 with an SDWA sign-extended byte).
template <int J>
__device__ __forceinline__ uint32_t i8_f32(uint32_t w) {
  return __float_as_uint(float(int32_t(w << (24 - 8 * J)) >> 24));
}

// ---- Q8_0 scores on MFMA ----------------------------------------------------
typedef float v4f __attribute__((ext_vector_type(4)));
// Four Q4_0 bytes (nibble n at element j, nibble m at element j + 16) as
// eight bf16 values 16 (n - 8), then 16 (m - 8), exactly: n ^ 8 read as a
// signed nibble is n - 8, and moved to the top of its byte it sign-extends
// through the same SDWA convert as an int8.  The factor 16 goes into d.
__device__ __forceinline__ uint4 nib8_bf16(uint32_t w) {
  const uint32_t x = w ^ 0x88888888u;
  const uint32_t lo = (x << 4) & 0xF0F0F0F0u, hi = x & 0xF0F0F0F0u;
  auto pair = [](uint32_t f0, uint32_t f1) { return __builtin_amdgcn_perm(f1, f0, 0x07060302u); };
  return make_uint4(pair(i8_f32<0>(lo), i8_f32<1>(lo)), pair(i8_f32<2>(lo), i8_f32<3>(lo)),
                    pair(i8_f32<0>(hi), i8_f32<1>(hi)), pair(i8_f32<2>(hi), i8_f32<3>(hi)));
}
// Four nibble bytes of a Q5 group and the fifth bits of their values (bit i
// of lo4: the low nibble of byte i; of hi4: its high nibble) as eight bf16
// values 8 (q - 16), low nibbles first, exactly: q << 3 fills a byte, its top
// bit flipped the byte read as int8 is 8 (q - 16).  The factor 8 goes into d.
__device__ __forceinline__ uint4 nib5_bf16(uint32_t w, uint32_t lo4, uint32_t hi4) {
  auto spread = [](uint32_t t) { return (__umul24(t, 0x204081u) & 0x01010101u) << 7; };  // bit i -> bit 8 i + 7
  const uint32_t lo = (((w << 3) & 0x78787878u) | spread(lo4)) ^ 0x80808080u;
  const uint32_t hi = (((w >> 1) & 0x78787878u) | spread(hi4)) ^ 0x80808080u;
  auto pair = [](uint32_t f0, uint32_t f1) { return __builtin_amdgcn_perm(f1, f0, 0x07060302u); };
  return make_uint4(pair(i8_f32<0>(lo), i8_f32<1>(lo)), pair(i8_f32<2>(lo), i8_f32<3>(lo)),
                    pair(i8_f32<0>(hi), i8_f32<1>(hi)), pair(i8_f32<2>(hi), i8_f32<3>(hi)));
}
// Q4_1 value d n + m taken as d (n - 8) + m', m' = m + 8 d (Q5_1: d q + m as
// d (q - 16) + m', m' = m + 16 d): the integer part is Q4_0's (Q5_0's), and
// m' sits near the group's mean, so neither part is much larger than the
// value (with m the group minimum the two would cancel).
template <int DT>
__device__ __forceinline__ float off_mprime(uint32_t dm) {
  constexpr float kMid = (DT == IT_Q5_1) ? 16.0f : 8.0f;
  return fmaf(kMid, f16_bits_to_f32(dm & 0xFFFFu), f16_bits_to_f32(dm >> 16));
}
// x = hi + mid + lo exactly, each part a bf16 (round to nearest even): the
// three parts carry the 24 significant bits of an fp32.  Two values per
// packed word (lo element first).  No inline asm here: the compiler's hazard
// checks do not look inside asm, and these words feed MFMA operands.  The
// low element comes back to fp32 through v_perm (hi << 16 written as a shift
// is turned into a second conversion of that element).
__device__ __forceinline__ void split3_bf16(float x0, float x1, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
  auto rne2 = [](float a, float b) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    bf2 p;
    p[0] = (__bf16)a;  // v_cvt_pk_bf16_f32
    p[1] = (__bf16)b;
    return __builtin_bit_cast(uint32_t, p);
  };
  auto lo_f = [](uint32_t w) { return __uint_as_float(__builtin_amdgcn_perm(0u, w, 0x01000C0Cu)); };
  auto hi_f = [](uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); };
  hi = rne2(x0, x1);
  const float r0 = x0 - lo_f(hi), r1 = x1 - hi_f(hi);
  mid = rne2(r0, r1);
  const float t0 = r0 - lo_f(mid), t1 = r1 - hi_f(mid);
  lo = rne2(t0, t1);
}
typedef short v4s __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4f mfma16k16(uint2 a, uint2 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(v4s, a), __builtin_bit_cast(v4s, b), c, 0, 0, 0);
}
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
__device__ __forceinline__ v4f mfma16_f16(uint4 a, uint4 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
}
// Signed byte J0 of w0 and byte J1 of w1 as an fp16 pair (lo = w0's),
// exactly: two SDWA converts, the second writing the high half in place.
#define IT_I8PAIR(J0, J1)                                                                               \
  asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_" #J0 "\n\t" \
      "v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_" #J1    \
      : "=&v"(r)                                                                                        \
      : "v"(w0), "v"(w1))
template <int J0, int J1>
__device__ __forceinline__ uint32_t i8pair_f16(uint32_t w0, uint32_t w1) {
  static_assert(J0 >= 0 && J0 < 4 && J1 >= 0 && J1 < 4, "byte");
  uint32_t r;
  if constexpr (J0 == 0 && J1 == 0) IT_I8PAIR(0, 0);
  else if constexpr (J0 == 1 && J1 == 1) IT_I8PAIR(1, 1);
  else if constexpr (J0 == 0 && J1 == 1) IT_I8PAIR(0, 1);
  else if constexpr (J0 == 2 && J1 == 3) IT_I8PAIR(2, 3);
  else static_assert(J0 < 0, "unused byte pair");
  return r;
}
#undef IT_I8PAIR
// Eight signed bytes as eight fp16, exactly.
__device__ __forceinline__ uint4 i8x8_f16(uint2 w) {
  return make_uint4(i8pair_f16<0, 1>(w.x, w.x), i8pair_f16<2, 3>(w.x, w.x), i8pair_f16<0, 1>(w.y, w.y),
                    i8pair_f16<2, 3>(w.y, w.y));
}
// x = hi + lo + r as fp16 parts, hi = fp16(x), lo = fp16(x - hi) (round to
// nearest even each), for the lanes' four values: |r| <= 2^-22 |x| for x
// in fp16's normal range (2^-14 .. 65504) and its residual too.
__device__ __forceinline__ void split2_f16(const float (&x)[4], uint2& hi, uint2& lo) {
  h2 h01, h23, l01, l23;
  h01[0] = (_Float16)x[0];
  h01[1] = (_Float16)x[1];
  h23[0] = (_Float16)x[2];
  h23[1] = (_Float16)x[3];
  l01[0] = (_Float16)(x[0] - (float)h01[0]);
  l01[1] = (_Float16)(x[1] - (float)h01[1]);
  l23[0] = (_Float16)(x[2] - (float)h23[0]);
  l23[1] = (_Float16)(x[3] - (float)h23[1]);
  hi = make_uint2(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23));
  lo = make_uint2(__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23));
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

// Inclusive prefix sum over the 64 lanes of a wave (DPP: row shifts within
// each 16-lane row, then row broadcasts of lanes 15 and 31).  Lanes a DPP
// source does not reach add 0 (bound_ctrl, or the disabled banks and rows,
// which return the old operand 0).
__device__ __forceinline__ int wave_inclusive_sum(int x) {
  int v = x + __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);          // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, x, 0x113, 0xf, 0xf, true);          // row_shr:3
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xe, false);         // row_shr:4, banks 1-3
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xc, false);         // row_shr:8, banks 2-3
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);         // row_bcast:15, rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);         // row_bcast:31, rows 2-3
  return v;
}

template <int DT, int D, int GC, int NW, int R>
__global__ __launch_bounds__(64 * NW) void paged_decode_split(DecodeArgs a) {
  using F = SplitFmt<DT, D>;
  constexpr int RB = F::kRow, GB = F::kGroup, SLOT = F::kSlot, NI = F::kDma, NL = F::kLoads;
  constexpr int PQ = F::kPieces, NQ = F::kQRegs, DPV = F::kDpv;
  constexpr bool k16 = F::k16, kQ = F::kQuant, kNib = F::kNib, kOff = F::kOff;
  // Q4_0 / Q4_1: the high nibbles enter as 16 (n - 8) (no shift), their q
  // (QK) and their tile's weights (P.V) carrying the 1/16.
  constexpr bool kHi16 = DT == IT_Q4_0 || DT == IT_Q4_1;
  constexpr int NT = 64 * NW;  // threads
  static_assert(GC >= 1 && GC <= 8, "1..8 heads per workgroup");
  static_assert(NW == 2 || NW == 4, "2 or 4 waves");
  static_assert(R >= 2 && R <= 4, "ring wait covers R = 2..4");
  static_assert((R - 2) * NL < 64, "vmcnt is 6 bits");

  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr size_t kRingAll = size_t(NW) * R * SLOT;
  constexpr size_t kRed = size_t(NW) * 8 * D * 4;
  char* const ring = smem;
  float* const sc = reinterpret_cast<float*>(smem + (kRingAll > kRed ? kRingAll : kRed));
  const int SP = a.partition + 16;  // plane stride (staggers heads over the banks)
  float* const s_mx = sc + GC * SP;  // [NW][8] partition max per wave and head
  float* const s_l = s_mx + NW * 8;  // [NW][8] probability sums
  uint32_t* const s_pp = reinterpret_cast<uint32_t*>(s_l + NW * 8);  // [NW][kScratch / 4]
  int32_t* const s_pages = reinterpret_cast<int32_t*>(s_pp + NW * (F::kScratch / 4));
  // Score of head h, token i (partition-relative): sc[h * SP + i].

  const int P = a.partition;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bs_mask = (1 << a.log2_bs) - 1;
  const int bs = bs_mask + 1;
  const int n_seqs = a.n_seqs, hc = a.n_kv_heads * a.chunks;

  int part, yc, b, ctx, st;
  if (a.compact) {
    // The non-empty (sequence, head chunk, partition) units, counted
    // sequence by sequence (T in all), are dealt to the XCDs in contiguous
    // ranges of q = ceil(T / 8): workgroup L (on XCD L % 8, the dispatcher
    // deals workgroups to the XCDs round-robin) takes unit (L % 8) q + L / 8.
    // So every XCD gets the same number of units whatever the contexts, and
    // the partitions of one (sequence, head chunk) run on one XCD: the
    // combine pass then reads each row's partial results from one XCD's
    // writes (measured 0.6 us faster per config-2 decode than units dealt
    // round-robin).  Every wave finds its unit itself: 64-wide prefix sums
    // of the sequences' unit counts.  A sequence whose start position is
    // negative has no units (latched).
    const int L = int(blockIdx.x);
    const int ln = int(threadIdx.x & 63);
    auto seq_units = [&](int s, int& c, int& t) {  // units of sequence s (0 past the end)
      c = t = 0;
      if (s >= n_seqs) return 0;
      c = a.ctx_lens[s];
      t = a.start_pos ? a.start_pos[s] : 0;
      const int nn = c - t;
      return (nn > 0 && t >= 0) ? min((nn + P - 1) / P, a.max_parts) * hc : 0;
    };
    // Pass 1: T.  The first 64 sequences' counts are kept for pass 2.
    int c0, t0v;
    const int cnt0 = seq_units(ln, c0, t0v);
    if (t0v < 0 && L == 0) atomicOr(a.err, kErrStart);
    const int incl0 = wave_inclusive_sum(cnt0);
    int T = __builtin_amdgcn_readlane(incl0, 63);
    for (int s0 = 64; s0 < n_seqs; s0 += 64) {
      int c, t;
      const int cnt = seq_units(s0 + ln, c, t);
      if (t < 0 && L == 0) atomicOr(a.err, kErrStart);
      T += __builtin_amdgcn_readlane(wave_inclusive_sum(cnt), 63);
    }
    const int q = (T + 7) >> 3;
    const int k = L >> 3;
    const int U = (L & 7) * q + k;  // this workgroup's unit
    if (k >= q || U >= T) return;   // uniform for the workgroup
    // Pass 2: the sequence holding unit U.
    int base = 0;
    b = -1;
    part = yc = ctx = st = 0;
    for (int s0 = 0; s0 < n_seqs; s0 += 64) {
      int cnt = cnt0, c = c0, t = t0v, incl = incl0;
      if (s0 > 0) {
        cnt = seq_units(s0 + ln, c, t);
        incl = wave_inclusive_sum(cnt);
      }
      const int total = __builtin_amdgcn_readlane(incl, 63);
      if (U < base + total) {
        // Inclusive prefixes do not decrease, so the lanes at or below U
        // are a prefix of the wave; the unit's sequence is the next lane.
        const int idx = int(__popcll(__builtin_amdgcn_ballot_w64(base + incl <= U)));
        const int r = U - base - __builtin_amdgcn_readlane(incl - cnt, idx);
        const int np = max(1, __builtin_amdgcn_readlane(cnt, idx) / hc);
        b = s0 + idx;
        ctx = __builtin_amdgcn_readlane(c, idx);
        st = __builtin_amdgcn_readlane(t, idx);
        yc = r / np;
        part = r - yc * np;
        break;
      }
      base += total;
    }
    // Past the last unit (uniform for the workgroup); the range checks keep
    // every index in bounds whatever the counts.
    if (b < 0 || b >= n_seqs || yc < 0 || yc >= hc || part < 0 || part >= a.max_parts) return;
  } else {
    part = blockIdx.x;
    yc = blockIdx.y;
    b = blockIdx.z;
    ctx = a.ctx_lens ? a.ctx_lens[b] : a.ctx_const;
    st = a.start_pos ? a.start_pos[b] : 0;
    if (st < 0) {  // skipped, as the gather skips it (uniform for the workgroup)
      if (tid == 0) atomicOr(a.err, kErrStart);
      return;
    }
  }
  const int kvh = yc / a.chunks;
  const int chunk = yc - kvh * a.chunks;
  const int head0 = kvh * a.group + chunk * GC;
  const int n = ctx - st;
  if (n <= 0 || part * P >= n) return;  // uniform for the workgroup
  if (part == a.max_parts - 1 && n > a.max_parts * P && threadIdx.x == 0)
    atomicOr(a.err, kErrCtx);  // context longer than the caller's max_tokens: tail ignored
  const int tok0 = st + part * P;
  const int nt = min(P, n - part * P);

  // Page indices (block * n_kv_heads + kvh) of the partition, via LDS.
  const int lb0 = tok0 >> a.log2_bs;
  const int nlb = ((tok0 + nt - 1) >> a.log2_bs) - lb0 + 1;  // <= max_pages
  for (int i = tid; i < nlb; i += NT) {
    const int lb = lb0 + i;
    int blk = lb;
    if (a.bt) {
      if (lb >= a.max_blocks) {
        atomicOr(a.err, kErrTable);
        blk = 0;
      } else {
        blk = a.bt[int64_t(b) * a.max_blocks + lb];
      }
    }
    if (blk < 0 || blk >= a.num_blocks) {
      atomicOr(a.err, kErrBlock);
      blk = 0;
    }
    s_pages[i] = blk * a.n_kv_heads + kvh;
  }

  // q in the QK layout: lane (r, k) holds, per head, words k, 16 + k, ... of
  // quarter r of the head dimension (packed 16-bit pairs, or fp32).
  const int qr_row = lane >> 4, qk_tok = lane & 15;
  uint32_t qv[GC][NQ];
  // Quantised formats: q is the A operand of v_mfma_f32_16x16x32_f16
  // instead, lane (kh, h) = (lane / 16, lane % 16) holding eight dims of
  // group ks of head h (zero for h >= GC): Q8_0 dims 32 ks + 8 kh .. + 8;
  // nibble formats dims 32 ks + 4 kh .. + 4 and 32 ks + 16 + 4 kh .. + 4 (the
  // low and high nibbles of bytes 4 kh .. + 4 of the group).
  constexpr int NK = kQ ? D / 32 : 1;  // 32-groups (MFMA k-steps) per row
  // q of head h scaled by 2^E_h (so that max |q| lies in [2^14, 2^15)) as
  // hi + lo fp16 parts; the scores are scaled back by 2^-E_h (exact).
  // Q4_0 / Q4_1 take the high-nibble dims' q divided by 16, against K
  // values 16 (n - 8).  sE[i]: 2^-E of head 4 (lane / 16) + i, the heads
  // this lane's scores belong to.
  uint4 qf[2][NK];
  float sE[4] = {1.0f, 1.0f, 1.0f, 1.0f};
  // Q4_1: sum of q over each 32-group, the A operand of the offset-term MFMA
  // (v_mfma_f32_16x16x16_bf16, k = group): lane (kh, h) holds groups
  // 4 kh .. + 4 of head h, split exactly into three bf16 parts.
  uint2 qs_a[3];
  if constexpr (!kQ) {
    const uint32_t* qp = static_cast<const uint32_t*>(a.q) +
                         (int64_t(b) * a.n_heads + head0) * (k16 ? D / 2 : D) + qr_row * (k16 ? D / 8 : D / 4) +
                         qk_tok;
#pragma unroll
    for (int g = 0; g < GC; ++g)
#pragma unroll
      for (int j = 0; j < NQ; ++j) qv[g][j] = qp[g * (k16 ? D / 2 : D) + 16 * j];
    // Consume q and the block-table loads before any DMA is issued (the
    // compiler's wait for them would not know about the ring loads), and
    // give the DPP readers of q their wait states.
#pragma unroll
    for (int g = 0; g < GC; ++g)
#pragma unroll
      for (int j = 0; j < NQ; ++j) asm volatile("" : "+v"(qv[g][j]));
  } else {
    const int hq = lane & 15;
    const float* qp = static_cast<const float*>(a.q) + (int64_t(b) * a.n_heads + head0 + (hq < GC ? hq : 0)) * D +
                      (kNib ? 4 : 8) * qr_row;
    float qsum[NK];
    int E = 0;
    {
      float4 x0[NK], x1[NK];
      float mx = 0.0f;
#pragma unroll
      for (int ks = 0; ks < NK; ++ks) {
        x0[ks] = *reinterpret_cast<const float4*>(qp + 32 * ks);
        x1[ks] = *reinterpret_cast<const float4*>(qp + 32 * ks + (kNib ? 16 : 4));
        if (hq >= GC) x0[ks] = x1[ks] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if constexpr (kHi16) {  // exact
          x1[ks].x *= 0.0625f, x1[ks].y *= 0.0625f, x1[ks].z *= 0.0625f, x1[ks].w *= 0.0625f;
        }
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(x0[ks].x), fabsf(x0[ks].y)), fmaxf(fabsf(x0[ks].z), fabsf(x0[ks].w))));
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(x1[ks].x), fabsf(x1[ks].y)), fmaxf(fabsf(x1[ks].z), fabsf(x1[ks].w))));
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16));  // the four lanes of head hq
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      // mx in [2^(e-1), 2^e): E = 15 - e; an all-zero (or non-finite) q keeps E = 0.
      E = (mx > 0.0f && mx <= FLT_MAX) ? 15 - __builtin_amdgcn_frexp_expf(mx) : 0;
#pragma unroll
      for (int ks = 0; ks < NK; ++ks) {
        // k order: Q5 interleaves the two nibbles of each byte (elements
        // e, e + 16), the others take the four x0 values, then x1's.
        const float x[8] = {x0[ks].x, F::kQ5 ? x1[ks].x : x0[ks].y, F::kQ5 ? x0[ks].y : x0[ks].z,
                            F::kQ5 ? x1[ks].y : x0[ks].w, F::kQ5 ? x0[ks].z : x1[ks].x,
                            F::kQ5 ? x1[ks].z : x1[ks].y, F::kQ5 ? x0[ks].w : x1[ks].z, x1[ks].w};
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          h2 hp, lp;
          const float y0 = __builtin_ldexpf(x[2 * j], E), y1 = __builtin_ldexpf(x[2 * j + 1], E);
          hp[0] = (_Float16)y0;
          hp[1] = (_Float16)y1;
          lp[0] = (_Float16)(y0 - (float)hp[0]);
          lp[1] = (_Float16)(y1 - (float)hp[1]);
          hw[j] = __builtin_bit_cast(uint32_t, hp);
          lw[j] = __builtin_bit_cast(uint32_t, lp);
        }
        qf[0][ks] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        qf[1][ks] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) sE[i] = __builtin_ldexpf(1.0f, -__shfl(E, 4 * qr_row + i));
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int ks = 0; ks < NK; ++ks)
          asm volatile("" : "+v"(qf[p][ks].x), "+v"(qf[p][ks].y), "+v"(qf[p][ks].z), "+v"(qf[p][ks].w));
    }
#pragma unroll
    for (int ks = 0; ks < NK && kOff; ++ks) {
      float4 x0 = *reinterpret_cast<const float4*>(qp + 32 * ks);
      float4 x1 = *reinterpret_cast<const float4*>(qp + 32 * ks + 16);
      if (hq >= GC) x0 = x1 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      qsum[ks] = ((x0.x + x0.y) + (x0.z + x0.w)) + ((x1.x + x1.y) + (x1.z + x1.w));
    }
    if constexpr (kOff) {
      float qg[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < NK; ++ks) {
        qsum[ks] += __shfl_xor(qsum[ks], 16);  // the four lanes of head hq
        qsum[ks] += __shfl_xor(qsum[ks], 32);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (ks == 4 * qr_row + j) qg[j] = __builtin_ldexpf(qsum[ks], E);  // the scores' 2^E
      }
      uint2 p0, p1, p2;
      split3_bf16(qg[0], qg[1], p0.x, p1.x, p2.x);
      split3_bf16(qg[2], qg[3], p0.y, p1.y, p2.y);
      qs_a[0] = p0, qs_a[1] = p1, qs_a[2] = p2;
    }
  }
  asm volatile("s_waitcnt vmcnt(0)\n\ts_nop 4" ::: "memory");
  lds_barrier();

  // This wave's groups: w, w + NW, ...; the stream is their K rows, then
  // their V rows.
  const int ng = (nt + kGroupTok - 1) / kGroupTok;
  const int ns = ng > wave ? (ng - 1 - wave) / NW + 1 : 0;
  const int S = 2 * ns;
  char* const my_ring = ring + size_t(wave) * R * SLOT;
  const uint32_t ring_m0 = lds_offset(my_ring);
  const uint32_t page_bytes = uint32_t(a.page_bytes);

  // Load stream item s (K or V group) into slot s % R: instruction j, lane i
  // moves bytes [1024 j + 16 i, +16) of the group's main plane, i.e. piece
  // slot ps of token row tt (K rows hold logical piece ps ^ (tt & kSwz)
  // there, quantised V rows ps ^ kVQuad ((tt / 4) % 4)); quantised formats
  // add dword loads of the group's scale rows.  Rows past the partition load
  // the group's first row as a stand-in.
  int lane_row[NI], lane_off_k[NI], lane_off_v[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int o = 1024 * j + 16 * lane;
    const int tt = o / RB, ps = (o % RB) / 16;
    lane_row[j] = tt;
    lane_off_k[j] = tt * RB + ((ps ^ (tt & F::kSwz)) << 4);
    lane_off_v[j] = tt * RB + ((ps ^ (F::kVQuad * ((tt >> 2) & 3))) << 4);
  }
  // Scale loads: load u moves bytes [256 u + 4 lane, +4) of the group's
  // scale rows (row s_row[u], byte s_col[u]) when that is inside them.
  constexpr int NS = F::kScaleLoads > 0 ? F::kScaleLoads : 1;
  int s_row[NS], s_col[NS];
  bool s_lane[NS];
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int sb = 256 * u + 4 * lane;
    s_lane[u] = sb < F::kScaleGroup;
    s_row[u] = kQ ? sb / (F::kScaleRow > 0 ? F::kScaleRow : 1) : 0;
    s_col[u] = kQ ? sb % (F::kScaleRow > 0 ? F::kScaleRow : 1) : 0;
  }
  auto issue = [&](int s) {
    const bool is_v = s >= ns;
    const int gi = is_v ? s - ns : s;
    const int tb = (gi * NW + wave) * kGroupTok;  // partition-relative first token
    const int t0 = tok0 + tb;
    const char* pool = is_v ? a.v_pool : a.k_pool;
    const uint32_t m0 = ring_m0 + uint32_t(s % R) * SLOT;
    const int in_page = t0 & bs_mask;
    if (in_page + kGroupTok <= bs) {
      // The whole group lies in one page: one uniform base, one add per load.
      const uint32_t page = uint32_t(__builtin_amdgcn_readfirstlane(s_pages[(t0 >> a.log2_bs) - lb0]));
      const char* pbase = pool + uint64_t(page) * page_bytes;
      const char* base = pbase + uint32_t(in_page * RB);
      if (tb + kGroupTok <= nt) {
        // Every row inside the partition: uniform bases, per-lane offsets
        // fixed for the kernel.
#pragma unroll
        for (int j = 0; j < NI; ++j)
          dma_b128_s(base, uint32_t(is_v ? lane_off_v[j] : lane_off_k[j]),
                     __builtin_amdgcn_readfirstlane(m0 + 1024u * j));
        if constexpr (kQ) {
          const char* sbase = pbase + uint32_t(bs * RB + in_page * F::kScaleRow);
#pragma unroll
          for (int u = 0; u < F::kScaleLoads; ++u)
            if (s_lane[u])
              dma_b32_s(sbase, uint32_t(s_row[u] * F::kScaleRow + s_col[u]),
                        __builtin_amdgcn_readfirstlane(m0 + uint32_t(GB + 256 * u)));
        }
      } else {
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          int off = is_v ? lane_off_v[j] : lane_off_k[j];
          if (tb + lane_row[j] >= nt) off -= lane_row[j] * RB;
          dma_b128(base + off, __builtin_amdgcn_readfirstlane(m0 + 1024u * j));
        }
        if constexpr (kQ) {
#pragma unroll
          for (int u = 0; u < F::kScaleLoads; ++u) {
            int row = s_row[u];
            if (tb + row >= nt) row = 0;
            const char* g = pbase + uint32_t(bs * RB + (in_page + row) * F::kScaleRow + s_col[u]);
            if (s_lane[u]) dma_b32(g, __builtin_amdgcn_readfirstlane(m0 + uint32_t(GB + 256 * u)));
          }
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int tt = lane_row[j];
        int tr = tb + tt;
        const int off = (is_v ? lane_off_v[j] : lane_off_k[j]) - tt * RB;  // piece offset within the row
        if (tr >= nt) tr = tb;
        const int t = tok0 + tr;
        const uint32_t page = uint32_t(s_pages[(t >> a.log2_bs) - lb0]);
        const char* g = pool + (uint64_t(page) * page_bytes + uint32_t((t & bs_mask) * RB + off));
        dma_b128(g, __builtin_amdgcn_readfirstlane(m0 + 1024u * j));
      }
      if constexpr (kQ) {
#pragma unroll
        for (int u = 0; u < F::kScaleLoads; ++u) {
          int tr = tb + s_row[u];
          if (tr >= nt) tr = tb;
          const int t = tok0 + tr;
          const uint32_t page = uint32_t(s_pages[(t >> a.log2_bs) - lb0]);
          const char* g =
              pool + (uint64_t(page) * page_bytes + uint32_t(bs * RB + (t & bs_mask) * F::kScaleRow + s_col[u]));
          if (s_lane[u]) dma_b32(g, __builtin_amdgcn_readfirstlane(m0 + uint32_t(GB + 256 * u)));
        }
      }
    }
  };
  // Before consuming item s: its loads are done (at most the items issued
  // after it are outstanding) and this wave's LDS reads are done, so the
  // slot read at step s-1 may be refilled.
  auto wait_item = [&](int s) {
    const int later = min(R - 2, S - 1 - s);  // items issued after s
    if (R >= 4 && later >= 2) asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)" ::"n"(2 * NL) : "memory");
    else if (R >= 3 && later >= 1) asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)" ::"n"(NL) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)" ::: "memory");
  };
  // Issue priority alternated item by item.  The oldest waves of a CU win
  // instruction arbitration at equal priority, and the memory pipe is
  // saturated here: the first workgroup dispatched to a CU ran its phases
  // 9% faster (config 2 at 4k) to 25% faster (ragged contexts) than its
  // three CU-mates, and the last, youngest ones set the kernel's end.
  // Alternating s_setprio by item parity (offset per workgroup) spreads the
  // advantage: measured split 43.45 -> 43.22 us at 4k, 26.48 -> 25.99 us
  // ragged.  (Reverse-age and issue-only priorities gained less; deeper
  // rings lost: 3 slots took 45.4 us at 4k.)  16/32-bit caches only, where
  // it was measured.
  auto age_fair = [&](int s) {
    if constexpr (!kQ) {
      if ((s ^ int(blockIdx.x >> 3)) & 1) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
  };
  for (int s = 0; s < R - 1 && s < S; ++s) issue(s);

  // ---------------- phase 1: scores -----------------------------------------
  const bool masked = a.mask != nullptr;
  const float qk_mult = masked ? 1.0f : a.scale_log2;
  // Head held by lane row r after the fold: {0, 2, 1, 3}[r] (+4 in s_b).
  const int h_a = ((qr_row & 1) << 1) | (qr_row >> 1);
  float m_a = -INFINITY, m_b = -INFINITY;
  float m_q[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};  // quantised: heads 4 qr_row + i
  // 0x64006400 held in a VGPR, so that (x & mask) | k6400 is one
  // v_and_or_b32 (a VOP3 reads at most one scalar operand here).
  uint32_t k6400 = 0x64006400u;
  asm volatile("" : "+v"(k6400));
  // Q5 QK: qh rotations that bring element 4 kh + i's fifth bit to bit 4.
  uint32_t rot5k[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) rot5k[i] = uint32_t(4 * qr_row + i - 4) & 31u;
  for (int s = 0; s < ns; ++s) {
    wait_item(s);
    age_fair(s);
    if (s + R - 1 < S) issue(s + R - 1);
    const char* slot = my_ring + (s % R) * SLOT;
    if constexpr (kQ) {
      // Scores on MFMA: S[h][t] = sum over 32-groups ks of f32(d[t][ks]) *
      // (q[h] . v[t]) over the group, the group dot product taken as two
      // exact fp16 passes (the hi and lo parts of q 2^E, against K values
      // exact in fp16) into one fp32 accumulator, scaled back by 2^-E.  Lane
      // (kh, t) reads bytes 8 kh .. + 8 of group ks of token t (nibble
      // formats: bytes 4 kh .. + 4 of the group's 16) and ends holding
      // S[4 kh + i][t], i = 0..3.
      const char* krow = slot + qk_tok * RB;
      const char* const kside = slot + GB + qk_tok * F::kScaleRow;
      uint16_t dsc[NK];
#pragma unroll
      for (int ks = 0; ks < NK; ++ks)
        dsc[ks] = *reinterpret_cast<const uint16_t*>(kside + F::kMetaOff + F::kMetaStride * ks);
      // Q5: the qh word of group ks (bit e: element e's fifth bit).
      uint32_t qh5[F::kQ5 ? NK : 1];
      if constexpr (F::kQ5) {
#pragma unroll
        for (int ks = 0; ks < NK; ++ks) qh5[ks] = *reinterpret_cast<const uint32_t*>(kside + 4 * ks);
      }
      // All K reads first; then the two passes of each group are software
      // pipelined across groups, so that no MFMA waits for the one before it.
      uint2 kr[NK];
#pragma unroll
      for (int ks = 0; ks < NK; ++ks) {
        if constexpr (kNib) {
          const int pc = ks ^ (qk_tok & F::kSwz);  // a Q4_0 group is one 16-byte piece
          kr[ks] = make_uint2(*reinterpret_cast<const uint32_t*>(krow + (pc << 4) + 4 * qr_row), 0u);
        } else {
          const int pc = (2 * ks + (qr_row >> 1)) ^ (qk_tok & F::kSwz);  // physical piece slot
          kr[ks] = *reinterpret_cast<const uint2*>(krow + (pc << 4) + 8 * (qr_row & 1));
        }
      }
      v4f acc[NK];
      uint4 kb[NK];
      {
        // q hi / lo parts against the exact fp16 K values, the two MFMAs of
        // a group a group apart.
        Unroll<0, NK + 1>::run([&](auto kc) {
          constexpr int k = decltype(kc)::value;
          if constexpr (k < NK) {
            if constexpr (F::kQ8) {
              kb[k] = i8x8_f16(kr[k]);
            } else if constexpr (F::kQ5) {
              // Pair i: elements e = 4 kh + i and e + 16, the two nibbles of
              // byte i (q holds the same order), values n + 16 b - 16 as the
              // fp16 bits 0x6400 | n | b << 4 (= 1024 + n + 16 b) - 1040,
              // exactly.  qh rotated right by e - 4 puts e's fifth bit on
              // bit 4 and e + 16's on bit 20.
              const uint32_t w = kr[k].x, w4 = w >> 4, qh = qh5[k];
              const h2 k1040 = {(_Float16)-1040.0f, (_Float16)-1040.0f};
              auto q5 = [&](int i) {
                // byte i of w (low nibble) and of w >> 4 (high nibble) into the halves
                uint32_t nibw = (__builtin_amdgcn_perm(w4, w, 0x0C040C00u + 0x00010001u * i) & 0x000F000Fu) | k6400;
                asm volatile("" : "+v"(nibw));  // two v_and_or, not and, and, or3
                const uint32_t z = __builtin_amdgcn_alignbit(qh, qh, rot5k[i]);
                return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, (z & 0x00100010u) | nibw) + k1040);
              };
              kb[k] = make_uint4(q5(0), q5(1), q5(2), q5(3));
            } else {
              // Bytes 0, 1 and 2, 3 into 16-bit halves; low nibbles n as
              // 0x6400 | n - 1032 = n - 8, high ones as 0x6400 | 16 n - 1152
              // = 16 (n - 8) (q of their dims carries 1/16), exactly.
              const uint32_t w = kr[k].x;
              const uint32_t p01 = __builtin_amdgcn_perm(0u, w, 0x0C010C00u), p23 = __builtin_amdgcn_perm(0u, w, 0x0C030C02u);
              const h2 k1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
              const h2 k1152 = {(_Float16)-1152.0f, (_Float16)-1152.0f};
              auto nib = [&](uint32_t x, uint32_t mask, h2 bias) {
                return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, (x & mask) | k6400) + bias);
              };
              kb[k] = make_uint4(nib(p01, 0x000F000Fu, k1032), nib(p23, 0x000F000Fu, k1032),
                                 nib(p01, 0x00F000F0u, k1152), nib(p23, 0x00F000F0u, k1152));
            }
            acc[k] = mfma16_f16(qf[0][k], kb[k], v4f{0.0f, 0.0f, 0.0f, 0.0f});
          }
          if constexpr (k >= 1) acc[k - 1] = mfma16_f16(qf[1][k - 1], kb[k - 1], acc[k - 1]);
        });
      }
      v4f sv = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < NK; ++ks) {
        const float d = f16_bits_to_f32(dsc[ks]);
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = fmaf(d, acc[ks][i], sv[i]);
      }
      if constexpr (kOff) {
        // + sum over groups G of m'_G(t) qsum[h][G]: lane (kh, t) holds
        // B[G = 4 kh + j][t] = m'_G(t), zero past the groups; both operands
        // in three exact bf16 parts.
        float mv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int G = 4 * qr_row + j;
          mv[j] = G < NK ? off_mprime<DT>(*reinterpret_cast<const uint32_t*>(kside + F::kMetaOff + 4 * (G < NK ? G : 0)))
                         : 0.0f;
        }
        uint2 mb[3];
        split3_bf16(mv[0], mv[1], mb[0].x, mb[1].x, mb[2].x);
        split3_bf16(mv[2], mv[3], mb[0].y, mb[1].y, mb[2].y);
#pragma unroll
        for (int p = 0; p < 3; ++p)
#pragma unroll
          for (int r = 0; r < 3; ++r) sv = mfma16k16(qs_a[p], mb[r], sv);
      }
      const int i_tok = (s * NW + wave) * kGroupTok + qk_tok;
      if (i_tok < nt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int h = 4 * qr_row + i;
          const float x = sv[i] * (qk_mult * sE[i]);  // sE: the head's 2^-E
          if (h < GC) sc[h * SP + i_tok] = x;
          m_q[i] = fmaxf(m_q[i], x);
        }
      }
      continue;
    }
    const char* row = slot + qk_tok * RB;
    float acc[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) acc[g] = 0.0f;
    uint4 kk[PQ];
#pragma unroll
    for (int i = 0; i < PQ; ++i) kk[i] = ld16(row + (((qr_row * PQ + i) ^ (qk_tok & F::kSwz)) << 4));
    {
      Unroll<0, PQ>::run([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        constexpr int w0 = 4 * i;  // first q word of the piece (mod 16: lane; / 16: VGPR)
        uint32_t qi[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) qi[g] = qv[g < GC ? g : 0][w0 / 16];
        qk_words<DT, GC, w0 % 16>(acc, qi, kk[i].x, kk[i].y, kk[i].z, kk[i].w);
      });
    }
    // v_permlane*_swap must not read the accumulators within a few wait
    // states of the asm that wrote them.
    asm volatile("s_nop 4" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(acc[4]), "+v"(acc[5]),
                 "+v"(acc[6]), "+v"(acc[7]));
    // Fold the four quarter sums: s_a rows hold heads {0,2,1,3}, s_b {4,6,5,7}.
    const float a01 = fold32(acc[0], acc[1]);
    const float a23 = GC > 2 ? fold32(acc[2], acc[3]) : 0.0f;
    const float s_a = fold16(a01, a23) * qk_mult;
    float s_b = 0.0f;
    if constexpr (GC > 4) {
      const float a45 = fold32(acc[4], acc[5]);
      const float a67 = GC > 6 ? fold32(acc[6], acc[7]) : 0.0f;
      s_b = fold16(a45, a67) * qk_mult;
    }
    const int i_tok = (s * NW + wave) * kGroupTok + qk_tok;
    if (i_tok < nt) {
      if (h_a < GC) sc[h_a * SP + i_tok] = s_a;
      if (GC > 4 && 4 + h_a < GC) sc[(4 + h_a) * SP + i_tok] = s_b;
      m_a = fmaxf(m_a, s_a);
      m_b = fmaxf(m_b, s_b);
    }
  }
  if constexpr (kQ) {
#pragma unroll
    for (int i = 0; i < 4; ++i) m_q[i] = group_max<16>(m_q[i]);
    if (qk_tok == 0 && qr_row < 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s_mx[wave * 8 + 4 * qr_row + i] = m_q[i];
    }
  } else {
    m_a = group_max<16>(m_a);
    m_b = group_max<16>(m_b);
    if (qk_tok == 0) {
      s_mx[wave * 8 + h_a] = m_a;
      s_mx[wave * 8 + 4 + h_a] = m_b;
    }
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

  // The softmax is folded into the PV loop: lane L computes the probabilities
  // of tokens 2 (L % 8) and 2 (L % 8) + 1 of the group for head L / 8 from the
  // partition max (16-bit caches round them, as a pair, to the cache's type:
  // the weights PV applies) and adds them to its running sum.
  const int h_l = lane >> 3, k_l = lane & 7;
  float m_l = s_mx[h_l];
#pragma unroll
  for (int w = 1; w < NW; ++w) m_l = fmaxf(m_l, s_mx[w * 8 + h_l]);
  const bool none_l = m_l == -INFINITY;  // every key skipped: zeros (flash_attn.rs:66-71)
  const float* const sc_l = sc + (h_l < GC ? h_l : 0) * SP;
  uint32_t* const pp_w = s_pp + wave * (F::kScratch / 4);
  float lsum = 0.0f;

  // ---------------- phase 3: P.V over the V groups ---------------------------
  float acc2[DPV][8];  // [dim of the lane][head]; heads >= GC stay 0
#pragma unroll
  for (int x = 0; x < DPV; ++x)
#pragma unroll
    for (int g = 0; g < 8; ++g) acc2[x][g] = 0.0f;
  // Quantised formats: P.V on MFMA, per 32-group G of the head dim
  // O[h][dim(G, c, n)] += sum_t p[h][t] f32(d[t][G]) v[t][dim(G, c, n)]
  // (tile c = 0, 1; column n; Q8_0 dim 32 G + 2 n + c from a 2-byte read,
  // nibble formats dim 32 G + 16 c + n, the two nibbles of byte n of the
  // group), in the fp16 form or the three-part bf16 form below.  Lane
  // (kq, hm) = (lane / 16, lane % 16) holds A[head hm][tokens 4 kq + j] and
  // B[tokens 4 kq + j][column hm] (the MFMA's k index runs over 4 kq + j in
  // both), and ends holding O[4 kq + i][column hm] of every tile.
  v4f o8[kQ ? NK : 1][2];
  v4f mo = {0.0f, 0.0f, 0.0f, 0.0f};  // Q4_1: sum_t p[4 kq + i][t] m'_hm(t)
  if constexpr (kQ) {
    const int hm = lane & 15, kq = qr_row;
#pragma unroll
    for (int g = 0; g < NK; ++g) o8[g][0] = o8[g][1] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    float m_h = -INFINITY;
    if (hm < GC) {
#pragma unroll
      for (int w = 0; w < NW; ++w) m_h = fmaxf(m_h, s_mx[w * 8 + hm]);
    }
    const bool none_h = m_h == -INFINITY;  // every key skipped, or a padding row
    const float* const sc_h = sc + (hm < GC ? hm : 0) * SP + 4 * kq;
    // One item of the partition, in the bf16 form if bf16_only; else in the
    // fp16 form, or, when that does not fit its scales, not at all: it then
    // returns false, having changed nothing but the item's wait and issue.
    auto v_item = [&](int s, auto bf16_only, bool redo) -> bool {
      if (!redo) {  // redo: the item's wait and issue are done
        wait_item(s);
        if (s + R - 1 < S) issue(s + R - 1);
      }
      const int gi = s - ns;
      const int tb = (gi * NW + wave) * kGroupTok;
      char* const slot = my_ring + (s % R) * SLOT;
      if (tb + kGroupTok > nt) {
        // Rows past the partition hold a stand-in row: each lane zeroes the
        // bytes its own loads brought (this wave's LDS ops stay in order).
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          const int o = 1024 * j + 16 * lane;
          if (tb + o / RB >= nt) *reinterpret_cast<uint4*>(slot + o) = make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < F::kScaleLoads; ++u)
          if (s_lane[u] && tb + s_row[u] >= nt) *reinterpret_cast<uint32_t*>(slot + GB + 256 * u + 4 * lane) = 0u;
      }
      const float4 sv = *reinterpret_cast<const float4*>(sc_h + tb);
      const float sj[4] = {sv.x, sv.y, sv.z, sv.w};
      float pj[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        pj[j] = (tb + 4 * kq + j < nt && !none_h) ? __builtin_amdgcn_exp2f(sj[j] - m_h) : 0.0f;
      const char* const vrow = slot + (4 * kq) * RB + (kNib ? 1 : 2) * hm;
      // The side rows of the lane's four tokens: their d words (NK fp16,
      // or (d, m) pairs), after the qh words for Q5.
      const char* const srow = slot + GB + (4 * kq) * F::kScaleRow;
      constexpr int SW = (F::kScaleRow > 0 ? F::kScaleRow - F::kMetaOff : 4) / 4;  // d dwords per token row
      uint32_t dw[4][SW];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const char* const dr = srow + j * F::kScaleRow + F::kMetaOff;
        if constexpr (SW % 4 == 0) {
#pragma unroll
          for (int c = 0; c < SW / 4; ++c) {
            const uint4 t = *reinterpret_cast<const uint4*>(dr + 16 * c);
            dw[j][4 * c] = t.x, dw[j][4 * c + 1] = t.y, dw[j][4 * c + 2] = t.z, dw[j][4 * c + 3] = t.w;
          }
        } else {
          const uint2 t = *reinterpret_cast<const uint2*>(dr);
          dw[j][0] = t.x, dw[j][1] = t.y;
        }
      }
      // fp16 d of group G for token 4 kq + j (Q4_1 / Q5_1 rows hold (d, m) pairs).
      auto dbits = [&](int j, auto gc) -> uint32_t {
        constexpr int G = decltype(gc)::value;
        if constexpr (kOff) return dw[j][G] & 0xFFFFu;
        else return G & 1 ? dw[j][G / 2] >> 16 : dw[j][G / 2] & 0xFFFFu;
      };
      // P.V in fp16, when every scale of the item is small enough that
      // |d v| <= 65504 (d below 512 where |v| <= 128: Q8_0's q, and Q4's
      // tile 1, which holds 16 (n - 8); d below 2048 for Q5's |q - 16| <=
      // 16; other items take the bf16 form below): B = d v is exact as
      // hi + lo fp16 parts (d has 11 significant bits and v at most 8), and
      // A = p 2^11 as two fp16 parts made once per item (p <= 1: every weight above 2^-13 keeps 22 bits,
      // smaller ones an absolute error below 2^-36).  Each tile takes two
      // v_mfma_f32_16x16x32_f16 whose k runs over (token, B part):
      // [A_hi A_hi] . [B_hi; B_lo] and [A_lo A_lo] . [B_hi; B_lo], every
      // product exact in the fp32 accumulator (11 x 11 significant bits).
      // K = 32 costs little more than K = 16 (measured 19 against 17
      // cycles), so a V item is 32 MFMAs instead of the bf16 form's 48.  The
      // two MFMAs of an accumulator are issued a group apart, so none waits
      // for the one before it.  (The offset term of Q4_1 / Q5_1 stays on
      // the bf16 form above.)
      bool f16_item;
      {
        // The 16 lanes of a token quad hold the same 4 SW scale words, so
        // each lane checks its share of them (one word for SW = 4) with a
        // read of its own, and the ballot covers the item.  |d| bits order
        // as the values (Q4_0's d = max / -8 and Q5_0's max / -16 take
        // either sign); Q4_1's and Q5_1's high halves are the offsets m, not
        // scales.  512: |v| <= 128 (Q8_0's q, Q4's 16 (n - 8)); 2048:
        // |v| <= 16 (Q5).
        constexpr unsigned kLim = F::kQ5 ? 0x6800u : 0x6000u;
        constexpr int NDW = 4 * SW;
        bool big = false;
#pragma unroll
        for (int r = 0; r < (NDW + 15) / 16; ++r) {
          const int i = (hm + 16 * r) % NDW;
          uint32_t w = *reinterpret_cast<const uint32_t*>(srow + (i / SW) * F::kScaleRow + F::kMetaOff + 4 * (i % SW));
          if constexpr (DT == IT_Q4_0 || DT == IT_Q5_0) w &= 0x7FFF7FFFu;
          big |= (w & 0xFFFFu) >= kLim || (!kOff && (w >> 16) >= kLim);
        }
        f16_item = __builtin_amdgcn_ballot_w64(big) == 0;  // uniform
      }
      if constexpr (!decltype(bf16_only)::value) {
        if (!f16_item) return false;  // before any state of the item changes
      }
      lsum += (pj[0] + pj[1]) + (pj[2] + pj[3]);
      if constexpr (kOff) {
        // The offset term: M[h][G] += sum over the item's tokens of p[h][t]
        // m'_G(t); B[t][G = hm] for the lane's four tokens, zero past the
        // groups; both operands in three exact bf16 parts.
        float mv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          mv[j] = hm < NK ? off_mprime<DT>(*reinterpret_cast<const uint32_t*>(slot + GB + (4 * kq + j) * F::kScaleRow +
                                                                               F::kMetaOff + 4 * (hm < NK ? hm : 0)))
                          : 0.0f;
        uint2 mb[3], pa[3];
        split3_bf16(mv[0], mv[1], mb[0].x, mb[1].x, mb[2].x);
        split3_bf16(mv[2], mv[3], mb[0].y, mb[1].y, mb[2].y);
        split3_bf16(pj[0], pj[1], pa[0].x, pa[1].x, pa[2].x);
        split3_bf16(pj[2], pj[3], pa[0].y, pa[1].y, pa[2].y);
#pragma unroll
        for (int p = 0; p < 3; ++p)
#pragma unroll
          for (int r = 0; r < 3; ++r) mo = mfma16k16(pa[p], mb[r], mo);
      }
      // The P.V weights carry 2^11 (exact; undone when the partials are
      // stored): the fp16 form below needs it, and the bf16 form keeps the
      // accumulators on the same scale.
#pragma unroll
      for (int j = 0; j < 4; ++j) pj[j] *= kQPScale;
      auto pv_f16 = [&](auto) {
        const uint32_t rot5 = uint32_t(hm - 4) & 31u;  // Q5: the fifth bits' rotation
        uint2 ah, al;
        split2_f16(pj, ah, al);
        const uint4 a_hi = make_uint4(ah.x, ah.y, ah.x, ah.y), a_lo = make_uint4(al.x, al.y, al.x, al.y);
        // B operands of group G (both tiles).
        auto bgroup = [&](auto gc, uint4 (&b)[2]) {
          constexpr int G = decltype(gc)::value;
          // fp16 d of group G for the token pairs (0, 1) and (2, 3).
          constexpr uint32_t kSel = (!kOff && (G & 1)) ? 0x07060302u : 0x05040100u;
          constexpr int GW = kOff ? G : G / 2;  // the dword holding it
          const h2 d01 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(dw[1][GW], dw[0][GW], kSel));
          const h2 d23 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(dw[3][GW], dw[2][GW], kSel));
          // v of the lane's four tokens as fp16 pairs, tile t: Q8_0 tile 0
          // even dims (byte 0 of each 2-byte read), tile 1 odd; nibble
          // formats tile 0 the low nibbles (element hm), tile 1 the high
          // (element 16 + hm).
          h2 v01[2], v23[2];
          if constexpr (F::kQ8) {
            const int vg = 32 * (G ^ kq);
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = *reinterpret_cast<const uint16_t*>(vrow + j * RB + vg);
            v01[0] = __builtin_bit_cast(h2, i8pair_f16<0, 0>(w[0], w[1]));
            v01[1] = __builtin_bit_cast(h2, i8pair_f16<1, 1>(w[0], w[1]));
            v23[0] = __builtin_bit_cast(h2, i8pair_f16<0, 0>(w[2], w[3]));
            v23[1] = __builtin_bit_cast(h2, i8pair_f16<1, 1>(w[2], w[3]));
          } else if constexpr (F::kQ5) {
            const int vg = 16 * (G ^ kq);
            us2 t01, t23;  // the group's byte of tokens (0, 1) and (2, 3), one per half
            t01[0] = *reinterpret_cast<const uint8_t*>(vrow + vg);
            t01[1] = *reinterpret_cast<const uint8_t*>(vrow + RB + vg);
            t23[0] = *reinterpret_cast<const uint8_t*>(vrow + 2 * RB + vg);
            t23[1] = *reinterpret_cast<const uint8_t*>(vrow + 3 * RB + vg);
            const uint32_t p01 = __builtin_bit_cast(uint32_t, t01), p23 = __builtin_bit_cast(uint32_t, t23);
            // qh of token j rotated right by hm - 4: bit 4 is element
            // hm's fifth bit (tile 0), bit 20 element 16 + hm's (tile 1).
            uint32_t r[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t qh = *reinterpret_cast<const uint32_t*>(srow + j * F::kScaleRow + 4 * G);
              r[j] = __builtin_amdgcn_alignbit(qh, qh, rot5);
            }
            // Values q - 16 = n + 16 b - 16 as the fp16 bits
            // 0x6400 | n | b << 4 (= 1024 + n + 16 b) - 1040, exactly; the
            // fifth bits of tokens (0, 1) / (2, 3) brought to bits 4 and
            // 20 by a byte permute.
            const h2 k1040 = {(_Float16)-1040.0f, (_Float16)-1040.0f};
            auto q5 = [&](uint32_t x, uint32_t z) {
              uint32_t nibw = (x & 0x000F000Fu) | k6400;
              asm volatile("" : "+v"(nibw));  // two v_and_or, not and, and, or3
              return __builtin_bit_cast(h2, (z & 0x00100010u) | nibw) + k1040;
            };
            v01[0] = q5(p01, __builtin_amdgcn_perm(r[1], r[0], 0x0C040C00u));
            v23[0] = q5(p23, __builtin_amdgcn_perm(r[3], r[2], 0x0C040C00u));
            v01[1] = q5(p01 >> 4, __builtin_amdgcn_perm(r[1], r[0], 0x0C060C02u));
            v23[1] = q5(p23 >> 4, __builtin_amdgcn_perm(r[3], r[2], 0x0C060C02u));
          } else {
            const int vg = 16 * (G ^ kq);
            // The group's byte of tokens (0, 1) and (2, 3), one per 16-bit
            // half.
            us2 t01, t23;
            t01[0] = *reinterpret_cast<const uint8_t*>(vrow + vg);
            t01[1] = *reinterpret_cast<const uint8_t*>(vrow + RB + vg);
            t23[0] = *reinterpret_cast<const uint8_t*>(vrow + 2 * RB + vg);
            t23[1] = *reinterpret_cast<const uint8_t*>(vrow + 3 * RB + vg);
            const uint32_t p01 = __builtin_bit_cast(uint32_t, t01), p23 = __builtin_bit_cast(uint32_t, t23);
            // Low nibble n as the fp16 bits 0x6400 | n = 1024 + n, high
            // nibble as 0x6400 | 16 n = 1024 + 16 n (one v_and_or each:
            // the 0x6400 word sits in a VGPR); then - 1032 and - 1152:
            // n - 8 and 16 (n - 8), exactly.  Tile 1 thus accumulates 16
            // times its values, undone where the partials are stored.
            const h2 k1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
            const h2 k1152 = {(_Float16)-1152.0f, (_Float16)-1152.0f};
            auto nib = [&](uint32_t x, uint32_t mask) { return __builtin_bit_cast(h2, (x & mask) | k6400); };
            v01[0] = nib(p01, 0x000F000Fu) + k1032, v23[0] = nib(p23, 0x000F000Fu) + k1032;
            v01[1] = nib(p01, 0x00F000F0u) + k1152, v23[1] = nib(p23, 0x00F000F0u) + k1152;
          }
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const h2 hi01 = v01[t] * d01, hi23 = v23[t] * d23;
            const h2 lo01 = __builtin_elementwise_fma(v01[t], d01, -hi01);
            const h2 lo23 = __builtin_elementwise_fma(v23[t], d23, -hi23);
            b[t] = make_uint4(__builtin_bit_cast(uint32_t, hi01), __builtin_bit_cast(uint32_t, hi23),
                              __builtin_bit_cast(uint32_t, lo01), __builtin_bit_cast(uint32_t, lo23));
          }
        };
        // Two groups at a time: their four A_hi MFMAs, then the four A_lo
        // ones, so an accumulator's second MFMA comes four after its first.
        Unroll<0, NK / 2>::run([&](auto pc) {
          constexpr int G0 = 2 * decltype(pc)::value;
          uint4 b0[2], b1[2];
          bgroup(std::integral_constant<int, G0>{}, b0);
          bgroup(std::integral_constant<int, G0 + 1>{}, b1);
          o8[G0][0] = mfma16_f16(a_hi, b0[0], o8[G0][0]);
          o8[G0][1] = mfma16_f16(a_hi, b0[1], o8[G0][1]);
          o8[G0 + 1][0] = mfma16_f16(a_hi, b1[0], o8[G0 + 1][0]);
          o8[G0 + 1][1] = mfma16_f16(a_hi, b1[1], o8[G0 + 1][1]);
          o8[G0][0] = mfma16_f16(a_lo, b0[0], o8[G0][0]);
          o8[G0][1] = mfma16_f16(a_lo, b0[1], o8[G0][1]);
          o8[G0 + 1][0] = mfma16_f16(a_lo, b1[0], o8[G0 + 1][0]);
          o8[G0 + 1][1] = mfma16_f16(a_lo, b1[1], o8[G0 + 1][1]);
        });
      };
      // The three-part bf16 form: A = p d split into three exact bf16
      // parts, B = v exact in bf16.
      auto pv_bf16 = [&](auto) {
        // B holds 16 (n - 8) (Q5: 8 (q - 16)); A = p d / 16 (/ 8) undoes the
        // factor, except in tile 1 of the formats with an fp16 form, whose
        // accumulators carry 16 times their values (see that form).
        constexpr bool kT1 = kHi16;
        float pt1[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) pt1[j] = pj[j];
        if constexpr (kNib) {
#pragma unroll
          for (int j = 0; j < 4; ++j) pj[j] *= F::kBScale;  // exact
        }
        Unroll<0, NK>::run([&](auto gc) {
          constexpr int G = decltype(gc)::value;
          // Byte offset of group G in the lane's rows (swizzled by token quad).
          const int vg = (kNib ? 16 : 32) * (G ^ kq);
          float x[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)  // p * d, one v_fma_mix_f32 each
            x[j] = fmaf(pj[j], f16_bits_to_f32(dbits(j, gc)), 0.0f);
          uint2 ah, am, al;
          split3_bf16(x[0], x[1], ah.x, am.x, al.x);
          split3_bf16(x[2], x[3], ah.y, am.y, al.y);
          uint2 th = ah, tm = am, tl = al;  // tile 1's A
          if constexpr (kT1) {
            float y[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) y[j] = fmaf(pt1[j], f16_bits_to_f32(dbits(j, gc)), 0.0f);
            split3_bf16(y[0], y[1], th.x, tm.x, tl.x);
            split3_bf16(y[2], y[3], th.y, tm.y, tl.y);
          }
          auto pair = [](uint32_t f0, uint32_t f1) { return __builtin_amdgcn_perm(f1, f0, 0x07060302u); };
          uint2 b0, b1;
          if constexpr (kNib) {
            uint32_t w = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) w |= uint32_t(*reinterpret_cast<const uint8_t*>(vrow + j * RB + vg)) << (8 * j);
            uint4 t;  // tokens 4 kq + j: low nibbles (tile 0), then high (tile 1)
            if constexpr (F::kQ5) {
              // Fifth bits of element hm (low nibble) and 16 + hm (high) of
              // each token, from the group's qh words.
              uint32_t lo4 = 0u, hi4 = 0u;
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const uint32_t qh = *reinterpret_cast<const uint32_t*>(srow + j * F::kScaleRow + 4 * G) >> hm;
                lo4 |= (qh & 1u) << j;
                hi4 |= ((qh >> 16) & 1u) << j;
              }
              t = nib5_bf16(w, lo4, hi4);
            } else {
              t = nib8_bf16(w);
            }
            b0 = make_uint2(t.x, t.y);
            b1 = make_uint2(t.z, t.w);
          } else {
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = *reinterpret_cast<const uint16_t*>(vrow + j * RB + vg);
            b0 = make_uint2(pair(i8_f32<0>(w[0]), i8_f32<0>(w[1])), pair(i8_f32<0>(w[2]), i8_f32<0>(w[3])));
            b1 = make_uint2(pair(i8_f32<1>(w[0]), i8_f32<1>(w[1])), pair(i8_f32<1>(w[2]), i8_f32<1>(w[3])));
          }
          o8[G][0] = mfma16k16(ah, b0, o8[G][0]);
          o8[G][1] = mfma16k16(th, b1, o8[G][1]);
          o8[G][0] = mfma16k16(am, b0, o8[G][0]);
          o8[G][1] = mfma16k16(tm, b1, o8[G][1]);
          o8[G][0] = mfma16k16(al, b0, o8[G][0]);
          o8[G][1] = mfma16k16(tl, b1, o8[G][1]);
          // As the fallback of the fp16 form, one group at a time: its
          // register use then stays below the fp16 loop's.
          __builtin_amdgcn_sched_barrier(0);
        });
      };
      if constexpr (!decltype(bf16_only)::value)
        pv_f16(0);
      else
        pv_bf16(0);
      return true;
    };
    // Items run in the first loop while every one takes the fp16 form: its
    // accumulators then pass from item to item in place.  (A loop whose
    // items may take either form merges two sets of MFMA results at its
    // latch: the register allocator then copies every accumulator there, 64
    // moves per item, and holds both sets.)  An item that needs the bf16
    // form ends it, and that item and the partition's remaining ones run in
    // the bf16 form.
    int s = ns;
    bool redo = false;
    for (; s < S; ++s)
      if (!v_item(s, std::false_type{}, false)) {
        redo = true;
        break;
      }
    for (; s < S; ++s) {
      v_item(s, std::true_type{}, redo);
      redo = false;
    }
    // Sum over the four token rows kq of head hm.
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
  }
  if constexpr (!kQ) {
    for (int s = ns; s < S; ++s) {
      wait_item(s);
      age_fair(s);
      if (s + R - 1 < S) issue(s + R - 1);
      const int gi = s - ns;
      const int tb = (gi * NW + wave) * kGroupTok;
      char* const slot = my_ring + (s % R) * SLOT;
      if (tb + kGroupTok > nt) {
        // Rows past the partition hold a stand-in row: each lane zeroes the
        // bytes its own loads brought (this wave's LDS ops stay in order).
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          const int o = 1024 * j + 16 * lane;
          if (tb + o / RB >= nt) *reinterpret_cast<uint4*>(slot + o) = make_uint4(0u, 0u, 0u, 0u);
        }
      }
      // Probabilities of the group: computed per lane, then read back with
      // token (pair) t in lane t of every row (same-wave LDS ops stay in order).
      uint32_t pv[8];
      {
        const int i0 = tb + 2 * k_l;
        const float2 sv = *reinterpret_cast<const float2*>(sc_l + i0);
        const float p0 = (i0 < nt && !none_l) ? __builtin_amdgcn_exp2f(sv.x - m_l) : 0.0f;
        const float p1 = (i0 + 1 < nt && !none_l) ? __builtin_amdgcn_exp2f(sv.y - m_l) : 0.0f;
        if constexpr (k16) {
          const uint32_t pp = pack16<DT>(p0, p1);
          lsum += lo16<DT>(pp) + hi16<DT>(pp);
          pp_w[lane] = pp;
        } else {
          lsum += p0 + p1;
          *reinterpret_cast<float2*>(pp_w + 2 * lane) = make_float2(p0, p1);
        }
#pragma unroll
        for (int g = 0; g < 8; ++g)
          pv[g] = k16 ? pp_w[(g < GC ? g : 0) * 8 + (qk_tok & 7)] : pp_w[(g < GC ? g : 0) * 16 + qk_tok];
      }
      if constexpr (k16) {
        Unroll<0, kGroupTok / 2>::run([&](auto jc) {
          constexpr int j = decltype(jc)::value;  // token pair
          if constexpr (DPV == 2) {
            const uint32_t w0 = *reinterpret_cast<const uint32_t*>(slot + (2 * j) * RB + 4 * lane);
            const uint32_t w1 = *reinterpret_cast<const uint32_t*>(slot + (2 * j + 1) * RB + 4 * lane);
            pv_words<DT, GC, j>(acc2[0], acc2[1], pv, __builtin_amdgcn_perm(w1, w0, 0x05040100u),
                                __builtin_amdgcn_perm(w1, w0, 0x07060302u));
          } else {
            const uint2 w0 = *reinterpret_cast<const uint2*>(slot + (2 * j) * RB + 8 * lane);
            const uint2 w1 = *reinterpret_cast<const uint2*>(slot + (2 * j + 1) * RB + 8 * lane);
            pv_words<DT, GC, j>(acc2[0], acc2[1], pv, __builtin_amdgcn_perm(w1.x, w0.x, 0x05040100u),
                                __builtin_amdgcn_perm(w1.x, w0.x, 0x07060302u));
            pv_words<DT, GC, j>(acc2[2], acc2[3], pv, __builtin_amdgcn_perm(w1.y, w0.y, 0x05040100u),
                                __builtin_amdgcn_perm(w1.y, w0.y, 0x07060302u));
          }
        });
      } else {
        Unroll<0, kGroupTok>::run([&](auto tc) {
          constexpr int t = decltype(tc)::value;  // token
          if constexpr (DPV == 2) {
            const uint2 w = *reinterpret_cast<const uint2*>(slot + t * RB + 8 * lane);
            pv_words<DT, GC, t>(acc2[0], acc2[1], pv, w.x, w.y);
          } else {
            const uint4 w = *reinterpret_cast<const uint4*>(slot + t * RB + 16 * lane);
            pv_words<DT, GC, t>(acc2[0], acc2[1], pv, w.x, w.y);
            pv_words<DT, GC, t>(acc2[2], acc2[3], pv, w.z, w.w);
          }
        });
      }
    }
  }

  // ---------------- across the waves, in a fixed order -----------------------
  if constexpr (kQ) {
    if (lane < 8) s_l[wave * 8 + lane] = lsum;
  } else {
    lsum = group_sum<8>(lsum);  // the 8 lanes of head h_l
    if (k_l == 0) s_l[wave * 8 + h_l] = lsum;
  }
  lds_barrier();  // every wave is done with its ring (its last wait was vmcnt(0))
  float* const red = reinterpret_cast<float*>(smem);  // [NW][GC][D]
  if constexpr (kQ) {
    const int hm = lane & 15;
    if constexpr (kOff) {
      // M[h][G] of this wave into its probability scratch (unused on this
      // path): [8 heads][8 groups] fp32.
      float* const s_mo = reinterpret_cast<float*>(s_pp + wave * (F::kScratch / 4));
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (4 * qr_row + i < GC && hm < NK) s_mo[(4 * qr_row + i) * 8 + hm] = mo[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * qr_row + i;
      if (h < GC) {
#pragma unroll
        for (int g = 0; g < NK; ++g) {
          float* const row = &red[(wave * GC + h) * D + 32 * g];
          // The weights carried 2^11 (exact).
          if constexpr (kNib) {
            // Tile 1 of Q4_0 / Q4_1 carries a further 16 (exact).
            constexpr float kS1 = kHi16 ? 1.0f / (16.0f * kQPScale) : 1.0f / kQPScale;
            row[hm] = o8[g][0][i] * (1.0f / kQPScale);
            row[16 + hm] = o8[g][1][i] * kS1;
          } else {
            *reinterpret_cast<float2*>(row + 2 * hm) =
                make_float2(o8[g][0][i] * (1.0f / kQPScale), o8[g][1][i] * (1.0f / kQPScale));
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      float* dst = &red[(wave * GC + g) * D + DPV * lane];
      if constexpr (DPV == 2) *reinterpret_cast<float2*>(dst) = make_float2(acc2[0][g], acc2[1][g]);
      else *reinterpret_cast<float4*>(dst) = make_float4(acc2[0][g], acc2[1][g], acc2[2][g], acc2[3][g]);
    }
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
    else o = (red[i] + red[GC * D + i]) + (red[2 * GC * D + i] + red[3 * GC * D + i]);
    const int g = i / D, d = i - g * D;
    if constexpr (kOff) {  // + the offset term of dim d's group, from every wave
      const float* const s_mo = reinterpret_cast<const float*>(s_pp);
#pragma unroll
      for (int w = 0; w < NW; ++w) o += s_mo[w * (F::kScratch / 4) + g * 8 + d / 32];
    }
    a.ws_o[(part_row + int64_t(g) * a.max_parts) * D + d] = o;
  }
}

}  // namespace itkv
