// it_quant.hpp -- the per-group KV quantisers shared by the append kernels
// (slot-mapped append and RoPE-then-append), device code.
//
// Eight consecutive lanes own one 32-element group of a token row, four
// floats each (lane l8 holds elements 4 l8 .. 4 l8 + 3).  Every lane of the
// group must make the call, live or not: the group reductions are DPP moves.
//
//  Q8_0  quantize_row_q8_0 (src/backend/arm/quant.rs:149-183, x86 path):
//        amax ignoring NaN, scale = amax / 127 (IEEE division), q =
//        roundf(x / scale) saturated to int8 (NaN -> 0), d = fp16(scale).
//  Q4_0  ggml's quantize_row_q4_0_ref (the reference carries the block,
//        types.rs:15-22, and its dequantisation, vec_dot.rs:425-440, but no
//        quantiser): max = the first element of largest magnitude, d =
//        max / -8, id = d ? 1/d : 0, nibble = min(15, (int8_t)(x id + 8.5f)).
//  Q4_1  ggml's quantize_row_q4_1_ref (the reference has only the block,
//        types.rs:24-32): min / max (strict compares: NaN never wins, the
//        first of equal values stays), d = (max - min) / 15, nibble =
//        min(15, (int8_t)((x - min) id + 0.5f)), d and m = min as fp16.
//  Q5_0  ggml's quantize_row_q5_0_ref (the reference has only the type id,
//        types.rs:116): Q4_0's max, d = max / -16, q = min(31, (int8_t)(x id
//        + 16.5f)).
//  Q5_1  ggml's quantize_row_q5_1_ref (types.rs:117): Q4_1's min / max, d =
//        (max - min) / 31, q = (uint8_t)((x - min) id + 0.5f), no clamp.
// Q4/Q5 products and sums are rounded separately (no FMA: this library
// builds with -ffp-contract=fast), and (int8_t) / (uint8_t) of NaN or an
// out-of-range value is 0, as x86's cvttss2si gives; byte j = nibble j |
// nibble (j + 16) << 4 (the low four bits of a Q5 value), and Q5's u32 qh
// holds bit 4 of element e's value at bit e.
#pragma once
#include <hip/hip_runtime.h>

#include <cfloat>
#include <type_traits>

#include "it_device.hpp"
#include "it_kv.h"

namespace itkv {

// fp32 -> fp16 bits as the oracle's (and the `half` crate's) from_f32:
// round to nearest even, subnormals kept, NaN quieted with its top payload.
__device__ __forceinline__ uint32_t f16_bits_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return ((u >> 16) & 0x8000u) | 0x7E00u | ((u & 0x7FFFFFu) >> 13);
  return f32_to_f16_bits(f);
}

// A rounded float32 product the compiler cannot fuse into an FMA.
__device__ __forceinline__ float mul_rn(float a, float b) {
  float r;
  asm("v_mul_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// What a lane stores: `qs` at its place in the group's main-plane bytes
// (Q8_0: four int8 at byte 4 l8; Q4 / Q5: four bytes at byte 4 l8, lanes
// 0-3 only) and, from lane 0, the group's scale word `meta` (Q8_0 / Q4_0 /
// Q5_0: fp16 d; Q4_1 / Q5_1: fp16 d | fp16 m << 16) and Q5's `qh`.
struct QuantGroup {
  uint32_t qs, meta, qh;
};

// Where the 4- and 5-bit formats keep a group's words in a page of bs rows:
// the nibble plane u8 [bs][d / 2], then per token a side row of
// (Q5 only) d/32 u32 qh words, then d/32 metadata words (fp16 d, or the
// (d, m) pair as one u32).
template <int DT>
struct NibFmt {
  static constexpr bool kQ5 = DT == IT_Q5_0 || DT == IT_Q5_1;
  static constexpr bool kMin = DT == IT_Q4_1 || DT == IT_Q5_1;     // (d, m) pairs
  static constexpr int kMeta = kMin ? 4 : 2;                        // metadata bytes per group
  static constexpr int kSide = kMeta + (kQ5 ? 4 : 0);               // side-row bytes per group
  static constexpr int kRecord = 16 + kSide;                        // ggml block bytes
  __host__ __device__ static constexpr int meta_off(int ng) { return kQ5 ? 4 * ng : 0; }
};

__device__ __forceinline__ int32_t q8_round(float x, float scale) {
  // quant.rs:176-178: (x / scale).round() as i32, clamped to [-128, 127];
  // IEEE division, round half away from zero, NaN -> 0 (Rust's saturating as).
  float r = roundf(x / scale);
  if (r != r) return 0;
  r = fminf(fmaxf(r, -128.0f), 127.0f);
  return int32_t(r);
}

// Whether a group's scale takes the fast quotient below: a normal scale
// whose reciprocal is normal too (amax 0, inf, NaN-free tiny or huge groups
// take the IEEE division for every element).
__device__ __forceinline__ bool q8_fast_scale(float scale) { return scale >= 0x1p-120f && scale <= 0x1p120f; }

// Why q8's fast path is exact: for |x| <= 127 scale (x an element of the
// group whose amax set the scale) and rs = v_rcp_f32(scale) (1 ulp), x rs
// lies within 127 (2^-23 + 2^-24) < 3.1e-5 of x / scale, and so does the
// IEEE quotient fl(x / scale) (within 127 2^-24).  When x rs is farther
// than 0.4999 from a half-integer, both lie strictly inside the unit
// interval around n = rint(x rs), so round(fl(x / scale)) = n, and |n| <=
// 127 needs no clamp.  Otherwise (near a tie, or NaN) the IEEE division
// decides.

// (int8_t)(r) and (uint8_t)(r) as ggml's x86 build computes them: truncate
// to int32 (NaN and out-of-range give 0x80000000), keep the low byte.
__device__ __forceinline__ int32_t trunc_i8(float r) {
  if (!(fabsf(r) < 2147483648.0f)) return 0;
  return int32_t(int8_t(int32_t(r)));
}
__device__ __forceinline__ int32_t trunc_u8(float r) {
  if (!(fabsf(r) < 2147483648.0f)) return 0;
  return int32_t(uint8_t(int32_t(r)));
}
// Q4's min(15, (int8_t)r), low byte.
__device__ __forceinline__ uint32_t q4_nibble(float r) { return uint32_t(min(trunc_i8(r), 15)) & 0xFFu; }

// The value of largest magnitude in an 8-lane group of four floats per lane
// (equal magnitudes: the lower element index; NaN never wins; none: 0).
__device__ __forceinline__ float group_absmax_first(const float (&xs)[4], int l8) {
  float am = 0.0f, mx = 0.0f;
  int im = 32;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a = fabsf(xs[e]);
    if (am < a) am = a, mx = xs[e], im = 4 * l8 + e;
  }
  auto step = [&](auto ctrl) {
    constexpr int C = decltype(ctrl)::value;
    const float a2 = dpp_f<C>(am), m2 = dpp_f<C>(mx);
    const int i2 = __builtin_amdgcn_mov_dpp(im, C, 0xF, 0xF, true);
    if (a2 > am || (a2 == am && i2 < im)) am = a2, mx = m2, im = i2;
  };
  step(std::integral_constant<int, kDppQuadXor1>{});
  step(std::integral_constant<int, kDppQuadXor2>{});
  step(std::integral_constant<int, kDppHalfMirror>{});
  return mx;
}

// Min and max of an 8-lane group (strict compares: NaN never wins, the
// first of equal values stays; FLT_MAX / -FLT_MAX when every element is NaN).
__device__ __forceinline__ void group_minmax(const float (&xs)[4], int l8, float& mn, float& mx) {
  mn = FLT_MAX, mx = -FLT_MAX;
  int imn = 32, imx = 32;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (xs[e] < mn) mn = xs[e], imn = 4 * l8 + e;
    if (xs[e] > mx) mx = xs[e], imx = 4 * l8 + e;
  }
  auto step = [&](auto ctrl) {
    constexpr int C = decltype(ctrl)::value;
    const float mn2 = dpp_f<C>(mn), mx2 = dpp_f<C>(mx);
    const int imn2 = __builtin_amdgcn_mov_dpp(imn, C, 0xF, 0xF, true);
    const int imx2 = __builtin_amdgcn_mov_dpp(imx, C, 0xF, 0xF, true);
    if (mn2 < mn || (mn2 == mn && imn2 < imn)) mn = mn2, imn = imn2;
    if (mx2 > mx || (mx2 == mx && imx2 < imx)) mx = mx2, imx = imx2;
  };
  step(std::integral_constant<int, kDppQuadXor1>{});
  step(std::integral_constant<int, kDppQuadXor2>{});
  step(std::integral_constant<int, kDppHalfMirror>{});
}

// OR of a word over an 8-lane group.
__device__ __forceinline__ uint32_t group_or8(uint32_t v) {
  v |= uint32_t(__builtin_amdgcn_mov_dpp(int(v), kDppQuadXor1, 0xF, 0xF, true));
  v |= uint32_t(__builtin_amdgcn_mov_dpp(int(v), kDppQuadXor2, 0xF, 0xF, true));
  v |= uint32_t(__builtin_amdgcn_mov_dpp(int(v), kDppHalfMirror, 0xF, 0xF, true));
  return v;
}

template <int DT>
__device__ __forceinline__ QuantGroup quant_group(float4 x, int l8) {
  const float xs[4] = {x.x, x.y, x.z, x.w};
  QuantGroup out{0u, 0u, 0u};
  if constexpr (DT == IT_Q8_0) {
    // amax (quant.rs:157-163, NaN ignored): an unsigned max of |x|'s bit
    // patterns orders every non-NaN value as fp32 does; a group holding a
    // NaN (bits above inf's; the max is group-uniform) takes the NaN-
    // skipping float max instead.
    const uint32_t kAbs = 0x7FFFFFFFu;
    uint32_t mb = max(max(__float_as_uint(x.x) & kAbs, __float_as_uint(x.y) & kAbs),
                      max(__float_as_uint(x.z) & kAbs, __float_as_uint(x.w) & kAbs));
    mb = max(mb, uint32_t(__builtin_amdgcn_mov_dpp(int(mb), kDppQuadXor1, 0xF, 0xF, true)));
    mb = max(mb, uint32_t(__builtin_amdgcn_mov_dpp(int(mb), kDppQuadXor2, 0xF, 0xF, true)));
    mb = max(mb, uint32_t(__builtin_amdgcn_mov_dpp(int(mb), kDppHalfMirror, 0xF, 0xF, true)));
    float amax = __uint_as_float(mb);
    if (mb > 0x7F800000u) {
      auto absn = [](float f) { return f == f ? fabsf(f) : 0.0f; };
      amax = group_max<8>(fmaxf(fmaxf(absn(x.x), absn(x.y)), fmaxf(absn(x.z), absn(x.w))));
    }
    if (amax != 0.0f) {  // quant.rs:166-170: an all-zero group stores d = 0, qs = 0
      // scale = amax / 127 (quant.rs:173): for a normal amax, a faithful
      // quotient and one exact-remainder correction give the IEEE quotient
      // (checked over every positive normal float on the host).
      constexpr float kR127 = 1.0f / 127.0f;
      float scale;
      if (amax >= 0x1p-100f && amax <= 0x1p100f) {
        const float y = mul_rn(amax, kR127);
        scale = fmaf(fmaf(-127.0f, y, amax), kR127, y);
      } else {
        scale = amax / 127.0f;
      }
      bool exact = !q8_fast_scale(scale);
      if (!exact) {
        // q = round(x / scale) (quant.rs:176-178) through rs = v_rcp_f32:
        // f = fma(x, rs, 1.5 2^23) holds n = rint(x rs) in its low byte
        // (as an int8), and |x rs - n| < 0.4999 makes n = round(fl(x /
        // scale)) (the argument above; sampled on the host too).
        const float rs = __builtin_amdgcn_rcpf(scale);
        constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23
        uint32_t fb[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float f = fmaf(xs[e], rs, kMagic);
          if (!(fabsf(fmaf(xs[e], rs, kMagic - f)) < 0.4999f)) exact = true;
          fb[e] = __float_as_uint(f);
        }
        out.qs = __builtin_amdgcn_perm(fb[1], fb[0], 0x0C0C0400u) | __builtin_amdgcn_perm(fb[3], fb[2], 0x04000C0Cu);
      }
      if (exact) {  // rare: a near-tie, a NaN, or a scale outside the fast range
        out.qs = 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e) out.qs |= (uint32_t(q8_round(xs[e], scale)) & 0xFFu) << (8 * e);
      }
      out.meta = f16_bits_rne(scale);
    }
  } else if constexpr (DT == IT_Q4_0) {
    const float d = group_absmax_first(xs, l8) / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) out.qs |= q4_nibble(mul_rn(xs[e], id) + 8.5f) << (8 * e);
    out.meta = f16_bits_rne(d);
  } else if constexpr (DT == IT_Q4_1) {
    float mn, mx;
    group_minmax(xs, l8, mn, mx);
    const float d = (mx - mn) / 15.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) out.qs |= q4_nibble(mul_rn(xs[e] - mn, id) + 0.5f) << (8 * e);
    out.meta = f16_bits_rne(d) | (f16_bits_rne(mn) << 16);
  } else {
    static_assert(DT == IT_Q5_0 || DT == IT_Q5_1, "Q8_0, Q4_0, Q4_1, Q5_0 or Q5_1");
    int32_t q[4];
    if constexpr (DT == IT_Q5_0) {
      const float d = group_absmax_first(xs, l8) / -16.0f;
      const float id = d != 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) q[e] = min(trunc_i8(mul_rn(xs[e], id) + 16.5f), 31);
      out.meta = f16_bits_rne(d);
    } else {
      float mn, mx;
      group_minmax(xs, l8, mn, mx);
      const float d = (mx - mn) / 31.0f;
      const float id = d != 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) q[e] = trunc_u8(mul_rn(xs[e] - mn, id) + 0.5f);
      out.meta = f16_bits_rne(d) | (f16_bits_rne(mn) << 16);
    }
    uint32_t hb = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      out.qs |= (uint32_t(q[e]) & 0xFu) << (8 * e);
      hb |= ((uint32_t(q[e]) >> 4) & 1u) << e;
    }
    out.qh = group_or8(hb << (4 * l8));
  }
  if constexpr (DT != IT_Q8_0) {
    // Lane i < 4 of the group takes lane i + 4's bytes (DPP row_shl:4):
    // byte j of the group = nibble j | nibble (j + 16) << 4.
    const uint32_t partner = uint32_t(__builtin_amdgcn_mov_dpp(int(out.qs), 0x104, 0xF, 0xF, true));
    out.qs |= (partner & 0x0F0F0F0Fu) << 4;
  }
  return out;
}

// Store a lane's part of a group into its page: token row `off` of a page of
// bs rows, head_dim d, vector cv of the row (group cv / 8, lane cv % 8).
template <int DT>
__device__ __forceinline__ void store_group(char* page, int64_t off, int64_t bs, int d, int cv, QuantGroup q) {
  const int g = cv >> 3, l8 = cv & 7;
  if constexpr (DT == IT_Q8_0) {
    *reinterpret_cast<uint32_t*>(page + off * d + cv * 4) = q.qs;
    if (l8 == 0) *reinterpret_cast<uint16_t*>(page + bs * d + (off * (d >> 5) + g) * 2) = uint16_t(q.meta);
  } else {
    using N = NibFmt<DT>;
    if (l8 < 4) *reinterpret_cast<uint32_t*>(page + off * (d >> 1) + g * 16 + l8 * 4) = q.qs;
    if (l8 == 0) {
      const int ng = d >> 5;
      char* const side = page + bs * (d >> 1) + off * (ng * N::kSide);
      if constexpr (N::kQ5) *reinterpret_cast<uint32_t*>(side + 4 * g) = q.qh;
      if constexpr (N::kMin)
        *reinterpret_cast<uint32_t*>(side + N::meta_off(ng) + 4 * g) = q.meta;
      else
        *reinterpret_cast<uint16_t*>(side + N::meta_off(ng) + 2 * g) = uint16_t(q.meta);
    }
  }
}

}  // namespace itkv
