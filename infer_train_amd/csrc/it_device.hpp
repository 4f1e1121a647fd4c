// it_device.hpp -- gfx950 device helpers shared by the KV kernels:
// 16-bit float widening/narrowing and wave64 cross-lane reductions built on
// DPP row operations (no LDS round trip inside a 16-lane row) and
// ds_swizzle / readlane across rows.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace itkv {

// A kernel that asks for more than 64 KiB of dynamic LDS must opt in, once
// per device.  `opted` holds one bit per device (one word per kernel
// instantiation): threads that race on a first call may both set the
// idempotent attribute, and none reads a torn flag.  Devices past 63 set
// it on every launch.
inline hipError_t opt_in_lds(const void* fn, int bytes, std::atomic<uint64_t>& opted) {
  int dev = -1;
  const uint64_t bit = (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) ? uint64_t(1) << dev : 0;
  if (bit && (opted.load(std::memory_order_acquire) & bit)) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) opted.fetch_or(bit, std::memory_order_release);
  return e;
}

// ---- 16-bit float conversions ---------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
// fp32 -> fp16 with v_cvt_f16_f32 (round to nearest even, fp16 subnormals
// kept: the default MODE register of a HIP kernel).
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// ---- DPP controls (gfx9 encoding) -----------------------------------------
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i -> 7-i within 8
constexpr int kDppRowRor8 = 0x128;    // lane i -> (i+8) mod 16 within 16

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  // Every control used here reads a lane of the same row, so bound_ctrl is
  // moot; setting it lets the compiler fold the move into the consuming
  // v_add/v_max (one DPP-modified VALU op per reduction step).
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
// xor-16 within each 32-lane half: ds_swizzle bit mode (and 0x1F, xor 0x10).
__device__ __forceinline__ float swz_xor16(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x401F));
}
__device__ __forceinline__ float swap_halves(float x) {
  // lane i <-> lane i^32 (ds_bpermute through the LDS crossbar, no memory).
  int lane = __lane_id();
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, x)));
}

// Sum over aligned groups of N lanes (N = 1..64, power of two); every lane
// of a group receives the group's sum.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += dpp_f<kDppQuadXor1>(x);
  if constexpr (N >= 4) x += dpp_f<kDppQuadXor2>(x);
  if constexpr (N >= 8) x += dpp_f<kDppHalfMirror>(x);
  if constexpr (N >= 16) x += dpp_f<kDppRowRor8>(x);
  if constexpr (N >= 32) x += swz_xor16(x);
  if constexpr (N >= 64) x += swap_halves(x);
  return x;
}
template <int N>
__device__ __forceinline__ float group_max(float x) {
  if constexpr (N >= 2) x = fmaxf(x, dpp_f<kDppQuadXor1>(x));
  if constexpr (N >= 4) x = fmaxf(x, dpp_f<kDppQuadXor2>(x));
  if constexpr (N >= 8) x = fmaxf(x, dpp_f<kDppHalfMirror>(x));
  if constexpr (N >= 16) x = fmaxf(x, dpp_f<kDppRowRor8>(x));
  if constexpr (N >= 32) x = fmaxf(x, swz_xor16(x));
  if constexpr (N >= 64) x = fmaxf(x, swap_halves(x));
  return x;
}

// Load helpers: 16-byte vector loads/stores on raw byte addresses.
__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }
// Streaming 16-byte accesses (nt: not kept in L2).  Measured on the data
// movers: nt loads make the bf16 page gather 26% faster (and the quantised
// gather, which reads 32-byte group pieces, 30% slower); nt stores help only
// the append's scattered row stores (2%) and slow contiguous or zeroing
// stores.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld16_nt(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st16_nt(void* p, uint4 v) {
  const u32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
}

}  // namespace itkv
