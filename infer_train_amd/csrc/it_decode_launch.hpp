// it_decode_launch.hpp -- compile-time dispatch of paged_decode_split over
// head_dim (128, 256) and heads per workgroup (1..8).
#pragma once
#include "it_decode.hpp"

namespace itkv {
// Largest dynamic LDS a decode workgroup may ask for (160 KiB per CU).
constexpr size_t kMaxDecodeLds = 160 * 1024;

template <int DT, int D, int GC>
hipError_t launch_decode_gc(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  const size_t smem = decode_lds_bytes(DT, GC, D, a.partition, a.max_pages);
  if (smem > kMaxDecodeLds) return hipErrorInvalidValue;
  if (smem > 64 * 1024) {
    // Above 64 KiB the kernel must opt in.  Idempotent, so a race between
    // threads setting it is harmless.
    static bool opted = false;
    if (!opted) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&paged_decode_split<DT, D, GC>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, int(kMaxDecodeLds));
      if (e != hipSuccess) return e;
      opted = true;
    }
  }
  hipLaunchKernelGGL((paged_decode_split<DT, D, GC>), grid, dim3(kDecodeThreads), smem, s, a);
  return hipGetLastError();
}

template <int DT, int D>
hipError_t launch_decode_d(int gc, const DecodeArgs& a, dim3 grid, hipStream_t s) {
  switch (gc) {
#define IT_GC_CASE(G) \
  case G: return launch_decode_gc<DT, D, G>(a, grid, s);
    IT_GC_CASE(1) IT_GC_CASE(2) IT_GC_CASE(3) IT_GC_CASE(4)
    IT_GC_CASE(5) IT_GC_CASE(6) IT_GC_CASE(7) IT_GC_CASE(8)
#undef IT_GC_CASE
    default: return hipErrorInvalidValue;
  }
}

template <int DT>
hipError_t launch_decode_typed(int d, int gc, const DecodeArgs& a, dim3 grid, hipStream_t s) {
  if (d == 128) return launch_decode_d<DT, 128>(gc, a, grid, s);
  if (d == 256) return launch_decode_d<DT, 256>(gc, a, grid, s);
  return hipErrorInvalidValue;
}

hipError_t launch_decode_bf16(int d, int gc, const DecodeArgs& a, dim3 grid, hipStream_t s);
hipError_t launch_decode_f16(int d, int gc, const DecodeArgs& a, dim3 grid, hipStream_t s);
hipError_t launch_decode_f32(int d, int gc, const DecodeArgs& a, dim3 grid, hipStream_t s);
hipError_t launch_decode_q8_0(int d, int gc, const DecodeArgs& a, dim3 grid, hipStream_t s);
}  // namespace itkv
