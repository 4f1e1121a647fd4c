// it_decode_launch.hpp -- compile-time dispatch of paged_decode_split over
// head_dim (128, 256) and heads per workgroup (1..8).
#pragma once
#include "it_decode.hpp"

namespace itkv {
template <int DT, int D>
hipError_t launch_decode_d(int gc, const DecodeArgs& a, dim3 grid, size_t smem, hipStream_t s) {
  switch (gc) {
#define IT_GC_CASE(G) \
  case G: hipLaunchKernelGGL((paged_decode_split<DT, D, G>), grid, dim3(kDecodeThreads), smem, s, a); break;
    IT_GC_CASE(1) IT_GC_CASE(2) IT_GC_CASE(3) IT_GC_CASE(4)
    IT_GC_CASE(5) IT_GC_CASE(6) IT_GC_CASE(7) IT_GC_CASE(8)
#undef IT_GC_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int DT>
hipError_t launch_decode_typed(int d, int gc, const DecodeArgs& a, dim3 grid, size_t smem, hipStream_t s) {
  if (d == 128) return launch_decode_d<DT, 128>(gc, a, grid, smem, s);
  if (d == 256) return launch_decode_d<DT, 256>(gc, a, grid, smem, s);
  return hipErrorInvalidValue;
}

hipError_t launch_decode_bf16(int d, int gc, const DecodeArgs& a, dim3 grid, size_t smem, hipStream_t s);
hipError_t launch_decode_f16(int d, int gc, const DecodeArgs& a, dim3 grid, size_t smem, hipStream_t s);
hipError_t launch_decode_f32(int d, int gc, const DecodeArgs& a, dim3 grid, size_t smem, hipStream_t s);
hipError_t launch_decode_q8_0(int d, int gc, const DecodeArgs& a, dim3 grid, size_t smem, hipStream_t s);
}  // namespace itkv
