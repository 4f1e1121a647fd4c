// it_decode_launch.hpp -- compile-time dispatch of paged_decode_split over
// head_dim (128, 256), heads per workgroup (1..8) and launch shape.
#pragma once
#include "it_decode.hpp"
#include "it_decode_split.hpp"

namespace itkv {
// Largest dynamic LDS a decode workgroup may ask for (160 KiB per CU).
constexpr size_t kMaxDecodeLds = 160 * 1024;

// Dynamic LDS of the split launch that serves these arguments.
inline size_t decode_smem_bytes(int32_t dt, int gc, int d, int partition, int max_pages, int64_t n_workgroups) {
  const SplitShape sh = split_shape(dt, d, gc, partition, max_pages, n_workgroups);
  return split_lds_bytes(dt, d, gc, partition, max_pages, sh.nw, sh.ring);
}

template <int DT, int D, int GC, int NW, int R>
hipError_t launch_split_shape(const DecodeArgs& a, dim3 grid, size_t smem, hipStream_t s) {
  if (smem > 64 * 1024) {
    static std::atomic<uint64_t> opted{0};
    const hipError_t e = opt_in_lds(reinterpret_cast<const void*>(&paged_decode_split<DT, D, GC, NW, R>),
                                    int(kMaxDecodeLds), opted);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((paged_decode_split<DT, D, GC, NW, R>), grid, dim3(64 * NW), smem, s, a);
  return hipGetLastError();
}

template <int DT, int D, int GC>
hipError_t launch_decode_gc(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  const int64_t n_wg = int64_t(grid.x) * grid.y * grid.z;
  const SplitShape sh = split_shape(DT, D, GC, a.partition, a.max_pages, n_wg);
  const size_t smem = split_lds_bytes(DT, D, GC, a.partition, a.max_pages, sh.nw, sh.ring);
  if (smem > kMaxDecodeLds) return hipErrorInvalidValue;
  if (sh.nw == 2) return launch_split_shape<DT, D, GC, 2, 2>(a, grid, smem, s);
  if (sh.ring == 4) return launch_split_shape<DT, D, GC, 4, 4>(a, grid, smem, s);
  if (sh.ring == 3) return launch_split_shape<DT, D, GC, 4, 3>(a, grid, smem, s);
  return launch_split_shape<DT, D, GC, 4, 2>(a, grid, smem, s);
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
hipError_t launch_decode_q4_0(int d, int gc, const DecodeArgs& a, dim3 grid, hipStream_t s);
hipError_t launch_decode_q4_1(int d, int gc, const DecodeArgs& a, dim3 grid, hipStream_t s);
hipError_t launch_decode_q5_0(int d, int gc, const DecodeArgs& a, dim3 grid, hipStream_t s);
hipError_t launch_decode_q5_1(int d, int gc, const DecodeArgs& a, dim3 grid, hipStream_t s);
}  // namespace itkv
