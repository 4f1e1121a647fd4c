// it_decode_bf16.hip -- instantiates the split-K decode kernels for BF16 caches
// (kept in its own translation unit so the instantiations build in parallel).
#include "it_decode.hpp"
#include "it_decode_launch.hpp"

namespace itkv {
hipError_t launch_decode_bf16(int d, int gc, const DecodeArgs& a, dim3 grid, hipStream_t s) {
  return launch_decode_typed<IT_BF16>(d, gc, a, grid, s);
}
}  // namespace itkv
