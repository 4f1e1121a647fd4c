// it_decode_f16.hip -- instantiates the split-K decode kernels for F16 caches
// (kept in its own translation unit so the instantiations build in parallel).
#include "it_decode.hpp"
#include "it_decode_launch.hpp"

namespace itkv {
hipError_t launch_decode_f16(int d, int gc, const DecodeArgs& a, dim3 grid, hipStream_t s) {
  return launch_decode_typed<IT_F16>(d, gc, a, grid, s);
}
}  // namespace itkv
