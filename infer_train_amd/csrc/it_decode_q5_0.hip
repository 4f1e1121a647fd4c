// it_decode_q5_0.hip -- instantiates the split-K decode kernels for Q5_0 caches
// (kept in its own translation unit so the instantiations build in parallel).
#include "it_decode.hpp"
#include "it_decode_launch.hpp"

namespace itkv {
hipError_t launch_decode_q5_0(int d, int gc, const DecodeArgs& a, dim3 grid, hipStream_t s) {
  return launch_decode_typed<IT_Q5_0>(d, gc, a, grid, s);
}
}  // namespace itkv
