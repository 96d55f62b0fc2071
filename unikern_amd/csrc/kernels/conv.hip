// Implicit-GEMM conv (placeholder launcher until the kernel lands).
#include "../launch.hpp"
namespace uk {
hipError_t launch_conv_igemm(const Plan&, const Shape&, Layout, const float*, const float*, const float*, float*,
                             hipStream_t) {
  return hipErrorNotSupported;
}
}  // namespace uk
