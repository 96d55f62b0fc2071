// Q8_0 skinny GEMM (placeholder launcher until the kernel lands).
#include "../launch.hpp"
namespace uk {
hipError_t launch_q8_gemm(const Plan&, const void*, const void*, float*, int64_t, int64_t, int64_t, hipStream_t) {
  return hipErrorNotSupported;
}
}  // namespace uk
