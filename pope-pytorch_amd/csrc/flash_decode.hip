// Split-K decode with PoPE (placeholder until the kernels land).
#include "pope_kernels.hpp"
namespace pope {
hipError_t launch_flash_decode(const DecodeParams&, int, hipStream_t) { return hipErrorInvalidValue; }
}  // namespace pope
