// Chunked encoder.  Under construction: returns an explicit error until the
// encoder kernels land.
#include "kernels.h"

namespace hz {
hipError_t run_deflate(hipStream_t, Scratch&, const u8*, u64, u8*, u64, u32, u32*) {
  return hipErrorNotSupported;
}
hipError_t run_deflate_batch(hipStream_t, Scratch&, const u8*, u64, const BatchFile*, u32, u8*, u64,
                             u32, u32*) {
  return hipErrorNotSupported;
}
}  // namespace hz
