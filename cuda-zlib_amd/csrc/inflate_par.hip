// General-route decode (parallel).  Under construction: returns an explicit
// error until the parallel kernels land.
#include "kernels.h"

namespace hz {
hipError_t run_inflate_general(hipStream_t, Scratch&, const u8*, u64, u8*, u64, u32, u32, u32*) {
  return hipErrorNotSupported;
}
}  // namespace hz
