// Small helper kernels: buffer fill and metadata writes.  The library clears
// memory with its own kernels (never a memset node) so its launches stay valid
// under HIP graph capture.
#include <atomic>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "kernels.h"

namespace hz {

namespace {
struct ProfileEntry {
  std::string name;
  hipEvent_t start, stop;
};
struct ProfileRegistry {
  std::atomic<bool> enabled{false};
  std::mutex mutex;
  std::vector<ProfileEntry> entries;
};
ProfileRegistry& profile_registry() {
  static ProfileRegistry* r = new ProfileRegistry;
  return *r;
}
}  // namespace

bool profiling_enabled() { return profile_registry().enabled.load(std::memory_order_relaxed); }

void profile_record(const char* name, hipEvent_t start, hipEvent_t stop) {
  ProfileRegistry& r = profile_registry();
  std::lock_guard<std::mutex> lock(r.mutex);
  r.entries.push_back({name, start, stop});
}

// Collect recorded launches into "name launches total_ms\n" lines, grouped by
// kernel in first-seen order; waits for each recorded stop event.
std::string profile_collect(bool reset) {
  ProfileRegistry& r = profile_registry();
  std::lock_guard<std::mutex> lock(r.mutex);
  std::vector<std::string> names;
  std::vector<double> totals;
  std::vector<unsigned long long> counts;
  for (const ProfileEntry& e : r.entries) {
    float ms = 0.f;
    if (hipEventSynchronize(e.stop) == hipSuccess) (void)hipEventElapsedTime(&ms, e.start, e.stop);
    size_t i = 0;
    while (i < names.size() && names[i] != e.name) ++i;
    if (i == names.size()) {
      names.push_back(e.name);
      totals.push_back(0.0);
      counts.push_back(0);
    }
    totals[i] += ms;
    counts[i] += 1;
  }
  if (reset) {
    for (const ProfileEntry& e : r.entries) {
      (void)hipEventDestroy(e.start);
      (void)hipEventDestroy(e.stop);
    }
    r.entries.clear();
  }
  std::string out;
  char line[256];
  for (size_t i = 0; i < names.size(); ++i) {
    std::snprintf(line, sizeof line, "%s %llu %.6f\n", names[i].c_str(), counts[i], totals[i]);
    out += line;
  }
  return out;
}

void profile_enable(bool on) { profile_registry().enabled.store(on); }

__global__ void fill_kernel(u8* dst, u8 value, u64 bytes) {
  const u64 tid = u64(blockIdx.x) * blockDim.x + threadIdx.x;
  const u64 stride = u64(gridDim.x) * blockDim.x;
  // Byte head up to 16-byte alignment, then 16-byte stores, then the tail.
  const uintptr_t addr = reinterpret_cast<uintptr_t>(dst);
  u64 head = (16 - (addr & 15)) & 15;
  if (head > bytes) head = bytes;
  for (u64 i = tid; i < head; i += stride) dst[i] = value;
  const u64 vec = (bytes - head) / 16;
  uint4* v = reinterpret_cast<uint4*>(dst + head);
  const u32 w = 0x01010101u * value;
  const uint4 pattern = make_uint4(w, w, w, w);
  for (u64 i = tid; i < vec; i += stride) v[i] = pattern;
  for (u64 i = head + vec * 16 + tid; i < bytes; i += stride) dst[i] = value;
}

__global__ void set_meta_kernel(u32* meta, u64 rows, u32 first, u32 second) {
  const u64 tid = u64(blockIdx.x) * blockDim.x + threadIdx.x;
  const u64 stride = u64(gridDim.x) * blockDim.x;
  for (u64 i = tid; i < rows; i += stride) {
    meta[2 * i] = first;
    meta[2 * i + 1] = second;
  }
}

hipError_t launch_fill(hipStream_t stream, void* dst, u8 value, u64 bytes) {
  if (!bytes) return hipSuccess;
  u64 blocks = (bytes / 16 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 2048) blocks = 2048;
  HZ_LAUNCH(fill_kernel, dim3(u32(blocks)), dim3(256), 0, stream,
                     static_cast<u8*>(dst), value, bytes);
  return hipGetLastError();
}

hipError_t launch_set_meta_rows(hipStream_t stream, u32* meta, u64 rows, u32 first, u32 second) {
  if (!rows) return hipSuccess;
  u64 blocks = (rows + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  HZ_LAUNCH(set_meta_kernel, dim3(u32(blocks)), dim3(256), 0, stream, meta, rows, first,
                     second);
  return hipGetLastError();
}

hipError_t launch_set_meta(hipStream_t stream, u32* meta, u32 first, u32 second) {
  return launch_set_meta_rows(stream, meta, 1, first, second);
}

}  // namespace hz
