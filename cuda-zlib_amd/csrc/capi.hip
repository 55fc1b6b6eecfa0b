// C-ABI entry points and the per-device workspace pool.
//
// Mirrors the reference's XLA FFI handlers and plain C exports
// (src/cuda_zlib/native/codec_ffi.cu:132-273, 958-1182): ABI-shape errors are
// returned, data errors go to the metadata buffer, scratch comes from one
// stream-ordered hipMemPool per device, and no call synchronises with the host.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/hip_zlib.h"
#include "kernels.h"

namespace hz {
namespace {

thread_local std::string g_last_error;

struct PoolEntry {
  int device;
  hipMemPool_t pool;
};

// A device buffer that calls carve their scratch from, kept between calls:
// a call takes an idle arena of its device whose last use was on the call's
// own stream or is already done (so that a call never waits for work on
// another stream), makes its stream wait for that use, and records its own
// use when it ends, so reuse needs no allocation and no host synchronisation.
struct Arena {
  int device;
  u8* base;
  u64 capacity;
  hipEvent_t last_use;
  hipStream_t last_stream;
  bool busy;
};

// A pinned host buffer for uploads (upload_to_device).
struct PinnedStage {
  void* host;
  u64 bytes;
  hipEvent_t done;  // recorded after the last copy out of it
  bool taken;
};

struct PoolRegistry {
  std::mutex mutex;
  std::vector<PoolEntry> pools;
  std::vector<PinnedStage> stages;
  std::vector<std::unique_ptr<Arena>> arenas;
  u64 retention = 1ull << 30;
};

// Process-lifetime registry; deliberately leaked so no HIP call runs at exit.
PoolRegistry& registry() {
  static PoolRegistry* r = new PoolRegistry;
  return *r;
}

hipError_t get_pool(int device, hipMemPool_t* out) {
  PoolRegistry& reg = registry();
  std::lock_guard<std::mutex> lock(reg.mutex);
  for (const PoolEntry& e : reg.pools)
    if (e.device == device) { *out = e.pool; return hipSuccess; }
  hipMemPoolProps props = {};
  props.allocType = hipMemAllocationTypePinned;
  props.handleTypes = hipMemHandleTypeNone;
  props.location.type = hipMemLocationTypeDevice;
  props.location.id = device;
  hipMemPool_t pool = nullptr;
  hipError_t err = hipMemPoolCreate(&pool, &props);
  if (err != hipSuccess) return err;
  u64 threshold = reg.retention;
  err = hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &threshold);
  if (err != hipSuccess) return err;
  // No reuse that would make one caller's stream wait for another's work
  // (memory freed on a stream whose work is still queued is not handed to
  // another stream).
  int no_waits = 0;
  err = hipMemPoolSetAttribute(pool, hipMemPoolReuseAllowInternalDependencies, &no_waits);
  if (err != hipSuccess) return err;
  reg.pools.push_back({device, pool});
  *out = pool;
  return hipSuccess;
}


}  // namespace

hipError_t upload_to_device(hipStream_t stream, void* dst, const void* src, u64 bytes) {
  if (!bytes) return hipSuccess;
  PoolRegistry& reg = registry();
  std::unique_lock<std::mutex> lock(reg.mutex);
  PinnedStage* stage = nullptr;
  for (PinnedStage& e : reg.stages)
    if (!e.taken && e.bytes >= bytes && hipEventQuery(e.done) == hipSuccess) {
      stage = &e;
      break;
    }
  if (!stage) {
    PinnedStage e = {nullptr, std::max<u64>(bytes, 64 << 10), nullptr, false};
    hipError_t err = hipHostMalloc(&e.host, e.bytes, hipHostMallocDefault);
    if (err != hipSuccess) return err;
    err = hipEventCreateWithFlags(&e.done, hipEventDisableTiming);
    if (err != hipSuccess) {
      (void)hipHostFree(e.host);
      return err;
    }
    reg.stages.push_back(e);
    stage = &reg.stages.back();
  }
  stage->taken = true;
  void* host = stage->host;
  hipEvent_t done = stage->done;
  const size_t index = size_t(stage - reg.stages.data());
  lock.unlock();
  std::memcpy(host, src, bytes);
  hipError_t err = hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, stream);
  if (err == hipSuccess) err = hipEventRecord(done, stream);
  lock.lock();
  // Given back only once its copy is ordered before `done` (else kept out of use).
  if (err == hipSuccess) reg.stages[index].taken = false;
  return err;
}

namespace {

bool find_pool(int device, hipMemPool_t* out) {
  PoolRegistry& reg = registry();
  std::lock_guard<std::mutex> lock(reg.mutex);
  for (const PoolEntry& e : reg.pools)
    if (e.device == device) { *out = e.pool; return true; }
  return false;
}

// Makes the stream's device current for the duration of a call.
class DeviceScope {
 public:
  hipError_t enter(hipStream_t stream) {
    hipError_t err = hipGetDevice(&previous_);
    if (err != hipSuccess) return err;
    int device = previous_;
    if (stream) {
      err = hipStreamGetDevice(stream, &device);
      if (err != hipSuccess) return err;
    }
    device_ = device;
    if (device != previous_) {
      err = hipSetDevice(device);
      if (err != hipSuccess) return err;
      switched_ = true;
    }
    return hipSuccess;
  }
  ~DeviceScope() {
    if (switched_) (void)hipSetDevice(previous_);
  }
  int device() const { return device_; }

 private:
  int previous_ = 0, device_ = 0;
  bool switched_ = false;
};

constexpr u64 kArenaGranule = 64ull << 20;
// Batch files of at least this many output bytes decode by parallel slices
// (a workgroup per file, in one launch beside the largest files); smaller
// ones by the serial one-wave decoder first.  With 256 the 4096-file batch
// took 1.14 ms, with 32 1.05 ms: the serial decoder's slowest small file
// (a lane-0 token loop) no longer precedes the parallel launch.
constexpr u64 kBatchWideBytes = 32;
// Single streams of the small route with at least this many output bytes are
// decoded by the parallel route first; the serial one-wave decoder (the
// reference's small route, codec_ffi.cu:681-693) runs only when that reports
// a failure, to give its status and its failed output (decoded prefix, then
// zeros).  Below it the serial decoder alone is faster than the launches.
constexpr u64 kSmallParallelBytes = 256;

// Stream-ordered scratch for one call, carved from an arena of the device
// (taken on the first allocation).  Requests the arena cannot hold come from
// the pool and are freed (stream-ordered) when the call ends; the arena is
// then grown to the call's total for later calls, within the retention
// budget.  Results stay valid for later work on the stream.
class Workspace final : public Scratch {
 public:
  Workspace(hipStream_t stream, hipMemPool_t pool, int device)
      : stream_(stream), pool_(pool), device_(device) {}
  int device() const { return device_; }
  hipError_t alloc_bytes(void** p, u64 bytes) override {
    *p = nullptr;
    bytes = scratch_round(bytes);
    if (!acquired_) {
      hipError_t err = acquire();
      if (err != hipSuccess) return err;
    }
    total_ += bytes;
    if (arena_ && used_ + bytes <= arena_->capacity) {
      *p = arena_->base + used_;
      used_ += bytes;
      return hipSuccess;
    }
    hipError_t err = hipMallocFromPoolAsync(p, bytes, pool_, stream_);
    if (err != hipSuccess) return err;
    allocations_.push_back(*p);
    return hipSuccess;
  }
  // Starts carving again from the arena's beginning: the work enqueued so
  // far keeps its scratch in stream order (later work on the stream runs
  // after it), so a call made of independent phases reuses one phase's
  // scratch for the next.  Pool allocations are freed on the stream.
  hipError_t rewind() {
    hipError_t first = hipSuccess;
    for (void* p : allocations_) {
      const hipError_t err = hipFreeAsync(p, stream_);
      if (first == hipSuccess) first = err;
    }
    allocations_.clear();
    peak_ = std::max(peak_, total_);
    total_ = 0;
    used_ = 0;
    return first;
  }
  hipError_t release() {
    hipError_t first = hipSuccess;
    auto keep = [&](hipError_t err) { if (first == hipSuccess) first = err; };
    for (void* p : allocations_) keep(hipFreeAsync(p, stream_));
    allocations_.clear();
    if (!acquired_) return first;
    acquired_ = false;
    total_ = std::max(peak_, total_);
    PoolRegistry& reg = registry();
    std::lock_guard<std::mutex> lock(reg.mutex);
    const u64 want = (total_ + kArenaGranule - 1) / kArenaGranule * kArenaGranule;
    u64 kept_bytes = 0;  // the device's arenas
    for (const auto& a : reg.arenas)
      if (a->device == device_) kept_bytes += a->capacity;
    if (!arena_ && kept_bytes + want <= reg.retention) {
      auto a = std::make_unique<Arena>();
      a->device = device_;
      a->base = nullptr;
      a->capacity = 0;
      a->last_stream = nullptr;
      a->busy = true;
      keep(hipEventCreateWithFlags(&a->last_use, hipEventDisableTiming));
      if (first != hipSuccess) return first;
      arena_ = a.get();
      reg.arenas.push_back(std::move(a));
    }
    if (arena_ && total_ > arena_->capacity) {
      // Grow for later calls: the old buffer is freed after this call's work.
      const u64 others = kept_bytes - arena_->capacity;  // the device's other arenas
      if (arena_->base) keep(hipFreeAsync(arena_->base, stream_));
      arena_->base = nullptr;
      arena_->capacity = 0;
      if (others + want <= reg.retention) {
        void* base = nullptr;
        hipError_t err = hipMallocFromPoolAsync(&base, want, pool_, stream_);
        keep(err);
        if (err == hipSuccess) {
          arena_->base = static_cast<u8*>(base);
          arena_->capacity = want;
        }
      }
    }
    if (arena_) {
      keep(hipEventRecord(arena_->last_use, stream_));
      arena_->last_stream = stream_;
      arena_->busy = false;
    }
    return first;
  }
  ~Workspace() override { (void)release(); }

 private:
  hipError_t acquire() {
    acquired_ = true;
    PoolRegistry& reg = registry();
    std::lock_guard<std::mutex> lock(reg.mutex);
    for (auto& a : reg.arenas)
      if (a->device == device_ && !a->busy &&
          (a->last_stream == stream_ || hipEventQuery(a->last_use) == hipSuccess)) {
        a->busy = true;
        arena_ = a.get();
        return hipStreamWaitEvent(stream_, arena_->last_use, 0);
      }
    return hipSuccess;
  }

  hipStream_t stream_;
  hipMemPool_t pool_;
  int device_;
  Arena* arena_ = nullptr;
  bool acquired_ = false;
  u64 used_ = 0, total_ = 0, peak_ = 0;
  std::vector<void*> allocations_;
};

int invalid(const char* message) {
  g_last_error = message;
  return HIP_ZLIB_INVALID_ARGUMENT;
}

template <typename Body>
int execute(hipStream_t stream, Body&& body) {
  try {
    DeviceScope scope;
    hipError_t err = scope.enter(stream);
    if (err != hipSuccess) return int(err);
    hipMemPool_t pool = nullptr;
    err = get_pool(scope.device(), &pool);
    if (err != hipSuccess) return int(err);
    Workspace ws(stream, pool, scope.device());
    err = body(ws);
    hipError_t rel = ws.release();
    return int(err != hipSuccess ? err : rel);
  } catch (...) {
    g_last_error = "native HIP codec handler exception";
    return HIP_ZLIB_INVALID_ARGUMENT;
  }
}

u64 chunk_count(u64 size, u64 chunk) { return std::max<u64>(1, (size + chunk - 1) / chunk); }

// Input bytes an open-ended member decode first looks at: at least this
// many, or four times the previous member's.  Discovery covers what a decode
// is given, so a window keeps a long run of small members linear in the
// input; a member that does not end inside its window is decoded again over
// the whole rest of the input.
constexpr u64 kMemberWindowMin = 16ull << 20;

// A concatenation of zlib streams or gzip members (HIP_ZLIB_FORMAT_MEMBERS):
// each member by an open-ended general-route decode into the output after
// the previous member's bytes, the host reading back (one stream
// synchronisation per member) where the member ended and how many bytes it
// produced.
hipError_t decode_members(hipStream_t stream, Workspace& ws, u32 format, int64_t max_candidates,
                          int64_t max_blocks, const uint8_t* input, uint64_t input_size,
                          uint8_t* output, uint64_t output_size, uint32_t* metadata) {
  if (output_size > kMaxBytes) return launch_set_meta(stream, metadata, kInvalidBounds, 0);
  hipError_t err = launch_fill(stream, output, 0, output_size);
  if (err != hipSuccess) return err;
  if (input_size > kMaxBytes || max_candidates < 1 || max_candidates > kMaxCandidates ||
      max_blocks < 1 || max_blocks > kMaxBlocks)
    return launch_set_meta(stream, metadata, kInvalidBounds, 0);
  const u64 fixed = format == kFormatGzip ? 18 : 8;
  u64 in_off = 0, out_off = 0, last_in = 0;
  u32 status = kOk;
  while (!status) {
    const u64 rest_in = input_size - in_off, rest_out = output_size - out_off;
    if (rest_in < fixed) {
      status = kTruncatedZlib;
      break;
    }
    u64 window = std::min(rest_in, std::max(kMemberWindowMin, 4 * last_in));
    u64 report_host[3] = {0, 0, 0};
    for (;;) {
      err = ws.rewind();
      if (err != hipSuccess) return err;
      u64* report = nullptr;
      u32* member_meta = nullptr;
      err = ws.alloc(&report, 3);
      if (err == hipSuccess) err = ws.alloc(&member_meta, 2);
      if (err != hipSuccess) return err;
      StreamFormat fmt;
      fmt.format = format;
      fmt.open = true;
      fmt.windowed = window < rest_in;
      fmt.report = report;
      err = run_inflate_general(stream, ws, input + in_off, window, output + out_off, rest_out,
                                u32(max_candidates), u32(max_blocks), member_meta, fmt);
      if (err == hipSuccess)
        err = hipMemcpyAsync(report_host, report, sizeof(report_host), hipMemcpyDeviceToHost,
                             stream);
      if (err == hipSuccess) err = hipStreamSynchronize(stream);
      if (err != hipSuccess) return err;
      if (report_host[0] && window < rest_in) {
        window = rest_in;  // the member may run past its window: decode it over all the rest
        continue;
      }
      break;
    }
    status = u32(report_host[0]);
    if (status) break;
    in_off += report_host[1];
    out_off += report_host[2];
    last_in = report_host[1];
    if (in_off >= input_size) break;
  }
  if (!status && out_off != output_size) status = kSizeMismatch;
  // A checksum mismatch keeps the output, as a single stream's does.
  if (status && status != kAdlerMismatch && status != kGzipCheckMismatch) {
    err = launch_fill(stream, output, 0, output_size);
    if (err != hipSuccess) return err;
  }
  return launch_set_meta(stream, metadata, status, 0);
}

}  // namespace
}  // namespace hz

using namespace hz;

extern "C" int HipZlibDecompress(hipStream_t stream, int64_t max_candidates, int64_t max_blocks,
                                 const uint8_t* input, uint64_t input_size, uint8_t* output,
                                 uint64_t output_size, uint32_t* metadata,
                                 uint64_t metadata_count) {
  if (!metadata || metadata_count != 2) return invalid("codec metadata must have shape (2,)");
  return execute(stream, [&](Workspace& ws) -> hipError_t {
    if (output_size > kMaxBytes) return launch_set_meta(stream, metadata, kInvalidBounds, 0);
    auto fail = [&](u32 status) -> hipError_t {
      hipError_t err = launch_fill(stream, output, 0, output_size);
      if (err != hipSuccess) return err;
      return launch_set_meta(stream, metadata, status, 0);
    };
    if (input_size > kMaxBytes || max_candidates < 1 || max_candidates > kMaxCandidates ||
        max_blocks < 1 || max_blocks > kMaxBlocks)
      return fail(kInvalidBounds);
    if (input_size < 8) return fail(kTruncatedZlib);
    const bool default_limits = max_candidates == kMaxCandidates && max_blocks == kMaxBlocks;
    // The reference's small route (codec_ffi.cu:681-693): tiny streams decode
    // serially in one wave; the others take the parallel route first, and the
    // serial decoder redoes only a failed one.  Everything else takes the
    // parallel route.
    if (default_limits && output_size <= 65536 && input_size <= 131072) {
      if (output_size < kSmallParallelBytes)
        return launch_inflate_single(stream, input, input_size, output, output_size,
                                     u32(max_blocks), metadata);
      hipError_t err = run_inflate_general(stream, ws, input, input_size, output, output_size,
                                           u32(max_candidates), u32(max_blocks), metadata);
      if (err != hipSuccess) return err;
      return launch_inflate_single(stream, input, input_size, output, output_size,
                                   u32(max_blocks), metadata, kFormatZlib, nullptr, 0, true);
    }
    return run_inflate_general(stream, ws, input, input_size, output, output_size,
                               u32(max_candidates), u32(max_blocks), metadata);
  });
}

extern "C" int HipZlibDecompressFormat(hipStream_t stream, int32_t format,
                                       const uint8_t* dictionary, uint64_t dictionary_size,
                                       int64_t max_candidates, int64_t max_blocks,
                                       const uint8_t* input, uint64_t input_size, uint8_t* output,
                                       uint64_t output_size, uint32_t* metadata,
                                       uint64_t metadata_count) {
  if (!metadata || metadata_count != 2) return invalid("codec metadata must have shape (2,)");
  const bool members = (format & HIP_ZLIB_FORMAT_MEMBERS) != 0;
  format &= ~HIP_ZLIB_FORMAT_MEMBERS;
  if (format != kFormatZlib && format != kFormatRaw && format != kFormatGzip)
    return invalid("unknown stream format (0 zlib, 1 raw DEFLATE, 2 gzip)");
  if (format == kFormatGzip && dictionary_size) return invalid("gzip streams take no dictionary");
  if (members && (format == kFormatRaw || dictionary_size))
    return invalid("concatenated members are zlib streams or gzip members, without a dictionary");
  if (dictionary_size && !dictionary) return invalid("missing preset dictionary");
  if (dictionary_size > kMaxBytes) return invalid("preset dictionary exceeds 2**32 - 1 bytes");
  if (members)
    return execute(stream, [&](Workspace& ws) -> hipError_t {
      return decode_members(stream, ws, u32(format), max_candidates, max_blocks, input, input_size,
                            output, output_size, metadata);
    });
  return execute(stream, [&](Workspace& ws) -> hipError_t {
    if (output_size > kMaxBytes) return launch_set_meta(stream, metadata, kInvalidBounds, 0);
    auto fail = [&](u32 status) -> hipError_t {
      hipError_t err = launch_fill(stream, output, 0, output_size);
      if (err != hipSuccess) return err;
      return launch_set_meta(stream, metadata, status, 0);
    };
    if (input_size > kMaxBytes || max_candidates < 1 || max_candidates > kMaxCandidates ||
        max_blocks < 1 || max_blocks > kMaxBlocks)
      return fail(kInvalidBounds);
    const u64 fixed = format == kFormatZlib ? 8 : format == kFormatGzip ? 18 : 0;
    if (input_size < fixed) return fail(kTruncatedZlib);
    const bool default_limits = max_candidates == kMaxCandidates && max_blocks == kMaxBlocks;
    if (default_limits && output_size <= 65536 && input_size <= 131072) {
      // As HipZlibDecompress's small route; with a dictionary, serially.
      if (output_size < kSmallParallelBytes || dictionary_size)
        return launch_inflate_single(stream, input, input_size, output, output_size,
                                     u32(max_blocks), metadata, u32(format), dictionary,
                                     dictionary_size);
      StreamFormat first;
      first.format = u32(format);
      hipError_t err = run_inflate_general(stream, ws, input, input_size, output, output_size,
                                           u32(max_candidates), u32(max_blocks), metadata, first);
      if (err != hipSuccess) return err;
      return launch_inflate_single(stream, input, input_size, output, output_size,
                                   u32(max_blocks), metadata, u32(format), nullptr, 0, true);
    }
    StreamFormat fmt;
    fmt.format = u32(format);
    fmt.dict = dictionary;
    fmt.dict_len = dictionary_size;
    if (!dictionary_size)
      return run_inflate_general(stream, ws, input, input_size, output, output_size,
                                 u32(max_candidates), u32(max_blocks), metadata, fmt);
    // With a dictionary the output is decoded behind its last window of
    // bytes (the history back-references may reach), then copied out.
    const u64 hist = std::min<u64>(dictionary_size, 32768);
    u8* ext = nullptr;
    hipError_t err = ws.alloc(&ext, hist + output_size);
    if (err != hipSuccess) return err;
    err = hipMemcpyAsync(ext, dictionary + (dictionary_size - hist), hist,
                         hipMemcpyDeviceToDevice, stream);
    if (err != hipSuccess) return err;
    fmt.out_base = hist;
    err = run_inflate_general(stream, ws, input, input_size, ext, output_size,
                              u32(max_candidates), u32(max_blocks), metadata, fmt);
    if (err != hipSuccess || !output_size) return err;
    return hipMemcpyAsync(output, ext + hist, output_size, hipMemcpyDeviceToDevice, stream);
  });
}

namespace {

// HipZlibCompress and HipZlibCompressIndependent: the same checks and
// outputs; `independent` limits every chunk's window to the chunk.
int compress_stream(hipStream_t stream, int64_t chunk_bytes, const uint8_t* input,
                    uint64_t input_size, uint8_t* output, uint64_t output_size, uint32_t* metadata,
                    uint64_t metadata_count, bool independent) {
  if (!metadata || metadata_count != 2) return invalid("codec metadata must have shape (2,)");
  return execute(stream, [&](Workspace& ws) -> hipError_t {
    if (output_size > kMaxBytes) return launch_set_meta(stream, metadata, 0, kInvalidBounds);
    // A rejected call returns a zeroed slot; an accepted one has the bytes
    // after its stream (or the whole slot, on failure) zeroed by run_deflate.
    auto reject = [&]() -> hipError_t {
      hipError_t err = launch_fill(stream, output, 0, output_size);
      if (err != hipSuccess) return err;
      return launch_set_meta(stream, metadata, 0, kInvalidBounds);
    };
    if (input_size > kMaxBytes || chunk_bytes < 256 || chunk_bytes > 65535) return reject();
    const u64 chunks = chunk_count(input_size, u64(chunk_bytes));
    if (2 * chunks - 1 > kMaxBlocks || input_size + chunks * 5 + 6 > kMaxBytes ||
        output_size != input_size + chunks * 5 + 6)
      return reject();
    return run_deflate(stream, ws, input, input_size, output, output_size, u32(chunk_bytes),
                       metadata, independent);
  });
}

}  // namespace

extern "C" int HipZlibCompress(hipStream_t stream, int64_t chunk_bytes, const uint8_t* input,
                               uint64_t input_size, uint8_t* output, uint64_t output_size,
                               uint32_t* metadata, uint64_t metadata_count) {
  return compress_stream(stream, chunk_bytes, input, input_size, output, output_size, metadata,
                         metadata_count, false);
}

extern "C" int HipZlibCompressIndependent(hipStream_t stream, int64_t chunk_bytes,
                                          const uint8_t* input, uint64_t input_size,
                                          uint8_t* output, uint64_t output_size,
                                          uint32_t* metadata, uint64_t metadata_count) {
  return compress_stream(stream, chunk_bytes, input, input_size, output, output_size, metadata,
                         metadata_count, true);
}

// ---- compression without allocation ------------------------------------------
// HipZlibCompressNoAlloc carves its scratch from this array instead of the
// pool.  Every GPU the library runs on holds its own copy for the life of the
// process; calls on one GPU share it, so calls that overlap on a GPU race.
// Host code never passes the array's name to a kernel: it uses the device
// address hipGetSymbolAddress returns for the current device.
constexpr u64 kNoAllocScratchBytes = 48ull << 20;
static __device__ __align__(256) u8 scratch[kNoAllocScratchBytes];

namespace hz {
namespace {

// Device address of `scratch` on `device` (which must be current), looked up
// once per device and kept.
hipError_t no_alloc_scratch(int device, void** out) {
  static std::mutex* mutex = new std::mutex;
  static std::vector<void*>* addresses = new std::vector<void*>;
  std::lock_guard<std::mutex> lock(*mutex);
  if (device < 0) return hipErrorInvalidDevice;
  if (addresses->size() <= size_t(device)) addresses->resize(size_t(device) + 1, nullptr);
  void*& slot = (*addresses)[size_t(device)];
  if (!slot) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return err;
    if (!p) return hipErrorInvalidSymbol;
    slot = p;
  }
  *out = slot;
  return hipSuccess;
}

}  // namespace
}  // namespace hz

extern "C" int HipZlibCompressNoAlloc(hipStream_t stream, int64_t chunk_bytes,
                                      const uint8_t* input, uint64_t input_size, uint8_t* output,
                                      uint64_t output_size, uint32_t* metadata,
                                      uint64_t metadata_count) {
  if (!metadata || metadata_count != 2) return invalid("codec metadata must have shape (2,)");
  // Calls HipZlibCompress would reject with status 23 get the same result.
  const bool bounds = output_size <= kMaxBytes && input_size <= kMaxBytes && chunk_bytes >= 256 &&
                      chunk_bytes <= 65535;
  u64 chunks = 1;
  bool accepted = bounds;
  if (bounds) {
    chunks = chunk_count(input_size, u64(chunk_bytes));
    accepted = 2 * chunks - 1 <= kMaxBlocks && input_size + chunks * 5 + 6 <= kMaxBytes &&
               output_size == input_size + chunks * 5 + 6;
  }
  if (accepted) {
    const u64 need = deflate_scratch_bytes(input_size, u32(chunk_bytes));
    if (need > kNoAllocScratchBytes) {
      g_last_error = "HipZlibCompressNoAlloc: this input needs " + std::to_string(need) +
                     " bytes of scratch, more than the " + std::to_string(kNoAllocScratchBytes) +
                     " bytes the no-allocation entry point holds; use HipZlibCompress";
      return HIP_ZLIB_INVALID_ARGUMENT;
    }
  }
  try {
    DeviceScope scope;
    hipError_t err = scope.enter(stream);
    if (err != hipSuccess) return int(err);
    if (output_size > kMaxBytes) return int(launch_set_meta(stream, metadata, 0, kInvalidBounds));
    if (!accepted) {
      err = launch_fill(stream, output, 0, output_size);
      if (err == hipSuccess) err = launch_set_meta(stream, metadata, 0, kInvalidBounds);
      return int(err);
    }
    void* region = nullptr;
    err = no_alloc_scratch(scope.device(), &region);
    if (err != hipSuccess) return int(err);
    FixedScratch fixed(region, kNoAllocScratchBytes);
    return int(run_deflate(stream, fixed, input, input_size, output, output_size,
                           u32(chunk_bytes), metadata));
  } catch (...) {
    g_last_error = "native HIP codec handler exception";
    return HIP_ZLIB_INVALID_ARGUMENT;
  }
}

extern "C" int HipZlibCompressBatch(hipStream_t stream, int64_t chunk_bytes,
                                    const int64_t* input_sizes, uint64_t files,
                                    const uint8_t* input, uint64_t input_size, uint8_t* output,
                                    uint64_t output_size, uint32_t* metadata,
                                    uint64_t metadata_rows, uint64_t metadata_cols) {
  if (!metadata || metadata_rows != files || metadata_cols != 2)
    return invalid("batch codec metadata must have shape (files, 2)");
  if (files && !input_sizes) return invalid("invalid argument: missing input sizes");
  // Layout validation mirrors codec_ffi.cu:1002-1045.
  std::vector<BatchFile> layout(files);
  u64 in_total = 0, out_total = 0, total_chunks = 0;
  bool bounds = chunk_bytes >= 256 && chunk_bytes <= 65535 && files <= kMaxBlocks;
  for (u64 f = 0; f < files; ++f) {
    if (input_sizes[f] < 0) return invalid("invalid argument: negative input size");
    const u64 size = u64(input_sizes[f]);
    const u64 chunks = bounds ? chunk_count(size, u64(chunk_bytes)) : 1;
    const u64 capacity = size + 5 * chunks + 6;
    layout[f] = {in_total, size, out_total, capacity};
    in_total += size;
    out_total += capacity;
    total_chunks += chunks;
    if (2 * chunks - 1 > kMaxBlocks) bounds = false;
  }
  if (in_total != input_size || out_total != output_size)
    return invalid("invalid argument: batch layout differs from buffer sizes");
  if (total_chunks > kMaxBlocks || in_total > kMaxBytes || out_total > kMaxBytes) bounds = false;
  return execute(stream, [&](Workspace& ws) -> hipError_t {
    hipError_t err = launch_fill(stream, output, 0, output_size);
    if (err != hipSuccess) return err;
    if (!bounds) return launch_set_meta_rows(stream, metadata, files, 0, kInvalidBounds);
    return run_deflate_batch(stream, ws, input, input_size, layout.data(), u32(files), output,
                             output_size, u32(chunk_bytes), metadata);
  });
}

extern "C" int HipZlibDecompressBatch(hipStream_t stream, const int64_t* input_sizes,
                                      uint64_t input_count, const int64_t* output_sizes,
                                      uint64_t output_count, const uint8_t* input,
                                      uint64_t input_size, const uint32_t* encoded_metadata,
                                      uint64_t encoded_rows, uint64_t encoded_cols,
                                      uint8_t* output, uint64_t output_size, uint32_t* metadata,
                                      uint64_t metadata_rows, uint64_t metadata_cols) {
  if (!metadata || metadata_rows != input_count || metadata_cols != 2)
    return invalid("batch codec metadata must have shape (files, 2)");
  if (!input_count || input_count != output_count)
    return invalid("input and output size lists must have matching nonempty lengths");
  if (encoded_rows && (encoded_rows != input_count || encoded_cols != 2 || !encoded_metadata))
    return invalid("encoded metadata must have shape (files, 2)");
  if (!input_sizes || !output_sizes) return invalid("invalid argument: missing size lists");
  std::vector<BatchFile> layout(input_count);
  u64 in_total = 0, out_total = 0;
  for (u64 f = 0; f < input_count; ++f) {
    if (input_sizes[f] < 0 || output_sizes[f] < 0)
      return invalid("invalid argument: negative size");
    layout[f] = {in_total, u64(input_sizes[f]), out_total, u64(output_sizes[f])};
    in_total += u64(input_sizes[f]);
    out_total += u64(output_sizes[f]);
  }
  if (in_total != input_size || out_total != output_size)
    return invalid("invalid argument: batch layout differs from buffer sizes");
  const u64 files = input_count;
  return execute(stream, [&](Workspace& ws) -> hipError_t {
    if (files > kMaxBlocks || in_total > kMaxBytes || out_total > kMaxBytes) {
      hipError_t err = launch_fill(stream, output, 0, output_size);
      if (err != hipSuccess) return err;
      return launch_set_meta_rows(stream, metadata, files, kInvalidBounds, 0);
    }
    // No fill of the output first: every file's bytes are written by its
    // decoder.  The serial one zeroes a file's slot before decoding (and a
    // slot with a bad encoded row); the parallel route writes all of a file
    // it accepts and hands every other file to the serial one.
    BatchFile* device_files = nullptr;
    hipError_t err = ws.alloc(&device_files, files);
    if (err != hipSuccess) return err;
    // Staged before the call returns, so the host vector may go out of scope.
    err = upload_to_device(stream, device_files, layout.data(), files * sizeof(BatchFile));
    if (err != hipSuccess) return err;
    const u32* encoded = encoded_rows ? encoded_metadata : nullptr;
    // Files of at least kBatchWideBytes go to the parallel route; the rest,
    // and any large file it hands back, to the serial one.
    // Largest files first: a file's workgroup decodes its blocks one after
    // another, so the longest decodes start while the grid fills and the
    // short ones fill in behind them.  The order only schedules work, so a
    // counting sort by size class (the power of two below the size and five
    // bits under it: classes within 3 %) stands in for a comparison sort,
    // whose host time for 4096 files (a few hundred microseconds) the GPU
    // waited on.  Files of one class keep their order.
    constexpr u32 kClasses = 2048;
    const auto size_class = [](u64 size) {  // size >= kBatchWideBytes >= 32
      const u32 e = 63u - u32(__builtin_clzll(size));
      return (e - 5u) * 32u + u32((size >> (e - 5u)) & 31u);
    };
    static_assert(kBatchWideBytes >= 32, "size classes start at 2^5");
    std::vector<u32> class_at(kClasses + 1, 0);
    u64 large_bits = 0, nlarge = 0;
    for (u64 f = 0; f < files; ++f)
      if (layout[f].out_size >= kBatchWideBytes) {
        ++class_at[kClasses - 1 - size_class(layout[f].out_size)];
        large_bits += layout[f].in_size * 8;
        ++nlarge;
      }
    for (u32 k = 0, run = 0; k <= kClasses; ++k) {
      const u32 c = class_at[k];
      class_at[k] = run;
      run += c;
    }
    std::vector<u32> large(nlarge);
    for (u64 f = 0; f < files; ++f)
      if (layout[f].out_size >= kBatchWideBytes)
        large[class_at[kClasses - 1 - size_class(layout[f].out_size)]++] = u32(f);
    if (large.empty())
      return launch_inflate_batch(stream, input, output, device_files, u32(files), kMaxBlocks,
                                  metadata, encoded, kBatchWideBytes);
    // The small files, then the large ones by the parallel route, all on the
    // caller's stream: a second stream would share one of the device's few
    // hardware queues with unrelated streams and wait behind their work.
    err = launch_inflate_batch(stream, input, output, device_files, u32(files), kMaxBlocks,
                               metadata, encoded, kBatchWideBytes);
    if (err != hipSuccess) return err;
    u32 *device_large = nullptr, *redo = nullptr;
    err = ws.alloc(&device_large, large.size());
    if (err == hipSuccess) err = ws.alloc(&redo, files);
    if (err != hipSuccess) return err;
    err = upload_to_device(stream, device_large, large.data(), large.size() * sizeof(u32));
    if (err != hipSuccess) return err;
    err = run_inflate_batch_wide(stream, ws, input, output, output_size, device_files,
                                 device_large, u32(large.size()), large_bits, encoded, kMaxBlocks,
                                 redo, metadata);
    if (err != hipSuccess) return err;
    return launch_inflate_batch(stream, input, output, device_files, u32(large.size()),
                                kMaxBlocks, metadata, encoded, ~0ull, device_large, redo);
  });
}

extern "C" int HipZlibSetWorkspaceRetention(uint64_t bytes) {
  PoolRegistry& reg = registry();
  std::lock_guard<std::mutex> lock(reg.mutex);
  if (!reg.pools.empty()) return invalid("workspace retention must be set before first use");
  reg.retention = bytes;
  return 0;
}

extern "C" int HipZlibWorkspacePoolStats(int device, uint64_t* stats) {
  if (!stats) return invalid("invalid argument: null stats");
  PoolRegistry& reg = registry();
  u64 retention, reserved = 0, used = 0, count = 0;
  {
    std::lock_guard<std::mutex> lock(reg.mutex);
    retention = reg.retention;
  }
  hipMemPool_t pool;
  if (find_pool(device, &pool)) {
    count = 1;
    hipError_t err = hipMemPoolGetAttribute(pool, hipMemPoolAttrReservedMemCurrent, &reserved);
    if (err != hipSuccess) return int(err);
    err = hipMemPoolGetAttribute(pool, hipMemPoolAttrUsedMemCurrent, &used);
    if (err != hipSuccess) return int(err);
  }
  stats[0] = retention;
  stats[1] = reserved;
  stats[2] = used;
  stats[3] = count;
  return 0;
}

extern "C" int HipZlibTrimWorkspacePool(int device) {
  hipMemPool_t pool;
  if (!find_pool(device, &pool)) return 0;
  // Idle arenas of the device leave the registry under the lock (no call can
  // take them any more); waiting for their last use and freeing them happen
  // after the lock is released, so calls on other streams are never held up
  // by this wait.
  std::vector<std::unique_ptr<Arena>> idle;
  {
    PoolRegistry& reg = registry();
    std::lock_guard<std::mutex> lock(reg.mutex);
    for (auto it = reg.arenas.begin(); it != reg.arenas.end();) {
      if ((*it)->device == device && !(*it)->busy) {
        idle.push_back(std::move(*it));
        it = reg.arenas.erase(it);
      } else {
        ++it;
      }
    }
  }
  int previous = 0;
  hipError_t first = hipGetDevice(&previous);
  if (first == hipSuccess && previous != device) first = hipSetDevice(device);
  auto keep = [&](hipError_t err) { if (first == hipSuccess) first = err; };
  for (auto& a : idle) {
    keep(hipEventSynchronize(a->last_use));
    // A synchronous free: the pool must hold the pages again before the trim.
    if (a->base) keep(hipFree(a->base));
    keep(hipEventDestroy(a->last_use));
  }
  if (first == hipSuccess) first = hipMemPoolTrimTo(pool, 0);
  if (previous != device) (void)hipSetDevice(previous);
  return int(first);
}

namespace hz {
std::string profile_collect(bool reset);
void profile_enable(bool on);
}  // namespace hz

extern "C" int HipZlibProfileEnable(int enabled) {
  hz::profile_enable(enabled != 0);
  return 0;
}

extern "C" uint64_t HipZlibProfileCollect(char* buffer, uint64_t capacity, int reset) {
  const std::string text = hz::profile_collect(reset != 0);
  if (buffer && capacity) {
    const uint64_t n = std::min<uint64_t>(capacity - 1, text.size());
    std::copy(text.data(), text.data() + n, buffer);
    buffer[n] = 0;
  }
  return text.size();
}

extern "C" const char* HipZlibErrorString(int code) {
  if (code == HIP_ZLIB_INVALID_ARGUMENT) return g_last_error.c_str();
  return hipGetErrorString(hipError_t(code));
}
