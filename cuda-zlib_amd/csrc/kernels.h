// Internal host-side launch interface between the C-ABI layer and the kernel
// translation units.  Every launcher enqueues on `stream` and returns the
// launch error; none of them synchronises with the host.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "deflate_common.h"

namespace hz {

struct BatchFile {
  u64 in_offset;
  u64 in_size;
  u64 out_offset;
  u64 out_size;
};

// util.hip: optional per-kernel timing.  When enabled, every launch made
// through HZ_LAUNCH is bracketed by HIP events on its stream; totals are read
// back (after the caller synchronises) through the C ABI.
bool profiling_enabled();
void profile_record(const char* name, hipEvent_t start, hipEvent_t stop);

#define HZ_LAUNCH(kernel, grid, block, shmem, stream, ...)                       \
  do {                                                                         \
    hipEvent_t hz_start_ = nullptr, hz_stop_ = nullptr;                        \
    const bool hz_prof_ = ::hz::profiling_enabled();                           \
    if (hz_prof_ && hipEventCreate(&hz_start_) == hipSuccess &&                \
        hipEventCreate(&hz_stop_) == hipSuccess)                               \
      (void)hipEventRecord(hz_start_, stream);                                 \
    hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);       \
    if (hz_prof_ && hz_stop_) {                                                \
      (void)hipEventRecord(hz_stop_, stream);                                  \
      ::hz::profile_record(#kernel, hz_start_, hz_stop_);                      \
    }                                                                          \
  } while (0)

hipError_t launch_fill(hipStream_t stream, void* dst, u8 value, u64 bytes);
// Host bytes to device memory in stream order, through pinned staging that
// is reused once the copy is done: the copy neither waits for nor holds up
// work on other streams (as the runtime's shared staging of pageable memory
// does), and the host source may be reused when it returns.
hipError_t upload_to_device(hipStream_t stream, void* dst, const void* src, u64 bytes);
hipError_t launch_set_meta(hipStream_t stream, u32* meta, u32 first, u32 second);
hipError_t launch_set_meta_rows(hipStream_t stream, u32* meta, u64 rows, u32 first, u32 second);

// inflate_wave.hip: serial-route decode (one wave per stream).
// format: kFormatZlib / kFormatRaw / kFormatGzip; dict (dict_len bytes, device)
// is the preset dictionary of a zlib stream with FDICT or the history of a
// raw stream (null and 0: none).  With `redo`, meta[0] already holds the
// parallel route's status for the same stream, and the serial decode runs
// only when it is not 0.
hipError_t launch_inflate_single(hipStream_t stream, const u8* in, u64 in_size, u8* out,
                                 u64 out_size, u32 max_blocks, u32* meta,
                                 u32 format = kFormatZlib, const u8* dict = nullptr,
                                 u64 dict_len = 0, bool redo = false);
// Files of at least skip_from output bytes are skipped; with `list`, only the
// listed files whose `redo` flag is set are decoded.
hipError_t launch_inflate_batch(hipStream_t stream, const u8* in, u8* out, const BatchFile* files,
                                u32 count, u32 max_blocks, u32* meta, const u32* encoded,
                                u64 skip_from = ~0ull, const u32* list = nullptr,
                                const u32* redo = nullptr);

// Every scratch buffer is a multiple of 256 bytes and 256-byte aligned.
inline u64 scratch_round(u64 bytes) { return ((bytes ? bytes : 1) + 255) & ~u64(255); }

// Scratch allocation interface used by multi-kernel routes.
struct Scratch {
  virtual hipError_t alloc_bytes(void** p, u64 bytes) = 0;
  template <typename T>
  hipError_t alloc(T** p, u64 count) {
    return alloc_bytes(reinterpret_cast<void**>(p), count * sizeof(T));
  }
  virtual ~Scratch() {}
};

// Wrapper of a stream for the general route: its format, the preset
// dictionary (device; a zlib stream with FDICT checks its Adler-32), and the
// number of history bytes that precede the stream's output in the output
// buffer (the dictionary's last bytes, placed there by the caller).
struct StreamFormat {
  u32 format = kFormatZlib;
  const u8* dict = nullptr;
  u64 dict_len = 0;
  u64 out_base = 0;
  // Open-ended decode of the first member of in[0..in_size): its stream may
  // end before in_size (other members follow its trailer) and produce at most
  // out_size bytes.  `report` (device, 3 x u64) then receives
  // [status, input bytes of the member, output bytes]; the output is not
  // cleared on failure.
  // `windowed`: in_size is a prefix of the member's input, so a stream the
  // fast path cannot accept reports kTruncated (1) at once, and the caller
  // decodes it again over all of its input.
  bool open = false;
  bool windowed = false;
  u64* report = nullptr;
};

// inflate_par.hip: general-route decode.  The stream's out_size bytes go to
// out[fmt.out_base ..]; callers guarantee in_size covers the wrapper's fixed
// fields (zlib 8 bytes, gzip 18).
hipError_t run_inflate_general(hipStream_t stream, Scratch& scratch, const u8* in, u64 in_size,
                               u8* out, u64 out_size, u32 max_candidates, u32 max_blocks,
                               u32* meta, const StreamFormat& fmt = StreamFormat());
// Batch files listed in `list` (device) decoded by parallel slices, one
// workgroup per file; a file that does not decode cleanly gets redo[f] = 1
// and is left for the serial decoder, the others get [0, 0] in meta.
// in_bits: total input bits of the listed files (sizes the slice pool).
hipError_t run_inflate_batch_wide(hipStream_t stream, Scratch& scratch, const u8* in, u8* out,
                                  u64 out_total, const BatchFile* files, const u32* list,
                                  u32 n, u64 in_bits, const u32* encoded, u32 max_blocks,
                                  u32* redo, u32* meta);

// Scratch carved from one caller-given device region; a request past its end
// fails with hipErrorOutOfMemory and carves nothing.
struct FixedScratch final : Scratch {
  u8* base;
  u64 capacity, used = 0;
  FixedScratch(void* region, u64 bytes) : base(static_cast<u8*>(region)), capacity(bytes) {}
  hipError_t alloc_bytes(void** p, u64 bytes) override {
    *p = nullptr;
    const u64 n = scratch_round(bytes);
    if (n > capacity - used) return hipErrorOutOfMemory;
    *p = base + used;
    used += n;
    return hipSuccess;
  }
};

// deflate.hip: chunked encode of one stream / a batch of streams.
// deflate_scratch_bytes: the scratch run_deflate takes for one stream.
u64 deflate_scratch_bytes(u64 in_size, u32 chunk_bytes);
// With `independent`, every chunk's LZ77 window is the chunk alone (no
// history from the bytes before it).
hipError_t run_deflate(hipStream_t stream, Scratch& scratch, const u8* in, u64 in_size, u8* out,
                       u64 capacity, u32 chunk_bytes, u32* meta, bool independent = false);
hipError_t run_deflate_batch(hipStream_t stream, Scratch& scratch, const u8* in, u64 in_total,
                             const BatchFile* files_host, u32 count, u8* out, u64 out_total,
                             u32 chunk_bytes, u32* meta);

}  // namespace hz
