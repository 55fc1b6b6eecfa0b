// Single-wave serial inflate: one 64-lane wavefront decodes one whole zlib
// stream.  Lane 0 walks the bit stream; the wave joins in for stored payload
// copies and long matches; the wave computes the Adler-32 check at the end.
//
// Serves the small-stream route and every file of a batch.  Semantics restate
// the reference's DecodeOneFile (native/batch_decode.cuh:123-296): statuses in
// stream order, failed output = decoded prefix followed by zeros, exact output
// size (11), no trailing body bytes (12), block cap (9), declared window (6).
#include "deflate_common.h"
#include "kernels.h"

namespace hz {

namespace {

constexpr u32 kWave = 64;
constexpr u32 kCoopMatch = 32;  // matches at least this long are copied by the wave

struct WaveShared {
  DecodeTables tables;
  union {
    u16 codes[320];  // table build scratch
    u32 runs[320];   // code-length runs of the header walk
  };
  u64 hdr_start;  // a dynamic header: the body bit after BTYPE
  u32 nl, nd, fixed, build_status;
  u32 action;  // 0 done, 1 match copy, 2 stored copy, 3 table build
  u32 error;
  u64 begin, length, distance, src;
  Frame frame;
};

// Wrapper of the stream a wave decodes: the format and, for zlib streams
// with a preset dictionary or raw streams, the dictionary whose last bytes
// precede the output as history.
struct WaveFormat {
  u32 format = kFormatZlib;
  const u8* dict = nullptr;
  u64 dict_len = 0;
};

// Copy a match of `length` bytes to out[begin..) from `d` bytes back.  Reads
// only the d-byte seed preceding `begin`, so an overlapping match never
// depends on this copy's own stores.
__device__ __forceinline__ void wave_match(u8* out, u64 begin, u64 d, u64 length, u32 lane) {
  const u64 first = begin - d;
  if (d == 1) {
    const u8 v = out[first];
    for (u64 j = lane; j < length; j += kWave) out[begin + j] = v;
    return;
  }
  u64 src = first + (lane % d);
  const u64 stride = kWave % d;
  for (u64 j = lane; j < length; j += kWave) {
    out[begin + j] = out[src];
    src += stride;
    if (src >= begin) src -= d;
  }
}

// Adler-32 of out[0..n) by one wave; result valid in lane 0.
__device__ u32 wave_adler(const u8* out, u64 n, u32 lane) {
  u64 s = 0, w = 0;
  // weight of byte i is (n - i) mod 65521; it drops by 64 per step.
  u64 weight = (n - lane) % kAdlerMod;
  const u64 step = kWave % kAdlerMod;
  u32 since = 0;
  for (u64 i = lane; i < n; i += kWave) {
    const u64 v = out[i];
    s += v;
    w += weight * v;
    weight = weight >= step ? weight - step : weight + kAdlerMod - step;
    if (++since == 4096) {  // keep sums far from overflow
      s %= kAdlerMod;
      w %= kAdlerMod;
      since = 0;
    }
  }
  s %= kAdlerMod;
  w %= kAdlerMod;
  for (u32 off = kWave / 2; off; off >>= 1) {
    s += __shfl_down(s, off, kWave);
    w += __shfl_down(w, off, kWave);
  }
  const u32 a = u32((s + 1) % kAdlerMod);
  const u32 b = u32((w + n) % kAdlerMod);
  return (b << 16) | a;
}

// CRC-32 of out[0..n) by one wave; result valid in lane 0.  Each lane takes a
// contiguous piece (register computed from 0), and pieces are joined by
// shuffles: left * x^(8 |right|) + right.
__device__ u32 wave_crc(const u8* out, u64 n, u32 lane) {
  const u64 piece = (n + kWave - 1) / kWave;
  const u64 lo = min<u64>(n, lane * piece), hi = min<u64>(n, lo + piece);
  u32 c = 0;
  for (u64 i = lo; i < hi; ++i) c = crc_byte_update(c, out[i]);
  u64 len = hi - lo;
  for (u32 width = 1; width < kWave; width <<= 1) {
    const u32 right = __shfl_down(c, width, kWave);
    const u64 right_len = __shfl_down(len, width, kWave);
    if ((lane & (2 * width - 1)) == 0 && lane + width < kWave) {
      c = crc_mul(c, crc_shift_bytes(right_len)) ^ right;
      len += right_len;
    }
  }
  return crc_finish(c, n);
}

// Decodes one stream with a 64-thread workgroup and writes [status, 0].
__device__ void inflate_one_wave(const u8* in, u64 in_size, u8* out, u64 out_size,
                                 u32 max_blocks, u32* meta, WaveShared& sh,
                                 const WaveFormat fmt = WaveFormat()) {
  const u32 lane = threadIdx.x;
  if (in_size > kMaxBytes || out_size > kMaxBytes || !max_blocks || max_blocks > kMaxBlocks) {
    if (!lane) { meta[0] = kInvalidBounds; meta[1] = 0; }
    return;
  }
  for (u64 i = lane; i < out_size; i += kWave) out[i] = 0;
  __syncthreads();

  // Lane-0 private parser state.
  u32 error = 0, final_block = 0, blocks = 0, window = 0;
  u64 produced = 0, body_bytes = 0;
  bool need_header = true, complete = false;
  BitIn r;
  if (!lane) {
    sh.action = 0;
    sh.error = parse_frame(in, in_size, fmt.format, fmt.dict_len > 0, sh.frame);
    // Only a zlib stream that asks for a dictionary (FDICT) uses one.
    if (fmt.format == kFormatZlib && !sh.frame.needs_dict) sh.frame.dict_id = 0;
  }
  __syncthreads();
  // The dictionary history a back-reference may reach (within the window).
  u64 hist = 0;
  if (!sh.error && (fmt.format == kFormatRaw || sh.frame.needs_dict)) {
    hist = fmt.dict_len;
    if (sh.frame.needs_dict) {
      const u32 id = wave_adler(fmt.dict, fmt.dict_len, lane);
      if (!lane && id != sh.frame.dict_id) sh.error = kDictionaryMismatch;
    }
  }
  __syncthreads();
  if (!lane) {
    error = sh.error;
    window = sh.frame.window;
    if (!error) {
      body_bytes = sh.frame.body_len;
      r.init(in + sh.frame.body, body_bytes, 0);
    }
  }

  while (true) {
    if (!lane) {
      u32 action = 0;
      if (sh.action == 3) error = sh.build_status;
      while (!error && !complete) {
        if (need_header) {
          if (blocks >= max_blocks) { error = kBlockCapacity; break; }
          ++blocks;
          u32 type;
          if (!r.take(1, final_block) || !r.take(2, type)) { error = kTruncated; break; }
          if (type == 3) { error = kReservedBlock; break; }
          if (type == 0) {
            r.seek((r.pos + 7) & ~u64(7));
            u32 n, comp;
            if (!r.take(16, n) || !r.take(16, comp)) { error = kTruncated; break; }
            if ((n ^ comp) != 0xffffu) { error = kBadSymbol; break; }
            if (n > out_size - produced) { error = kOutputOverflow; break; }
            if (u64(n) * 8 > r.avail()) { error = kTruncated; break; }
            sh.begin = produced;
            sh.length = n;
            sh.src = (r.pos >> 3) + sh.frame.body;
            produced += n;
            r.seek(r.pos + u64(n) * 8);
            complete = final_block != 0;
            action = 2;
            break;
          }
          // The wave reads a dynamic header's code lengths and builds the
          // tables (action 3); lane 0 resumes after the header.
          need_header = false;
          sh.nl = 288;
          sh.nd = 32;
          sh.hdr_start = r.pos;
          sh.fixed = type == 1;
          action = 3;
          break;
        }
        u32 lit = 0, length = 0, distance = 0;
        error = decode_token(sh.tables, r, window, lit, length, distance);
        if (error) break;
        if (!length) {  // end of block
          complete = final_block != 0;
          need_header = true;
          continue;
        }
        if (length > out_size - produced) { error = kOutputOverflow; break; }
        if (!distance) { out[produced++] = u8(lit); continue; }
        if (distance > produced + hist) { error = kBadDistance; break; }
        if (distance > produced) {
          // Reaches into the dictionary: byte by byte, sources in the
          // dictionary or (for an overlapping copy) in this copy's period.
          const i64 first = i64(produced) - i64(distance);
          for (u32 j = 0; j < length; ++j) {
            const i64 s = first + i64(j % distance);
            out[produced + j] = s < 0 ? fmt.dict[i64(fmt.dict_len) + s] : out[s];
          }
          produced += length;
          continue;
        }
        if (length >= kCoopMatch) {
          sh.begin = produced;
          sh.length = length;
          sh.distance = distance;
          produced += length;
          action = 1;
          break;
        }
        u64 src = produced - distance;
        const u64 first = src;
        for (u32 j = 0; j < length; ++j) {
          out[produced + j] = out[src];
          if (++src == produced) src = first;
        }
        produced += length;
      }
      if (!action && !error) {
        if (produced != out_size) error = kSizeMismatch;
        else if ((r.pos + 7) / 8 != body_bytes) error = kExtent;
      }
      sh.action = action;
      sh.error = error;
    }
    __syncthreads();
    const u32 action = sh.action;
    if (!action) break;
    if (action == 1) {
      wave_match(out, sh.begin, sh.distance, sh.length, lane);
    } else if (action == 2) {
      for (u64 j = lane; j < sh.length; j += kWave) out[sh.begin + j] = in[sh.src + j];
    } else {
      // Same tables and statuses as build_fixed_tables / build_dynamic_tables.
      const bool fixed = sh.fixed;
      u32 err = kOk;
      if (fixed) {
        for (u32 i = lane; i < 320; i += kWave)
          sh.tables.lens[i] = i < 144 ? 8 : i < 256 ? 9 : i < 280 ? 7 : i < 288 ? 8 : 5;
      } else {
        // The lengths by the wave walk over the body's dwords from the one
        // holding the header (at most 256 of them, so positions stay small),
        // or by lane 0's serial parse where the walk cannot finish there.
        const u64 start = sh.hdr_start, len = sh.frame.body_len;
        const uintptr_t addr = reinterpret_cast<uintptr_t>(in + sh.frame.body);
        const u64 lead = u64(addr & 3u) * 8;  // body bit b is bit b + lead of the dwords
        const u64 all = (u64(addr & 3u) + len + 3) >> 2;
        const u64 first = (start + lead) >> 5;
        const u32* words = reinterpret_cast<const u32*>(addr & ~uintptr_t(3)) + first;
        const u64 bit0 = first * 32 - lead;
        const u32 count = u32(min(all - first, u64(256)));
        u32 nl = 0, nd = 0, p = 0, lim = 0;
        u64 after = start;
        if (!header_prelude_wave(words, bit0, count, sh.tables, len, start, nl, nd, err, after, p,
                                 lim)) {
          err = kHeaderWalkStuck;
        } else if (!err) {
          err = header_lengths_wave(words, sh.tables, sh.runs, nl + nd, p, lim);
          after = bit0 + p;
        }
        if (err == kHeaderWalkStuck) {  // uniform
          if (!lane) {
            r.seek(start);
            err = parse_dynamic_lengths(sh.tables, r, nl, nd);
            sh.nl = nl;
            sh.nd = nd;
            sh.build_status = err;
            after = r.pos;
          }
          __syncthreads();
          err = sh.build_status;
          nl = sh.nl;
          nd = sh.nd;
        }
        if (!lane) {
          r.seek(after);
          sh.nl = nl;
          sh.nd = nd;
        }
      }
      __syncthreads();
      if (!err)
        err = huff_build_wave(sh.tables.ll, sh.tables.lens, sh.nl, false, true, 15, sh.codes,
                              &sh.build_status);
      if (!err)
        err = huff_build_wave(sh.tables.dd, sh.tables.lens + sh.nl, sh.nd, !fixed, true, 15,
                              sh.codes, &sh.build_status);
      if (!lane) sh.build_status = err;
    }
    __syncthreads();
  }

  u32 status = sh.error;
  if (!status && sh.frame.check == kCheckAdler) {
    const u32 got = wave_adler(out, out_size, lane);
    if (!lane && got != sh.frame.wanted) status = kAdlerMismatch;
  } else if (!status && sh.frame.check == kCheckCrc) {
    const u32 got = wave_crc(out, out_size, lane);
    if (!lane && (got != sh.frame.wanted || u32(out_size) != sh.frame.isize))
      status = kGzipCheckMismatch;
  }
  if (!lane) {
    meta[0] = status;
    meta[1] = 0;
  }
}

// Copies n bytes with the wave: dwords when both ends are dword-aligned,
// bytes otherwise.
__device__ __forceinline__ void wave_copy(u8* dst, const u8* src, u64 n, u32 lane) {
  u64 i = lane;
  if (!((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 3u)) {
    const u64 words = n >> 2;
    for (; i < words; i += kWave)
      reinterpret_cast<u32*>(dst)[i] = reinterpret_cast<const u32*>(src)[i];
    i = (words << 2) + lane;
  }
  for (; i < n; i += kWave) dst[i] = src[i];
}

// inflate_one_wave with the output, and the stream when it fits too, copied
// into `stage` (LDS, 16-byte aligned, `capacity` bytes).  Lane 0's walk then
// waits on LDS rather than on global memory for each dword of the bit stream
// and for each source byte of a short match.  `out` receives the same bytes
// as an unstaged decode: the staged output starts zeroed and is copied whole.
__device__ void inflate_staged(const u8* in, u64 in_size, u8* out, u64 out_size, u32 max_blocks,
                               u32* meta, WaveShared& sh, u8* stage, u64 capacity,
                               const WaveFormat fmt = WaveFormat()) {
  const u32 lane = threadIdx.x;
  const u64 out_room = (out_size + 15) & ~u64(15), in_room = (in_size + 15) & ~u64(15);
  // Invalid limits leave `out` untouched, so they stay on the direct path.
  const bool staged = max_blocks && max_blocks <= kMaxBlocks && in_size <= kMaxBytes &&
                      out_room <= capacity;
  const u8* src = in;
  if (staged && out_room + in_room <= capacity) {
    u8* copy = stage + out_room;
    wave_copy(copy, in, in_size, lane);
    // The dword reads of the bit reader see zeros, not stale bytes, past the end.
    if (lane < in_room - in_size) copy[in_size + lane] = 0;
    src = copy;
  }
  __syncthreads();
  inflate_one_wave(src, in_size, staged ? stage : out, out_size, max_blocks, meta, sh, fmt);
  if (staged) {
    __syncthreads();
    wave_copy(out, stage, out_size, lane);
  }
}

// LDS staging capacities: the one-stream kernel (one workgroup, streams of at
// most 64 KiB of output on the small route) and the batch kernel (many
// resident workgroups; files under 256 B of output).
constexpr u64 kSingleStage = 128 * 1024;
constexpr u64 kBatchStage = 2048;

}  // namespace

// With `redo`, the stream was already decoded by the parallel route, which
// left its status in meta[0]: the kernel decodes it again only when that
// status is not 0, to give the serial route's status and failed output.
__global__ __launch_bounds__(64) void inflate_single_kernel(const u8* in, u64 in_size, u8* out,
                                                            u64 out_size, u32 max_blocks,
                                                            u32* meta, u32 format, const u8* dict,
                                                            u64 dict_len, u32 redo) {
  __shared__ WaveShared sh;
  __shared__ __align__(16) u8 stage[kSingleStage];
  if (redo && !meta[0]) return;  // uniform
  WaveFormat fmt;
  fmt.format = format;
  fmt.dict = dict;
  fmt.dict_len = dict_len;
  inflate_staged(in, in_size, out, out_size, max_blocks, meta, sh, stage, kSingleStage, fmt);
}

// One workgroup per file.  With encoded metadata (compression's
// [length, status] rows), a file's stream length comes from its row and a
// failed or oversized slot is zeroed with status 22/23 (batch_decode.cuh:298-328).
// Files of at least `skip_from` output bytes are left to the parallel
// large-file route.  With `list`, only the listed files flagged in `redo`
// are decoded (the large files that route handed back).
__global__ __launch_bounds__(64) void inflate_batch_kernel(const u8* in, u8* out,
                                                           const BatchFile* files, u32 count,
                                                           u32 max_blocks, u32* meta,
                                                           const u32* encoded, u64 skip_from,
                                                           const u32* list, const u32* redo) {
  __shared__ WaveShared sh;
  __shared__ __align__(16) u8 stage[kBatchStage];
  for (u32 i = blockIdx.x; i < count; i += gridDim.x) {
    const u32 f = list ? list[i] : i;
    if (list ? !redo[f] : files[f].out_size >= skip_from) continue;  // uniform
    const BatchFile file = files[f];
    u64 in_size = file.in_size;
    if (encoded) {
      const u32 enc_len = encoded[2 * u64(f)];
      const u32 enc_status = encoded[2 * u64(f) + 1];
      u32 error = enc_status ? u32(kCompressionOverflow) : (enc_len > file.in_size ? u32(kInvalidBounds) : 0u);
      if (file.out_size > kMaxBytes) error = kInvalidBounds;
      if (error) {
        if (file.out_size <= kMaxBytes)
          for (u64 i = threadIdx.x; i < file.out_size; i += kWave) out[file.out_offset + i] = 0;
        if (!threadIdx.x) {
          meta[2 * u64(f)] = error;
          meta[2 * u64(f) + 1] = 0;
        }
        __syncthreads();
        continue;
      }
      in_size = enc_len;
    }
    inflate_staged(in + file.in_offset, in_size, out + file.out_offset, file.out_size, max_blocks,
                   meta + 2 * u64(f), sh, stage, kBatchStage);
    __syncthreads();
  }
}

hipError_t launch_inflate_single(hipStream_t stream, const u8* in, u64 in_size, u8* out,
                                 u64 out_size, u32 max_blocks, u32* meta, u32 format,
                                 const u8* dict, u64 dict_len, bool redo) {
  HZ_LAUNCH(inflate_single_kernel, dim3(1), dim3(kWave), 0, stream, in, in_size, out,
                     out_size, max_blocks, meta, format, dict, dict_len, redo ? 1u : 0u);
  return hipGetLastError();
}

hipError_t launch_inflate_batch(hipStream_t stream, const u8* in, u8* out, const BatchFile* files,
                                u32 count, u32 max_blocks, u32* meta, const u32* encoded,
                                u64 skip_from, const u32* list, const u32* redo) {
  if (!count) return hipSuccess;
  const u32 grid = count < 65536u ? count : 65536u;
  HZ_LAUNCH(inflate_batch_kernel, dim3(grid), dim3(kWave), 0, stream, in, out, files, count,
                     max_blocks, meta, encoded, skip_from, list, redo);
  return hipGetLastError();
}

}  // namespace hz
