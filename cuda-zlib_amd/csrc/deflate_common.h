// Shared device-side building blocks of the HIP zlib/DEFLATE codec (gfx950).
//
// Everything here is header-only and included by each kernel translation unit.
// Status codes are the codec's metadata contract (src/cuda_zlib/_decode_kernels.py:36-50
// and native/codec_ffi.cu:51-62 in the reference); bit/Huffman semantics follow
// RFC 1951 plus the reference's exact error rules (_decode_kernels.py:69-296).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hz {

typedef uint8_t u8;
typedef uint16_t u16;
typedef uint32_t u32;
typedef uint64_t u64;
typedef int32_t i32;
typedef int64_t i64;

// ---- status contract -------------------------------------------------------
enum Status : u32 {
  kOk = 0,
  kTruncated = 1,          // bits ran out inside a header, symbol or payload
  kReservedBlock = 2,      // BTYPE == 3
  kBadTree = 3,            // over/under-subscribed code, HLIT > 286, EOB length 0
  kBadSymbol = 4,          // LL 286/287, distance 30/31, invalid code, LEN/NLEN
  kBadRepeat = 5,          // code-length repeat before a length or past the end
  kBadDistance = 6,        // distance beyond history or the declared window
  kOutputOverflow = 7,     // decoded output exceeds the declared size
  kBlockCapacity = 9,      // more blocks than max_blocks
  kUndiscovered = 10,      // dynamic block boundary not among the candidates
  kSizeMismatch = 11,      // final decoded size differs from the declared size
  kExtent = 12,            // block end/trailing-byte mismatch
  kTruncatedZlib = 14,
  kInvalidHeader = 15,
  kUnsupportedGzip = 16,
  kUnsupportedDictionary = 17,
  kCandidateOverflow = 18,
  kInitialBlockMissing = 19,
  kReferenceDepth = 20,
  kAdlerMismatch = 21,
  kCompressionOverflow = 22,
  kInvalidBounds = 23,
  // Statuses of the wrapper formats the reference does not decode (gzip,
  // raw DEFLATE, preset dictionaries); the zlib entry points never give them.
  kGzipCheckMismatch = 24,  // gzip CRC-32 or ISIZE differs from the output
  kDictionaryMismatch = 25, // the preset dictionary's Adler-32 is not the DICTID
};

constexpr u64 kMaxBytes = 0xffffffffull;   // per-buffer bound (4 GiB - 1)
constexpr u32 kMaxCandidates = 262144;
constexpr u32 kMaxBlocks = 262144;
constexpr u32 kAdlerMod = 65521;

// ---- RFC 1951 length/distance alphabets (closed forms) ----------------------
// Length symbol 257+i: base and extra bits.  i<8: 3+i, 0 extra; i==28: 258.
__host__ __device__ __forceinline__ u32 length_extra(u32 i) {
  return (i < 8 || i == 28) ? 0u : (i >> 2) - 1u;
}
__host__ __device__ __forceinline__ u32 length_base(u32 i) {
  return i < 8 ? i + 3u : (i == 28 ? 258u : 3u + ((4u + (i & 3u)) << ((i >> 2) - 1u)));
}
// Distance symbol d (0..29).
__host__ __device__ __forceinline__ u32 dist_extra(u32 d) {
  return d < 4 ? 0u : (d >> 1) - 1u;
}
__host__ __device__ __forceinline__ u32 dist_base(u32 d) {
  return d < 4 ? d + 1u : 1u + ((2u + (d & 1u)) << ((d >> 1) - 1u));
}

__host__ __device__ __forceinline__ u32 bit_reverse(u32 code, u32 len) {
  return __builtin_bitreverse32(code) >> (32 - len);
}

// Bytes b .. b+3 of (hi:lo) (b < 4): v_alignbyte_b32 in GPU code.
__host__ __device__ __forceinline__ u32 funnel_bytes(u32 hi, u32 lo, u32 b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_alignbyte(hi, lo, b);
#else
  return u32(((u64(hi) << 32) | lo) >> (8 * (b & 3u)));
#endif
}

// Dot product of the four bytes of x with the four bytes of w (v_dot4_u32_u8).
__host__ __device__ __forceinline__ u32 byte_dot(u32 x, u32 w) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_udot4(x, w, 0u, false);
#else
  u32 d = 0;
  for (u32 k = 0; k < 32; k += 8) d += ((x >> k) & 0xffu) * ((w >> k) & 0xffu);
  return d;
#endif
}

// The low 32 bits of (hi:lo) >> s for s < 32: v_alignbit_b32 in GPU code;
// the same value by shifts in the host build of the readers (CPU bounds tests).
__host__ __device__ __forceinline__ u32 funnel32(u32 hi, u32 lo, u32 s) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_alignbit(hi, lo, s);
#else
  return u32(((u64(hi) << 32) | lo) >> (s & 31u));
#endif
}

// ---- bit input --------------------------------------------------------------
// LSB-first reader over a byte range [data, data + bytes).  The reader loads
// aligned dwords only, and only dwords that hold at least one byte of the
// range, so it never touches a page outside the caller's buffer.  `pos` counts
// consumed bits from the start of the range; `avail()` is what remains.  Bits
// past the range may be garbage inside `buf`; every consumer checks avail()
// before committing, which reproduces the reference's "error 1 on over-read".
struct BitIn {
  const u32* words;
  u64 base_bit;   // bit offset of data[0] inside words[0]
  u64 total;      // valid bits in the range
  u64 pos;        // consumed bits
  u64 buf;        // bits [pos, pos + cnt)
  u32 cnt;
  u64 wnext;      // next dword index to load
  u64 wlimit;     // dwords holding range bytes

  __host__ __device__ __forceinline__ void init(const u8* data, u64 bytes, u64 start_bit) {
    const uintptr_t addr = reinterpret_cast<uintptr_t>(data);
    words = reinterpret_cast<const u32*>(addr & ~uintptr_t(3));
    base_bit = u64(addr & 3u) * 8u;
    total = bytes * 8u;
    wlimit = (u64(addr & 3u) + bytes + 3u) >> 2;
    seek(start_bit);
  }
  __host__ __device__ __forceinline__ void refill() {
    while (cnt <= 32) {
      const u64 v = wnext < wlimit ? u64(words[wnext]) : 0ull;
      buf |= v << cnt;
      cnt += 32;
      ++wnext;
    }
  }
  __host__ __device__ __forceinline__ void seek(u64 p) {
    pos = p;
    const u64 a = base_bit + p;
    wnext = a >> 5;
    buf = 0;
    cnt = 0;
    refill();
    const u32 skip = u32(a & 31u);
    buf >>= skip;
    cnt -= skip;
    refill();
  }
  __host__ __device__ __forceinline__ u64 avail() const { return pos <= total ? total - pos : 0; }
  // Callers guarantee n <= 32 and have checked avail() where it matters.
  __host__ __device__ __forceinline__ u32 peek(u32 n) const {
    return n ? u32(buf & ((1ull << n) - 1ull)) : 0u;
  }
  __host__ __device__ __forceinline__ void drop(u32 n) {
    buf >>= n;
    cnt -= n;
    pos += n;
    if (cnt <= 32) refill();
  }
  // take(n): returns false (truncation) when fewer than n bits remain.
  __host__ __device__ __forceinline__ bool take(u32 n, u32& v) {
    if (u64(n) > avail()) return false;
    v = peek(n);
    drop(n);
    return true;
  }
};

// LSB-first reader over words staged in LDS, with 32-bit positions relative to
// word 0 (a stage holds at most a few hundred kilobits).  `limit` is the
// relative bit position of the body end (saturated), so avail() keeps the
// body's truncation semantics; words past `nwords` read as zero.
struct StagedBits {
  const u32* words;
  u32 nwords;
  u32 pos;
  u32 limit;
  u64 buf;
  u32 cnt;
  u32 wnext;

  __host__ __device__ __forceinline__ void refill() {
    while (cnt <= 32) {
      const u64 v = wnext < nwords ? u64(words[wnext]) : 0ull;
      buf |= v << cnt;
      cnt += 32;
      ++wnext;
    }
  }
  __host__ __device__ __forceinline__ void seek(u32 p) {
    pos = p;
    wnext = p >> 5;
    buf = 0;
    cnt = 0;
    refill();
    const u32 skip = p & 31u;
    buf >>= skip;
    cnt -= skip;
    refill();
  }
  __host__ __device__ __forceinline__ u32 avail() const { return pos < limit ? limit - pos : 0u; }
  __host__ __device__ __forceinline__ u32 peek(u32 n) const {
    return n ? u32(buf & ((1ull << n) - 1ull)) : 0u;
  }
  __host__ __device__ __forceinline__ void drop(u32 n) {
    buf >>= n;
    cnt -= n;
    pos += n;
    if (cnt <= 32) refill();
  }
  __host__ __device__ __forceinline__ bool take(u32 n, u32& v) {
    if (n > avail()) return false;
    v = peek(n);
    drop(n);
    return true;
  }
};

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for
// every outstanding global store of the wave; kernels whose threads never
// exchange data through global memory within the launch (their stores are
// read by later launches) use this instead and keep stores in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---- canonical Huffman decode tables ---------------------------------------
// Primary LUT entry (u32): bits 0..3 code length (0 = no short code here),
// bits 16..31 symbol.  Codes longer than the primary width are decoded from
// the per-length bounds (long_code).  `maximum` is the longest code length
// (0 for an empty tree).
//
// With v the next 15 bits read as an MSB-first code value and first[l] the
// first canonical code of length l, limit[l] = (first[l] + count[l]) << (15 - l)
// is the first 15-bit value past the length-l codes.  The limits never
// decrease with l (lengths past `maximum` repeat the last one), so the code
// length is the least l with v < limit[l], and its symbol is
// symbols[base[l] + (v >> (15 - l))] with base[l] = (symbols before length l)
// - first[l], modulo 2^16.
template <int N, int P>
struct HuffTable {
  u16 count[16];
  u16 limit[16];  // also the serial build's scratch until the bounds are set
  u16 base[16];
  u16 symbols[N];
  u32 primary[1 << P];
  u32 maximum;
};

// limit and base from count (lengths 1..15; entry 0 unused).  Only the
// tables a build accepts are decoded, so over-subscribed counts may wrap.
template <int N, int P>
__host__ __device__ inline void huff_bounds(HuffTable<N, P>& t) {
  u32 first = 0, index = 0;
  t.limit[0] = 0;
  t.base[0] = 0;
  for (u32 l = 1; l < 16; ++l) {
    const u32 c = t.count[l];
    t.limit[l] = u16((first + c) << (15 - l));
    t.base[l] = u16(index - first);
    index += c;
    first = (first + c) << 1;
  }
}

// Code-length alphabet order (RFC 1951 3.2.7), 5 bits per entry, packed so
// device code indexes registers rather than a private array.
__host__ __device__ __forceinline__ u32 cl_order(u32 i) {
  return i < 12 ? u32((0x22caa324e804a30ull >> (5 * i)) & 31)
                : u32((0x3c2e1346cull >> (5 * (i - 12))) & 31);
}

// Build from code lengths.  empty_ok: all-zero lengths allowed (distance tree).
// single_ok: an incomplete code consisting of one length-1 code is allowed.
// Returns 0 or kBadTree.  Must be called by one thread.  Semantics follow the
// reference's Huffman::build (_decode_kernels.py:141-183).
template <int N, int P>
__host__ __device__ u32 huff_build(HuffTable<N, P>& t, const u8* lens, u32 n, bool empty_ok,
                          bool single_ok, u32 limit) {
  for (u32 i = 0; i < 16; ++i) t.count[i] = 0;
  t.maximum = 0;
  if (n > u32(N)) return kBadTree;
  for (u32 i = 0; i < n; ++i) {
    const u32 l = lens[i];
    if (l > limit) return kBadTree;
    ++t.count[l];
    if (l > t.maximum) t.maximum = l;
  }
  if (!t.maximum) {
    huff_bounds(t);
    return empty_ok ? 0u : u32(kBadTree);
  }
  i32 left = 1;
  for (u32 l = 1; l <= limit; ++l) {
    left = (left << 1) - i32(t.count[l]);
    if (left < 0) return kBadTree;
  }
  if (left && !(single_ok && t.maximum == 1 && t.count[1] == 1)) return kBadTree;
  u16* slot = t.limit;  // next symbol slot of each length
  slot[1] = 0;
  for (u32 l = 1; l < 15; ++l) slot[l + 1] = slot[l] + t.count[l];
  for (u32 i = 0; i < n; ++i)
    if (lens[i]) t.symbols[slot[lens[i]]++] = u16(i);
  huff_bounds(t);
  for (u32 i = 0; i < (1u << P); ++i) t.primary[i] = 0;
  u32 code = 0, index = 0;
  for (u32 l = 1; l <= u32(P); ++l) {
    for (u32 j = 0; j < t.count[l]; ++j) {
      const u32 rev = bit_reverse(code + j, l);
      const u32 e = (u32(t.symbols[index + j]) << 16) | l;
      for (u32 k = rev; k < (1u << P); k += 1u << l) t.primary[k] = e;
    }
    index += t.count[l];
    code = (code + t.count[l]) << 1;
  }
  return 0;
}

// A code longer than the primary LUT (or none) at the next bits `b` (LSB
// first), after a LUT miss.  Returns the symbol and its length, or -1 with
// `err`: kTruncated when the code, or any code up to `maximum` bits when none
// matches, needs more than `avail` bits; kBadSymbol when no code matches.
// A LUT miss leaves v >= limit[l] for every l <= P (P >= 7), so only lengths
// 8..15 are compared; a length is decided by its own first l bits, so bits
// past `avail` never change a result that fits in `avail`.
template <int N, int P>
__host__ __device__ __forceinline__ i32 long_code(const HuffTable<N, P>& t, u32 b, u32 avail,
                                                  u32& len_out, u32& err) {
  static_assert(P >= 7, "long_code compares lengths 8..15 only");
  const u32 v = bit_reverse(b & 0x7fffu, 15);
  u32 n = 0;
#pragma unroll
  for (u32 l = 8; l < 16; ++l) n += u32(t.limit[l]) <= v ? 1u : 0u;
  if (n == 8) {
    err = t.maximum > avail ? kTruncated : kBadSymbol;
    return -1;
  }
  const u32 len = 8 + n;
  if (len > avail) {
    err = kTruncated;
    return -1;
  }
  len_out = len;
  return i32(t.symbols[(u32(t.base[len]) + (v >> (15 - len))) & 0xffffu]);
}

// Decode one symbol.  Returns the symbol (>= 0), or -1 with `err` set to
// kTruncated (bits ran out first) or kBadSymbol (no code matches within
// `maximum` bits).  Matches the reference's LUT-plus-canonical decode exactly,
// including its behaviour at the end of the bit range.
template <int N, int P, class Reader>
__host__ __device__ __forceinline__ i32 huff_decode(const HuffTable<N, P>& t, Reader& r, u32& err) {
  const u32 e = t.primary[r.peek(P)];
  const u32 l = e & 15u;
  if (l) {
    if (u64(l) > r.avail()) { err = kTruncated; return -1; }
    r.drop(l);
    return i32(e >> 16);
  }
  // Long codes and invalid prefixes.
  const u64 avail = r.avail();
  u32 len = 0;
  const i32 sym = long_code(t, u32(r.buf), avail > 0xffffffffull ? 0xffffffffu : u32(avail), len, err);
  if (sym >= 0) r.drop(len);
  return sym;
}

struct DecodeTables {
  HuffTable<288, 10> ll;
  HuffTable<32, 8> dd;
  HuffTable<19, 7> cl;
  u8 lens[320];
};

// Fixed Huffman tables (RFC 1951 3.2.6).
__host__ __device__ inline u32 build_fixed_tables(DecodeTables& t) {
  for (u32 i = 0; i < 288; ++i) t.lens[i] = i < 144 ? 8 : i < 256 ? 9 : i < 280 ? 7 : 8;
  u32 err = huff_build(t.ll, t.lens, 288, false, true, 15);
  if (err) return err;
  for (u32 i = 0; i < 32; ++i) t.lens[i] = 5;
  return huff_build(t.dd, t.lens, 32, false, true, 15);
}

// Code-length code table from 19 packed 3-bit lengths (symbol s at bits 3s):
// counts and next codes live in packed registers, so no private arrays.
// The code must be complete (RFC 1951 allows no other).  Returns 0 or kBadTree.
__host__ __device__ inline u32 build_cl_table(HuffTable<19, 7>& t, u64 pack) {
  u64 cnt = 0;  // byte l = number of symbols of length l
  for (u32 s = 0; s < 19; ++s) cnt += 1ull << (8 * ((pack >> (3 * s)) & 7));
  u32 kraft = 0, maximum = 0;
  for (u32 l = 1; l < 8; ++l) {
    const u32 c = u32(cnt >> (8 * l)) & 0xff;
    kraft += c << (7 - l);
    if (c) maximum = l;
  }
  for (u32 l = 0; l < 16; ++l) t.count[l] = l < 8 ? u16((cnt >> (8 * l)) & 0xff) : 0;
  t.maximum = maximum;
  if (kraft != 128) return kBadTree;
  huff_bounds(t);
  u64 next = 0, offs = 0;  // byte l: next code / next symbol slot for length l
  u32 code = 0, slot = 0;
  for (u32 l = 1; l < 8; ++l) {
    code = (code + (l > 1 ? u32(cnt >> (8 * (l - 1))) & 0xff : 0u)) << 1;
    next |= u64(code) << (8 * l);
    offs |= u64(slot) << (8 * l);
    slot += u32(cnt >> (8 * l)) & 0xff;
  }
  for (u32 s = 0; s < 19; ++s) {
    const u32 l = (pack >> (3 * s)) & 7;
    if (!l) continue;
    const u32 c = u32(next >> (8 * l)) & 0xff;
    next += 1ull << (8 * l);
    t.symbols[u32(offs >> (8 * l)) & 0xff] = u16(s);
    offs += 1ull << (8 * l);
    const u32 e = (s << 16) | l;
    for (u32 k = bit_reverse(c, l); k < 128; k += 1u << l) t.primary[k] = e;
  }
  return kOk;
}

// Dynamic block header (RFC 1951 3.2.7) up to the code lengths: reads HLIT,
// HDIST, HCLEN and the code-length code, then decodes the nl + nd lengths into
// t.lens.  Reader positioned after BTYPE.  Error order follows the reference's
// dynamic_tables (_decode_kernels.py:240-283).
__host__ __device__ inline u32 parse_dynamic_lengths(DecodeTables& t, BitIn& r, u32& nl, u32& nd) {
  u32 hlit, hdist, hclen;
  if (!r.take(5, hlit) || !r.take(5, hdist) || !r.take(4, hclen)) return kTruncated;
  nl = hlit + 257;
  nd = hdist + 1;
  const u32 nc = hclen + 4;
  if (nl > 286) return kBadTree;
  u64 pack = 0;
  for (u32 i = 0; i < nc; ++i) {
    u32 v;
    if (!r.take(3, v)) return kTruncated;
    pack |= u64(v) << (3 * cl_order(i));
  }
  u32 err = build_cl_table(t.cl, pack);
  if (err) return err;
  u32 i = 0;
  while (i < nl + nd) {
    u32 e = 0;
    const i32 sym = huff_decode(t.cl, r, e);
    if (sym < 0) return e;
    if (sym < 16) { t.lens[i++] = u8(sym); continue; }
    u32 repeat, value, x;
    if (sym == 16) {
      if (!i) return kBadRepeat;
      if (!r.take(2, x)) return kTruncated;
      repeat = x + 3;
      value = t.lens[i - 1];
    } else if (sym == 17) {
      if (!r.take(3, x)) return kTruncated;
      repeat = x + 3;
      value = 0;
    } else {
      if (!r.take(7, x)) return kTruncated;
      repeat = x + 11;
      value = 0;
    }
    if (repeat > nl + nd - i) return kBadRepeat;
    for (u32 j = 0; j < repeat; ++j) t.lens[i++] = u8(value);
  }
  if (!t.lens[256]) return kBadTree;
  return kOk;
}

// Dynamic block header (RFC 1951 3.2.7), reader positioned after BTYPE.
__host__ __device__ inline u32 build_dynamic_tables(DecodeTables& t, BitIn& r) {
  u32 nl, nd;
  u32 err = parse_dynamic_lengths(t, r, nl, nd);
  if (err) return err;
  err = huff_build(t.ll, t.lens, nl, false, true, 15);
  if (err) return err;
  return huff_build(t.dd, t.lens + nl, nd, true, true, 15);
}

// Wave-cooperative table build for a 64-thread workgroup (one wavefront).
// Length counts, per-length ranks and canonical codes come from ballots over
// 64-symbol chunks; lane 0 only checks the Kraft sum over 15 lengths.  Same
// validity rules and table contents as huff_build.  `scratch` holds >= 320
// u16 in LDS (codes, then offsets/next codes); every lane must call it and
// every lane gets the status.
template <int N, int P, bool kOneWave = false>
__device__ u32 huff_build_wave(HuffTable<N, P>& t, const u8* lens, u32 n, bool empty_ok,
                               bool single_ok, u32 limit, u16* scratch, u32* status) {
  // kOneWave: called by wave 0 of a larger workgroup (wave-level syncs only).
  auto sync = [] {
    if (kOneWave) wave_sync();
    else __syncthreads();
  };
  const u32 lane = threadIdx.x;
  u16* codes = scratch;
  u16* offs = scratch + 288;
  u16* next = scratch + 304;
  // Counts: lane l (< 16) accumulates the number of symbols of length l.
  u32 cnt = 0;
  for (u32 base = 0; base < n; base += 64) {
    const u32 sym = base + lane;
    const u32 l = sym < n ? lens[sym] : 16u;
    for (u32 len = 0; len < 16; ++len) {
      const u64 b = __ballot(l == len);
      if (lane == len) cnt += __popcll(b);
    }
  }
  if (lane < 16) t.count[lane] = u16(cnt);
  // Kraft sum, offsets and first codes by scans over lanes 1..15.  With
  // weights count[l] << (15 - l), the serial running balance of huff_build
  // goes negative exactly when the total passes 2^15 (the partial sums only
  // grow), the code is complete exactly at 2^15, and the first code of
  // length l is the exclusive weighted sum below l shifted down by 15 - l
  // (exact: every term below l is a multiple of 2^(16 - l)).
  {
    const bool used = lane >= 1 && lane <= limit && lane < 16;
    const u32 c = used ? cnt : 0u;
    u32 wsum = c << (15 - (lane & 15)), csum = c;
#pragma unroll
    for (u32 o = 1; o < 16; o <<= 1) {
      const u32 wy = __shfl_up(wsum, o, 64), cy = __shfl_up(csum, o, 64);
      if (lane >= o) {
        wsum += wy;
        csum += cy;
      }
    }
    const u32 total = u32(__builtin_amdgcn_readlane(int(wsum), 15));
    const u64 lens_used = __ballot(used && cnt);
    const u64 over_limit = __ballot(lane > limit && lane < 16 && cnt);
    const u32 maximum = lens_used ? 63u - u32(__builtin_clzll(lens_used)) : 0u;
    const u32 ones = u32(__builtin_amdgcn_readlane(int(cnt), 1));
    if (lane >= 1 && lane < 16) {
      const u32 first = (wsum - (c << (15 - lane))) >> (15 - lane);
      offs[lane] = u16(csum - c);
      next[lane] = u16(first);
      // The inclusive weighted sum is the length's limit (see HuffTable).
      t.limit[lane] = u16(wsum);
      t.base[lane] = u16(csum - c - first);
    }
    if (!lane) {
      t.limit[0] = 0;
      t.base[0] = 0;
    }
    if (!lane) {
      u32 st = kOk;
      if (n > u32(N) || over_limit) st = kBadTree;
      t.maximum = maximum;
      if (!st && !maximum && !empty_ok) st = kBadTree;
      if (!st && maximum) {
        if (total > 32768u) st = kBadTree;
        else if (total != 32768u && !(single_ok && maximum == 1 && ones == 1)) st = kBadTree;
      }
      *status = st;
    }
  }
  for (u32 i = lane; i < (1u << P); i += 64) t.primary[i] = 0;
  sync();
  const u32 st = *status;
  if (!st && t.maximum) {
    // Symbols in (length, symbol) order and canonical codes; lane l (< 16)
    // carries the running count of length-l symbols seen in earlier chunks.
    u32 running = 0;
    for (u32 base = 0; base < n; base += 64) {
      const u32 sym = base + lane;
      const u32 l = sym < n ? lens[sym] : 0u;
      u32 rank = 0, chunk = 0;
      for (u32 len = 1; len < 16; ++len) {
        const u64 b = __ballot(l == len);
        if (l == len) rank = __popcll(b & ((1ull << lane) - 1));
        if (lane == len) chunk = __popcll(b);
      }
      const u32 before = __shfl(running, l, 64);
      if (l) {
        t.symbols[offs[l] + before + rank] = u16(sym);
        codes[sym] = u16(next[l] + before + rank);
      }
      running += chunk;
    }
  }
  sync();
  if (!st) {
    for (u32 s = lane; s < n; s += 64) {
      const u32 l = lens[s];
      if (!l || l > u32(P)) continue;
      const u32 e = (s << 16) | l;
      for (u32 k = bit_reverse(codes[s], l); k < (1u << P); k += 1u << l) t.primary[k] = e;
    }
  }
  sync();
  return st;
}

// One literal/length token after the LL symbol.  Returns kOk and sets
// length/distance (length 0 = EOB, distance 0 = literal in `lit`), or an error.
// Order of checks follows the reference's token decode (_decode_kernels.py:393-420).
template <class Reader>
__host__ __device__ __forceinline__ u32 decode_token(const DecodeTables& t, Reader& r, u32 window, u32& lit,
                                             u32& length, u32& distance) {
  u32 err = 0;
  const i32 sym = huff_decode(t.ll, r, err);
  length = 0;
  distance = 0;
  if (sym < 0) return err;
  if (sym < 256) { lit = u32(sym); length = 1; return kOk; }
  if (sym == 256) return kOk;
  if (sym > 285) return kBadSymbol;
  const u32 li = u32(sym) - 257;
  u32 x = 0;
  if (!r.take(length_extra(li), x)) return kTruncated;
  length = length_base(li) + x;
  const i32 ds = huff_decode(t.dd, r, err);
  if (ds < 0) return err;
  if (ds > 29) return kBadSymbol;
  if (!r.take(dist_extra(u32(ds)), x)) return kTruncated;
  distance = dist_base(u32(ds)) + x;
  if (distance > window) return kBadDistance;
  return kOk;
}

// ---- fast token decoding ---------------------------------------------------
// After a table build, the primary LUT can be rewritten into a format that
// resolves a token's class and constants with one lookup:
//   literal/length: bits 0-3 code length (0: no code of <= P bits here),
//     bits 4-5 kind, bits 8-15 literal byte or length extra-bit count,
//     bits 16-31 length base;
//   distance: bits 0-3 code length, bits 4-7 extra-bit count, bit 8 invalid
//     symbol (30, 31), bits 16-31 distance base.
// Codes longer than P bits and invalid prefixes take the canonical walk over
// count/symbols, which the rewrite leaves untouched.
enum : u32 { kKindLit = 0, kKindLen = 1, kKindEob = 2, kKindBad = 3 };

__host__ __device__ __forceinline__ u32 fast_ll_entry(u32 sym, u32 l) {
  if (sym < 256) return l | (sym << 8);
  if (sym == 256) return l | (kKindEob << 4);
  if (sym > 285) return l | (kKindBad << 4);
  const u32 li = sym - 257;
  return l | (kKindLen << 4) | (length_extra(li) << 8) | (length_base(li) << 16);
}

__host__ __device__ __forceinline__ u32 fast_d_entry(u32 sym, u32 l) {
  if (sym > 29) return l | 0x100u;
  return l | (dist_extra(sym) << 4) | (dist_base(sym) << 16);
}

// Rewrite a built table's primary LUT (threads `first`, `first + step`, ...).
template <int N, int P>
__host__ __device__ void fast_format(HuffTable<N, P>& t, bool literal_length, u32 first, u32 step) {
  for (u32 i = first; i < (1u << P); i += step) {
    const u32 e = t.primary[i];
    const u32 l = e & 15u;
    if (l) t.primary[i] = literal_length ? fast_ll_entry(e >> 16, l) : fast_d_entry(e >> 16, l);
  }
}

// LSB-first reader over LDS words with 32-bit positions: two words in
// registers, extraction by funnel shift.  kChecked: avail() is the distance to
// `limit` (the body end); otherwise the caller guarantees that no consumed bit
// lies past the body end, and avail() is unbounded.  Words are read up to
// index (pos >> 5) + 1, which the caller keeps inside the word array.
template <bool kChecked>
struct WordBits {
  const u32* words;
  u32 w, lo, hi, off, limit;
  __host__ __device__ __forceinline__ void seek(u32 p) {
    w = p >> 5;
    off = p & 31u;
    lo = words[w];
    hi = words[w + 1];
  }
  __host__ __device__ __forceinline__ u32 pos() const { return (w << 5) + off; }
  __host__ __device__ __forceinline__ u32 bits32() const { return funnel32(hi, lo, off); }
  __host__ __device__ __forceinline__ void drop(u32 n) {  // n <= 32
    off += n;
    if (off >= 32) {
      off -= 32;
      lo = hi;
      ++w;
      hi = words[w + 1];
    }
  }
  __host__ __device__ __forceinline__ u32 avail() const {
    if (!kChecked) return 0xffffffffu;
    const u32 p = pos();
    return p < limit ? limit - p : 0u;
  }
};

// One token with fast-format tables; same results and error order as
// decode_token over the standard format (a distance is at most 32768).
template <class R>
__host__ __device__ __forceinline__ u32 fast_token(const HuffTable<288, 10>& ll, const HuffTable<32, 8>& dd,
                                          R& r, u32& lit, u32& length, u32& distance) {
  length = 0;
  distance = 0;
  u32 b = r.bits32();
  u32 e = ll.primary[b & 1023u];
  u32 l = e & 15u;
  if (!l) {
    u32 err = 0;
    const i32 sym = long_code(ll, b, r.avail(), l, err);
    if (sym < 0) return err;
    e = fast_ll_entry(u32(sym), l);
  }
  if (l > r.avail()) return kTruncated;
  r.drop(l);
  const u32 kind = (e >> 4) & 3u;
  if (kind == kKindLit) {
    lit = (e >> 8) & 0xffu;
    length = 1;
    return kOk;
  }
  if (kind == kKindEob) return kOk;
  if (kind == kKindBad) return kBadSymbol;
  const u32 nx = (e >> 8) & 15u;
  if (nx > r.avail()) return kTruncated;
  b = r.bits32();
  length = (e >> 16) + (b & ((1u << nx) - 1u));
  r.drop(nx);
  b = r.bits32();
  u32 d = dd.primary[b & 255u];
  u32 dl = d & 15u;
  if (!dl) {
    u32 err = 0;
    const i32 sym = long_code(dd, b, r.avail(), dl, err);
    if (sym < 0) return err;
    d = fast_d_entry(u32(sym), dl);
  }
  if (dl > r.avail()) return kTruncated;
  r.drop(dl);
  if (d & 0x100u) return kBadSymbol;
  const u32 dx = (d >> 4) & 15u;
  if (dx > r.avail()) return kTruncated;
  b = r.bits32();
  distance = (d >> 16) + (b & ((1u << dx) - 1u));
  r.drop(dx);
  return kOk;
}

// LSB-first reader over LDS words holding four words (128 bits) in
// registers: the next token's lookups need only the first two (taken from
// the old four), and the last two are reloaded on every advance for the
// token after, so the load latency overlaps the next token's table
// lookups.  advance(n) takes n <= 64.
// Words are read up to index (pos >> 5) + 3, which the caller keeps inside
// the word array; bits past the body end are never consumed when kChecked.
template <bool kChecked>
struct Win4 {
  const u32* words;
  u32 w, off, x0, x1, x2, x3, limit;
  __host__ __device__ __forceinline__ void seek(u32 p) {
    w = p >> 5;
    off = p & 31u;
    x0 = words[w];
    x1 = words[w + 1];
    x2 = words[w + 2];
    x3 = words[w + 3];
  }
  __host__ __device__ __forceinline__ u32 pos() const { return (w << 5) + off; }
  __host__ __device__ __forceinline__ u32 bits32() const { return funnel32(x1, x0, off); }
  __host__ __device__ __forceinline__ u64 bits64() const {
    return u64(funnel32(x1, x0, off)) |
           (u64(funnel32(x2, x1, off)) << 32);
  }
  __host__ __device__ __forceinline__ u32 avail() const {
    if (!kChecked) return 0xffffffffu;
    const u32 p = pos();
    return p < limit ? limit - p : 0u;
  }
  __host__ __device__ __forceinline__ void advance(u32 n) {
    const u32 o = off + n;
    const u32 adv = o >> 5;  // 0, 1 or 2
    off = o & 31u;
    w += adv;
    u32 c0 = x0, c1 = x1, c2 = x2, c3 = x3;
    // Opaque register values: keeps the compiler from turning the selects
    // below into a load through a selected pointer (into private memory).
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("" : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3));
#endif
    x0 = adv >= 2 ? c2 : adv ? c1 : c0;
    x1 = adv >= 2 ? c3 : adv ? c2 : c1;
    x2 = words[w + 2];  // first used by the next advance
    x3 = words[w + 3];
  }
};

// One literal or match with fast-format tables when both codes hit their
// primary LUTs: every class is resolved with selects rather than branches
// (the distance lookup is made for literals too and ignored).  Returns false,
// leaving the reader where it was, for anything else (a longer code, an end
// of block, an invalid symbol, or bits too close to the limit): the caller
// then decodes that token with fast_token.  The token takes n <= 41 bits.
template <bool kChecked>
__host__ __device__ __forceinline__ bool quick_token(const HuffTable<288, 10>& ll, const HuffTable<32, 8>& dd,
                                            Win4<kChecked>& r, u32& length, u32& lit_or_dist) {
  const u64 b = r.bits64();
  const u32 b32 = u32(b);
  const u32 e = ll.primary[b32 & 1023u];
  const u32 l = e & 15u;
  const u32 kind = (e >> 4) & 3u;
  const u32 is_len = kind == kKindLen ? ~0u : 0u;  // masks, not branches
  const u32 nx = (e >> 8) & 15u & is_len;
  const u32 s = l + nx;  // <= 20
  const u32 d = dd.primary[(b32 >> s) & 255u];
  const u32 dl = d & 15u, dx = (d >> 4) & 15u;
  const u32 n = l + ((nx + dl + dx) & is_len);
  const u32 dist_ok = (dl != 0) & ((d >> 8) ^ 1u);
  bool ok = ((l != 0) & (kind <= kKindLen) & (~is_len | dist_ok) & 1u) != 0;
  if (kChecked) ok = ok && n <= r.avail();
  const u32 match_len = (e >> 16) + ((b32 >> l) & ((1u << nx) - 1u));
  length = (match_len & is_len) | (1u & ~is_len);
  const u32 dist = (d >> 16) + u32((b >> (s + dl)) & ((1u << dx) - 1u));
  lit_or_dist = (dist & is_len) | ((e >> 8) & 0xffu & ~is_len);
  r.advance(ok ? n : 0u);
  return ok;
}

// quick_token, extended to literal pairs: when the token is a literal whose
// successor is also a literal in the primary LUT and starts before `stop`,
// both are taken from the same window bits (the second lookup, which for a
// match reads its distance code, then reads the next literal/length code).
// Returns the tokens taken: 0 (nothing; the caller decodes with
// fast_token), 1 (length/x as quick_token gives them) or 2 (two literals:
// x and lit2, the second starting `first_bits` after the first).  The pair
// takes n <= 30 bits.
template <bool kChecked>
__host__ __device__ __forceinline__ u32 quick_pair(const HuffTable<288, 10>& ll, const HuffTable<32, 8>& dd,
                                          Win4<kChecked>& r, u32 stop, u32& length, u32& x,
                                          u32& lit2, u32& first_bits) {
  const u64 b = r.bits64();
  const u32 b32 = u32(b);
  const u32 e = ll.primary[b32 & 1023u];
  const u32 l = e & 15u;
  const u32 kind = (e >> 4) & 3u;
  const bool is_len = kind == kKindLen;
  const u32 nx = is_len ? (e >> 8) & 15u : 0u;
  const u32 s = l + nx;  // <= 20
  // One lookup serves both cases: a match's distance code, or the code
  // after a literal.
  const u32* p2 = is_len ? &dd.primary[(b32 >> s) & 255u] : &ll.primary[u32(b >> l) & 1023u];
  const u32 e2 = *p2;
  const u32 l2 = e2 & 15u, dx = (e2 >> 4) & 15u;
  const bool lit = kind == kKindLit && l != 0;
  bool pair = lit && l2 != 0 && dx == kKindLit && r.pos() + l < stop;  // dx: the code's kind
  if (kChecked) pair = pair && l + l2 <= r.avail();
  const bool dist_ok = l2 != 0 && !(e2 & 0x100u);
  const u32 n = is_len ? s + l2 + dx : l + (pair ? l2 : 0u);
  bool ok = lit || (is_len && l != 0 && dist_ok);
  if (kChecked) ok = ok && n <= r.avail();
  length = is_len ? (e >> 16) + ((b32 >> l) & ((1u << nx) - 1u)) : 1u;
  x = is_len ? (e2 >> 16) + u32((b >> (s + l2)) & ((1u << dx) - 1u)) : (e >> 8) & 0xffu;
  lit2 = (e2 >> 8) & 0xffu;
  first_bits = l;
  r.advance(ok ? n : 0u);
  return ok ? (pair ? 2u : 1u) : 0u;
}

// fast_token over the window's registers: the same results, errors and
// error order, but every bit comes from bits64() (a token takes at most 48
// bits), so a token that misses quick_pair costs its table reads only, not
// the word loads of a second reader.  On success the window moves past the
// token (an EOB included); on an error it stays where it was.
template <bool kChecked>
__host__ __device__ __forceinline__ u32 window_token(const HuffTable<288, 10>& ll,
                                                    const HuffTable<32, 8>& dd, Win4<kChecked>& r,
                                                    u32& lit, u32& length, u32& distance) {
  length = 0;
  distance = 0;
  const u64 b = r.bits64();
  const u32 avail = r.avail();
  u32 e = ll.primary[u32(b) & 1023u];
  u32 l = e & 15u;
  if (!l) {
    u32 err = 0;
    const i32 sym = long_code(ll, u32(b), avail, l, err);
    if (sym < 0) return err;
    e = fast_ll_entry(u32(sym), l);
  }
  if (l > avail) return kTruncated;
  u32 used = l;
  const u32 kind = (e >> 4) & 3u;
  if (kind == kKindLit || kind == kKindEob) {
    if (kind == kKindLit) {
      lit = (e >> 8) & 0xffu;
      length = 1;
    }
    r.advance(used);
    return kOk;
  }
  if (kind == kKindBad) return kBadSymbol;
  const u32 nx = (e >> 8) & 15u;
  if (nx > avail - used) return kTruncated;
  length = (e >> 16) + (u32(b >> used) & ((1u << nx) - 1u));
  used += nx;
  const u32 bd = u32(b >> used);
  u32 d = dd.primary[bd & 255u];
  u32 dl = d & 15u;
  if (!dl) {
    u32 err = 0;
    const i32 sym = long_code(dd, bd, avail - used, dl, err);
    if (sym < 0) return err;
    d = fast_d_entry(u32(sym), dl);
  }
  if (dl > avail - used) return kTruncated;
  used += dl;
  if (d & 0x100u) return kBadSymbol;
  const u32 dx = (d >> 4) & 15u;
  if (dx > avail - used) return kTruncated;
  distance = (d >> 16) + (u32(b >> used) & ((1u << dx) - 1u));
  r.advance(used + dx);
  return kOk;
}

// quick_pair extended to a third literal after a pair (a third lookup in
// the same window bits, taken when that code too is a literal in the primary
// table and starts before `stop`): returns 0-3 tokens taken; with 3, lit3 is
// the third literal.  The second and third literals start first_bits and
// pair_bits after the first token's start.
template <bool kChecked>
__host__ __device__ __forceinline__ u32 quick_triple(const HuffTable<288, 10>& ll,
                                                     const HuffTable<32, 8>& dd, Win4<kChecked>& r,
                                                     u32 stop, u32& length, u32& x, u32& lit2,
                                                     u32& lit3, u32& first_bits, u32& pair_bits) {
  const u32 p = r.pos();
  const u64 b = r.bits64();
  const u32 got = quick_pair<kChecked>(ll, dd, r, stop, length, x, lit2, first_bits);
  const u32 l12 = r.pos() - p;  // both codes
  pair_bits = l12;
  if (got != 2) return got;
  const u32 e3 = ll.primary[u32(b >> l12) & 1023u];
  const u32 l3 = e3 & 15u;
  bool third = l3 != 0 && ((e3 >> 4) & 3u) == kKindLit && p + l12 < stop;
  if (kChecked) third = third && l3 <= r.avail();
  lit3 = (e3 >> 8) & 0xffu;
  r.advance(third ? l3 : 0u);
  return third ? 3u : 2u;
}

// Adler-32 partial sums of output bytes as they are produced: S = sum of the
// bytes, W = sum of (end - position) * byte, where `end` is the stream's end
// position, so that a byte at stream position i weighs n - i.  W is reduced
// mod 65521 before it can wrap.
struct AdlerAcc {
  u64 s = 0, w = 0;
  __host__ __device__ __forceinline__ void add_byte(u32 x, u64 weight) {
    s += x;
    w += weight * x;
    if (w >> 62) w %= kAdlerMod;
  }
  // add_byte without the reduction: the caller folds (below) before w can
  // pass 2^63 (a weight stays below 2^34, a product below 2^42).
  __host__ __device__ __forceinline__ void add_byte_unfolded(u32 x, u64 weight) {
    s += x;
    w += weight * x;
  }
  __host__ __device__ __forceinline__ void fold() { w %= kAdlerMod; }
  // Sixteen bytes whose first weighs `weight0` (each next one 1 less).
  __host__ __device__ __forceinline__ void add16(const uint4& q, u64 weight0) {
    const u32 words[4] = {q.x, q.y, q.z, q.w};
    u32 cs = 0, cl = 0;
#pragma unroll
    for (u32 k = 0; k < 4; ++k) {
      const u32 ws = byte_dot(words[k], 0x01010101u);
      cs += ws;
      cl += byte_dot(words[k], 0x03020100u) + 4 * k * ws;
    }
    s += cs;
    w += weight0 * cs - cl;
    if (w >> 62) w %= kAdlerMod;
  }
};

// dst[0, n) = src[0, n) by threads first, first + step, ...: bytes up to
// dst's first 16-byte boundary, then 16-byte stores of source dwords
// realigned with v_alignbyte, then the tail bytes.  Source dwords are read
// only while they lie before src_end.
// With `acc`, every copied byte is also added to the Adler-32 sums; the
// destination's first byte weighs `weight0`.
__host__ __device__ __forceinline__ void copy_bytes(u8* dst, const u8* src, u64 n, const u8* src_end,
                                           u32 first, u32 step, AdlerAcc* acc = nullptr,
                                           u64 weight0 = 0) {
  const u64 align = (16 - (reinterpret_cast<uintptr_t>(dst) & 15)) & 15;
  const u64 head = n < align ? n : align;
  for (u64 i = first; i < head; i += step) {
    dst[i] = src[i];
    if (acc) acc->add_byte(src[i], weight0 - i);
  }
  const uintptr_t s0 = reinterpret_cast<uintptr_t>(src + head);
  const u32* s32 = reinterpret_cast<const u32*>(s0 & ~uintptr_t(3));
  const u32 sh = u32(s0 & 3);
  // Block j reads dwords j*4 .. j*4 + 4 of s32: all of them before src_end.
  const u64 avail_words = (reinterpret_cast<uintptr_t>(src_end) - (s0 & ~uintptr_t(3))) / 4;
  u64 blocks = (n - head) / 16;
  if (avail_words < 5) blocks = 0;
  else if (blocks > (avail_words - 5) / 4 + 1) blocks = (avail_words - 5) / 4 + 1;
  for (u64 j = first; j < blocks; j += step) {
    const u32* q = s32 + 4 * j;
    const u32 x0 = q[0], x1 = q[1], x2 = q[2], x3 = q[3], x4 = q[4];
    uint4 o;
    o.x = funnel_bytes(x1, x0, sh);
    o.y = funnel_bytes(x2, x1, sh);
    o.z = funnel_bytes(x3, x2, sh);
    o.w = funnel_bytes(x4, x3, sh);
    *reinterpret_cast<uint4*>(dst + head + 16 * j) = o;
    if (acc) acc->add16(o, weight0 - head - 16 * j);
  }
  for (u64 i = head + 16 * blocks + first; i < n; i += step) {
    dst[i] = src[i];
    if (acc) acc->add_byte(src[i], weight0 - i);
  }
}

// zlib wrapper (RFC 1950) checks, in the reference's precedence order.
__host__ __device__ __forceinline__ u32 check_framing(const u8* in, u64 size, u32& window,
                                                       u32& wanted) {
  window = 0;
  wanted = 0;
  if (size < 8) return kTruncatedZlib;
  const u32 cmf = in[0], flg = in[1];
  if (cmf == 0x1f && flg == 0x8b) return kUnsupportedGzip;
  if ((cmf & 15) != 8 || (cmf >> 4) > 7 || (cmf * 256 + flg) % 31) return kInvalidHeader;
  if (flg & 32) return kUnsupportedDictionary;
  window = 1u << ((cmf >> 4) + 8);
  wanted = (u32(in[size - 4]) << 24) | (u32(in[size - 3]) << 16) | (u32(in[size - 2]) << 8) |
           u32(in[size - 1]);
  return kOk;
}

// ---- fixed-Huffman tokens without tables ----------------------------------------
// One token of a fixed-Huffman block (RFC 1951 3.2.6) at the low bits of `b`
// (LSB first; at least 31 meaningful bits, the longest fixed token).  The
// first nine stream bits, reversed, are the code MSB first: 7-bit codes
// 0000000-0010111 are symbols 256-279, 8-bit 00110000-10111111 literals
// 0-143 and 11000000-11000111 symbols 280-287, 9-bit 110010000-111111111
// literals 144-255.  Distance codes are five bits.  Returns kKindLit (value =
// the byte), kKindLen (length, value = distance), kKindEob or kKindBad
// (symbols 286-287, distance codes 30-31), and the bits the token takes.
__host__ __device__ __forceinline__ u32 fixed_token(u64 b, u32& nbits, u32& length, u32& value) {
  const u32 r9 = __builtin_bitreverse32(u32(b)) >> 23;
  u32 sym, l;
  if ((r9 >> 2) < 24) {
    sym = 256 + (r9 >> 2);
    l = 7;
  } else if ((r9 >> 1) < 0xC0) {
    sym = (r9 >> 1) - 0x30;
    l = 8;
  } else if ((r9 >> 1) < 0xC8) {
    sym = 280 + ((r9 >> 1) - 0xC0);
    l = 8;
  } else {
    sym = r9 - 256;  // 0x190 -> 144
    l = 9;
  }
  length = 1;
  value = sym;
  nbits = l;
  if (sym < 256) return kKindLit;
  if (sym == 256) return kKindEob;
  if (sym > 285) return kKindBad;
  const u32 li = sym - 257, e = length_extra(li);
  length = length_base(li) + (u32(b >> l) & ((1u << e) - 1u));
  l += e;
  const u32 d = __builtin_bitreverse32(u32(b >> l)) >> 27;
  l += 5;
  nbits = l;
  if (d > 29) return kKindBad;
  const u32 de = dist_extra(d);
  value = dist_base(d) + (u32(b >> l) & ((1u << de) - 1u));
  nbits = l + de;
  return kKindLen;
}

// ---- wrapper formats -----------------------------------------------------------
// zlib (RFC 1950), raw DEFLATE (RFC 1951 alone) and gzip (RFC 1952, one
// member).  The drop-in zlib entry points use kFormatZlib without a
// dictionary, whose statuses are the reference's (check_framing above).
enum Format : u32 { kFormatZlib = 0, kFormatRaw = 1, kFormatGzip = 2 };
enum Check : u32 { kCheckNone = 0, kCheckAdler = 1, kCheckCrc = 2 };

struct Frame {
  u64 body;      // first body byte
  u64 body_len;  // body bytes, up to the trailer
  u32 window;    // largest allowed back-reference distance
  u32 check;     // trailer check (Check)
  u32 wanted;    // expected Adler-32 or CRC-32
  u32 isize;     // gzip: output size mod 2^32
  u32 dict_id;   // zlib with FDICT: the DICTID
  u32 needs_dict;
};

// CRC-32 (the gzip polynomial, reflected: bit 31 holds x^0) ---------------------
constexpr u32 kCrcPoly = 0xEDB88320u;

__host__ __device__ __forceinline__ u32 crc_byte_update(u32 c, u32 byte) {
  c ^= byte;
#pragma unroll
  for (u32 k = 0; k < 8; ++k) c = (c >> 1) ^ ((c & 1u) ? kCrcPoly : 0u);
  return c;
}

// a * b mod P over GF(2), both in the reflected representation.
__host__ __device__ inline u32 crc_mul(u32 a, u32 b) {
  u32 p = 0;
  for (u32 i = 0; i < 32; ++i) {
    if ((a >> (31 - i)) & 1u) p ^= b;
    b = (b >> 1) ^ ((b & 1u) ? kCrcPoly : 0u);  // b * x
  }
  return p;
}

// x^(8n) mod P: the factor that appends n bytes after a register value.
__host__ __device__ inline u32 crc_shift_bytes(u64 n) {
  u32 r = 1u << 31;   // x^0
  u32 f = 1u << 23;   // x^8
  while (n) {
    if (n & 1u) r = crc_mul(r, f);
    f = crc_mul(f, f);
    n >>= 1;
  }
  return r;
}

// CRC-32 of a message from `linear`, its register value computed from 0 (no
// initial or final inversion): the initial all-ones register contributes
// ~0 * x^(8n), and the result is inverted.
__host__ __device__ inline u32 crc_finish(u32 linear, u64 n) {
  return ~(crc_mul(0xffffffffu, crc_shift_bytes(n)) ^ linear);
}

// Parses the wrapper of a `size`-byte stream in `format`.  `have_dict` says
// whether the caller supplied a preset dictionary.  Statuses follow the zlib
// route's order: truncated wrapper 14, bad header 15, gzip magic under zlib 16,
// a preset dictionary nobody supplied 17.
// With `fields_at`, a gzip header's FNAME, FCOMMENT and FHCRC fields are
// left to the caller: *fields_at is where they start (0 when the header has
// none), and f holds everything else (f.body and f.body_len are set once
// the fields are parsed).  Without it, they are parsed here, byte by byte.
__host__ __device__ inline u32 parse_frame(const u8* in, u64 size, u32 format, bool have_dict,
                                           Frame& f, u64* fields_at = nullptr) {
  if (fields_at) *fields_at = 0;
  f.body = 0;
  f.body_len = 0;
  f.window = 32768;
  f.check = kCheckNone;
  f.wanted = 0;
  f.isize = 0;
  f.dict_id = 0;
  f.needs_dict = 0;
  if (format == kFormatRaw) {
    f.body_len = size;
    return kOk;
  }
  if (format == kFormatZlib) {
    u32 window, wanted;
    const u32 st = check_framing(in, size, window, wanted);
    const bool fdict = st == kUnsupportedDictionary;
    if (st && !(fdict && have_dict)) return st;
    f.window = fdict ? 1u << ((in[0] >> 4) + 8) : window;
    f.check = kCheckAdler;
    f.wanted = (u32(in[size - 4]) << 24) | (u32(in[size - 3]) << 16) | (u32(in[size - 2]) << 8) |
               u32(in[size - 1]);
    f.body = 2;
    if (fdict) {
      if (size < 12) return kTruncatedZlib;
      f.needs_dict = 1;
      f.dict_id = (u32(in[2]) << 24) | (u32(in[3]) << 16) | (u32(in[4]) << 8) | u32(in[5]);
      f.body = 6;
    }
    f.body_len = size - f.body - 4;
    return kOk;
  }
  // gzip: ID1 ID2 CM FLG MTIME(4) XFL OS [XLEN extra] [name\0] [comment\0] [CRC16],
  // body, CRC-32 and ISIZE (little endian).
  if (size < 18) return kTruncatedZlib;
  if (in[0] != 0x1f || in[1] != 0x8b || in[2] != 8 || (in[3] & 0xe0)) return kInvalidHeader;
  const u32 flg = in[3];
  const u64 limit = size - 8;  // the header ends before the trailer
  u64 p = 10;
  if (flg & 4) {
    if (p + 2 > limit) return kTruncatedZlib;
    p += 2 + (u64(in[p]) | (u64(in[p + 1]) << 8));
    if (p > limit) return kTruncatedZlib;
  }
  f.check = kCheckCrc;
  f.wanted = u32(in[size - 8]) | (u32(in[size - 7]) << 8) | (u32(in[size - 6]) << 16) |
             (u32(in[size - 5]) << 24);
  f.isize = u32(in[size - 4]) | (u32(in[size - 3]) << 8) | (u32(in[size - 2]) << 16) |
            (u32(in[size - 1]) << 24);
  if (fields_at && (flg & (2 | 8 | 16))) {
    *fields_at = p;
    return kOk;
  }
  for (u32 field = 8; field <= 16; field <<= 1) {  // FNAME, then FCOMMENT
    if (!(flg & field)) continue;
    while (p < limit && in[p]) ++p;
    if (p >= limit) return kTruncatedZlib;
    ++p;
  }
  if (flg & 2) {
    if (p + 2 > limit) return kTruncatedZlib;
    u32 c = 0xffffffffu;
    for (u64 i = 0; i < p; ++i) c = crc_byte_update(c, in[i]);
    if (((~c) & 0xffffu) != (u32(in[p]) | (u32(in[p + 1]) << 8))) return kInvalidHeader;
    p += 2;
  }
  f.body = p;
  f.body_len = limit - p;
  return kOk;
}

__device__ __forceinline__ u32 lane_id() { return __lane_id(); }

// Lanes below this one in the wave.
__device__ __forceinline__ u64 lanemask_lt() {
  const u32 lane = lane_id();
  return lane ? (~0ull >> (64 - lane)) : 0ull;
}

// Status of a wave header walk that would read past its words.
constexpr u32 kHeaderWalkStuck = 0xffffffffu;

// Position of code-length symbol s in the header's order of lengths (the
// inverse of cl_order), 5 bits per symbol.
__device__ __forceinline__ u32 cl_index(u32 s) {
  return s < 12 ? u32((0x520c429d2b6be23ull >> (5 * s)) & 31)
                : u32((0x820941ccull >> (5 * (s - 12))) & 31);
}

// 32 bits from bit q of a dword array (words q/32 and q/32 + 1).
__device__ __forceinline__ u32 stage_bits(const u32* words, u32 q) {
  return __builtin_amdgcn_alignbit(words[(q >> 5) + 1], words[q >> 5], q & 31);
}

// Fields and code-length code of a dynamic header, by the whole wave, from
// `count` dwords in which body bit b is bit b - bit0 (mod 2^64); `start` is
// the body bit after BTYPE.  Returns false when a read could pass the
// given words or the body end (the caller then runs parse_dynamic_lengths
// from the same start, so statuses and their order are that function's);
// otherwise sets err (kBadTree: HLIT above 29 or an incomplete code-length
// code, as build_cl_table rules) and `after` (the bit after the fields read),
// and with err == 0 the code-length table's
// primary LUT is built and p (first length's bit in the words) / lim (read
// limit there) / nl / nd describe the walk over the lengths.  Lane s < 19 holds symbol s: its length, its rank among the
// symbols of that length (ballots) and so its canonical code, whose LUT
// entries it fills.
template <class Tables>  // DecodeTables, or any type with its `cl` table and `lens`
__device__ inline bool header_prelude_wave(const u32* words, u64 bit0, u32 count,
                                           Tables& tables, u64 len, u64 start, u32& nl,
                                           u32& nd, u32& err, u64& after, u32& p, u32& lim32) {
  const u32 lane = lane_id();
  // A read of bit q touches words q/32 and q/32 + 1.
  const u64 staged = count > 1 ? u64(count - 1) * 32 : 0;
  const u64 body_end = len * 8 - bit0;
  const u64 lim = min(staged, body_end);
  const u64 q0 = start - bit0;
  if (q0 + 14 > lim) return false;
  const u32 f = stage_bits(words, u32(q0));
  const u32 hlit = f & 31u, hdist = (f >> 5) & 31u, hclen = (f >> 10) & 15u;
  nl = hlit + 257;
  nd = hdist + 1;
  const u32 nc = hclen + 4;
  after = start + 14;
  if (nl > 286) {
    err = kBadTree;
    return true;
  }
  if (q0 + 14 + 3 * nc > lim) return false;
  after += 3 * nc;
  u32 l = 0;
  if (lane < 19) {
    const u32 k = cl_index(lane);
    if (k < nc) l = stage_bits(words, u32(q0 + 14 + 3 * k)) & 7u;
  }
  // Kraft sum and the first canonical code of each length.
  u32 kraft = 0, code = 0, mine = 0, count_prev = 0;
#pragma unroll
  for (u32 k = 1; k < 8; ++k) {
    const u64 b = __ballot(l == k);
    const u32 c = u32(__popcll(b));
    code = (code + count_prev) << 1;  // first code of length k
    if (l == k) mine = code + u32(__popcll(b & lanemask_lt()));
    count_prev = c;
    kraft += c << (7 - k);
  }
  if (kraft != 128) {  // the code must be complete
    err = kBadTree;
    return true;
  }
  if (l) {
    const u32 e = (lane << 16) | l;
    for (u32 k = bit_reverse(mine, l); k < 128; k += 1u << l) tables.cl.primary[k] = e;
  }
  p = u32(q0 + 14 + 3 * nc);
  lim32 = u32(lim);
  err = kOk;
  wave_sync();
  return true;
}

// The code lengths of a dynamic header by the whole wave, after
// header_prelude_wave.  The code-length code is complete, so every 7-bit
// pattern starts a code: each lane decodes the symbol (and extra bits) at its
// own bit of a 64-bit batch.  The true path through the batch (its offsets,
// from 0, one hop per symbol) is the only serial part; the path lanes then
// place their runs together: the lengths before each (a prefix sum of the
// repeat counts), the value a 16 repeats (the last other symbol before it, a
// max scan), and the first path symbol that ends the walk (unreadable within
// the limit, a 16 first, a repeat past the end, or the last length).
// Lanes then fill the lengths from the runs (`runs`: LDS, >= 320 entries).
// Returns kOk, an error status (the one parse_dynamic_lengths gives: every
// read on the path lies before the limit), or kHeaderWalkStuck when the walk
// would read past it.  `p` advances to the bit after the lengths.
template <class Tables>
__device__ inline u32 header_lengths_wave(const u32* words, Tables& tables, u32* runs, u32 total,
                                   u32& p, u32 lim) {
  const u32 lane = lane_id();
  u32 i = 0, prev = 0, nruns = 0;
  while (i < total) {
    // This lane's symbol at bit p + lane: its advance (0: past the limit),
    // symbol and repeat count.
    const u32 q = p + lane;
    u32 adv = 0, sym = 0, rep = 1;
    if (q + 14 <= lim) {
      const u32 b = stage_bits(words, q);
      const u32 e = tables.cl.primary[b & 127];
      const u32 l = e & 15u;
      sym = e >> 16;
      const u32 x = b >> l;
      adv = sym < 16 ? l : sym == 16 ? l + 2 : sym == 17 ? l + 3 : l + 7;
      rep = sym < 16 ? 1u : sym == 16 ? 3 + (x & 3u) : sym == 17 ? 3 + (x & 7u) : 11 + (x & 127u);
      if (!l) adv = 0;
    }
    // The path's offsets (uniform hops).
    u64 path = 0;
    u32 off = 0;
    while (off < 64) {
      const u32 a = u32(__builtin_amdgcn_readlane(int(adv), int(off)));
      path |= 1ull << off;
      if (!a) break;
      off += a;
    }
    const bool on = (path >> lane) & 1;
    // Lengths before each path symbol.
    const u32 r_on = on ? rep : 0u;
    u32 incl = r_on;
#pragma unroll
    for (u32 o = 1; o < 64; o <<= 1) {
      const u32 y = __shfl_up(incl, o, 64);
      if (lane >= o) incl += y;
    }
    const u32 before = i + incl - r_on;
    // The first path symbol that ends the walk, and how.
    const bool stuck = !adv;
    const bool bad = (sym == 16 && before == 0) || before + rep > total;
    const u64 term = __ballot(on && (stuck || bad || before + rep == total));
    const u32 end = term ? u32(__builtin_ctzll(term)) : 64u;
    if (end < 64) {
      if (__builtin_amdgcn_readlane(int(stuck), int(end))) return kHeaderWalkStuck;
      if (__builtin_amdgcn_readlane(int(bad), int(end))) return kBadRepeat;
    }
    const u64 valid = end < 64 ? path & ((2ull << end) - 1) : path;
    // The value a 16 repeats: that of the last other path symbol before it
    // (17 and 18 give 0), or the value carried from the earlier batches.
    int last = (valid >> lane) & 1 && sym != 16 ? int(lane) : -1;
#pragma unroll
    for (u32 o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(last, o, 64);
      if (lane >= o && y > last) last = y;
    }
    const u32 src_sym = u32(__shfl(int(sym), last < 0 ? 0 : last, 64));
    const u32 base = last < 0 ? prev : src_sym < 16 ? src_sym : 0u;
    const u32 value = sym < 16 ? sym : sym == 16 ? base : 0u;
    if ((valid >> lane) & 1)
      runs[nruns + __popcll(valid & lanemask_lt())] = before | (value << 9) | (rep << 13);
    nruns += u32(__popcll(valid));
    const u32 tail = 63 - u32(__builtin_clzll(valid));
    i = u32(__builtin_amdgcn_readlane(int(before + rep), int(tail)));
    prev = u32(__builtin_amdgcn_readlane(int(value), int(tail)));
    p += end < 64 ? end + u32(__builtin_amdgcn_readlane(int(adv), int(end))) : off;
  }
  wave_sync();
  u32 status = kOk;
  for (u32 k = lane; k < nruns; k += 64) {
    const u32 e = runs[k];
    const u32 first = e & 511u, value = (e >> 9) & 15u, r = e >> 13;
    for (u32 j = 0; j < r; ++j) tables.lens[first + j] = u8(value);
  }
  wave_sync();
  if (!tables.lens[256]) status = kBadTree;
  wave_sync();
  return status;
}

}  // namespace hz
