// General-route decode: any valid zlib stream, parallel over Deflate blocks.
//
// Pipeline (all on one stream, no host synchronisation):
//   frame      framing checks, declared window, wanted Adler-32
//   discover   every bit offset: bit-parallel prefilter (BTYPE, HLIT, a
//              complete code-length code); ordered compaction (per-workgroup
//              lists, scan, gather) into a dense sorted array; exact header
//              validation with lanes refilled from the array (long headers
//              to a wave-per-header pass); valid offsets in order
//   headers    one wave per candidate: parse its header, build and store its
//              decode tables
//   describe   one 256-lane workgroup per candidate: speculative slices of
//              its blocks decoded in parallel, merged where decodings meet,
//              give every slice's true entry and output offset, the segment
//              end, size and status (up to the next candidate)
//   chain      one workgroup: path from bit 0 through the segment graph,
//              output prefixes; any anomaly defers to the exact walk
//   exact      serial walk with the reference's status precedence (runs only
//              when the fast chain did not accept the stream)
//   emit       one 256-lane workgroup per accepted segment decodes its slices
//              in parallel, writing output in place; a byte copied from
//              before its slice's start is marked unresolved with its root
//   resolve    rounds over the unresolved bitmask, each following up to 32
//              root links per byte
//   adler      vectorised Adler-32 partials, then the final status
//
// Status semantics restate the reference's general route: framing
// (native/codec_ffi.cu:304-329) > candidate overflow (344-360) > exact chain
// (select_chain, _decode_kernels.py:1226-1408) > emission history/window
// (parse_block<Emit>, 683-781; EmissionStatus codec_ffi.cu:405-435) > Adler-32
// (467-483).  Failed output is all zeros except on an Adler-32 mismatch.
#include <algorithm>

#include "deflate_common.h"
#include "kernels.h"

namespace hz {
namespace {

constexpr u32 kWave = 64;
constexpr u32 kNone = 0xffffffffu;
constexpr u32 kDiscThreads = 256;
constexpr u32 kDiscBytesPerThread = 8;
constexpr u32 kDiscRange = kDiscThreads * kDiscBytesPerThread;  // bytes per workgroup
constexpr u32 kDiscCap = 64;                                      // local list capacity
constexpr u32 kCoopMatch = 32;

struct State {
  u32 status;        // first error (framing, discovery, chain/exact)
  u32 window;
  u32 wanted;
  u32 chain_ok;      // fast chain accepted the stream
  u64 candidates;    // dynamic candidates + bit 0 (sorted list length)
  u64 seeds;         // stored-endpoint seeds (counted for the overflow check)
  u64 accepted;      // number of accepted segments
  u32 emit_status;
  u32 pad;
  u64 unresolved[2]; // unresolved bytes after emission / after the last resolve round
  u64 recs_used;     // block records handed out by describe
  u64 groups_used;   // 64-slot slice groups handed out by describe
  u64 precount;      // entries of the dense pre-candidate array
  u64 tables_used;   // stored per-block decode tables
  u64 dense_count;   // ranges whose valid headers alone overflow their list (kind 2)
  u64 start_bit;     // body bit of the first block (0 unless a wrapper field precedes it)
  u64 floor;         // lowest output position a back-reference may read (history allowed: 0)
  u32 isize;         // gzip: the trailer's ISIZE
  u32 pad2;
  // Open-ended decode (one member of a concatenation): the accepted path's
  // end bit and output bytes, which the trailer and the next member follow.
  u64 stream_end;
  u64 produced;
  // Long fixed-Huffman runs: regions deferred by describe, run records and
  // tile slots handed out by the walk.
  u64 fix_regions;
  u64 fix_runs;
  u64 fix_rt;
  u64 fix_tasks;  // remainder tasks queued by the summary pass
  u64 emit_units;  // emission units of long fixed runs queued for the unit pass
};

// An open-ended decode's stream may end before the input does (other members
// follow it) and produce fewer bytes than the output holds; `trailer` is the
// wrapper's trailer length, which must fit after the last block.  A
// `windowed` decode sees only a prefix of the input: when the fast chain does
// not accept it, it reports kTruncated at once (no exact walk), and the
// caller decodes the member again over the whole input.
struct OpenEnd {
  u32 open;
  u32 trailer;
  u32 windowed;
};

struct Segment {
  u64 start;      // bit offset of the first block
  u64 end;        // bit offset after the last block
  u64 prefix;     // output offset
  u64 size;       // output bytes
  u32 rec_first;  // first block record, or kNone: emit serially
  u32 rec_count;
};

// One block of a described segment; records of a segment are linked through
// `next`.  A fixed/dynamic block's token range is split into `lanes` slices
// held in linked groups of 64 slots: slice i of a group decodes tokens from
// slice_entry[64 * group + i] up to the next slice's entry (the last slice
// ends at the EOB) and writes at block output offset slice_off[64 * group + i].
struct BlockRec {
  u64 start;      // bit offset of the block header
  u64 data;       // first token bit (stored: first payload bit)
  u64 end;        // bit after the block
  u64 size;       // output bytes
  u32 type;
  u32 lanes;      // slices (fixed/dynamic)
  u32 group;      // first slice group
  u32 next;       // next record of the segment, or kNone
  u32 table;      // stored fast-format tables (BlockTables), or kNone
  u32 pad;
};

// Literal/length and distance tables of one block in the fast LUT format,
// stored by describe for emission.
struct BlockTables {
  HuffTable<288, 10> ll;
  HuffTable<32, 8> dd;
  u32 pad[2];
};

constexpr u32 kStageBytes = 16384;                 // LDS bitstream window per wave
constexpr u32 kStageMargin = 64;                   // bytes staged past the last slice
constexpr u32 kStageWords = (kStageBytes + kStageMargin) / 4 + 4;
constexpr u64 kMaxSlice = (u64(kStageBytes) * 8) / 64;
constexpr u32 kHeaderBytes = 640;  // > longest dynamic header (< 566 bytes)
constexpr u32 kHeaderWords = kHeaderBytes / 4 + 4;

// LDS copy of a bitstream range: words[] are consecutive aligned dwords of
// the input; body bit `bit0` is the first bit of words[0] (mod 2^64).
template <u32 W>
struct StageT {
  u32 words[W];
  u64 bit0;
  u32 count;
};
using Stage = StageT<kStageWords>;

// Stage the body bytes covering bits [bit0, bit1) plus `margin` bytes into LDS
// (capped at the body end and at the stage capacity).  Every thread of the
// workgroup takes part.
template <u32 W>
__device__ __forceinline__ void stage_range(const u8* body, u64 len, u64 bit0, u64 bit1, StageT<W>& sg,
                            u64 margin = kStageMargin) {
  const uintptr_t base = reinterpret_cast<uintptr_t>(body);
  const u64 first_word = (base + (bit0 >> 3)) >> 2;
  u64 last_byte = (bit1 + 7) / 8 + margin;
  if (last_byte > len) last_byte = len;
  const u64 end_word = (base + last_byte + 3) >> 2;  // words holding body bytes only
  u64 words = end_word > first_word ? end_word - first_word : 0;
  if (words > W) words = W;
  const u32* g = reinterpret_cast<const u32*>(first_word << 2);
  // Eight loads per thread in flight before the first store.
  constexpr u32 kBatch = 8;
  for (u64 i0 = threadIdx.x; i0 < words; i0 += kBatch * blockDim.x) {
    u32 x[kBatch];
#pragma unroll
    for (u32 j = 0; j < kBatch; ++j) {
      const u64 i = i0 + u64(j) * blockDim.x;
      x[j] = i < words ? g[i] : 0u;
    }
#pragma unroll
    for (u32 j = 0; j < kBatch; ++j) {
      const u64 i = i0 + u64(j) * blockDim.x;
      if (i < words) sg.words[i] = x[j];
    }
  }
  if (!threadIdx.x) {
    sg.count = u32(words);
    sg.bit0 = (first_word << 5) - (u64(base) << 3);  // body bit of word 0, mod 2^64
  }
}

// Reader over staged words whose positions are body bits; bits outside the
// staged words read as zero and avail() still reflects the real body end.
template <u32 W>
__device__ __forceinline__ BitIn staged_reader(const StageT<W>& sg, u64 len, u64 pos) {
  BitIn r;
  r.words = sg.words;
  r.base_bit = u64(0) - sg.bit0;
  r.total = len * 8;
  r.wlimit = sg.count;
  r.seek(pos);
  return r;
}

// True if the staged words hold every byte of bits [bit0, bit1) plus margin
// (or up to the body end).
template <u32 W>
__device__ __forceinline__ bool staged_covers(const StageT<W>& sg, const u8* body, u64 len,
                                              u64 bit0, u64 bit1, u64 margin = kStageMargin) {
  const u64 lo = sg.bit0, have = u64(sg.count) * 32;
  u64 need_end = ((bit1 + 7) / 8 + margin) * 8;
  if (need_end > len * 8) need_end = len * 8;
  return bit0 >= lo && bit0 - lo < have && need_end - lo <= have;
}

// 64 bits of the body starting at bit `pos` from the stage (zeros outside).
template <u32 W>
__device__ __forceinline__ u64 staged_u64(const StageT<W>& sg, u64 pos) {
  const u64 a = pos - sg.bit0;
  const u64 w = a >> 5;
  const u32 sh = u32(a & 31);
  const u64 w0 = w < sg.count ? sg.words[w] : 0u;
  const u64 w1 = w + 1 < sg.count ? sg.words[w + 1] : 0u;
  const u64 w2 = w + 2 < sg.count ? sg.words[w + 2] : 0u;
  const u64 lo = w0 | (w1 << 32);
  return sh ? (lo >> sh) | (w2 << (64 - sh)) : lo;
}


__device__ __forceinline__ u64 load_window_word(const u8* body, u64 len, u64 byte) {
  // Eight bytes starting at `byte`; bytes past the body read as zero.
  u64 v = 0;
  if (byte + 8 <= len) {
#pragma unroll
    for (u32 j = 0; j < 8; ++j) v |= u64(body[byte + j]) << (8 * j);
  } else {
    for (u32 j = 0; j < 8; ++j)
      if (byte + j < len) v |= u64(body[byte + j]) << (8 * j);
  }
  return v;
}

__device__ __forceinline__ u64 funnel(u64 lo, u64 hi, u32 k) {
  return k ? (lo >> k) | (hi << (64 - k)) : lo;
}

// Copy of the literal/length and distance tables, as words, by threads
// first, first + kStep, ...: every load of a thread is issued before its
// stores, so the copy waits for memory once.
template <u32 kStep>
__device__ __forceinline__ void copy_tables(u32* dll, u32* ddd, const u32* sll, const u32* sdd,
                                            u32 first) {
  constexpr u32 kL = sizeof(HuffTable<288, 10>) / 4, kD = sizeof(HuffTable<32, 8>) / 4;
  constexpr u32 kRl = (kL + kStep - 1) / kStep, kRd = (kD + kStep - 1) / kStep;
  u32 vl[kRl], vd[kRd];
#pragma unroll
  for (u32 k = 0; k < kRl; ++k) vl[k] = first + k * kStep < kL ? sll[first + k * kStep] : 0u;
#pragma unroll
  for (u32 k = 0; k < kRd; ++k) vd[k] = first + k * kStep < kD ? sdd[first + k * kStep] : 0u;
#pragma unroll
  for (u32 k = 0; k < kRl; ++k)
    if (first + k * kStep < kL) dll[first + k * kStep] = vl[k];
#pragma unroll
  for (u32 k = 0; k < kRd; ++k)
    if (first + k * kStep < kD) ddd[first + k * kStep] = vd[k];
}

// Exact validity of a dynamic header whose BTYPE bits were already checked:
// the same outcome as building all three tables (huff_build rules), computed
// with Kraft sums instead of tables.  `lut` is a thread's 128-entry LDS table
// with entries `stride` bytes apart (interleaved across threads, so the
// threads of a wave hit different banks).
__device__ __forceinline__ bool dynamic_header_fields_valid(BitIn& r, u8* lut, u32 stride) {
  u32 hlit, hdist, hclen;
  if (!r.take(5, hlit) || !r.take(5, hdist) || !r.take(4, hclen)) return false;
  const u32 nl = hlit + 257, nd = hdist + 1, nc = hclen + 4;
  if (nl > 286) return false;
  u64 pack = 0;  // 3-bit length per code-length symbol
  u32 kraft = 0;
  for (u32 i = 0; i < nc; ++i) {
    u32 v;
    if (!r.take(3, v)) return false;
    pack |= u64(v) << (3 * cl_order(i));
    if (v) kraft += 128u >> v;
  }
  if (kraft != 128) return false;
  // Canonical codes of the code-length alphabet into a 7-bit LUT (entry =
  // symbol | length << 5); counts and next codes packed in registers.
  u64 cnt = 0;
  for (u32 s = 0; s < 19; ++s) cnt += 1ull << (8 * ((pack >> (3 * s)) & 7));
  u64 next = 0;
  u32 code = 0;
  for (u32 l = 1; l < 8; ++l) {
    code = (code + (l > 1 ? u32(cnt >> (8 * (l - 1))) & 0xff : 0u)) << 1;
    next |= u64(code) << (8 * l);
  }
  for (u32 s = 0; s < 19; ++s) {
    const u32 l = (pack >> (3 * s)) & 7;
    if (!l) continue;
    const u32 c = u32(next >> (8 * l)) & 0xff;
    next += 1ull << (8 * l);
    for (u32 k = bit_reverse(c, l); k < 128; k += 1u << l) lut[k * stride] = u8(s | (l << 5));
  }
  u32 ll_kraft = 0, ll_nnz = 0, d_kraft = 0, d_nnz = 0, eob = 0, prev = 0;
  u32 i = 0;
  const u32 total = nl + nd;
  while (i < total) {
    const u32 e = lut[r.peek(7) * stride];
    const u32 l = e >> 5, sym = e & 31;
    if (u64(l) > r.avail()) return false;
    r.drop(l);
    u32 repeat, value, x;
    if (sym < 16) {
      repeat = 1;
      value = sym;
    } else if (sym == 16) {
      if (!i) return false;
      if (!r.take(2, x)) return false;
      repeat = x + 3;
      value = prev;
    } else if (sym == 17) {
      if (!r.take(3, x)) return false;
      repeat = x + 3;
      value = 0;
    } else {
      if (!r.take(7, x)) return false;
      repeat = x + 11;
      value = 0;
    }
    if (repeat > total - i) return false;
    if (value) {
      const u32 in_ll = i < nl ? min(repeat, nl - i) : 0u;
      const u32 in_d = repeat - in_ll;
      ll_kraft += in_ll << (15 - value);
      ll_nnz += in_ll;
      d_kraft += in_d << (15 - value);
      d_nnz += in_d;
      if (i <= 256 && 256 < i + repeat) eob = 1;
      // Kraft sums only grow: an oversubscribed code can never become valid.
      if (ll_kraft > (1u << 15) || d_kraft > (1u << 15)) return false;
    }
    prev = value;
    i += repeat;
  }
  if (!eob) return false;
  const bool ll_ok = ll_kraft == (1u << 15) || (ll_nnz == 1 && ll_kraft == (1u << 14));
  const bool d_ok = d_nnz == 0 || d_kraft == (1u << 15) || (d_nnz == 1 && d_kraft == (1u << 14));
  return ll_ok && d_ok;
}

// Exact validity of the dynamic header at `start` (BTYPE already checked),
// reading global memory.
__device__ bool dynamic_header_valid(const u8* body, u64 len, u64 start, u8* lut, u32 stride) {
  BitIn r;
  r.init(body, len, start + 3);
  return dynamic_header_fields_valid(r, lut, stride);
}

// Stored-block endpoint seed at `byte` (counted like the reference's discovery,
// _decode_kernels.py:1019-1038).
__device__ __forceinline__ bool stored_seed(const u8* body, u64 len, u64 byte) {
  if (!byte || len - byte < 5) return false;
  const u32 n = body[byte] | (u32(body[byte + 1]) << 8);
  const u32 comp = body[byte + 2] | (u32(body[byte + 3]) << 8);
  if ((n ^ comp) != 0xffffu || u64(n) + 4 >= len - byte) return false;
  u32 before = u32(body[byte - 1]) << 8;
  if (byte >= 2) before |= body[byte - 2];
  bool possible = false;
  for (u32 gap = 3; gap <= 10; ++gap)
    if (byte * 8 >= gap && ((before >> (17 - gap)) & 3u) == 0) possible = true;
  return possible && ((body[byte + 4 + n] >> 1) & 3u) == 1;
}

// stage_range split in two, so that a range's words can be loaded into
// registers (kPer per thread) while the previous range is still in use, and
// stored into the stage later.
template <u32 W, u32 kPer>
struct StagePrefetch {
  u32 x[kPer];
  u64 first_word;
  u32 words;
  __device__ __forceinline__ void load(const u8* body, u64 len, u64 bit0, u64 bit1, u64 margin) {
    const uintptr_t base = reinterpret_cast<uintptr_t>(body);
    first_word = (base + (bit0 >> 3)) >> 2;
    u64 last_byte = (bit1 + 7) / 8 + margin;
    if (last_byte > len) last_byte = len;
    const u64 end_word = (base + last_byte + 3) >> 2;  // words holding body bytes only
    u64 n = end_word > first_word ? end_word - first_word : 0;
    words = u32(n > W ? W : n);
    const u32* g = reinterpret_cast<const u32*>(first_word << 2);
#pragma unroll
    for (u32 j = 0; j < kPer; ++j) {
      const u32 i = threadIdx.x + j * blockDim.x;
      x[j] = i < words ? g[i] : 0u;
    }
  }
  __device__ __forceinline__ void store(StageT<W>& sg, const u8* body) const {
#pragma unroll
    for (u32 j = 0; j < kPer; ++j) {
      const u32 i = threadIdx.x + j * blockDim.x;
      if (i < words) sg.words[i] = x[j];
    }
    if (!threadIdx.x) {
      sg.count = words;
      sg.bit0 = (first_word << 5) - (u64(reinterpret_cast<uintptr_t>(body)) << 3);
    }
  }
};

// Bytes past a workgroup's range staged for the prefilter: the fields it
// reads end 3 + 14 + 57 bits after a position of the range's last byte.
constexpr u32 kPreMargin = 24;
constexpr u32 kPreStageWords = (kDiscRange + kPreMargin + 32) / 4;
constexpr u32 kSurvivorCap = 1024;  // prefilter survivors a wave checks per pass
using PreStage = StageT<kPreStageWords>;
// Pre-candidate entries: bit offset, plus this flag once the header is known valid.
constexpr u64 kValidBit = 1ull << 62;
constexpr u64 kPosMask = kValidBit - 1;
constexpr u32 kKindShift = 30;  // wg_count: count | kind << 30
constexpr u32 kCountMask = (1u << kKindShift) - 1;

// Kraft sums of three 3-bit code lengths (index: l0 | l1 << 3 | l2 << 6).
__device__ __forceinline__ void build_kraft3(u16* kraft3) {
  for (u32 i = threadIdx.x; i < 512; i += blockDim.x) {
    u32 k = 0;
    for (u32 j = 0; j < 3; ++j) {
      const u32 l = (i >> (3 * j)) & 7;
      if (l) k += 128u >> l;
    }
    kraft3[i] = u16(k);
  }
}

// Prefilter of the 64 bit offsets of bytes [b0, b0 + 8): BTYPE == 2,
// HLIT <= 29 and a complete code-length code (Kraft sum of the HCLEN lengths
// == 128).  Every valid dynamic header passes; about 0.1 % of random offsets
// do.  Bit offset 0 is excluded (it is always a candidate).
// The offsets of a thread's 64 (body bits 8*b0 .. 8*b0+63) that may be
// candidates: those after `s0`, the first block's bit.  `first` gets s0's own
// bit when it lies here: it is always a candidate, whatever its block type.
__device__ __forceinline__ u64 start_mask(u64 s0, u64 b0, u64& first) {
  const u64 lo = b0 * 8;
  first = 0;
  if (s0 >= lo + 64) return 0;
  u64 m = s0 > lo ? ~0ull << (s0 - lo) : ~0ull;
  if (s0 >= lo) {
    first = 1ull << (s0 - lo);
    m &= ~first;
  }
  return m;
}

__device__ u64 prefilter_mask(u64 len, u64 b0, const PreStage& sg, const u16* kraft3, u64 s0) {
  if (b0 >= len) return 0;
  const u64 w0 = staged_u64(sg, b0 * 8), w1 = staged_u64(sg, b0 * 8 + 64),
            w2 = staged_u64(sg, b0 * 8 + 128);
  // Bit k of s_j is stream bit (8*b0 + k + j).
  const u64 s1 = funnel(w0, w1, 1), s2 = funnel(w0, w1, 2);
  const u64 s4 = funnel(w0, w1, 4), s5 = funnel(w0, w1, 5);
  const u64 s6 = funnel(w0, w1, 6), s7 = funnel(w0, w1, 7);
  u64 m = ~s1 & s2 & ~(s4 & s5 & s6 & s7);  // BTYPE == 2 and HLIT <= 29
  const u64 bits_left = (len - b0) * 8;
  if (bits_left < 64) m &= (1ull << bits_left) - 1;
  u64 first;
  m &= start_mask(s0, b0, first);
  u64 out = 0;
  while (m) {
    const u32 k = __builtin_ctzll(m);
    m &= m - 1;
    const u64 a = funnel(w0, w1, k), b = funnel(w1, w2, k);
    const u32 nc = u32((a >> 13) & 15) + 4;
    const u64 lens = ((a >> 17) | (b << 47)) & ((1ull << (3 * nc)) - 1);
    u32 kraft = 0;
#pragma unroll
    for (u32 j = 0; j < 7; ++j) kraft += kraft3[(lens >> (9 * j)) & 511];
    if (kraft == 128) out |= 1ull << k;
  }
  return out;
}

// Exact header validation of the prefiltered offsets in `pre` (global reads).
__device__ u64 validate_mask(const u8* body, u64 len, u64 b0, u64 pre, u8* lut, u32 stride) {
  u64 valid = 0;
  while (pre) {
    const u32 k = __builtin_ctzll(pre);
    pre &= pre - 1;
    if (dynamic_header_valid(body, len, b0 * 8 + k, lut, stride)) valid |= 1ull << k;
  }
  return valid;
}

__device__ __forceinline__ u32 block_exclusive_scan(u32 v, u32* sh, u32& total) {
  // 256-thread exclusive scan: wave shuffles, then the four wave totals.
  const u32 t = threadIdx.x, lane = lane_id(), wave = t >> 6;
  u32 incl = v;
#pragma unroll
  for (u32 off = 1; off < 64; off <<= 1) {
    const u32 y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  if (lane == 63) sh[wave] = incl;
  __syncthreads();
  u32 before = 0;
  total = 0;
#pragma unroll
  for (u32 w = 0; w < kDiscThreads / 64; ++w) {
    const u32 c = sh[w];
    before += w < wave ? c : 0u;
    total += c;
  }
  __syncthreads();  // sh is reused by the next scan
  return before + incl - v;
}

// Exclusive scan of `count` u32 values (each masked by `mask`) into u64
// offsets by one 1024-thread workgroup; returns the total.  Tiles of
// kScanPer values per thread are staged in LDS with coalesced loads (padded
// so that the per-thread reads of consecutive values hit distinct banks),
// summed per thread, scanned by wave shuffles and combined over the 16 waves.
constexpr u32 kScanThreads = 1024;
constexpr u32 kScanPer = 8;
constexpr u32 kScanTile = kScanThreads * kScanPer;
struct ScanShared {
  u32 v[kScanTile + kScanTile / kScanPer];
  u32 wave[kScanThreads / 64];
};
__device__ __forceinline__ u32 scan_slot(u32 e) { return e + e / kScanPer; }

__device__ u64 wg_exclusive_scan(const u32* in, u32 mask, u64 count, u64* out, ScanShared& sh) {
  const u32 t = threadIdx.x, lane = lane_id(), wave = t >> 6;
  u64 carry = 0;
  // The next tile's values load while the current tile is scanned.
  u32 x[kScanPer];
#pragma unroll
  for (u32 k = 0; k < kScanPer; ++k) {
    const u64 e = k * kScanThreads + t;
    x[k] = e < count ? in[e] & mask : 0u;
  }
  for (u64 base = 0; base < count; base += kScanTile) {
    const u32 m = count - base < kScanTile ? u32(count - base) : kScanTile;
#pragma unroll
    for (u32 k = 0; k < kScanPer; ++k) sh.v[scan_slot(k * kScanThreads + t)] = x[k];
#pragma unroll
    for (u32 k = 0; k < kScanPer; ++k) {
      const u64 e = base + kScanTile + k * kScanThreads + t;
      x[k] = e < count ? in[e] & mask : 0u;
    }
    lds_barrier();  // LDS only: the next tile's loads stay in flight
    u32 mine = 0;
#pragma unroll
    for (u32 k = 0; k < kScanPer; ++k) mine += sh.v[scan_slot(t * kScanPer + k)];
    u32 incl = mine;
#pragma unroll
    for (u32 off = 1; off < 64; off <<= 1) {
      const u32 y = __shfl_up(incl, off, 64);
      if (lane >= off) incl += y;
    }
    if (lane == 63) sh.wave[wave] = incl;
    lds_barrier();
    u64 run = carry, tile_total = 0;
#pragma unroll
    for (u32 w = 0; w < kScanThreads / 64; ++w) {
      const u32 c = sh.wave[w];
      if (w < wave) run += c;
      tile_total += c;
    }
    run += incl - mine;
#pragma unroll
    for (u32 k = 0; k < kScanPer; ++k) {
      const u32 e = t * kScanPer + k;
      if (e < m) out[base + e] = run;
      run += sh.v[scan_slot(e)];
    }
    carry += tile_total;
    lds_barrier();  // the next tile reuses sh
  }
  return carry;
}

}  // namespace

// A gzip header's FNAME, FCOMMENT and FHCRC fields from `p` (RFC 1952 2.3.1),
// by the whole 256-thread workgroup, with the statuses parse_frame gives:
// each field's terminating zero is searched 4 KiB at a time (16 bytes a
// thread), and the header's CRC-32 (for FHCRC) is summed a piece per thread
// and the pieces joined by GF(2) shifts, so that a hostile header as long as
// the input costs a parallel pass, not a serial one.  Returns the status;
// f.body and f.body_len on success.
__device__ u32 gzip_fields_group(const u8* in, u64 size, u64 p, Frame& f, u64& zmin, u32* table,
                                 u32* piece) {
  const u32 t = threadIdx.x;
  const u32 flg = in[3];
  const u64 limit = size - 8;
  for (u32 field = 8; field <= 16; field <<= 1) {  // FNAME, then FCOMMENT
    if (!(flg & field)) continue;
    u64 zero_at = limit;
    for (u64 base = p; base < limit; base += 16 * 256) {  // uniform
      if (!t) zmin = limit;
      __syncthreads();
      const u64 q = base + 16 * u64(t);
      for (u32 j = 0; j < 16 && q + j < limit; ++j)
        if (!in[q + j]) {
          atomicMin(reinterpret_cast<unsigned long long*>(&zmin), q + j);
          break;
        }
      __syncthreads();
      zero_at = zmin;
      __syncthreads();  // every thread has read zmin before it is reset
      if (zero_at < limit) break;  // uniform
    }
    if (zero_at >= limit) return kTruncatedZlib;
    p = zero_at + 1;
  }
  if (flg & 2) {
    if (p + 2 > limit) return kTruncatedZlib;
    table[t] = crc_byte_update(0, t);
    __syncthreads();
    // Thread t: the register (from 0) of bytes [t c, (t + 1) c) of [0, p).
    const u64 c = (p + 255) / 256, lo = min(p, u64(t) * c), hi = min(p, lo + c);
    u32 reg = 0;
    for (u64 i = lo; i < hi; ++i) reg = table[(reg ^ in[i]) & 255u] ^ (reg >> 8);
    piece[t] = reg;
    __syncthreads();
    if (!t) {
      const u32 shift = crc_shift_bytes(c);
      u32 all = 0;
      for (u32 k = 0; k < 256 && u64(k) * c < p; ++k) {
        const u64 len = min(p, u64(k + 1) * c) - u64(k) * c;
        all = crc_mul(all, len == c ? shift : crc_shift_bytes(len)) ^ piece[k];
      }
      piece[0] = crc_finish(all, p);
    }
    __syncthreads();
    if ((piece[0] & 0xffffu) != (u32(in[p]) | (u32(in[p + 1]) << 8))) return kInvalidHeader;
    p += 2;
  }
  if (!t) {
    f.body = p;
    f.body_len = limit - p;
  }
  return kOk;
}

// Wrapper checks and the state's initial values.  `body_off` is where the
// host-side launches place the body (2 for zlib, 10 for gzip, 0 for raw); a
// wrapper field between it and the first block (a zlib DICTID, gzip's
// optional fields) becomes start_bit.  A zlib stream with FDICT checks the
// dictionary's Adler-32 against its DICTID (the workgroup sums the bytes).
// Every workgroup also zeroes its grid-stride share of zero[0..zero_words):
// the scratch that later kernels accumulate into (Adler-32 pairs, resolve
// counts, the first unresolved bitmap).
__global__ __launch_bounds__(256) void g_frame(const u8* in, u64 in_size, u32 format,
                                               const u8* dict, u64 dict_len, u64 body_off,
                                               u64 out_base, State* st, u32* zero,
                                               u64 zero_words) {
  __shared__ Frame frame;
  __shared__ u32 status;
  __shared__ u64 red[2][4];
  __shared__ u64 fields_at, zmin;
  __shared__ u32 crc_table[256], crc_piece[256];
  const u32 t = threadIdx.x, lane = lane_id(), wave = t >> 6;
  {
    const u64 stride = u64(gridDim.x) * blockDim.x;
    for (u64 i = u64(blockIdx.x) * blockDim.x + t; i < zero_words; i += stride) zero[i] = 0;
  }
  if (blockIdx.x) return;
  if (!t) status = parse_frame(in, in_size, format, dict_len > 0, frame, &fields_at);
  __syncthreads();
  if (!status && fields_at) {  // uniform: gzip's optional fields, by the workgroup
    const u32 s = gzip_fields_group(in, in_size, fields_at, frame, zmin, crc_table, crc_piece);
    __syncthreads();
    if (!t) status = s;
    __syncthreads();
  }
  if (!status && frame.needs_dict) {  // uniform
    u64 s = 0, w = 0;
    for (u64 i = t; i < dict_len; i += 256) {
      s += dict[i];
      w += ((dict_len - i) % kAdlerMod) * dict[i];
    }
    s %= kAdlerMod;
    w %= kAdlerMod;
    for (u32 off = 32; off; off >>= 1) {
      s += __shfl_down(s, off, 64);
      w += __shfl_down(w, off, 64);
    }
    if (!lane) {
      red[0][wave] = s;
      red[1][wave] = w;
    }
    __syncthreads();
    if (!t) {
      const u32 a = u32((red[0][0] + red[0][1] + red[0][2] + red[0][3] + 1) % kAdlerMod);
      const u32 b =
          u32((red[1][0] + red[1][1] + red[1][2] + red[1][3] + dict_len % kAdlerMod) % kAdlerMod);
      if (((b << 16) | a) != frame.dict_id) status = kDictionaryMismatch;
    }
  }
  if (t) return;
  st->status = status;
  st->window = frame.window;
  st->wanted = frame.wanted;
  st->isize = frame.isize;
  st->start_bit = status ? 0 : (frame.body - body_off) * 8;
  // The dictionary's bytes before out_base are history only for a raw stream
  // given one or a zlib stream that asks for it (FDICT).
  st->floor = (format == kFormatRaw || frame.needs_dict) ? 0 : out_base;
  st->chain_ok = 0;
  st->candidates = 0;
  st->seeds = 0;
  st->accepted = 0;
  st->emit_status = 0;
  st->unresolved[0] = 0;
  st->unresolved[1] = 0;
  st->recs_used = 0;
  st->groups_used = 0;
  st->precount = 0;
  st->tables_used = 0;
  st->dense_count = 0;
  st->stream_end = 0;
  st->produced = 0;
  st->fix_regions = 0;
  st->fix_runs = 0;
  st->fix_rt = 0;
  st->fix_tasks = 0;
  st->emit_units = 0;
}

// Discovery pass 1, per 2 KiB range: prefiltered offsets in order (kind 0,
// validated later one per lane).  A range with more than kDiscCap of them
// validates them itself and keeps the valid ones (kind 1), or, when even those
// overflow, leaves them to the gather pass (kind 2).  Also counts
// stored-endpoint seeds.  Workgroups take ranges grid-stride.
__global__ __launch_bounds__(256) void g_discover(const u8* body, u64 len, State* st,
                                                  u32* wg_count, u64* wg_list, u32* dense,
                                                  u32* block_total, u64 groups, u64 per_block) {
  // The prefilter's lists are dead once its result is read, before any
  // validation uses the tables.
  __shared__ union {
    u8 luts[128][kDiscThreads];
    struct {
      u16 surv[kDiscThreads / 64][kSurvivorCap];  // per wave: offsets left to check
      u32 pass[kDiscRange * 8 / 32];              // prefilter result, one bit per offset
    };
  } lds;
  __shared__ u32 scan[kDiscThreads];
  __shared__ u16 kraft3[512];
  __shared__ PreStage sg;
  auto& luts = lds.luts;
  auto& surv = lds.surv;
  auto& pass = lds.pass;
  if (st->status) return;
  const u64 s0 = st->start_bit;
  const u32 t = threadIdx.x, lane = lane_id(), wave = t >> 6;
  build_kraft3(kraft3);
  u32 seeds = 0;
  // The next range's words are loaded while the current range is checked.
  static_assert(kPreStageWords <= 3 * kDiscThreads, "three words per thread hold a range");
  StagePrefetch<kPreStageWords, 3> next;
  // This workgroup's ranges: per_block consecutive ones.
  const u64 r0 = u64(blockIdx.x) * per_block, r1 = min(groups, r0 + per_block);
  u32 entries = 0;  // listed entries of the block's ranges
  if (r0 < r1) next.load(body, len, r0 * kDiscRange * 8, (r0 + 1) * kDiscRange * 8, kPreMargin);
  for (u64 wg = r0; wg < r1; ++wg) {
    next.store(sg, body);
    for (u32 i = t; i < kDiscRange * 8 / 32; i += kDiscThreads) pass[i] = 0;
    __syncthreads();
    // Words past the staged ones read as zero, as body bits past the end do.
    for (u32 i = sg.count + t; i < kPreStageWords; i += kDiscThreads) sg.words[i] = 0;
    __syncthreads();
    if (wg + 1 < r1)
      next.load(body, len, (wg + 1) * kDiscRange * 8, (wg + 2) * kDiscRange * 8, kPreMargin);
    const u64 b0 = wg * kDiscRange + u64(t) * kDiscBytesPerThread;
    // The range starts at stage byte `a` (the stage begins at the aligned word
    // holding it); this thread's 64 offsets start at stage word 2t.
    const u32 a = u32((reinterpret_cast<uintptr_t>(body) + wg * kDiscRange) & 3);
    const u32 x0 = sg.words[2 * t], x1 = sg.words[2 * t + 1], x2 = sg.words[2 * t + 2],
              x3 = sg.words[2 * t + 3], x4 = sg.words[2 * t + 4];
    const u64 w0 = u64(__builtin_amdgcn_alignbyte(x1, x0, a)) |
                   (u64(__builtin_amdgcn_alignbyte(x2, x1, a)) << 32);
    const u64 w1 = u64(__builtin_amdgcn_alignbyte(x3, x2, a)) |
                   (u64(__builtin_amdgcn_alignbyte(x4, x3, a)) << 32);
    u64 m = 0, first = 0;
    const u64 allowed = start_mask(s0, b0, first);
    if (b0 < len) {
      // Bit k of s_j is stream bit (8*b0 + k + j): BTYPE == 2 and HLIT <= 29.
      const u64 s1 = funnel(w0, w1, 1), s2 = funnel(w0, w1, 2);
      const u64 s4 = funnel(w0, w1, 4), s5 = funnel(w0, w1, 5);
      const u64 s6 = funnel(w0, w1, 6), s7 = funnel(w0, w1, 7);
      m = ~s1 & s2 & ~(s4 & s5 & s6 & s7);
      const u64 bits_left = (len - b0) * 8;
      if (bits_left < 64) m &= (1ull << bits_left) - 1;
      m &= allowed;
    }
    // Stored-endpoint seeds: LEN/NLEN complement in the staged bytes first.
  #pragma unroll
    for (u32 j = 0; j < kDiscBytesPerThread; ++j) {
      const u32 x = u32(funnel(w0, w1, 8 * j));
      if (((x ^ (x >> 16)) & 0xffffu) == 0xffffu && b0 + j < len && stored_seed(body, len, b0 + j))
        ++seeds;
    }
    // Complete code-length code (Kraft sum of the HCLEN lengths == 128) for
    // the survivors, compacted per wave so that every lane checks one.
    const u32 wave_bit0 = wave * 64 * 64;  // first offset of the wave's span (range-relative)
    for (;;) {
      const u32 cnt = __popcll(m);
      u32 incl = cnt;
  #pragma unroll
      for (u32 off = 1; off < 64; off <<= 1) {
        const u32 y = __shfl_up(incl, off, 64);
        if (lane >= off) incl += y;
      }
      const u32 total = __shfl(incl, 63, 64), excl = incl - cnt;
      if (!total) break;
      const u32 take = excl >= kSurvivorCap ? 0u : min(cnt, kSurvivorCap - excl);
      for (u32 k = 0; k < take; ++k) {
        const u32 bit = __builtin_ctzll(m);
        m &= m - 1;
        surv[wave][excl + k] = u16(lane * 64 + bit);
      }
      wave_sync();
      const u32 n = min(total, kSurvivorCap);
      for (u32 i = lane; i < n; i += 64) {
        const u32 o = wave_bit0 + surv[wave][i];
        const u32 P = 8 * a + o, wi = P >> 5, sh = P & 31;
        const u32 y0 = sg.words[wi], y1 = sg.words[wi + 1], y2 = sg.words[wi + 2],
                  y3 = sg.words[wi + 3];
        const u32 A = __builtin_amdgcn_alignbit(y1, y0, sh);
        const u32 B = __builtin_amdgcn_alignbit(y2, y1, sh);
        const u32 C = __builtin_amdgcn_alignbit(y3, y2, sh);
        const u32 nc = ((A >> 13) & 15u) + 4;
        const u64 lens =
            (u64(A >> 17) | (u64(B) << 15) | (u64(C) << 47)) & ((1ull << (3 * nc)) - 1);
        u32 kraft = 0;
  #pragma unroll
        for (u32 j = 0; j < 7; ++j) kraft += kraft3[(lens >> (9 * j)) & 511];
        if (kraft == 128) atomicOr(&pass[o >> 5], 1u << (o & 31));
      }
      wave_sync();  // the list is refilled next
    }
    __syncthreads();
    u64 mask = u64(pass[2 * t]) | (u64(pass[2 * t + 1]) << 32);
    const u64 flag = first;  // the first block is always a candidate
    mask |= first;
    u64 valid_flag = flag;
    u32 total;
    u32 base = block_exclusive_scan(__popcll(mask), scan, total);
    u32 kind = 0;
    if (total > kDiscCap) {
      mask = validate_mask(body, len, b0, mask & ~flag, &luts[0][threadIdx.x], kDiscThreads) | flag;
      valid_flag = mask;
      base = block_exclusive_scan(__popcll(mask), scan, total);
      kind = total > kDiscCap ? 2u : 1u;
    }
    if (!threadIdx.x) {
      wg_count[wg] = total | (kind << kKindShift);
      if (kind == 2)
        dense[atomicAdd(reinterpret_cast<unsigned long long*>(&st->dense_count), 1ull)] = u32(wg);
    }
    entries += total;
    if (kind < 2) {
      while (mask) {
        const u32 k = __builtin_ctzll(mask);
        mask &= mask - 1;
        wg_list[wg * kDiscCap + base++] = (b0 * 8 + k) | ((valid_flag >> k) & 1 ? kValidBit : 0);
      }
    }
    __syncthreads();  // the next range reuses the stage and the lists
  }
  if (!t) block_total[blockIdx.x] = entries;
  if (seeds) atomicAdd(reinterpret_cast<unsigned long long*>(&st->seeds), seeds);
}

// Offset in the dense array of range wg's list: its block's base plus the
// lists of the block's earlier ranges (lanes load their counts, a wave sum
// adds them).  Every lane of the wave calls it.
__device__ __forceinline__ u64 range_offset(const u32* wg_count, const u64* block_base, u64 wg,
                                            u64 per_block) {
  const u64 b = wg / per_block, first = b * per_block;
  u32 before = 0;
  for (u64 j = first + lane_id(); j < wg; j += 64) before += wg_count[j] & kCountMask;
  for (u32 off = 32; off; off >>= 1) before += __shfl_xor(before, off, 64);
  return block_base[b] + before;
}

// Pre-candidates one validation wave takes: the fewest (a power of two up to
// kValPerWave) that spread them over at most kValResident waves, so that a
// few pre-candidates get a wave each (a wave then waits for one walk, not
// for a lane's several), and many take kValPerWave a wave, a lane walking a
// few headers one after another.  The launch has more than kValResident
// waves, and enough for n / kValPerWave.
constexpr u32 kValPerWave = 128;
constexpr u64 kValResident = 2048;
// Up to this many pre-candidates a wave, the wave walks each header with all
// its lanes (val_wave) rather than a lane a header.
constexpr u32 kValWaveChunk = 4;
__host__ __device__ inline u32 val_chunk(u64 n) {
  u32 c = 1;
  while (c < kValPerWave && n > u64(c) * kValResident) c <<= 1;
  return c;
}

// Discovery pass 2: one workgroup scans the per-block entry totals into
// offsets of the dense pre-candidate array.  When validation waves will take
// fewer than kValPerWave pre-candidates each, several add into one range's
// valid count, which is cleared here.
__global__ __launch_bounds__(1024) void g_discover_scan(State* st, const u32* block_total,
                                                        u64* block_base, u64 blocks,
                                                        u64 pre_capacity, u32* range_valid) {
  __shared__ ScanShared sh;
  if (st->status) return;
  const u64 total = wg_exclusive_scan(block_total, ~0u, blocks, block_base, sh);
  if (total <= pre_capacity && val_chunk(total) < kValPerWave)  // uniform
    for (u64 i = threadIdx.x; i < (total + kValPerWave - 1) / kValPerWave; i += blockDim.x)
      range_valid[i] = 0;
  if (threadIdx.x == 0) {
    st->precount = total;
    // Only kind-2 ranges (valid headers alone overflowing a range) can push the
    // total past the capacity, and then the valid candidates alone exceed the
    // candidate limit.
    if (total > pre_capacity) st->status = kCandidateOverflow;
  }
}

// Discovery pass 3: the per-range lists in order into the dense array, one
// wave per range (kind-2 ranges are left to pass 3b).
__global__ __launch_bounds__(256) void g_discover_gather(const State* st, const u32* wg_count,
                                                         const u64* wg_list, const u64* block_base,
                                                         u64* pre, u64 groups, u64 per_block) {
  if (st->status) return;
  const u64 wg = u64(blockIdx.x) * (kDiscThreads / 64) + (threadIdx.x >> 6);
  if (wg >= groups) return;
  const u32 c = wg_count[wg], lane = lane_id();
  if ((c >> kKindShift) >= 2) return;
  const u64 off = range_offset(wg_count, block_base, wg, per_block);
  if (lane < (c & kCountMask)) pre[off + lane] = wg_list[wg * kDiscCap + lane];
}

// Discovery pass 3b: kind-2 ranges (listed by pass 1) recompute and
// validate their offsets straight into the dense array.
__global__ __launch_bounds__(256) void g_discover_dense(const u8* body, u64 len, const State* st,
                                                        const u32* dense, const u32* wg_count,
                                                        const u64* block_base, u64* pre,
                                                        u64 per_block) {
  __shared__ u64 range_off;
  __shared__ u8 luts[128][kDiscThreads];
  __shared__ u32 scan[kDiscThreads];
  __shared__ u16 kraft3[512];
  __shared__ PreStage sg;
  if (st->status) return;
  const u64 n = st->dense_count;
  if (blockIdx.x >= n) return;
  build_kraft3(kraft3);
  for (u64 k = blockIdx.x; k < n; k += gridDim.x) {
    const u64 wg = dense[k];
    if (threadIdx.x < 64) {
      const u64 o = range_offset(wg_count, block_base, wg, per_block);
      if (!threadIdx.x) range_off = o;
    }
    stage_range(body, len, wg * kDiscRange * 8, (wg + 1) * kDiscRange * 8, sg, kPreMargin);
    __syncthreads();
    const u64 b0 = wg * kDiscRange + u64(threadIdx.x) * kDiscBytesPerThread;
    const u64 s0 = st->start_bit;
    u64 first;
    start_mask(s0, b0, first);
    u64 mask = validate_mask(body, len, b0, prefilter_mask(len, b0, sg, kraft3, s0),
                             &luts[0][threadIdx.x], kDiscThreads);
    mask |= first;
    u32 total;
    u32 at = block_exclusive_scan(__popcll(mask), scan, total);  // (its barrier publishes range_off)
    const u64 off = range_off;
    while (mask) {
      const u32 b = __builtin_ctzll(mask);
      mask &= mask - 1;
      pre[off + at++] = (b0 * 8 + b) | kValidBit;
    }
    __syncthreads();  // the next range reuses the stage
  }
}

namespace {

// Discovery pass 4 works on one wave per workgroup: every lane validates
// pre-candidates of the wave's range one after another, taking the next
// unvalidated entry whenever it finishes (every kValRound symbols), so a
// long header walk does not idle the other lanes.  A lane's header bits
// are copied into its LDS window and its code-length symbols are decoded
// arithmetically from the canonical code (no per-candidate table); a walk
// that reaches the window's end reloads the window from its position.
constexpr u32 kValRound = 16;                       // symbols between refills
constexpr u32 kValWindowWords = 32;                 // LDS window per lane (dwords)
constexpr u32 kValUsableBits = (kValWindowWords - 3) * 32;  // a read touches words pos/32 .. +2

struct ValShared {
  u32 win[kValWindowWords][64];  // header bits of each lane's candidate
};

// Header walk of one lane (RFC 1951 3.2.7): the same accept/reject rules as
// dynamic_header_fields_valid, over the lane's window.
struct ValWalk {
  u32 x0, x1, x2;    // window words w, w+1, w+2 (x2 loaded for the next advance)
  u32 w, off;        // window position
  u32 limit;         // window-relative bit limit
  bool body_end;     // limit is the body end (else the window is reloaded there)
  u64 bit0;          // body bit of window bit 0
  u32 nl, total, i, prev, eob, ll_kraft, d_kraft, ll_nnz, d_nnz;
  // Canonical code-length code (val_start): la[0..2] hold the left-justified
  // 7-bit starts of the codes of lengths 2..7 as 16-bit fields; lp and bp the
  // starts and the sorted rank of the first symbol of each length l (8-bit
  // fields at 8 * l); slo/shi the symbols sorted by (length, symbol), 5 bits
  // each (ranks 0-11 and 12-18).
  u32 la0, la1, la2;
  u64 lp, bp, slo, shi;
  // Code-length symbol and its length at the next bits `b` (the code is
  // complete, so every 7-bit pattern starts a code).
  __device__ __forceinline__ u32 symbol(u32 b, u32& l) const {
    const u32 rv = __builtin_bitreverse32(b) >> 25;  // code bits MSB first
    const u32 r = (rv | (rv << 16)) | 0x80008000u;   // bit 15 of each field: rv >= start
    l = 1 + __builtin_popcount((r - la0) & 0x80008000u) + __builtin_popcount((r - la1) & 0x80008000u) +
        __builtin_popcount((r - la2) & 0x80008000u);
    const u32 start = u32(lp >> (8 * l)) & 0xffu;
    const u32 rank = (u32(bp >> (8 * l)) & 0xffu) + ((rv - start) >> (7 - l));
    return rank < 12 ? u32(slo >> (5 * rank)) & 31u : u32(shi >> (5 * (rank - 12))) & 31u;
  }
  __device__ __forceinline__ u32 pos() const { return (w << 5) + off; }
  __device__ __forceinline__ u32 bits() const { return __builtin_amdgcn_alignbit(x1, x0, off); }
  __device__ __forceinline__ void seek(const ValShared& sh, u32 lane, u32 p) {
    w = p >> 5;
    off = p & 31u;
    x0 = sh.win[w][lane];
    x1 = sh.win[w + 1][lane];
    x2 = sh.win[w + 2][lane];
  }
  __device__ __forceinline__ void advance(const ValShared& sh, u32 lane, u32 n) {  // n < 32
    const u32 o = off + n;
    const u32 adv = o >> 5;
    off = o & 31u;
    w += adv;
    u32 c1 = x1, c2 = x2;
    asm volatile("" : "+v"(c1), "+v"(c2));
    x0 = adv ? c1 : x0;
    x1 = adv ? c2 : c1;
    x2 = sh.win[min(w + 2, kValWindowWords - 1)][lane];
  }
};

enum : u32 { kValRunning = 0, kValValid = 1, kValInvalid = 2, kValLong = 3 };

// The lane's window: body bits from the dword holding bit `pos`, the walk
// positioned at `pos`.  kBatch window words are loaded at a time (all of
// them for a new candidate; fewer registers for a reload mid-walk).
template <u32 kBatch>
__device__ __forceinline__ void val_window(const u8* body, u64 len, u64 pos, ValShared& sh,
                                           u32 lane, ValWalk& v) {
  static_assert(kValWindowWords % kBatch == 0, "whole batches");
  const uintptr_t base = reinterpret_cast<uintptr_t>(body);
  const uintptr_t first = (base + (pos >> 3)) & ~uintptr_t(3);
  const uintptr_t end = base + len;  // body bytes end here
  const u32* g = reinterpret_cast<const u32*>(first);
  if (first + 4 * kValWindowWords <= end) {
#pragma unroll 1
    for (u32 j0 = 0; j0 < kValWindowWords; j0 += kBatch) {
      u32 x[kBatch];  // a batch of loads in flight at once
#pragma unroll
      for (u32 j = 0; j < kBatch; ++j) x[j] = g[j0 + j];
#pragma unroll
      for (u32 j = 0; j < kBatch; ++j) sh.win[j0 + j][lane] = x[j];
    }
  } else {
    for (u32 j = 0; j < kValWindowWords; ++j) {
      const uintptr_t a = first + 4 * j;
      u32 x = 0;
      if (a + 4 <= end) x = g[j];
      else
        for (u32 b = 0; b < 4; ++b)
          if (a + b < end) x |= u32(*reinterpret_cast<const u8*>(a + b)) << (8 * b);
      sh.win[j][lane] = x;
    }
  }
  const u32 p0 = u32((base + (pos >> 3) - first) * 8 + (pos & 7));  // window bit of `pos`
  // Window bit of the body end (0 when even `pos` lies past it: nothing fits).
  const u64 rel_end = u64(p0) + len * 8 > pos ? u64(p0) + len * 8 - pos : 0;
  v.body_end = rel_end <= kValUsableBits;
  v.limit = v.body_end ? u32(rel_end) : kValUsableBits;
  v.bit0 = pos - p0;
  v.seek(sh, lane, p0);
}

// Load candidate `pos` (its BTYPE already known to be 2) into the lane's
// window and parse HLIT/HDIST/HCLEN and the code-length code.  Returns
// kValRunning or a final verdict.
__device__ u32 val_start(const u8* body, u64 len, u64 pos, ValShared& sh, u32 lane, ValWalk& v) {
  val_window<kValWindowWords>(body, len, pos + 3, sh, lane, v);
  // 14 + 57 bits of fields fit in the usable window (p0 < 32).
  if (v.pos() + 14 > v.limit) return kValInvalid;  // only at the body end
  const u32 f = v.bits();
  const u32 hlit = f & 31u, hdist = (f >> 5) & 31u, hclen = (f >> 10) & 15u;
  v.advance(sh, lane, 14);
  v.nl = hlit + 257;
  v.total = v.nl + hdist + 1;
  if (v.nl > 286) return kValInvalid;
  const u32 nc = hclen + 4;
  if (v.pos() + 3 * nc > v.limit) return kValInvalid;
  // The 3 * nc <= 57 bits of code-length-code lengths, read at once from the
  // three window words in registers, then skipped in two advances.
  const u64 field = u64(__builtin_amdgcn_alignbit(v.x1, v.x0, v.off)) |
                    (u64(__builtin_amdgcn_alignbit(v.x2, v.x1, v.off)) << 32);
  v.advance(sh, lane, 3 * nc - 3 * (nc >> 1));
  v.advance(sh, lane, 3 * (nc >> 1));
  u64 pack = 0;
  u32 kraft = 0;
#pragma unroll
  for (u32 i = 0; i < 19; ++i) {
    const u32 x = i < nc ? u32(field >> (3 * i)) & 7u : 0u;
    pack |= u64(x) << (3 * cl_order(i));
    kraft += x ? 128u >> x : 0u;
  }
  if (kraft != 128) return kValInvalid;
  // Canonical code parameters (see ValWalk).
  u64 cnt = 0;
  for (u32 s = 0; s < 19; ++s) cnt += 1ull << (8 * ((pack >> (3 * s)) & 7));
  u64 lp = 0, bp = 0;
  u32 start = 0, rank = 0;
  for (u32 l = 1; l < 8; ++l) {
    lp |= u64(start) << (8 * l);
    bp |= u64(rank) << (8 * l);
    const u32 c = u32(cnt >> (8 * l)) & 0xffu;
    start += c << (7 - l);
    rank += c;
  }
  u64 nr = bp, slo = 0, shi = 0;
  for (u32 s = 0; s < 19; ++s) {
    const u32 l = (pack >> (3 * s)) & 7;
    const u32 r = u32(nr >> (8 * l)) & 0xffu;
    nr += l ? 1ull << (8 * l) : 0ull;
    slo |= (l && r < 12) ? u64(s) << (5 * r) : 0ull;
    shi |= (l && r >= 12) ? u64(s) << (5 * (r - 12)) : 0ull;
  }
  v.lp = lp;
  v.bp = bp;
  v.slo = slo;
  v.shi = shi;
  const auto start_of = [&](u32 l) { return u32(lp >> (8 * l)) & 0xffu; };
  v.la0 = start_of(2) | (start_of(3) << 16);
  v.la1 = start_of(4) | (start_of(5) << 16);
  v.la2 = start_of(6) | (start_of(7) << 16);
  v.i = 0;
  v.prev = 0;
  v.eob = 0;
  v.ll_kraft = v.d_kraft = v.ll_nnz = v.d_nnz = 0;
  return kValRunning;
}

// One code-length symbol of the walk.  kValLong: the symbol does not fit in
// the window (nothing taken).
__device__ __forceinline__ u32 val_step(const ValShared& sh, u32 lane, ValWalk& v) {
  const u32 b = v.bits();
  u32 l;
  const u32 sym = v.symbol(b, l);
  const bool rep = sym >= 16, r16 = sym == 16, r18 = sym == 18;
  const u32 xbits = rep ? (r16 ? 2u : r18 ? 7u : 3u) : 0u;
  const u32 need = l + xbits;
  if (v.pos() + need > v.limit) return v.body_end ? kValInvalid : kValLong;
  const u32 x = (b >> l) & ((1u << xbits) - 1u);
  v.advance(sh, lane, need);
  // Every case computed with selects; a rejected walk ends here anyway.
  const u32 repeat = rep ? x + (r18 ? 11u : 3u) : 1u;
  const u32 value = r16 ? v.prev : rep ? 0u : sym;
  const u32 i = v.i;
  const bool nz = value != 0;
  const u32 in_ll = i < v.nl ? min(repeat, v.nl - i) : 0u;
  const u32 in_d = repeat - in_ll;
  v.ll_kraft += nz ? in_ll << (15 - value) : 0u;
  v.d_kraft += nz ? in_d << (15 - value) : 0u;
  v.ll_nnz += nz ? in_ll : 0u;
  v.d_nnz += nz ? in_d : 0u;
  v.eob |= (nz && i <= 256 && 256 < i + repeat) ? 1u : 0u;
  v.prev = value;
  v.i = i + repeat;
  // Kraft sums only grow: an oversubscribed code can never become valid.
  const bool bad = (r16 && i == 0) || repeat > v.total - i || v.ll_kraft > (1u << 15) ||
                   v.d_kraft > (1u << 15);
  if (bad) return kValInvalid;
  if (v.i < v.total) return kValRunning;
  const bool ll_ok = v.ll_kraft == (1u << 15) || (v.ll_nnz == 1 && v.ll_kraft == (1u << 14));
  const bool d_ok =
      v.d_nnz == 0 || v.d_kraft == (1u << 15) || (v.d_nnz == 1 && v.d_kraft == (1u << 14));
  return v.eob && ll_ok && d_ok ? kValValid : kValInvalid;
}

}  // namespace

// What the wave-wide header walk of g_validate needs: the code-length code,
// the lengths, the staged header and the walk's runs.
struct ValHeadTables {
  HuffTable<19, 7> cl;
  u8 lens[320];
};
struct ValWaveShared {
  ValHeadTables tables;
  StageT<kHeaderWords> stage;
  u32 runs[320];
};

// A wave's single pre-candidate at bit `pos` (its BTYPE known to be 2, its
// header staged whole before the body end): walked by the whole wave as
// g_headers walks a header (lanes decode speculatively, the true path taken
// by scalar hops), then the verdict val_step gives: the code-length code
// complete, every run inside the lengths, a code for symbol 256, and
// literal/length and distance codes complete (or a single code of length 1;
// no distance codes at all is allowed too).
__device__ bool val_wave(const u8* body, u64 len, u64 pos, ValWaveShared& w) {
  const u32 lane = lane_id();
  stage_range(body, len, pos, pos + 8, w.stage, kHeaderBytes);
  __syncthreads();
  u32 nl = 0, nd = 0, err = kOk, p = 0, lim = 0;
  u64 after = 0;
  if (!header_prelude_wave(w.stage.words, w.stage.bit0, w.stage.count, w.tables, len, pos + 3, nl,
                           nd, err, after, p, lim) ||
      err)
    return false;
  if (header_lengths_wave(w.stage.words, w.tables, w.runs, nl + nd, p, lim)) return false;
  u32 llk = 0, lln = 0, dk = 0, dn = 0;  // Kraft sums in units of 2^-15, nonzero counts
  for (u32 k = lane; k < nl + nd; k += 64) {
    const u32 l = w.tables.lens[k];
    const u32 wt = l ? 1u << (15 - l) : 0u;
    if (k < nl) {
      llk += wt;
      lln += l != 0;
    } else {
      dk += wt;
      dn += l != 0;
    }
  }
  for (u32 off = 32; off; off >>= 1) {
    llk += __shfl_xor(llk, off, 64);
    lln += __shfl_xor(lln, off, 64);
    dk += __shfl_xor(dk, off, 64);
    dn += __shfl_xor(dn, off, 64);
  }
  const bool ll_ok = llk == (1u << 15) || (lln == 1 && llk == (1u << 14));
  const bool d_ok = dn == 0 || dk == (1u << 15) || (dn == 1 && dk == (1u << 14));
  return ll_ok && d_ok;
}

// Discovery pass 4 (one wave per workgroup; see above).  Valid entries get
// kValidBit; wave_valid[r] counts the valid entries of pre-candidates
// [kValPerWave r, kValPerWave (r + 1)), written by the wave that takes them
// all or added by the waves that share them (val_chunk).
__global__ __launch_bounds__(64) void g_validate(const u8* body, u64 len, State* st, u64* pre,
                                                 u32* wave_valid) {
  __shared__ union {
    ValShared lanes;
    ValWaveShared wave;
  } shu;
  ValShared& sh = shu.lanes;
  if (st->status) return;
  const u64 n = st->precount;
  const u32 chunk = val_chunk(n);
  const u64 q0 = u64(blockIdx.x) * chunk;
  if (q0 >= n) return;
  const u64 q1 = min<u64>(q0 + chunk, n);
  const u32 lane = lane_id();
  if (chunk <= kValWaveChunk && (pre[q1 - 1] & kPosMask) / 8 + kHeaderBytes + 16 <= len) {
    // Few pre-candidates a wave: the whole wave walks each header in turn
    // (one lane's walk would take a symbol a step), unless a header could
    // reach the body end, where the lane walk's exact limits apply (the
    // entries are in order, so the last one is the one to check).
    u32 found_here = 0;
    for (u64 q = q0; q < q1; ++q) {
      const u64 e = pre[q];
      const bool valid = (e & kValidBit) || val_wave(body, len, e & kPosMask, shu.wave);
      if (valid && !(e & kValidBit) && !lane) pre[q] = e | kValidBit;
      found_here += valid ? 1u : 0u;
      __syncthreads();  // the next header reuses the stage
    }
    if (!lane && found_here) atomicAdd(&wave_valid[q0 / kValPerWave], found_here);
    return;
  }
  u64 cursor = q0;  // next unassigned entry (uniform)
  u64 ci = 0;
  bool active = false;
  ValWalk v;
  u32 found = 0;  // this lane's valid verdicts
  for (;;) {
    // Give every idle lane the next entry that needs a walk.
    for (;;) {
      const u64 idle = __ballot(!active);
      if (!idle || cursor >= q1) break;
      if (!active) {
        ci = cursor + __popcll(idle & lanemask_lt());
        if (ci < q1) {
          const u64 e = pre[ci];
          if (e & kValidBit) ++found;  // validated by discovery
          else active = val_start(body, len, e & kPosMask, sh, lane, v) == kValRunning;
        }
      }
      cursor += __popcll(idle);
    }
    if (!__ballot(active)) break;
    // A walk that reaches its window's end pauses for the rest of the round
    // and reloads the window after it (one copy of the reload, outside the
    // unrolled steps); the step it could not take is taken next round.
    bool reload = false;
    for (u32 k = 0; k < kValRound; ++k) {
      if (active) {
        const u32 r = val_step(sh, lane, v);
        if (r != kValRunning) {
          active = false;
          if (r == kValValid) {
            pre[ci] |= kValidBit;
            ++found;
          }
          reload = r == kValLong;
        }
      }
    }
    if (reload) {
      val_window<8>(body, len, v.bit0 + v.pos(), sh, lane, v);
      active = true;
    }
  }
  for (u32 off = 32; off; off >>= 1) found += __shfl_xor(found, off, 64);
  if (!lane) {
    if (chunk == kValPerWave) wave_valid[blockIdx.x] = found;
    else if (found) atomicAdd(&wave_valid[q0 / kValPerWave], found);
  }
}

// Discovery pass 5: valid entries in order into the candidate array, one
// 256-entry block (two validation waves) per workgroup.  The block's offset
// is the sum of the earlier waves' valid counts, added up by the workgroup;
// the workgroup holding the last entry sets the candidate count and checks
// the candidate limit (valid headers + bit 0 + stored seeds, as the
// reference counts them).
__global__ __launch_bounds__(256) void g_valid_scatter(State* st, const u64* pre,
                                                       const u32* wave_valid, u64* cand,
                                                       u64 cand_capacity, u64 max_candidates) {
  static_assert(kDiscThreads % kValPerWave == 0, "a block covers whole validation waves");
  __shared__ u32 wave_count[kDiscThreads / 64];
  __shared__ u64 red[kDiscThreads / 64];
  if (st->status) return;
  const u64 n = st->precount;
  if (u64(blockIdx.x) * kDiscThreads >= n) return;
  const u32 t = threadIdx.x, wave = t >> 6, lane = lane_id();
  // Valid entries before the block: the validation waves before its first.
  const u64 before_waves = u64(blockIdx.x) * (kDiscThreads / kValPerWave);
  u64 part = 0;
  for (u64 w = t; w < before_waves; w += 4 * kDiscThreads) {
    const u64 w1 = w + kDiscThreads, w2 = w + 2 * kDiscThreads, w3 = w + 3 * kDiscThreads;
    const u32 a = wave_valid[w];
    const u32 b = w1 < before_waves ? wave_valid[w1] : 0u;
    const u32 c = w2 < before_waves ? wave_valid[w2] : 0u;
    const u32 d = w3 < before_waves ? wave_valid[w3] : 0u;
    part += u64(a) + b + c + d;
  }
  for (u32 off = 32; off; off >>= 1) part += __shfl_xor(part, off, 64);
  const u64 i = u64(blockIdx.x) * kDiscThreads + t;
  const u64 e = i < n ? pre[i] : 0;
  const bool valid = i < n && (e & kValidBit);
  const u64 bal = __ballot(valid);
  if (!lane) {
    wave_count[wave] = __popcll(bal);
    red[wave] = part;
  }
  __syncthreads();
  u64 at = 0;
  for (u32 w = 0; w < kDiscThreads / 64; ++w) at += red[w];
  const u64 block_base = at;
  for (u32 w = 0; w < wave; ++w) at += wave_count[w];
  at += __popcll(bal & lanemask_lt());
  if (valid && at < cand_capacity) cand[at] = e & kPosMask;
  if (!t && (u64(blockIdx.x) + 1) * kDiscThreads >= n) {
    u64 total = block_base;
    for (u32 w = 0; w < kDiscThreads / 64; ++w) total += wave_count[w];
    st->candidates = total;
    st->tables_used = total;  // table slots 0 .. total-1 belong to the candidates
    if (total + st->seeds > max_candidates) st->status = kCandidateOverflow;
  }
}

namespace {

// Lower bound of `key` in the sorted candidate array.
// First index at or after `from` whose candidate is >= key, when every
// entry before `from` is known to be below `key` (the list is sorted):
// galloping from `from`, so an answer close to it costs one or two loads
// instead of a full binary search of dependent loads.
__device__ u64 lower_bound_from(const u64* cand, u64 n, u64 from, u64 key) {
  if (from >= n || cand[from] >= key) return from;
  u64 below = from, step = 1;  // cand[below] < key
  while (below + step < n && cand[below + step] < key) {
    below += step;
    step <<= 1;
  }
  u64 lo = below + 1, hi = below + step < n ? below + step : n;  // answer in [lo, hi]
  while (lo < hi) {
    const u64 mid = lo + (hi - lo) / 2;
    if (cand[mid] < key) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// Count-only parse of one block at r.pos (the reference's parse_block with
// Emit=false): limit bounds this block's output, distances are checked
// against the maximum window only.
__device__ u32 describe_block(BitIn& r, DecodeTables& t, u64 limit, u32& final_block, u64& size) {
  size = 0;
  u32 type;
  if (!r.take(1, final_block) || !r.take(2, type)) return kTruncated;
  if (type == 3) return kReservedBlock;
  if (type == 0) {
    r.seek((r.pos + 7) & ~u64(7));
    u32 n, comp;
    if (!r.take(16, n) || !r.take(16, comp)) return kTruncated;
    if ((n ^ comp) != 0xffffu) return kBadSymbol;
    if (n > limit) return kOutputOverflow;
    if (u64(n) * 8 > r.avail()) return kTruncated;
    r.seek(r.pos + u64(n) * 8);
    size = n;
    return kOk;
  }
  u32 err = type == 1 ? build_fixed_tables(t) : build_dynamic_tables(t, r);
  if (err) return err;
  u64 produced = 0;
  for (;;) {
    u32 lit, length, distance;
    err = decode_token(t, r, 32768u, lit, length, distance);
    if (err) break;
    if (!length) break;
    if (!distance) {
      if (produced >= limit) { err = kOutputOverflow; break; }
      ++produced;
      continue;
    }
    if (length > limit - produced) { err = kOutputOverflow; break; }
    produced += length;
  }
  size = produced;
  return err;
}

// ---- long fixed-Huffman runs ------------------------------------------------
// A fixed block has a 3-bit header, so discovery cannot find where one starts,
// and a run of fixed blocks (Z_FIXED data, a text segment of the stress
// stream) would otherwise belong to the segment of the candidate before it and
// be described by one workgroup.  Instead describe defers such a run (a
// "region"), and three passes decode it across the whole GPU:
//   summaries  every 2 KiB tile of the region, from each of the 32 bit
//              offsets at which the tile's first token can start (a fixed
//              token is at most 31 bits): where decoding leaves the tile,
//              bytes produced, headers crossed, first EOB, or how it ended
//   walk       one wave per region chains the summaries from the run's first
//              token (stored blocks between runs parsed in place), giving the
//              true entry and output offset of every tile, the segment's end
//              and block records; a tile without a summary is decoded there
//   slices     every tile on a run decodes once more from its true entry to
//              place the 512-bit emission slices inside it
// Emission then decodes a run's slices like a block's, crossing the fixed
// headers inside a slice.  The reference keeps per-2 KiB-tile summaries of 32
// entries for its serial chain walk (FixedSummary, scan_fixed_region,
// _decode_kernels.py:376-472, 1181-1207, 1274).
constexpr u32 kFixTileBits = 16384;
constexpr u32 kFixEntries = 32;
constexpr u32 kFixSliceBits = 512;
constexpr u32 kFixTileSlices = kFixTileBits / kFixSliceBits;
constexpr u32 kFixProbeTokens = 512;  // tokens a fixed block is probed before it is deferred
constexpr u32 kFixSyncBits = 256;     // entries decoded apart before those that meet share a task
constexpr u32 kFixMarginBytes = 64;   // staged past a tile: its last token, an EOB and a header
constexpr u32 kFixStageWords = (2 * kFixTileBits / 8 + kFixMarginBytes) / 4 + 4;
enum : u32 { kFixGo = 0, kFixEnd = 1, kFixHeader = 2, kFixError = 3 };
constexpr u32 kFixInFinal = 0x10;       // kind flag: the exit lies inside the final block
constexpr u16 kFixNoEob = 0xffffu;
constexpr u32 kSegPaused = 0x40000000u;  // seg_flags: the segment continues in a fixed run
constexpr u32 kSegRecsLost = 0x20000000u;  // seg_flags with kSegPaused: records ran out
constexpr u32 kRecFixedRun = 1u;         // BlockRec.pad: slices cross fixed block headers

// Decoding from one entry bit of one tile (tile-relative bit positions).
struct FixSummary {
  u32 bytes;      // output bytes up to the exit or terminal
  u32 eob_bytes;  // output bytes before the first EOB
  u16 exit;       // kFixGo: first token start at or after the tile's end; else the terminal
                  // bit (kFixEnd: after the final EOB; kFixHeader: the non-fixed header;
                  // kFixError: the failing token)
  u16 eob;        // bit after the first EOB, or kFixNoEob
  u16 blocks;     // block headers crossed (all fixed, non-final or final)
  u8 kind;        // kFix* | kFixInFinal
  u8 status;      // kFixError: the status
};
static_assert(sizeof(FixSummary) == 16, "summary layout");

// The rest of one tile for the entries whose decodes reached the same token
// start `p` (tile-relative, at or after kFixSyncBits) in the same state.
struct FixTask {
  u64 tile;
  u32 entries;  // bit e: entry e
  u16 p;
  u16 in_final;
};
static_assert(sizeof(FixTask) == 16, "task layout");

// A decode's summary from its prefix p (which ended, kind kFixGo, where r
// starts) and the rest r.
__device__ __forceinline__ FixSummary fix_join(const FixSummary& p, const FixSummary& r) {
  FixSummary s;
  const bool had_eob = p.eob != kFixNoEob;
  s.bytes = p.bytes + r.bytes;
  s.eob_bytes = had_eob ? p.eob_bytes : p.bytes + r.eob_bytes;
  s.exit = r.exit;
  s.eob = had_eob ? p.eob : r.eob;
  s.blocks = u16(p.blocks + r.blocks);
  s.kind = r.kind;
  s.status = r.status;
  return s;
}

// A run of fixed blocks on a walked path, for the slice pass: its slices are
// the 512-bit windows b0 .. b0 + lanes - 1 (slice i starts at the first token
// at or after bit 512 * (b0 + i); slice 0 at the run's first token).
struct FixRun {
  u64 tok;      // first token bit
  u64 end;      // bit after the last EOB
  u64 b0;
  u32 lanes;
  u32 group;    // first of the run's consecutive slice groups
};

// Tiles k .. k + tiles - 1 of a run: the first one's true entry and the
// run's output bytes before it (the others' follow from the summaries).
struct FixTile {
  u64 pos;
  u32 off;
  u32 run;    // kNone: unused slot
  u32 k;      // tile index
  u32 tiles;  // 1, or a group's tiles walked in one step
};

// The walk's step over a group of kFixGroupTiles marked tiles from one entry
// state (entry bit e < 32 of the group's first tile, in the final block or
// not): the tile summaries composed.
constexpr u32 kFixGroupTiles = 16;
struct FixGroupSum {
  u32 bytes;   // output bytes up to the group's end or its terminal
  u32 blocks;  // block headers crossed
  u16 exit;    // as a tile summary's, relative to the last tile walked
  u8 kind;     // as a tile summary's (kFixInFinal: the state after the group)
  u8 tiles;    // tiles walked (the terminal's included); 0: step tile by tile
  u8 status;
  u8 pad[3];
};
static_assert(sizeof(FixGroupSum) == 16, "group summary layout");

// 64 bits starting at stage bit p, words past `n` reading as zero.
struct FixPeek {
  const u32* w;
  u32 n;
  __device__ __forceinline__ u64 operator()(u32 p) const {
    const u32 i = p >> 5, sh = p & 31u;
    const u64 x0 = i < n ? w[i] : 0u, x1 = i + 1 < n ? w[i + 1] : 0u, x2 = i + 2 < n ? w[i + 2] : 0u;
    const u64 lo = x0 | (x1 << 32);
    return sh ? (lo >> sh) | (x2 << (64 - sh)) : lo;
  }
};

// 64 bits at bit p of words in memory for one thread's forward decode: 128
// bits in registers and the next 64 in flight, loaded when the position
// moves past the first 64 (so a load has a few tokens of decoding to arrive).
// Positions must not decrease by more than the window or jump more than 64
// bits past it without a reload, which seek() does.  Words past `n` read as
// zero.
struct FixStream {
  const u32* w;
  u32 n;
  u32 i0;  // even word index of `cur`
  u64 cur, nxt, pend;
  __device__ __forceinline__ u64 pair(u32 i) const {
    return u64(i < n ? w[i] : 0u) | (u64(i + 1 < n ? w[i + 1] : 0u) << 32);
  }
  __device__ __forceinline__ void seek(u32 p) {
    i0 = (p >> 5) & ~1u;
    cur = pair(i0);
    nxt = pair(i0 + 2);
    pend = pair(i0 + 4);
  }
  __device__ __forceinline__ u64 operator()(u32 p) {
    const u32 at = p - i0 * 32u;  // wraps when p precedes the window
    if (at >= 128) {
      seek(p);
    } else if (at >= 64) {
      cur = nxt;
      nxt = pend;
      i0 += 2;
      pend = pair(i0 + 4);
    }
    const u32 sh = p - i0 * 32u;
    return sh ? (cur >> sh) | (nxt << (64 - sh)) : cur;
  }
};

// Fixed-Huffman decode from token start `p` until the first token start at or
// after `stop`, crossing non-final and final fixed headers, within `body_end`
// (stage bits past it do not exist).  `in_final`: the decode starts inside the
// stream's final block, so its first EOB ends the stream.  Positions in the
// result are relative to `rel0`.  With kMaxTokens, a decode that has taken
// that many tokens stops as if it had reached `stop` (the probe).
template <u32 kMaxTokens = 0, class Peek>
__device__ __forceinline__ FixSummary fix_scan(Peek& pk, u32 p, u32 stop, u32 body_end,
                                               bool in_final, u32 rel0) {
  FixSummary s;
  s.bytes = 0;
  s.eob_bytes = 0;
  s.eob = kFixNoEob;
  s.blocks = 0;
  s.status = 0;
  u32 kind = kFixGo, tokens = 0;
  for (;;) {
    if (p >= stop || (kMaxTokens && tokens == kMaxTokens)) break;
    ++tokens;
    const u64 b = pk(p);
    u32 nb, length, value;
    const u32 k = fixed_token(b, nb, length, value);
    if (k == kKindBad || p + nb > body_end) {
      kind = kFixError;
      s.status = k == kKindBad ? kBadSymbol : kTruncated;
      break;
    }
    if (k == kKindEob) {
      const u32 q = p + 7;
      if (s.eob == kFixNoEob) {
        s.eob = u16(q - rel0);
        s.eob_bytes = s.bytes;
      }
      if (in_final) {
        kind = kFixEnd;
        p = q;
        break;
      }
      if (q + 3 > body_end) {
        kind = kFixError;
        s.status = kTruncated;
        p = q;
        break;
      }
      const u32 h = u32(pk(q)) & 7u;  // BFINAL, then BTYPE
      if ((h >> 1) != 1u) {
        kind = kFixHeader;
        p = q;
        break;
      }
      ++s.blocks;
      in_final = h & 1u;
      p = q + 3;
      continue;
    }
    s.bytes += length;
    p += nb;
  }
  s.exit = u16(p - rel0);
  s.kind = u8(kind | (kind == kFixGo && in_final ? kFixInFinal : 0u));
  return s;
}

constexpr u32 kNoMerge = 0xffffffffu;
constexpr u32 kDescEvents = 4;           // events a slice decode records (it stops at the last)
constexpr u16 kNoEvent = 0xffffu;

// ---- describe: one 256-thread workgroup per candidate ----------------------
constexpr u32 kDescThreads = 256;
constexpr u32 kDescWaves = kDescThreads / 64;
constexpr u32 kVisitBits = 512;  // a slice records every token start (slices <= 512 bits)
constexpr u32 kVisitWords = kVisitBits / 64;
constexpr u32 kDescMinSlice = 192;  // > longest token (48 bits); short slices rarely resynchronize
constexpr u32 kDescMaxSlice = kVisitBits;
static_assert(u64(kDescThreads) * kDescMaxSlice <= u64(kStageBytes) * 8, "describe stage too small");

struct DescShared {
  DecodeTables tables;
  Stage stage;
  union {
    u16 codes[320];                        // scratch of cooperative table builds (headers only)
    u64 visit[kVisitWords][kDescThreads];  // token starts of each slice's own decode (word-major:
                                           // lanes touch consecutive banks)
  };
  u32 xpos[kDescThreads];                // stage-relative end of each slice decode
  u32 count[kDescThreads];               // bytes of each slice decode
  // Events (an EOB or an undecodable token) met by each slice decode, as
  // offsets from the slice start; the decode steps over them (past the EOB,
  // or one bit) and stops at the kDescEvents-th.  Only an event on the true
  // token path ends the block.
  u8 evn[kDescThreads];                  // events recorded
  u16 evp[kDescEvents][kDescThreads];
  u16 evq[kDescThreads];                 // lane 0 and merged lanes: first event at or after
                                         // the entry, or kNoEvent
  u32 merge[kDescThreads];               // offset from s_j where lane j-1's continuation met
                                         // lane j's tokens, or kNoMerge
  u32 merge2[kDescThreads];              // offset from s_j where lane j-2's continuation met
                                         // lane j's tokens after crossing slice j-1 (bits 0-8;
                                         // bits 9-31: lane j's bytes before it), or kNoMerge
  u32 tail[kDescThreads];                // bytes of lane j's continuation up to its merge
  union {
    // Phases 1-3: bytes lane j produced by the tokens starting in visit words
    // 0..w (read for w <= 6: at most 32 * 7 tokens of <= 258 bytes, 16 bits).
    u16 ck[kVisitWords][kDescThreads];
    u32 hruns[320];  // block_header: code-length runs of the wave walk
    struct {
      u32 before[kDescThreads];   // bytes lane j produced before its merge point
      u32 prefix[kDescThreads];   // inclusive prefix of per-slice bytes
      u32 entry[kDescThreads];    // stage-relative true entry of each slice
      u32 off[kDescThreads];      // block output offset of each slice
      u32 runbase[kDescThreads];  // run starts: off of lane k = runbase + prefix[k-1]
    };
  };
  u64 brk[kDescWaves], evm[kDescWaves], runs[kDescWaves], serial[kDescWaves];
  u32 wsum[kDescWaves];
  // control written by lane 0 (block_header interface: pos, d0, end, size, type, ...)
  u64 pos, d0, hint, end, size, round;
  u32 slice, need, table;
  u32 type, final_block, status, nl, nd, go, build_status, group, lanes;
};
// Three describe workgroups share a CU at this size; at 53 768 bytes only
// two did (measured on MI355X: the describe pass took 27 % longer), so the
// layout stays within 26 * 2 KiB.
static_assert(sizeof(DescShared) <= 26 * 2048, "describe LDS no longer fits three workgroups per CU");

__device__ __forceinline__ bool desc_visited(const DescShared& sh, u32 lane, u32 off) {
  return off < kVisitBits && ((sh.visit[off >> 6][lane] >> (off & 63)) & 1);
}

// Body end relative to the stage's word 0 (saturated).
__device__ __forceinline__ u32 stage_limit(const Stage& sg, u64 len) {
  const u64 lim = len * 8 - sg.bit0;  // modular: bit0 may precede the body by < 32 bits
  return lim > 0xffffffffull ? 0xffffffffu : u32(lim);
}

template <bool kChecked>
__device__ __forceinline__ WordBits<kChecked> word_bits(const Stage& sg, u32 limit, u32 pos) {
  WordBits<kChecked> r;
  r.words = sg.words;
  r.limit = limit;
  r.seek(pos);
  return r;
}

template <bool kChecked>
__device__ __forceinline__ Win4<kChecked> win4(const Stage& sg, u32 limit, u32 pos) {
  Win4<kChecked> r;
  r.words = sg.words;
  r.limit = limit;
  r.seek(pos);
  return r;
}

// One token with the full decoder (long codes, end of block, errors) at the
// window's position; on success the window moves past it.
template <bool kChecked>
__device__ __forceinline__ u32 full_token(const DecodeTables& t, Win4<kChecked>& r, u32& length,
                                       u32& lit, u32& distance) {
  return window_token<kChecked>(t.ll, t.dd, r, lit, length, distance);
}

// Token-level decode from r.pos() until it reaches `stop`.  An event (an EOB
// or an undecodable token) is recorded in evp (offset from win0) and stepped
// over: past the EOB, or by one bit for an error; the decode stops at the
// kDescEvents-th event.  Every token start in [win0, stop)
// (stop - win0 <= kVisitBits) is recorded in `visit`, and ck[w] ends as the
// bytes produced by the tokens starting in visit words 0..w.  Both are stored
// on every token, which is cheaper than branching on word changes.
template <bool kChecked>
__device__ void desc_slice(const DecodeTables& t, Win4<kChecked>& r, u32 stop, u64* visit,
                           u32 win0, u32& count, u32& nev, u16* evp, u16* ck) {
  u32 produced = 0, cw = 0;
  u64 bits = 0;
  nev = 0;
  for (u32 w = 0; w < kVisitWords; ++w) visit[w * kDescThreads] = 0;
  for (;;) {
    const u32 p = r.pos();
    if (p >= stop) break;
    const u32 off = p - win0;
    const u32 w = off >> 6;
    bits = (w == cw ? bits : 0ull) | (1ull << (off & 63));
    cw = w;
    visit[w * kDescThreads] = bits;
    u32 length, x, x2, l1;
    const u32 got = quick_pair<kChecked>(t.ll, t.dd, r, stop, length, x, x2, l1);
    if (!got) {
      u32 lit, distance;
      const u32 err = full_token<kChecked>(t, r, length, lit, distance);
      if (err || !length) {
        evp[nev * kDescThreads] = u16(off);
        if (++nev == kDescEvents) break;
        if (err) r.seek(p + 1);
        length = 0;
      }
    }
    produced += length;  // <= 512 tokens of <= 258 bytes per slice
    ck[w * kDescThreads] = u16(produced);  // read back for words 0..6 only: < 2^16
    if (got == 2) {
      // The pair's second literal starts l1 bits after the first (before stop).
      const u32 off2 = off + l1, w2 = off2 >> 6;
      bits = (w2 == cw ? bits : 0ull) | (1ull << (off2 & 63));
      cw = w2;
      visit[w2 * kDescThreads] = bits;
      ++produced;
      ck[w2 * kDescThreads] = u16(produced);
    }
  }
  count = produced;
}

// Bytes produced by decoding tokens from `from` up to token start `to`.
template <bool kChecked>
__device__ u32 desc_bytes_between(const DecodeTables& t, const Stage& sg, u32 limit, u32 from, u32 to) {
  Win4<kChecked> r = win4<kChecked>(sg, limit, from);
  u32 bytes = 0;
  while (r.pos() < to) {
    const u32 p = r.pos();
    u32 length, x, x2, l1;
    const u32 got = quick_pair<kChecked>(t.ll, t.dd, r, to, length, x, x2, l1);
    bytes += got >> 1;  // a pair's second literal
    if (!got) {
      u32 lit, distance;
      // Events are stepped over as desc_slice does.
      const u32 err = full_token<kChecked>(t, r, length, lit, distance);
      if (err) r.seek(p + 1);
      if (err || !length) length = 0;
    }
    bytes += length;
  }
  return bytes;
}

// Bytes lane `lane` produced from its slice start s0 up to its token start
// s0 + m: the checkpoint of m's visit word plus the few tokens from that
// word's first token start.
template <bool kChecked>
__device__ __forceinline__ u32 desc_bytes_before(const DescShared& sh, u32 lane, u32 limit, u32 s0,
                                                 u32 m) {
  const u32 w = m >> 6;
  const u32 base = w ? u32(sh.ck[w - 1][lane]) : 0u;  // a token starts in every word before m
  const u32 first = (w << 6) + u32(__builtin_ctzll(sh.visit[w][lane]));
  return base + desc_bytes_between<kChecked>(sh.tables, sh.stage, limit, s0 + first, s0 + m);
}

// First set bit at index >= from in a kDescThreads-bit mask, or kDescThreads.
__device__ __forceinline__ u32 next_bit(const u64* mask, u32 from) {
  for (u32 w = from >> 6; w < kDescWaves; ++w) {
    u64 m = mask[w];
    if (w == (from >> 6)) m &= ~0ull << (from & 63);
    if (m) return w * 64 + __builtin_ctzll(m);
  }
  return kDescThreads;
}

// Last set bit at index <= at (the mask has bit 0 set).
__device__ __forceinline__ u32 prev_bit(const u64* mask, u32 at) {
  for (u32 w = at >> 6;; --w) {
    u64 m = mask[w];
    if (w == (at >> 6) && (at & 63) != 63) m &= (2ull << (at & 63)) - 1;
    if (m) return w * 64 + 63 - __builtin_clzll(m);
    if (!w) return 0;
  }
}

// Reads a block header at sh.pos from the stage: lane 0 the block type and a
// stored block's fields, wave 0 a dynamic block's code lengths (the wave walk,
// or lane 0's serial parse where the walk cannot finish within the stage or
// without kWalk, which leaves sh.hruns out of the shared layout); then wave 0
// builds the fixed/dynamic tables.  Sets
// sh.type, sh.final_block, sh.status, sh.d0 (first token or payload bit) and,
// for stored blocks, sh.end/sh.size.
template <bool kOneWave = false, bool kFast = false, bool kWalk = true, typename Shared>
__device__ void block_header(const u8* body, u64 len, u64 limit, Shared& sh) {
  const u32 lane = threadIdx.x;
  if (!staged_covers(sh.stage, body, len, sh.pos, sh.pos + 4096)) {
    __syncthreads();
    stage_range(body, len, sh.pos, sh.pos + 64 * kMaxSlice, sh.stage);
  }
  __syncthreads();
  if (!lane) {
    BitIn r = staged_reader(sh.stage, len, sh.pos);
    u32 type = 0, fin = 0, err = 0;
    sh.nl = sh.nd = 0;
    if (!r.take(1, fin) || !r.take(2, type)) err = kTruncated;
    else if (type == 3) err = kReservedBlock;
    else if (type == 0) {
      r.seek((r.pos + 7) & ~u64(7));
      u32 nlen, comp;
      if (!r.take(16, nlen) || !r.take(16, comp)) err = kTruncated;
      else if ((nlen ^ comp) != 0xffffu) err = kBadSymbol;
      else if (nlen > limit) err = kOutputOverflow;
      else if (u64(nlen) * 8 > r.avail()) err = kTruncated;
      else {
        sh.end = r.pos + u64(nlen) * 8;
        sh.size = nlen;
      }
    } else if (type == 1) {
      sh.nl = 288;
      sh.nd = 32;
    }
    sh.d0 = r.pos;  // a dynamic block: the bit after BTYPE
    sh.type = type;
    sh.final_block = fin;
    sh.status = err;
  }
  __syncthreads();
  if (sh.type == 2 && !sh.status) {
    const u64 start = sh.d0;
    if constexpr (kWalk) {
      if (lane < 64) {
        u32 nl = 0, nd = 0, err = kOk, p = 0, lim = 0;
        u64 after = start;
        if (!header_prelude_wave(sh.stage.words, sh.stage.bit0, sh.stage.count, sh.tables, len,
                                 start, nl, nd, err, after, p, lim)) {
          err = kHeaderWalkStuck;
        } else if (!err) {
          err = header_lengths_wave(sh.stage.words, sh.tables, sh.hruns, nl + nd, p, lim);
          after = sh.stage.bit0 + p;
        }
        if (!lane) {
          sh.status = err;
          sh.nl = nl;
          sh.nd = nd;
          sh.d0 = after;
        }
      }
    } else {
      if (!lane) sh.status = kHeaderWalkStuck;
    }
    __syncthreads();
    if (!lane && sh.status == kHeaderWalkStuck) {
      BitIn r = staged_reader(sh.stage, len, start);
      u32 nl = 0, nd = 0;
      sh.status = parse_dynamic_lengths(sh.tables, r, nl, nd);
      sh.nl = nl;
      sh.nd = nd;
      sh.d0 = r.pos;
    }
    __syncthreads();
  }
  if (sh.type && !sh.status) {
    // The tables are built by one wave (wave 0 of a larger workgroup).
    if (!kOneWave || lane < 64) {
      const bool fixed = sh.type == 1;
      if (fixed) {
        for (u32 i = lane; i < 320; i += 64)
          sh.tables.lens[i] = i < 144 ? 8 : i < 256 ? 9 : i < 280 ? 7 : i < 288 ? 8 : 5;
        if (kOneWave) wave_sync();
        else __syncthreads();
      }
      u32 err = huff_build_wave<288, 10, kOneWave>(sh.tables.ll, sh.tables.lens, sh.nl, false,
                                                   true, 15, sh.codes, &sh.build_status);
      if (!err)
        err = huff_build_wave<32, 8, kOneWave>(sh.tables.dd, sh.tables.lens + sh.nl, sh.nd, !fixed,
                                               true, 15, sh.codes, &sh.build_status);
      if (!lane) sh.status = err;
      if (kFast && !err) {
        wave_sync();
        fast_format(sh.tables.ll, true, lane, 64);
        fast_format(sh.tables.dd, false, lane, 64);
      }
    }
    __syncthreads();
  }
}

// State of one block's description across rounds (meaningful in thread 0).
struct DescRun {
  u64 e_abs, total, end;
  u32 status, lanes_total, group, last_group;
  bool done, keep;
};

// One round of describe_tokens: 256 slices of `slice` bits from round_abs.
template <bool kChecked>
__device__ void describe_round(u64 len, u64 limit, DescShared& sh, State* st, u64* slice_entry,
                               u32* slice_off, u32* group_link, u64 group_capacity, DescRun& run,
                               u64 round_abs, u32 slice) {
  const u32 t = threadIdx.x, lane = lane_id(), wave = t >> 6;
  const u32 blim = stage_limit(sh.stage, len);
  const u32 r0 = u32(round_abs - sh.stage.bit0);
  const u32 s0 = r0 + t * slice;
  {  // 1. speculative slices, then 2. continuation into the next slice (and,
     // when it meets none of that slice's tokens, into the one after)
    Win4<kChecked> r = win4<kChecked>(sh.stage, blim, s0);
    u32 cnt, nev;
    desc_slice<kChecked>(sh.tables, r, s0 + slice, &sh.visit[0][t], s0, cnt, nev, &sh.evp[0][t],
                         &sh.ck[0][t]);
    sh.xpos[t] = r.pos();
    sh.count[t] = cnt;
    sh.evn[t] = u8(nev);
    __syncthreads();
    u32 merge = kNoMerge, merge2 = kNoMerge, tail = 0;
    // A decode stopped at its last event did not reach its slice end.
    if (t + 1 < kDescThreads && nev < kDescEvents) {
      u32 k = t + 1, sk = s0 + slice;
      for (;;) {
        const u32 off = r.pos() - sk;
        if (off >= slice) {
          if (k == t + 1 && k + 1 < kDescThreads) {
            ++k;
            sk += slice;
            continue;
          }
          break;
        }
        const bool seen = desc_visited(sh, k, off);
        u32 length, x, x2, l1;
        const u32 got = quick_pair<kChecked>(sh.tables.ll, sh.tables.dd, r, sk + slice, length, x,
                                             x2, l1);
        if (seen) {
          if (k == t + 1) merge = off;
          else merge2 = off;
          break;
        }
        if (!got) {
          u32 lit, distance;
          if (full_token<kChecked>(sh.tables, r, length, lit, distance) || !length) break;
        }
        tail += length;
        if (got == 2) {
          // A pair's second literal (inside slice k) may be where they meet.
          if (desc_visited(sh, k, off + l1)) {
            if (k == t + 1) merge = off + l1;
            else merge2 = off + l1;
            break;
          }
          ++tail;
        }
      }
    }
    if (t + 1 < kDescThreads) sh.merge[t + 1] = merge;
    if (t + 2 < kDescThreads) sh.merge2[t + 2] = merge2;
    sh.tail[t] = tail;
    if (!t) sh.merge[0] = kNoMerge;
    if (t < 2) sh.merge2[t] = kNoMerge;
  }
  __syncthreads();
  // 3. bytes before the merge point(s) of each lane's own decode; per-slice
  // bytes of a merged run (own bytes after the merge point plus the
  // continuation when the next lane merged), their prefix sum, and the break
  // and event masks.
  const u32 m1 = sh.merge[t], m2 = sh.merge2[t];
  // The first event at or after the entry of lane 0 (the slice start) or of
  // a merged lane (its merge point) lies on the true path and ends the block.
  u32 q = kNoEvent;
  if (t == 0 || m1 != kNoMerge) {
    const u32 from = t == 0 ? 0u : m1;
    const u32 n = sh.evn[t];
    for (u32 i = n; i-- > 0;) {
      const u32 o = sh.evp[i][t];
      q = o >= from ? o : q;
    }
  }
  sh.evq[t] = u16(q);
  u32 before = 0, at_event = 0;
#pragma nounroll
  for (u32 pass = 0; pass < 3; ++pass) {  // one call site keeps register use down
    const u32 m = pass == 0 ? m1 : pass == 1 ? m2 : (q == kNoEvent ? kNoMerge : q);
    if (m == kNoMerge) continue;
    const u32 v = desc_bytes_before<kChecked>(sh, t, blim, s0, m);
    if (pass == 0) before = v;
    else if (pass == 1) sh.merge2[t] = m2 | (v << 9);
    else at_event = v;
  }
  __syncthreads();  // the checkpoints share storage with the arrays below
  sh.before[t] = before;
  u32 bsl = sh.count[t] - before;
  if (q != kNoEvent) bsl = at_event - before;
  else if (t + 1 < kDescThreads && sh.merge[t + 1] != kNoMerge) bsl += sh.tail[t];
  u32 x = bsl;
  for (u32 o = 1; o < 64; o <<= 1) {
    const u32 y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) sh.wsum[wave] = x;
  const u64 bm = __ballot(t > 0 && sh.merge[t] == kNoMerge);
  const u64 em = __ballot(q != kNoEvent);
  if (!lane) {
    sh.brk[wave] = bm;
    sh.evm[wave] = em;
    sh.runs[wave] = 0;
    sh.serial[wave] = 0;
  }
  __syncthreads();
  for (u32 w = 0; w < wave; ++w) x += sh.wsum[w];
  sh.prefix[t] = x;
  __syncthreads();
  if (!t) {  // 4. runs and breaks
    u32 event_at = kNoMerge;  // stage position of the true event that ends the block
    u32 lanes = kDescThreads;
    u32 e = r0;         // true position
    u64 T = run.total;  // block bytes before e
    u32 j = 0;          // run start: lane j's own decode is true from e on
    u32 j_entry = r0;   // true entry of slice j
    u64 j_off = T;      // output offset of slice j's entry
    u32 j_bytes = 0;    // bytes lane j's decode produced before e
    bool round_done = false, done = false;
    while (!round_done && !done) {
      const u32 sj = r0 + j * slice;
      sh.entry[j] = j_entry;
      sh.off[j] = u32(j_off);
      sh.runs[j >> 6] |= 1ull << (j & 63);
      // Lane j's first event at or after e is on the true path.
      u32 qj = kNoEvent;
      for (u32 i = sh.evn[j]; i-- > 0;) {
        const u32 o = sh.evp[i][j];
        qj = sj + o >= e ? o : qj;
      }
      if (qj != kNoEvent) {
        T += desc_bytes_between<kChecked>(sh.tables, sh.stage, blim, sj, sj + qj) - j_bytes;
        event_at = sj + qj;
        lanes = j + 1;
        done = true;
        break;
      }
      // Lane j from e to its slice end, plus its continuation when lane j+1
      // merged; merged lanes after it add their per-slice bytes.
      const u32 bj = sh.count[j] - j_bytes +
                     (j + 1 < kDescThreads && sh.merge[j + 1] != kNoMerge ? sh.tail[j] : 0u);
      sh.runbase[j] = u32(T + bj - sh.prefix[j]);
      const u32 b = next_bit(sh.brk, j + 1), E = next_bit(sh.evm, j + 1);
      if (E < b) {
        T += bj + (sh.prefix[E] - sh.prefix[j]);
        event_at = r0 + E * slice + sh.evq[E];
        lanes = E + 1;
        done = true;
        break;
      }
      T += bj + (sh.prefix[b - 1] - sh.prefix[j]);
      e = sh.xpos[b - 1];
      if (b == kDescThreads) break;
      const u32 m2 = b + 1 < kDescThreads ? sh.merge2[b + 1] : kNoMerge;
      if (m2 != kNoMerge) {
        // Break at lane b, bridged by lane b-1's continuation: slice b starts
        // at the true position, and the run resumes at lane b+1's merge point.
        sh.entry[b] = e;
        sh.off[b] = u32(T);
        sh.serial[b >> 6] |= 1ull << (b & 63);
        T += sh.tail[b - 1];
        j = b + 1;
        j_entry = r0 + j * slice + (m2 & 511u);
        j_off = T;
        j_bytes = m2 >> 9;
        e = j_entry;
        continue;
      }
      // Break at lane b: decode serially from the true position until it
      // meets the tokens of a later lane.
      u32 k = b;
      for (;;) {
        if (k >= kDescThreads) { round_done = true; break; }
        const u32 sk = r0 + k * slice;
        const u32 k_entry = e;
        const u64 k_off = T;
        bool synced = false;
        WordBits<kChecked> r = word_bits<kChecked>(sh.stage, blim, e);
        for (;;) {
          const u32 off = e - sk;
          if (desc_visited(sh, k, off)) { synced = true; break; }
          if (off >= slice) break;
          u32 lit, length, distance;
          const u32 err = fast_token(sh.tables.ll, sh.tables.dd, r, lit, length, distance);
          if (err) { run.status = err; run.end = sh.stage.bit0 + e; done = true; break; }
          if (!length) { run.end = sh.stage.bit0 + r.pos(); done = true; break; }
          T += length;
          e = r.pos();
        }
        if (done || !synced) {
          // Slice k decoded serially (entirely, or up to the block end).
          sh.entry[k] = k_entry;
          sh.off[k] = u32(k_off);
          sh.serial[k >> 6] |= 1ull << (k & 63);
          if (done) { lanes = k + 1; break; }
          ++k;
          continue;
        }
        // Lane k's own decode is true from e: a run starts there.
        j = k;
        j_entry = k_entry;
        j_off = k_off;
        j_bytes = desc_bytes_between<kChecked>(sh.tables, sh.stage, blim, sk, e);
        break;
      }
    }
    if (event_at != kNoMerge) {
      // An EOB (the block's end) or an undecodable token (its status).
      WordBits<kChecked> r = word_bits<kChecked>(sh.stage, blim, event_at);
      u32 lit, length, distance;
      const u32 err = fast_token(sh.tables.ll, sh.tables.dd, r, lit, length, distance);
      if (err) run.status = err;
      run.end = sh.stage.bit0 + (err ? event_at : r.pos());
    }
    if (!done && T > limit) {
      run.status = kOutputOverflow;
      run.end = sh.stage.bit0 + e;
      done = true;
    }
    if (!done && sh.stage.bit0 + e >= len * 8) {
      run.status = kTruncated;
      run.end = sh.stage.bit0 + e;
      done = true;
    }
    run.total = T;
    run.e_abs = sh.stage.bit0 + e;
    run.done = done;
    // Slice groups for this round's lanes (consecutive ids, 64 slices each).
    const u32 ng = (lanes + 63) / 64;
    u32 g = kNone;
    if (run.keep) {
      const u64 gi = atomicAdd(reinterpret_cast<unsigned long long*>(&st->groups_used), u64(ng));
      if (gi + ng <= group_capacity) {
        g = u32(gi);
        if (run.last_group == kNone) run.group = g;
        else group_link[run.last_group] = g;
        for (u32 i = 0; i + 1 < ng; ++i) group_link[g + i] = g + i + 1;
        group_link[g + ng - 1] = kNone;
        run.last_group = g + ng - 1;
      } else {
        run.keep = false;
        run.group = kNone;
      }
    }
    run.lanes_total += lanes;
    sh.group = g;
    sh.lanes = lanes;
    sh.go = done ? 0u : 1u;
  }
  __syncthreads();
  // Entries and offsets of the merged lanes; slice groups.
  const u32 lanes = sh.lanes, g = sh.group;
  if (t < lanes) {
    u32 entry, off;
    if (((sh.runs[wave] | sh.serial[wave]) >> lane) & 1) {
      entry = sh.entry[t];
      off = sh.off[t];
    } else {
      const u32 j = prev_bit(sh.runs, t);
      entry = s0 + sh.merge[t];
      off = sh.runbase[j] + sh.prefix[t - 1];
    }
    if (g != kNone) {
      slice_entry[u64(g) * 64 + t] = sh.stage.bit0 + entry;
      slice_off[u64(g) * 64 + t] = off;
    }
  }
  __syncthreads();
}

// Describe the tokens of the fixed/dynamic block whose tables are built and
// whose tokens start at sh.d0.  Each round covers 256 slices of `slice` bits:
//   1. every lane decodes its slice speculatively, recording its token starts;
//   2. every lane continues past its slice end until it meets a token start
//      of the next lane (a merge: from there the two decodings coincide);
//   3. every lane counts the bytes it produced before its merge point;
//   4. a prefix sum gives every slice's output offset.  Lane 0 starts at the
//      round's true entry; a run of merged slices needs no further work, and
//      lane 0 decodes serially only where a merge is missing (a "break"),
//      until the true tokens meet the next lane's tokens.
// Rounds away from the body end decode without truncation checks.
// Results: sh.status, sh.end (bit after the EOB), sh.size, and slice groups
// (sh.group = kNone if capacity ran out; emission then decodes serially).
__device__ __forceinline__ void describe_tokens(const u8* body, u64 len, u64 limit,
                                                DescShared& sh, State* st, u64* slice_entry,
                                                u32* slice_off, u32* group_link,
                                                u64 group_capacity) {
  const u32 t = threadIdx.x;
  DescRun run;
  run.e_abs = sh.d0;
  run.total = 0;
  run.end = 0;
  run.status = 0;
  run.lanes_total = 0;
  run.group = kNone;
  run.last_group = kNone;
  run.done = false;
  run.keep = true;
  for (;;) {
    if (!t) {
      // Up to the hint (the next candidate) the slices spread the span evenly.
      const u64 span =
          sh.hint > run.e_abs ? sh.hint - run.e_abs : u64(kDescThreads) * kDescMaxSlice;
      // Rounds of equal slices, as few as the visit window allows.
      const u64 per_round = u64(kDescThreads) * kDescMaxSlice;
      const u64 rounds = (span + per_round - 1) / per_round;
      u64 slice = (span + kDescThreads * rounds - 1) / (kDescThreads * rounds);
      if (slice < kDescMinSlice) slice = kDescMinSlice;
      if (slice > kDescMaxSlice) slice = kDescMaxSlice;
      sh.slice = u32(slice);
      sh.go = run.done ? 0u : 1u;
      sh.round = run.e_abs;
      sh.need = !staged_covers(sh.stage, body, len, run.e_abs,
                               run.e_abs + u64(kDescThreads) * slice);
    }
    __syncthreads();
    if (!sh.go) break;
    const u64 round_abs = sh.round;
    const u32 slice = sh.slice;
    if (sh.need) {
      stage_range(body, len, round_abs, round_abs + u64(kDescThreads) * slice, sh.stage);
      __syncthreads();
    }
    // Unchecked decoding needs every bit a round can read (its slices, one
    // slice of continuation and a token of overshoot) before the body end.
    const bool near_end = round_abs + u64(kDescThreads + 1) * slice + 64 > len * 8;
    if (near_end)
      describe_round<true>(len, limit, sh, st, slice_entry, slice_off, group_link,
                           group_capacity, run, round_abs, slice);
    else
      describe_round<false>(len, limit, sh, st, slice_entry, slice_off, group_link,
                            group_capacity, run, round_abs, slice);
  }
  if (!t) {
    sh.status = run.status;
    sh.end = run.end;
    sh.size = run.total;
    sh.group = run.keep ? run.group : kNone;
    sh.lanes = run.lanes_total;
  }
  __syncthreads();
}

}  // namespace

namespace {

struct HeaderShared {
  DecodeTables tables;
  StageT<kHeaderWords> stage;
  u16 codes[320];
  u32 runs[320];  // code-length runs of the wave walk: first index | value << 9 | repeat << 13
  u64 d0;
  u32 status, type, fin, nl, nd, build_status;
  u32 walk;  // the wave walk runs
};

}  // namespace

// One wave per candidate (below the table capacity): parse its dynamic
// header, build the literal/length and distance tables in the fast format
// into the candidate's table slot, and record the first token bit and flags
// (hdr_info: status | BFINAL << 8 | BTYPE << 9).  Bit 0 is a candidate
// whatever its block type: a stored or fixed block there is only recorded
// (BTYPE != 2, no tables) and g_describe parses it itself.
__global__ __launch_bounds__(64) void g_headers(const u8* body, u64 len, const State* st,
                                                const u64* cand, BlockTables* tables,
                                                u64 table_capacity, u64* hdr_d0, u32* hdr_info) {
  __shared__ HeaderShared sh;
  if (st->status) return;
  const u32 lane = threadIdx.x;
  const u64 n = min<u64>(st->candidates, table_capacity);
  for (u64 c = blockIdx.x; c < n; c += gridDim.x) {
    const u64 pos = cand[c];
    stage_range(body, len, pos, pos + 8, sh.stage, kHeaderBytes);
    __syncthreads();
    // Lane 0 reads BFINAL and BTYPE; the wave reads the fields and the
    // code-length code and walks the lengths; lane 0 falls back to the
    // serial parser when the walk cannot finish within the staged words.
    const u64 start = pos + 3;
    if (!lane) {
      BitIn r = staged_reader(sh.stage, len, pos);
      u32 fin = 0, type = 0;
      sh.status = !r.take(1, fin) || !r.take(2, type) ? kTruncated : kOk;
      sh.type = type;
      sh.fin = fin;
      sh.nl = 0;
      sh.nd = 0;
      sh.d0 = r.pos;
      sh.walk = 0;
    }
    __syncthreads();
    u32 p = 0, lim = 0;  // the wave walk's start and read limit (stage bits)
    if (!sh.status && sh.type == 2) {
      u32 nl = 0, nd = 0, err = kOk;
      u64 after = start;
      const bool staged = header_prelude_wave(sh.stage.words, sh.stage.bit0, sh.stage.count,
                                              sh.tables, len, start, nl, nd, err, after, p, lim);
      if (!lane) {
        sh.status = staged ? err : kHeaderWalkStuck;
        sh.walk = staged && !err;
        sh.nl = nl;
        sh.nd = nd;
        sh.d0 = after;
      }
    }
    __syncthreads();
    if (sh.walk) {
      const u32 st_walk =
          header_lengths_wave(sh.stage.words, sh.tables, sh.runs, sh.nl + sh.nd, p, lim);
      if (!lane) {
        sh.status = st_walk;
        sh.d0 = sh.stage.bit0 + p;
      }
    }
    __syncthreads();
    if (!lane && sh.status == kHeaderWalkStuck) {
      BitIn r = staged_reader(sh.stage, len, start);
      u32 nl = 0, nd = 0;
      sh.status = parse_dynamic_lengths(sh.tables, r, nl, nd);
      sh.nl = nl;
      sh.nd = nd;
      sh.d0 = r.pos;
    }
    __syncthreads();
    u32 err = sh.status;
    if (!err && sh.type == 2) {
      err = huff_build_wave(sh.tables.ll, sh.tables.lens, sh.nl, false, true, 15, sh.codes,
                            &sh.build_status);
      if (!err)
        err = huff_build_wave(sh.tables.dd, sh.tables.lens + sh.nl, sh.nd, true, true, 15,
                              sh.codes, &sh.build_status);
      if (!err) {
        fast_format(sh.tables.ll, true, lane, 64);
        fast_format(sh.tables.dd, false, lane, 64);
      }
      __syncthreads();
      if (!err) {
        const u32* src_ll = reinterpret_cast<const u32*>(&sh.tables.ll);
        const u32* src_dd = reinterpret_cast<const u32*>(&sh.tables.dd);
        u32* dst_ll = reinterpret_cast<u32*>(&tables[c].ll);
        u32* dst_dd = reinterpret_cast<u32*>(&tables[c].dd);
        copy_tables<64>(dst_ll, dst_dd, src_ll, src_dd, lane);
      }
    }
    if (!lane) {
      hdr_d0[c] = sh.d0;
      hdr_info[c] = err | (sh.fin << 8) | (sh.type << 9);
    }
    __syncthreads();
  }
}

namespace {

// Marks tiles k0 .. k1 of the summary bitmap.
__device__ void fix_mark_tiles(u32* need, u64 k0, u64 k1) {
  for (u64 w = k0 >> 5; w <= (k1 >> 5); ++w) {
    const u32 lo = w == (k0 >> 5) ? ~0u << (k0 & 31) : ~0u;
    const u32 hi = w == (k1 >> 5) ? ~0u >> (31 - (k1 & 31)) : ~0u;
    atomicOr(need + w, lo & hi);
  }
}

// Candidates a region's marking looks past (their segments failed: header
// look-alikes inside the run's data) before it stops and leaves the rest of
// the run to the walk.
constexpr u32 kFixMarkScan = 4096;

}  // namespace

// One workgroup per candidate: describe the candidate's segment (its block and
// the following stored/fixed blocks up to the next candidate) with parallel
// token decoding, and record per-block slices for emission.  A fixed block
// whose decode is still going after kFixProbeTokens tokens starts a region:
// the segment stops there (kSegPaused; seg_end = the block's header bit,
// seg_last = its last block record) and g_fix_walk continues it from where
// workgroup's records go on (g_fix_mark marks the tiles to summarise).
__global__ __launch_bounds__(kDescThreads) void g_describe(
    const u8* body, u64 len, const u64* cand, State* st, u64 out_size, u64* seg_end,
    u64* seg_size, u32* seg_blocks, u32* seg_next, u32* seg_flags, u32* seg_rec, BlockRec* recs,
    u64 rec_capacity, u64* slice_entry, u32* slice_off, u32* group_link, u64 group_capacity,
    BlockTables* tables, u64 table_capacity, const u64* hdr_d0, const u32* hdr_info,
    u32* seg_last, u32* region_cand) {
  __shared__ DescShared sh;
  if (st->status) return;
  const u32 t = threadIdx.x;
  const u64 n = st->candidates;
  for (u64 c = blockIdx.x; c < n; c += gridDim.x) {
    u64 produced = 0;
    u32 blocks = 0, status = 0, final_block = 0, next = kNone, first_rec = kNone, last_rec = kNone;
    bool paused = false;
    // Thread 0: every candidate before this index lies at or before sh.pos
    // (the list is sorted and sh.pos only grows).
    u64 search_from = c + 1;
    bool recs_ok = true;
    // The candidate's own dynamic header was parsed by g_headers (tables in
    // slot c); any other block type at bit 0 is parsed below.  Its position,
    // header results and tables load at once (one memory latency).
    const u32 info0 = c < table_capacity ? hdr_info[c] : 0u;
    const bool pre0 = c < table_capacity && ((info0 >> 9) & 3u) == 2;
    if (!t) {
      sh.pos = cand[c];
      sh.stage.count = 0;
      sh.stage.bit0 = 0;
      if (pre0) {
        sh.status = info0 & 0xffu;
        sh.final_block = (info0 >> 8) & 1u;
        sh.type = (info0 >> 9) & 3u;
        sh.d0 = hdr_d0[c];
      }
    }
    if (pre0) {
      const u32* src_ll = reinterpret_cast<const u32*>(&tables[c].ll);
      const u32* src_dd = reinterpret_cast<const u32*>(&tables[c].dd);
      u32* dst_ll = reinterpret_cast<u32*>(&sh.tables.ll);
      u32* dst_dd = reinterpret_cast<u32*>(&sh.tables.dd);
      copy_tables<kDescThreads>(dst_ll, dst_dd, src_ll, src_dd, t);
    }
    __syncthreads();
    bool first = true;
    for (;;) {
      const bool pre = first && pre0;
      if (!pre) block_header<true, true>(body, len, out_size, sh);
      first = false;
      if (sh.type == 1 && !sh.status) {  // uniform
        // Probe the fixed run: a long one becomes a region.  Decoding garbage
        // (a header look-alike's block) meets an invalid code within a few
        // dozen tokens, so regions start only on real fixed data.  The scan is
        // inlined: as an outlined call it cost the pass a fifth of its time.
        constexpr u64 kProbeBits = u64(kFixProbeTokens) * 34;
        if (!staged_covers(sh.stage, body, len, sh.d0, sh.d0 + kProbeBits)) {
          __syncthreads();
          stage_range(body, len, sh.pos, sh.pos + 64 * kMaxSlice, sh.stage);
          __syncthreads();
        }
        if (!t) {
          const FixPeek pk{sh.stage.words, sh.stage.count};
          const u32 d0 = u32(sh.d0 - sh.stage.bit0);
          const FixSummary f = fix_scan<kFixProbeTokens>(pk, d0, 0xffffffffu,
                                                         stage_limit(sh.stage, len),
                                                         sh.final_block != 0, d0);
          sh.need = (f.kind & 15u) == kFixGo ? 1u : 0u;
          if (sh.need) {
            const u64 r = atomicAdd(reinterpret_cast<unsigned long long*>(&st->fix_regions), 1ull);
            region_cand[r] = u32(c);
            paused = true;
          }
        }
        __syncthreads();
        if (sh.need) break;  // uniform
      }
      if (!t && sh.type && !sh.status) {
        const u64 idx = lower_bound_from(cand, n, search_from, sh.pos + 1);
        search_from = idx;
        sh.hint = idx < n ? cand[idx] : len * 8;
        sh.group = kNone;
        sh.lanes = 0;
        if (pre) sh.table = u32(c);
        else {
          const u64 ti = atomicAdd(reinterpret_cast<unsigned long long*>(&st->tables_used), 1ull);
          sh.table = ti < table_capacity ? u32(ti) : kNone;
        }
      }
      __syncthreads();
      if (!pre && sh.type && !sh.status && sh.table != kNone) {
        // The block's tables for emission (raw words of both HuffTables).
        const u32* src_ll = reinterpret_cast<const u32*>(&sh.tables.ll);
        const u32* src_dd = reinterpret_cast<const u32*>(&sh.tables.dd);
        u32* dst_ll = reinterpret_cast<u32*>(&tables[sh.table].ll);
        u32* dst_dd = reinterpret_cast<u32*>(&tables[sh.table].dd);
        copy_tables<kDescThreads>(dst_ll, dst_dd, src_ll, src_dd, t);
      }
      if (sh.type && !sh.status)
        describe_tokens(body, len, out_size, sh, st, slice_entry, slice_off, group_link,
                        group_capacity);
      if (!t) {
        ++blocks;
        const u32 bstatus = sh.status;
        // Whether the block ends on a candidate, looked up before the record
        // is reserved so that the two memory latencies overlap.
        const u64 end_idx = lower_bound_from(cand, n, search_from, sh.end);
        const bool end_is_cand = end_idx < n && cand[end_idx] == sh.end;
        if (bstatus) status = bstatus;
        else {
          produced += sh.size;
          if (recs_ok) {
            const u64 ri = atomicAdd(reinterpret_cast<unsigned long long*>(&st->recs_used), 1ull);
            if (ri >= rec_capacity || ri >= kNone || (sh.type != 0 && sh.group == kNone)) {
              recs_ok = false;
            } else {
              BlockRec rec;
              rec.start = sh.pos;
              rec.data = sh.d0;
              rec.end = sh.end;
              rec.size = sh.size;
              rec.type = sh.type;
              rec.lanes = sh.type ? sh.lanes : 0;
              rec.group = sh.type ? sh.group : kNone;
              rec.next = kNone;
              rec.table = sh.type ? sh.table : kNone;
              rec.pad = 0;
              recs[ri] = rec;
              if (last_rec == kNone) first_rec = u32(ri);
              else recs[last_rec].next = u32(ri);
              last_rec = u32(ri);
            }
          }
          if (produced > out_size) status = kOutputOverflow;
          else if (sh.final_block) final_block = 1;
          else {
            const u64 p = sh.end;
            search_from = end_idx;
            if (end_is_cand) next = u32(end_idx);
            else {
              BitIn h;
              h.init(body, len, p);
              u32 f, type;
              if (h.take(1, f) && h.take(2, type) && type == 2) status = kUndiscovered;
              else if (blocks >= kMaxBlocks) status = kBlockCapacity;
            }
          }
        }
        sh.pos = sh.end;
        sh.go = (status || final_block || next != kNone) ? 0u : 1u;
      }
      __syncthreads();
      if (!sh.go) break;
    }
    if (!t) {
      if (paused) {
        seg_end[c] = sh.pos;
        seg_size[c] = produced;
        seg_blocks[c] = blocks;
        seg_next[c] = kNone;
        seg_flags[c] = kSegPaused | (recs_ok ? 0u : kSegRecsLost);
        seg_rec[c] = first_rec;
        seg_last[c] = last_rec;
      } else {
        seg_end[c] = sh.end;
        seg_size[c] = produced;
        seg_blocks[c] = blocks;
        seg_next[c] = next;
        seg_flags[c] = status | (final_block ? 0x80000000u : 0u);
        seg_rec[c] = recs_ok ? first_rec : kNone;
      }
    }
    __syncthreads();
  }
}

// Marks the tiles of every region for g_fix_sum: from the region's start to
// the first later candidate whose own segment did not fail (header
// look-alikes inside a run fail), at most kFixMarkScan candidates on.
__global__ __launch_bounds__(256) void g_fix_mark(const State* st, const u64* cand, u64 len,
                                                  const u64* seg_end, const u32* seg_flags,
                                                  const u32* region_cand, u32* fix_need,
                                                  u64 tiles) {
  if (st->status) return;
  const u64 regions = st->fix_regions, n = st->candidates;
  for (u64 r = threadIdx.x; r < regions; r += blockDim.x) {
    const u32 c = region_cand[r];
    const u64 x = seg_end[c];
    u64 j = lower_bound_from(cand, n, c + 1, x + 1);
    u64 h = len * 8;
    for (u32 k = 0; j < n; ++j, ++k) {
      if (k == kFixMarkScan || (seg_flags[j] & 0xffffu) == 0) {
        h = cand[j];
        break;
      }
    }
    if (tiles) fix_mark_tiles(fix_need, x / kFixTileBits, min<u64>(h / kFixTileBits, tiles - 1));
  }
}

namespace {

__device__ __forceinline__ u64 wave_fetch_add(u64* p, u64 v) {
  u64 old = 0;
  if (!lane_id()) old = atomicAdd(reinterpret_cast<unsigned long long*>(p), v);
  return __shfl(old, 0, 64);
}

// One wave's tile pair for g_fix_sum.  Every entry decodes to the first token
// start at or after kFixSyncBits; entries that reach the same one in the same
// state decode the same rest of the tile, which the lowest of them queues as
// one task for g_fix_rem (with the queue full, each entry decodes it here).
// The summaries of queued entries hold their prefixes until g_fix_rem joins
// the rest.  Fixed codes resynchronize slowly: after 256 bits the 32 entries
// of a tile typically still follow one to three token paths.
__device__ void fix_sum_pair(const u8* body, u64 len, const u32* need, FixSummary* sum, u64 tiles,
                             u64 k0, u32 pair, u32* w, u32 lane, State* st, FixTask* tasks,
                             u64 task_capacity) {
  // The wave stages body bits [k0 T, (k0 + 2) T) and the margin.
  const uintptr_t base = reinterpret_cast<uintptr_t>(body);
  const u64 byte0 = k0 * (kFixTileBits / 8);
  const u64 first_word = (base + byte0) >> 2;
  u64 last_byte = byte0 + 2 * (kFixTileBits / 8) + kFixMarginBytes;
  if (last_byte > len) last_byte = len;
  const u64 end_word = (base + last_byte + 3) >> 2;
  const u32 nwords = u32(min<u64>(end_word > first_word ? end_word - first_word : 0, kFixStageWords));
  const u32* g = reinterpret_cast<const u32*>(first_word << 2);
  wave_sync();  // the previous pair's reads of the stage are done
  for (u32 i = lane; i < nwords; i += 64) w[i] = g[i];
  wave_sync();
  const u32 half = lane >> 5, e = lane & 31u;
  const u64 k = k0 + half;
  const bool mine = k < tiles && ((pair >> half) & 1u);
  const u32 skew = u32((base + byte0) & 3u) * 8;  // stage bit of body bit k0 T
  const u32 rel = skew + half * kFixTileBits;
  const u32 body_end = u32(min<u64>(len * 8 - k0 * kFixTileBits + skew, 0xffffffffull));
  const FixPeek pk{w, nwords};
  FixSummary f{};
  if (mine) f = fix_scan(pk, rel + e, rel + kFixSyncBits, body_end, false, rel);
  const bool go = mine && (f.kind & 15u) == kFixGo;
  const u32 key = go ? u32(f.exit) | ((f.kind & kFixInFinal) ? 1u << 16 : 0u) | (half << 17) : ~0u;
  // Each lane's representative: the lowest lane with its key.
  u32 rep = lane, entries = 0;
  for (u64 todo = __ballot(go); todo;) {
    const u32 l = u32(__builtin_ctzll(todo));
    const u32 kl = __shfl(key, int(l), 64);
    const u64 same = __ballot(key == kl);
    todo &= ~same;
    if (key == kl) rep = l;
    if (lane == l) entries = u32(same >> (32 * half));
  }
  const bool lead = go && rep == lane;
  const u64 leads = __ballot(lead);
  const u64 slot0 = leads ? wave_fetch_add(&st->fix_tasks, u64(__popcll(leads))) : 0;
  const u64 slot = slot0 + u64(__popcll(leads & ((1ull << lane) - 1)));
  const bool queued = lead && slot < task_capacity;
  if (queued) {
    FixTask tk;
    tk.tile = k;
    tk.entries = entries;
    tk.p = f.exit;
    tk.in_final = (f.kind & kFixInFinal) ? 1 : 0;
    tasks[slot] = tk;
  }
  const u64 taken = __ballot(queued);
  if (go && !((taken >> rep) & 1u))
    f = fix_join(f, fix_scan(pk, rel + f.exit, rel + kFixTileBits, body_end,
                             (f.kind & kFixInFinal) != 0, rel));
  if (mine) sum[k * kFixEntries + e] = f;
}

}  // namespace

// Summaries of the marked tiles (one wave per two tiles: lane e decodes the
// first tile from its entry bit e, lane 32 + e the second), over the tiles
// and a margin staged in LDS.  Waves take tile pairs grid-stride.
__global__ __launch_bounds__(256) void g_fix_sum(const u8* body, u64 len, State* st,
                                                 const u32* need, FixSummary* sum, u64 tiles,
                                                 FixTask* tasks, u64 task_capacity) {
  __shared__ u32 words[kDescThreads / 64][kFixStageWords];
  if (st->status || !st->fix_regions) return;
  const u32 lane = lane_id(), wave = threadIdx.x >> 6;
  const u64 waves = u64(gridDim.x) * (kDescThreads / 64);
  for (u64 k0 = (u64(blockIdx.x) * (kDescThreads / 64) + wave) * 2; k0 < tiles; k0 += 2 * waves) {
    const u32 pair = (need[k0 >> 5] >> (k0 & 31)) & 3u;  // k0 is even: one need word
    if (pair)
      fix_sum_pair(body, len, need, sum, tiles, k0, pair, words[wave], lane, st, tasks,
                   task_capacity);
  }
}

// The queued rests of tiles: one thread per task decodes from the task's
// token start to the tile's end (the body read through the cache) and joins
// the result to the summaries of the task's entries.
__global__ __launch_bounds__(256) void g_fix_rem(const u8* body, u64 len, const State* st,
                                                 const FixTask* tasks, u64 task_capacity,
                                                 FixSummary* sum) {
  if (st->status || !st->fix_regions) return;
  const u64 n = min<u64>(st->fix_tasks, task_capacity);
  const uintptr_t base = reinterpret_cast<uintptr_t>(body);
  for (u64 i = u64(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += u64(gridDim.x) * blockDim.x) {
    const FixTask tk = tasks[i];
    // The tile and its margin, as g_fix_sum staged them.
    const u64 byte0 = tk.tile * (kFixTileBits / 8);
    const u64 first_word = (base + byte0) >> 2;
    u64 last_byte = byte0 + kFixTileBits / 8 + kFixMarginBytes;
    if (last_byte > len) last_byte = len;
    const u64 end_word = (base + last_byte + 3) >> 2;
    const u32 nwords = u32(end_word > first_word ? end_word - first_word : 0);
    const u32 skew = u32((base + byte0) & 3u) * 8;
    const u32 body_end = u32(min<u64>(len * 8 - tk.tile * kFixTileBits + skew, 0xffffffffull));
    FixStream pk;
    pk.w = reinterpret_cast<const u32*>(first_word << 2);
    pk.n = nwords;
    pk.seek(skew + tk.p);
    const FixSummary r =
        fix_scan(pk, skew + tk.p, skew + kFixTileBits, body_end, tk.in_final != 0, skew);
    for (u32 m = tk.entries; m; m &= m - 1) {
      FixSummary* s = sum + tk.tile * kFixEntries + __builtin_ctz(m);
      *s = fix_join(*s, r);
    }
  }
}

// Group summaries for the walk: one thread per (group of kFixGroupTiles
// wholly marked tiles, entry state) composes the group's tile summaries as
// the walk would step them (in the final block, a tile's first EOB ends the
// stream).
__global__ __launch_bounds__(256) void g_fix_groups(const State* st, const u32* need,
                                                    const FixSummary* sum, u64 tiles,
                                                    FixGroupSum* groups) {
  if (st->status || !st->fix_regions) return;
  const u64 n = tiles / kFixGroupTiles * 64;
  for (u64 i = u64(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += u64(gridDim.x) * blockDim.x) {
    const u64 k0 = i / 64 * kFixGroupTiles;
    if (((need[k0 >> 5] >> (k0 & 31)) & 0xffffu) != 0xffffu) continue;  // stepped tile by tile
    u32 e = u32(i & 31), bytes = 0, blocks = 0;
    bool fin = (i & 32) != 0;
    FixGroupSum r;
    r.exit = 0;
    r.kind = 0;
    r.tiles = 0;
    r.status = 0;
    for (u32 j = 0; j < kFixGroupTiles; ++j) {
      FixSummary f = sum[(k0 + j) * kFixEntries + e];
      if (fin && f.eob != kFixNoEob) {
        f.kind = kFixEnd;
        f.exit = f.eob;
        f.bytes = f.eob_bytes;
        f.blocks = 0;
      }
      bytes += f.bytes;
      blocks += f.blocks;
      if ((f.kind & 15u) != kFixGo) {
        r.exit = f.exit;
        r.kind = f.kind;
        r.tiles = u8(j + 1);
        r.status = f.status;
        break;
      }
      fin = fin || (f.kind & kFixInFinal) != 0;
      if (f.exit < kFixTileBits || f.exit - kFixTileBits >= kFixEntries) break;  // no jump (r.tiles 0)
      if (j + 1 == kFixGroupTiles) {
        r.exit = f.exit;
        r.kind = u8(kFixGo | (fin ? kFixInFinal : 0u));
        r.tiles = u8(kFixGroupTiles);
      }
      e = f.exit - kFixTileBits;
    }
    r.bytes = bytes;
    r.blocks = blocks;
    groups[i] = r;
  }
}



namespace {

constexpr u32 kFixBatch = 16;  // tiles of summaries a walk holds in LDS at once

struct FixWalkShared {
  FixSummary batch[kFixBatch][kFixEntries];
  u32 words[kFixStageWords / 2 + 8];  // one tile and its margin, for decodes without a summary
};

// An atomic add by lane 0, its old value given to every lane.
}  // namespace

// One wave per region: continue the paused segment from the fixed block at
// its seg_end.  Every lane follows the same walk (uniform loads; lane 0
// stores), and the wave loads summaries and stages tiles together.  Fixed
// runs are followed by summaries (a tile entered at a bit offset above 31, or
// not marked, is decoded from the stage); stored blocks are parsed in place;
// the segment ends at a final block, at a block boundary that is a candidate,
// or at an error, as describe ends it.  Each finished run gets a block record
// (kRecFixedRun) with consecutive slice groups and a FixRun; each of its tiles
// a FixTile slot for g_fix_slices.  When records, groups or slots run out the
// segment keeps no records (serial emission).
__global__ __launch_bounds__(64) void g_fix_walk(
    const u8* body, u64 len, State* st, const u64* cand, const u32* need, const FixSummary* sum,
    u64 tiles, u64* seg_end, u64* seg_size, u32* seg_blocks, u32* seg_next, u32* seg_flags,
    u32* seg_rec, const u32* seg_last, const u32* region_cand, BlockRec* recs, u64 rec_capacity,
    FixRun* runs, u64 run_capacity, FixTile* rt, u64 rt_capacity, u32* group_link,
    u64 group_capacity, u64 out_size, const FixGroupSum* groups) {
  __shared__ FixWalkShared sh;
  if (st->status) return;
  const u64 regions = st->fix_regions;
  const u64 n = st->candidates;
  const u32 lane = lane_id();
  const uintptr_t base = reinterpret_cast<uintptr_t>(body);
  for (u64 ri = blockIdx.x; ri < regions; ri += gridDim.x) {
    const u32 c = region_cand[ri];
    u64 pos = seg_end[c];  // the header of the region's first fixed block
    u64 out = seg_size[c];
    u64 blocks = seg_blocks[c];
    bool recs_ok = !(seg_flags[c] & kSegRecsLost);
    u32 first_rec = seg_rec[c], last_rec = seg_last[c];
    u64 search_from = c + 1;
    const u64 start_pos = pos;
    bool at_header = true, in_final = false, final_seg = false;
    u32 status = 0, next = kNone;
    bool run_on = false;
    u64 run_hdr = 0, run_tok = 0, run_out0 = 0;
    u32 run_id = kNone;
    u64 slot_base = 0;
    u32 slot_used = 64;
    bool chunk = false;  // slots slot_base .. +63 are this walk's (unused ones marked at the end)
    FixTile mine;        // lane l: slot l of the chunk, stored when the chunk is done
    u64 batch_k = ~0ull;
    u64 need_at = ~0ull;  // index of the cached word of the tile marks
    u32 need_word = 0;
    // Finishes the open run at bit `e_end`: its record, slice groups and FixRun.
    auto close_run = [&](u64 e_end) {
      run_on = false;
      if (run_id == kNone || !recs_ok) return;
      const u64 b0 = run_tok / kFixSliceBits, bl = (e_end - 1) / kFixSliceBits;
      const u64 lanes = bl - b0 + 1, ng = (lanes + 63) / 64;
      const u64 g = wave_fetch_add(&st->groups_used, ng);
      const u64 ri2 = wave_fetch_add(&st->recs_used, 1);
      if (g + ng > group_capacity || ri2 >= rec_capacity || ri2 >= kNone || lanes >= kNone) {
        recs_ok = false;
        return;
      }
      for (u64 i = lane; i < ng; i += 64) group_link[g + i] = i + 1 < ng ? u32(g + i + 1) : kNone;
      if (!lane) {
        FixRun fr;
        fr.tok = run_tok;
        fr.end = e_end;
        fr.b0 = b0;
        fr.lanes = u32(lanes);
        fr.group = u32(g);
        runs[run_id] = fr;
        BlockRec rec;
        rec.start = run_hdr;
        rec.data = run_tok;
        rec.end = e_end;
        rec.size = out - run_out0;
        rec.type = 1;
        rec.lanes = u32(lanes);
        rec.group = u32(g);
        rec.next = kNone;
        rec.table = kNone;
        rec.pad = kRecFixedRun;
        recs[ri2] = rec;
        if (last_rec != kNone) recs[last_rec].next = u32(ri2);
      }
      if (last_rec == kNone) first_rec = u32(ri2);
      last_rec = u32(ri2);
    };
    for (;;) {
      if (at_header) {
        if (pos != start_pos) {  // a block boundary: a candidate there ends the segment
          const u64 idx = lower_bound_from(cand, n, search_from, pos);
          search_from = idx;
          if (idx < n && cand[idx] == pos) {
            next = u32(idx);
            break;
          }
        }
        BitIn h;
        h.init(body, len, pos);
        u32 fin = 0, type = 0;
        if (!h.take(1, fin) || !h.take(2, type)) { status = kTruncated; break; }
        if (type == 3) { status = kReservedBlock; break; }
        if (type == 2) { status = kUndiscovered; break; }
        if (++blocks > kMaxBlocks) { status = kBlockCapacity; break; }
        if (type == 1) {
          if (!run_on) {
            run_on = true;
            run_hdr = pos;
            run_tok = pos + 3;
            run_out0 = out;
            run_id = kNone;
            if (recs_ok) {
              const u64 id = wave_fetch_add(&st->fix_runs, 1);
              if (id < run_capacity) {
                run_id = u32(id);
                if (!lane) runs[id].lanes = 0;  // until the run is finished
              } else {
                recs_ok = false;
              }
            }
          }
          in_final = fin != 0;
          pos += 3;
          at_header = false;
          continue;
        }
        // A stored block (RFC 1951 3.2.4), as describe_block reads it.
        if (run_on) close_run(pos);
        h.seek((h.pos + 7) & ~u64(7));
        u32 nlen = 0, comp = 0;
        if (!h.take(16, nlen) || !h.take(16, comp)) { status = kTruncated; break; }
        if ((nlen ^ comp) != 0xffffu) { status = kBadSymbol; break; }
        if (nlen > out_size - out) { status = kOutputOverflow; break; }
        if (u64(nlen) * 8 > h.avail()) { status = kTruncated; break; }
        if (recs_ok) {
          const u64 ri2 = wave_fetch_add(&st->recs_used, 1);
          if (ri2 >= rec_capacity || ri2 >= kNone) {
            recs_ok = false;
          } else {
            if (!lane) {
              BlockRec rec;
              rec.start = pos;
              rec.data = h.pos;
              rec.end = h.pos + u64(nlen) * 8;
              rec.size = nlen;
              rec.type = 0;
              rec.lanes = 0;
              rec.group = kNone;
              rec.next = kNone;
              rec.table = kNone;
              rec.pad = 0;
              recs[ri2] = rec;
              if (last_rec != kNone) recs[last_rec].next = u32(ri2);
            }
            if (last_rec == kNone) first_rec = u32(ri2);
            last_rec = u32(ri2);
          }
        }
        out += nlen;
        pos = h.pos + u64(nlen) * 8;
        if (fin) {
          final_seg = true;
          break;
        }
        continue;
      }
      // Inside a fixed run, at the token start `pos` of tile k.
      if (pos >= len * 8) { status = kTruncated; break; }
      const u64 k = pos / kFixTileBits;
      const u32 e = u32(pos - k * kFixTileBits);
      if (k < tiles && (k >> 5) != need_at) {  // the walk's tiles advance: one load per 32
        need_at = k >> 5;
        need_word = need[need_at];
      }
      const bool have = e < kFixEntries && k < tiles && ((need_word >> (k & 31)) & 1u);
      // At the first tile of a group of marked tiles: the whole group in one
      // step, unless the output or block limit fails inside it (then tile by
      // tile, which finds the failing tile).
      FixGroupSum gs;
      bool jump = false;
      if (have && k % kFixGroupTiles == 0 && k + kFixGroupTiles <= tiles &&
          ((need_word >> (k & 31)) & 0xffffu) == 0xffffu) {
        gs = groups[k / kFixGroupTiles * 64 + e + (in_final ? 32 : 0)];
        jump = gs.tiles != 0 && out + gs.bytes <= out_size && blocks + gs.blocks <= kMaxBlocks;
      }
      if (recs_ok && run_id != kNone) {
        if (slot_used == 64) {
          if (chunk) rt[slot_base + lane] = mine;  // the full chunk, one slot a lane
          slot_base = wave_fetch_add(&st->fix_rt, 64);
          slot_used = 0;
          chunk = slot_base + 64 <= rt_capacity;
          if (!chunk) {
            // Mark what fits of the chunk unused, and keep no records.
            if (slot_base + lane < rt_capacity) rt[slot_base + lane].run = kNone;
            recs_ok = false;
          }
        }
        if (recs_ok) {
          if (lane == slot_used) {
            mine.pos = pos;
            mine.off = u32(out - run_out0);
            mine.run = run_id;
            mine.k = u32(k);
            mine.tiles = jump ? gs.tiles : 1u;
          }
          ++slot_used;
        }
      }
      if (jump) {
        out += gs.bytes;
        blocks += gs.blocks;
        pos = (k + gs.tiles - 1) * kFixTileBits + gs.exit;
        const u32 kind = gs.kind & 15u;
        if (kind == kFixGo) {
          in_final = (gs.kind & kFixInFinal) != 0;
        } else if (kind == kFixEnd) {
          close_run(pos);
          final_seg = true;
          break;
        } else if (kind == kFixHeader) {
          close_run(pos);
          at_header = true;
        } else {
          status = gs.status ? gs.status : u32(kBadSymbol);
          break;
        }
        continue;
      }
      FixSummary f;
      if (have) {
        if (k < batch_k || k >= batch_k + kFixBatch) {
          // The next kFixBatch tiles' summaries, 16 bytes a load.
          const uint4* src = reinterpret_cast<const uint4*>(sum + k * kFixEntries);
          uint4* dst = reinterpret_cast<uint4*>(&sh.batch[0][0]);
          const u64 avail = min<u64>(kFixBatch, tiles - k) * kFixEntries;
          for (u32 i = lane; i < kFixBatch * kFixEntries; i += 64)
            if (i < avail) dst[i] = src[i];
          wave_sync();
          batch_k = k;
        }
        f = sh.batch[k - batch_k][e];
        if (in_final && f.eob != kFixNoEob) {
          // The stream's last block ends at its first EOB.
          f.kind = kFixEnd;
          f.exit = f.eob;
          f.bytes = f.eob_bytes;
          f.blocks = 0;
        }
      } else {
        // Decode from the stage: tile k and its margin.
        const u64 byte0 = k * (kFixTileBits / 8);
        const u64 first_word = (base + byte0) >> 2;
        u64 last_byte = byte0 + kFixTileBits / 8 + kFixMarginBytes;
        if (last_byte > len) last_byte = len;
        const u64 end_word = (base + last_byte + 3) >> 2;
        const u32 nwords = u32(min<u64>(end_word > first_word ? end_word - first_word : 0,
                                        kFixStageWords / 2 + 8));
        const u32* gw = reinterpret_cast<const u32*>(first_word << 2);
        wave_sync();  // earlier reads of the stage are done
        for (u32 i = lane; i < nwords; i += 64) sh.words[i] = gw[i];
        wave_sync();
        const u32 skew = u32((base + byte0) & 3u) * 8;
        const u64 body_end = len * 8 - k * kFixTileBits + skew;
        const FixPeek pk{sh.words, nwords};
        f = fix_scan(pk, skew + e, skew + kFixTileBits, u32(min<u64>(body_end, 0xffffffffull)),
                     in_final, skew);
      }
      out += f.bytes;
      blocks += f.blocks;
      if (out > out_size) { status = kOutputOverflow; break; }
      if (blocks > kMaxBlocks) { status = kBlockCapacity; break; }
      const u32 kind = f.kind & 15u;
      if (kind == kFixGo) {
        in_final = (f.kind & kFixInFinal) != 0 || (have && in_final);
        pos = k * kFixTileBits + f.exit;
      } else if (kind == kFixEnd) {
        pos = k * kFixTileBits + f.exit;
        close_run(pos);
        final_seg = true;
        break;
      } else if (kind == kFixHeader) {
        pos = k * kFixTileBits + f.exit;
        close_run(pos);
        at_header = true;
      } else {
        pos = k * kFixTileBits + f.exit;
        status = f.status ? f.status : u32(kBadSymbol);
        break;
      }
    }
    // The last chunk: its used slots, and its unused ones marked.
    if (chunk) {
      if (lane < slot_used) rt[slot_base + lane] = mine;
      else rt[slot_base + lane].run = kNone;
    }
    if (!lane) {
      seg_end[c] = pos;
      seg_size[c] = out;
      seg_blocks[c] = u32(min<u64>(blocks, 0xffffffffull));
      seg_next[c] = next;
      seg_flags[c] = status | (final_seg && !status ? 0x80000000u : 0u);
      seg_rec[c] = recs_ok ? first_rec : kNone;
    }
    wave_sync();
  }
}

// Slices of the walked runs: one thread per tile slot decodes the tile from
// its true entry and places the slices whose 512-bit windows start inside
// it (slice b - b0 of the run starts at the first token at or after bit
// 512 b; where the run ends first, at the run's end, with nothing to decode).
__global__ __launch_bounds__(256) void g_fix_slices(const u8* body, u64 len, const State* st,
                                                    const FixTile* rt, u64 rt_capacity,
                                                    const FixRun* runs, u64 run_capacity,
                                                    const FixSummary* sum, u64* slice_entry,
                                                    u32* slice_off) {
  if (st->status || !st->fix_regions) return;
  const u64 used = min<u64>(st->fix_rt, rt_capacity);
  const u64 nruns = min<u64>(st->fix_runs, run_capacity);
  const uintptr_t base = reinterpret_cast<uintptr_t>(body);
  const u32* words = reinterpret_cast<const u32*>(base & ~uintptr_t(3));
  const u64 skew = u64(base & 3u) * 8;
  const u64 nwords = (u64(base & 3u) + len + 3) / 4;
  for (u64 i = u64(blockIdx.x) * blockDim.x + threadIdx.x; i < used * kFixGroupTiles;
       i += u64(gridDim.x) * blockDim.x) {
    // Tile j of slot i / kFixGroupTiles.
    const FixTile ft = rt[i / kFixGroupTiles];
    const u32 j = u32(i % kFixGroupTiles);
    if (ft.run == kNone || ft.run >= nruns || j >= ft.tiles) continue;
    const FixRun run = runs[ft.run];
    if (!run.lanes) continue;
    // The tile's true entry and offset: through the summaries of the tiles
    // before it in the group (inside a group every tile but the last is
    // left at its end, so the final-block rule never applies to them).
    const u64 k = u64(ft.k) + j;
    u64 p = ft.pos;
    u32 off = ft.off;
    if (j) {
      u32 e = u32(ft.pos - u64(ft.k) * kFixTileBits);
      for (u32 q = 0; q < j; ++q) {
        const FixSummary f = sum[(u64(ft.k) + q) * kFixEntries + e];
        off += f.bytes;
        e = u32(f.exit) - kFixTileBits;
      }
      p = k * kFixTileBits + e;
    }
    const u64 bl = run.b0 + run.lanes - 1;
    const u64 bf = max<u64>(run.b0, k * kFixTileSlices);
    const u64 bt = min<u64>(bl, k * kFixTileSlices + kFixTileSlices - 1);
    const u64 at = u64(run.group) * 64 - run.b0;  // slice index of window b: at + b
    slice_entry[at + bf] = p;
    slice_off[at + bf] = off;
    // Windows up to bt; the tile whose decode reaches the run's end also
    // places the windows after it (the run's last EOB may end past the tile).
    const u64 tile_end = (k + 1) * kFixTileBits;
    // The body read from the tile's first word on (bit p at p - tile + skew).
    const u64 tile0 = k * kFixTileBits, w0 = tile0 / 32;
    FixStream in;
    in.w = words + w0;
    in.n = u32(min<u64>(nwords > w0 ? nwords - w0 : 0, 0xffffffffull));
    in.seek(u32(p - tile0 + skew));
    for (u64 b = bf + 1; b <= bl;) {
      if (p >= run.end || (b <= bt && p >= b * kFixSliceBits)) {
        if (p > run.end) p = run.end;
        slice_entry[at + b] = p;
        slice_off[at + b] = off;
        ++b;
        continue;
      }
      if (b > bt && p >= tile_end) break;  // the next tile places the rest
      // 64 body bits at p (bits past the body's words read as zero).
      const u64 bits = in(u32(p - tile0 + skew));
      u32 nb, length, value;
      const u32 kind = fixed_token(bits, nb, length, value);
      if (kind == kKindBad) {
        p = run.end;  // never on a walked run; emission then reports an extent error
        continue;
      }
      if (kind == kKindEob) {
        p = p + 7 >= run.end ? run.end : p + 10;  // past the next fixed header
        continue;
      }
      off += length;
      p += nb;
    }
  }
}

constexpr u32 kChainLdsNodes = 12288;  // candidates whose exits g_chain keeps in LDS

// One 1024-thread workgroup: path from candidate 0, output prefixes and
// acceptance of the whole chain.  Thread t owns the candidates [lo, hi) of
// range t.  When the candidates fit in LDS (kChainLdsNodes), a thread keeps
// its candidates' links, sizes and block counts in registers, loaded at once,
// and walks them in candidate order (a link always points to a later
// candidate), so no step waits on a chain of dependent loads.
__global__ __launch_bounds__(1024) void g_chain(State* st, const u64* __restrict__ cand,
                                                const u64* __restrict__ seg_end,
                                                const u64* __restrict__ seg_size,
                                                const u32* __restrict__ seg_blocks,
                                                const u32* __restrict__ seg_next,
                                                const u32* __restrict__ seg_flags,
                                                const u32* __restrict__ seg_rec,
                                                u32* __restrict__ exit_node, u64 len,
                                                u64 out_size, u32 max_blocks,
                                                Segment* __restrict__ acc, u64 out_base,
                                                OpenEnd open) {
  constexpr u32 kPer = kChainLdsNodes / 1024;  // candidates per thread in LDS mode
  __shared__ u32 entry[1024];
  __shared__ u64 psize[1024], pblocks[1024], pcount[1024];
  __shared__ u32 lexit[kChainLdsNodes];  // exit_node in LDS when the candidates fit
  __shared__ u32 wexit[kChainLdsNodes];  // first node outside the wave's span (LDS mode)
  __shared__ u32 wentry[16];
  __shared__ u32 last_node, last_wave, path_end;
  __shared__ u32 ok;
  if (st->status) return;
  const u32 t = threadIdx.x;
  const u64 n = st->candidates;
  if (!n) {  // no candidate (bit 0 always is one): nothing to accept
    if (!t) {
      st->chain_ok = 0;
      st->accepted = 0;
    }
    return;
  }
  const bool in_lds = n <= kChainLdsNodes;
  const u64 per = (n + 1023) / 1024;
  const u64 lo = min<u64>(n, u64(t) * per), hi = min<u64>(n, lo + per);
  u32 bl[kPer];
  u64 sz[kPer];
#pragma unroll
  for (u32 i = 0; i < kPer; ++i) {
    const u64 c = lo + i;
    const bool mine = in_lds && c < hi;
    if (mine) wexit[c] = seg_next[c];  // the links, staged in LDS
    sz[i] = mine ? seg_size[c] : 0ull;
    bl[i] = mine ? seg_blocks[c] : 0u;
  }
  if (in_lds) {  // uniform
    // 1. exits: first node outside [lo, hi) reached from each node.
#pragma unroll
    for (u32 j = 0; j < kPer; ++j) {
      const u64 c = lo + kPer - 1 - j;
      if (c < hi) {
        const u32 x = wexit[c];
        lexit[c] = (x == kNone || x >= hi) ? x : lexit[x];
      }
    }
  } else {
    for (u64 c = hi; c-- > lo;) {
      const u32 x = seg_next[c];
      exit_node[c] = (x == kNone || x >= hi) ? x : exit_node[x];
    }
  }
  entry[t] = kNone;
  if (t < 16) wentry[t] = kNone;
  if (!t) path_end = kNone;
  __syncthreads();
  // 2. entry node of every range on the path from node 0.
  if (in_lds) {
    // Exits from each wave's span (64 ranges) by pointer doubling, then a
    // walk over the 16 spans, then one walk per wave inside its span.
    const u32 wave = t >> 6;
    const u64 whi = min<u64>(n, (u64(wave) * 64 + 64) * per);
    for (u64 c = lo; c < hi; ++c) wexit[c] = lexit[c];
    __syncthreads();
    for (u32 round = 0; round < 7; ++round) {  // 2^7 > 64 ranges per span
      for (u64 c = lo; c < hi; ++c) {
        const u32 y = wexit[c];
        if (y != kNone && y < whi) wexit[c] = wexit[y];
      }
      __syncthreads();
    }
    const u32 span = u32(per) * 64;
    if (!t) {
      u32 cur = 0, lw = 0;
      while (cur != kNone) {
        lw = cur / span;
        wentry[lw] = cur;
        cur = wexit[cur];
      }
      last_wave = lw;
    }
    __syncthreads();
    if ((t & 63) == 0 && wentry[wave] != kNone) {
      u32 cur = wentry[wave], last = cur;
      while (cur != kNone && cur < whi) {
        entry[cur / u32(per)] = cur;
        last = cur;
        cur = lexit[cur];
      }
      if (wave == last_wave) last_node = last;
    }
  } else if (!t) {
    // Walk ranges from node 0 (one dependent global read per range).
    u32 cur = 0;
    u32 last = 0;
    while (cur != kNone) {
      entry[per ? u32(cur / per) : 0] = cur;
      last = cur;
      cur = exit_node[cur];
    }
    last_node = last;
  }
  __syncthreads();
  // The links again, into LDS (wexit is done with; a thread reads back only
  // its own candidates'): independent loads, one latency.
  u32* lnext = wexit;
  if (in_lds) {
#pragma unroll
    for (u32 i = 0; i < kPer; ++i)
      if (lo + i < hi) lnext[lo + i] = seg_next[lo + i];
  }
  // 3. mark path nodes inside each range and sum their sizes; the range
  // where the path ends records its last node.
  u64 s = 0, b = 0, k = 0;
  if (in_lds) {
    u32 cur = entry[t];
#pragma unroll
    for (u32 i = 0; i < kPer; ++i) {
      const u64 c = lo + i;
      if (c < hi && c == cur) {
        s += sz[i];
        b += bl[i];
        ++k;
        cur = lnext[c];
        if (cur == kNone) path_end = u32(c);
      }
    }
  } else {
    u32 cur = entry[t];
    while (cur != kNone && cur < hi) {
      s += seg_size[cur];
      b += seg_blocks[cur];
      ++k;
      cur = seg_next[cur];
    }
  }
  // Inclusive prefix sums over the 1024 ranges: wave scans by shuffles, then
  // the earlier waves' totals (one barrier in between).
  {
    const u32 lane = t & 63, wave = t >> 6;
    u64 xs = s, xb = b, xk = k;
#pragma unroll
    for (u32 off = 1; off < 64; off <<= 1) {
      const u64 ys = __shfl_up(xs, off, 64), yb = __shfl_up(xb, off, 64),
                yk = __shfl_up(xk, off, 64);
      if (lane >= off) {
        xs += ys;
        xb += yb;
        xk += yk;
      }
    }
    if (lane == 63) {
      psize[wave] = xs;
      pblocks[wave] = xb;
      pcount[wave] = xk;
    }
    __syncthreads();
    u64 ws = 0, wb = 0, wk = 0;
    for (u32 w = 0; w < wave; ++w) {
      ws += psize[w];
      wb += pblocks[w];
      wk += pcount[w];
    }
    __syncthreads();
    psize[t] = ws + xs;
    pblocks[t] = wb + xb;
    pcount[t] = wk + xk;
    __syncthreads();
  }
  if (!t) {
    // The path's last node: recorded in LDS mode, else followed by next
    // pointers inside the last entered range.
    u32 z = last_node;
    if (in_lds && path_end != kNone) z = path_end;
    else
      while (seg_next[z] != kNone) z = seg_next[z];
    const u32 flags = seg_flags[z];
    const u64 total = psize[1023], blocks = pblocks[1023], count = pcount[1023];
    const u64 end_byte = (seg_end[z] + 7) / 8;
    const bool fits = open.open ? total <= out_size && end_byte + open.trailer <= len
                                : total == out_size && end_byte == len;
    const bool good = (flags & 0x7fffffffu) == 0 && (flags & 0x80000000u) && fits &&
                      blocks <= max_blocks;
    ok = good ? 1u : 0u;
    st->chain_ok = ok;
    st->accepted = good ? count : 0;
    if (good) {
      st->stream_end = seg_end[z];
      st->produced = total;
    }
  }
  __syncthreads();
  if (!ok) return;
  // 4. write accepted segments in order.
  u64 offset = out_base + psize[t] - s, index = pcount[t] - k;
  if (in_lds) {
    u32 cur = entry[t];
#pragma unroll
    for (u32 i = 0; i < kPer; ++i) {
      const u64 c = lo + i;
      if (c < hi && c == cur) {
        acc[index].start = cand[c];
        acc[index].end = seg_end[c];
        acc[index].prefix = offset;
        acc[index].size = sz[i];
        acc[index].rec_first = seg_rec[c];
        acc[index].rec_count = bl[i];
        offset += sz[i];
        ++index;
        cur = lnext[c];
      }
    }
  } else {
    u32 cur = entry[t];
    while (cur != kNone && cur < hi) {
      acc[index].start = cand[cur];
      acc[index].end = seg_end[cur];
      acc[index].prefix = offset;
      acc[index].size = seg_size[cur];
      acc[index].rec_first = seg_rec[cur];
      acc[index].rec_count = seg_blocks[cur];
      offset += seg_size[cur];
      ++index;
      cur = seg_next[cur];
    }
  }
}

namespace {
struct WalkShared {
  DecodeTables tables;
  u8 lut[128];
};
}  // namespace

// Exact serial walk (the reference's select_chain precedence); runs only when
// the fast chain did not accept the stream.  On success it rebuilds the
// accepted list one block per entry.
__global__ __launch_bounds__(64) void g_exact_walk(const u8* body, u64 len, State* st,
                                                   u64 out_size, u32 max_blocks, Segment* acc,
                                                   u64 out_base, OpenEnd open) {
  __shared__ WalkShared sh;
  if (st->status || st->chain_ok || threadIdx.x) return;
  if (open.windowed) {
    st->status = kTruncated;
    return;
  }
  const u64 start = st->start_bit;
  u64 next = start, output = 0, n = 0;
  u32 status = 0;
  for (;;) {
    if (n >= max_blocks) { status = kBlockCapacity; break; }
    BitIn h;
    h.init(body, len, next);
    u32 f, type;
    if (!h.take(1, f) || !h.take(2, type)) { status = kTruncated; break; }
    if (type == 3) { status = kReservedBlock; break; }
    u64 limit = out_size - output;
    if (next == start || type == 2) {
      if (next != start && !dynamic_header_valid(body, len, next, sh.lut, 1)) {
        status = kUndiscovered;
        break;
      }
      limit = out_size;
    }
    BitIn r;
    r.init(body, len, next);
    u32 final_block;
    u64 size;
    status = describe_block(r, sh.tables, limit, final_block, size);
    if (status) break;
    const u64 end = r.pos;
    if (end <= next || end > len * 8) { status = kExtent; break; }
    if (size > out_size - output) { status = kOutputOverflow; break; }
    acc[n].start = next;
    acc[n].end = end;
    acc[n].prefix = out_base + output;
    acc[n].size = size;
    acc[n].rec_first = kNone;
    acc[n].rec_count = 1;
    ++n;
    output += size;
    next = end;
    if (final_block) {
      if (open.open) {
        // The member's trailer must follow its last block.
        if ((next + 7) / 8 + open.trailer > len) status = kTruncatedZlib;
      } else if (output != out_size) {
        status = kSizeMismatch;
      } else if ((next + 7) / 8 != len) {
        status = kExtent;
      }
      break;
    }
  }
  st->status = status;
  st->accepted = status ? 0 : n;
  st->stream_end = next;
  st->produced = output;
}

namespace {

struct EmitShared {
  DecodeTables tables;
  u32 action;
  u32 error;
  u64 begin, length, distance, src;
  u32 done;
};

__device__ __forceinline__ bool bit_get(const u32* bits, u64 i) {
  const u32 w = __hip_atomic_load(bits + (i >> 5), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return (w >> (i & 31)) & 1u;
}
// Resolve groups: the 2048 output bytes of 64 bitmap words, one resolve wave's
// share.  A byte per group marks a group that may hold unresolved bytes;
// resolve rounds skip the others.
constexpr u32 kResolveGroupShift = 11;
__device__ __forceinline__ void mark_groups(u8* marks, u64 first, u64 n) {
  if (!marks || !n) return;
  for (u64 g = first >> kResolveGroupShift; g <= (first + n - 1) >> kResolveGroupShift; ++g)
    marks[g] = 1;
}

__device__ __forceinline__ void bit_set(u32* bits, u64 i) {
  atomicOr(bits + (i >> 5), 1u << (i & 31));
}

// Copies one output byte from `src` to `dst` inside a segment starting at
// `seg`; sources outside the segment or still unresolved make the byte
// unresolved.  Returns true when the byte was queued.
// Written bytes are added to Adler-32 sums S (s) and W (w), a byte at output
// position p weighing end - p.
__device__ __forceinline__ bool copy_byte(u8* out, u32* roots, u32* unres, u64 seg, u64 dst,
                                          u64 src, u64& s, u64& w, u64 end) {
  if (src < seg) {
    roots[dst] = u32(src);
    bit_set(unres, dst);
    return true;
  }
  if (bit_get(unres, src)) {
    roots[dst] = roots[src];
    bit_set(unres, dst);
    return true;
  }
  const u8 v = out[src];
  out[dst] = v;
  s += v;
  w += (end - dst) * v;
  if (w >> 62) w %= kAdlerMod;
  return false;
}

// Adler-32 pairs are added (atomically) into this many slots per producing
// kernel, so that g_finish sums a few hundred pairs whatever the grids.
constexpr u32 kAdlerSlots = 64;

// Sum of a workgroup's per-thread Adler-32 pairs, reduced mod 65521 (valid
// in thread 0); `red` holds two u64 per wave.
__device__ __forceinline__ void adler_block_sum(u64& s, u64& w, u64 (*red)[16]) {
  const u32 t = threadIdx.x, waves = blockDim.x / 64;
  s %= kAdlerMod;
  w %= kAdlerMod;
  for (u32 off = 32; off; off >>= 1) {
    s += __shfl_down(s, off, 64);
    w += __shfl_down(w, off, 64);
  }
  if (lane_id() == 0) {
    red[0][t >> 6] = s;
    red[1][t >> 6] = w;
  }
  __syncthreads();
  if (!t) {
    s = w = 0;
    for (u32 k = 0; k < waves; ++k) {
      s += red[0][k];
      w += red[1][k];
    }
    s %= kAdlerMod;
    w %= kAdlerMod;
  }
}

}  // namespace

// One wave per accepted segment: lane 0 parses, the wave copies stored
// payloads and long matches.  Output positions are absolute.
__global__ __launch_bounds__(64) void g_emit_serial(const u8* body, u64 len, State* st,
                                                    const Segment* acc, u8* out, u32* roots,
                                                    u32* unres, u64 out_end, u64* parts,
                                                    u8* marks) {
  __shared__ EmitShared sh;
  __shared__ u64 red[2][16];
  if (st->status) return;
  const u32 lane = threadIdx.x;
  const u64 segments = st->accepted;
  const u32 window = st->window;
  u64 as = 0, aw = 0;  // Adler-32 sums of the bytes this lane writes
  for (u64 si = blockIdx.x; si < segments; si += gridDim.x) {
    const Segment seg = acc[si];
    if (seg.rec_first != kNone) continue;
    // Lane-0 parser state.
    BitIn r;
    u64 produced = 0;
    u32 error = 0, final_block = 0;
    bool need_header = true, complete = false;
    if (!lane) r.init(body, len, seg.start);
    while (true) {
      if (!lane) {
        u32 action = 0;
        while (!error && !complete) {
          if (need_header) {
            // Deterministic re-parse of a described segment: it ends exactly at seg.end.
            if (r.pos >= seg.end) { complete = true; break; }
            u32 type;
            if (!r.take(1, final_block) || !r.take(2, type) || type == 3) { error = kExtent; break; }
            if (type == 0) {
              r.seek((r.pos + 7) & ~u64(7));
              u32 nlen, comp;
              if (!r.take(16, nlen) || !r.take(16, comp) || u64(nlen) * 8 > r.avail()) {
                error = kExtent;
                break;
              }
              if (nlen > seg.size - produced) { error = kExtent; break; }
              sh.begin = seg.prefix + produced;
              sh.length = nlen;
              sh.src = r.pos >> 3;
              produced += nlen;
              r.seek(r.pos + u64(nlen) * 8);
              if (r.pos >= seg.end) complete = true;
              action = 2;
              break;
            }
            const u32 terr = type == 1 ? build_fixed_tables(sh.tables) : build_dynamic_tables(sh.tables, r);
            if (terr) { error = kExtent; break; }
            need_header = false;
          }
          u32 lit = 0, length = 0, distance = 0;
          if (decode_token(sh.tables, r, 32768u, lit, length, distance)) { error = kExtent; break; }
          if (!length) {
            need_header = true;
            continue;
          }
          const u64 dst = seg.prefix + produced;
          // Described and emitted parses agree; the guard keeps writes inside
          // the segment even if they did not.
          if (length > seg.size - produced) { error = kExtent; break; }
          if (!distance) {
            out[dst] = u8(lit);
            as += lit;
            aw += (out_end - dst) * lit;
            if (aw >> 62) aw %= kAdlerMod;
            ++produced;
            continue;
          }
          if (distance > window || distance > dst - st->floor) { error = kBadDistance; break; }
          if (length >= kCoopMatch) {
            sh.begin = dst;
            sh.length = length;
            sh.distance = distance;
            produced += length;
            action = 1;
            break;
          }
          for (u32 j = 0; j < length; ++j) {
            const u64 src = dst - distance + (j % distance);
            if (copy_byte(out, roots, unres, seg.prefix, dst + j, src, as, aw, out_end)) {
              atomicAdd(reinterpret_cast<unsigned long long*>(&st->unresolved[0]), 1ull);
              mark_groups(marks, dst + j, 1);
            }
          }
          produced += length;
        }
        sh.action = action;
        sh.error = error;
      }
      __syncthreads();
      const u32 action = sh.action;
      if (!action) break;
      const u64 begin = sh.begin, length = sh.length;
      if (action == 1) {
        const u64 d = sh.distance;
        for (u64 j0 = 0; j0 < length; j0 += kWave) {
          const u64 j = j0 + lane;
          bool queued = false;
          if (j < length)
            queued = copy_byte(out, roots, unres, seg.prefix, begin + j, begin - d + (j % d), as,
                               aw, out_end);
          if (queued) mark_groups(marks, begin + j, 1);
          const u64 bal = __ballot(queued);
          if (!lane && bal)
            atomicAdd(reinterpret_cast<unsigned long long*>(&st->unresolved[0]), u64(__popcll(bal)));
        }
      } else {
        for (u64 j = lane; j < length; j += kWave) {
          const u8 v = body[sh.src + j];
          out[begin + j] = v;
          as += v;
          aw += (out_end - begin - j) * v;
          if (aw >> 62) aw %= kAdlerMod;
        }
      }
      __syncthreads();
    }
    if (!lane && sh.error) atomicMax(&st->emit_status, sh.error);
    __syncthreads();
  }
  // Most workgroups emit nothing here (segments without block records are
  // rare): skip the reduction when no lane wrote a byte.
  if (__ballot((as | aw) != 0) == 0) return;
  adler_block_sum(as, aw, red);
  if (!lane) {
    const u32 slot = blockIdx.x % kAdlerSlots;
    atomicAdd(reinterpret_cast<unsigned long long*>(&parts[2 * slot]), as);
    atomicAdd(reinterpret_cast<unsigned long long*>(&parts[2 * slot + 1]), aw);
  }
}

namespace {
constexpr u32 kEmitThreads = kDescThreads;
// Longest slice emission accepts, in bits (describe's slices are at most
// 512 bits plus a token, a fixed run's windows 512 bits plus a token and an
// end of block with its header): a longer one is an extent error.
constexpr u64 kMaxEmitSlice = 4096;

// Below this many accepted segments every block's rounds are spread over the
// grid as units (a workgroup per round); above it a segment's workgroup emits
// its blocks' rounds itself, loading each block's tables once.
constexpr u64 kSpreadSegments = 512;

// One emission round: slices first .. first + 255 (at most) of record `rec`,
// whose output starts at block_out, in slice groups from `group` on.
// rec = kNone: a slot reserved past the queue's end, skipped.
struct EmitUnit {
  u64 block_out;
  u32 rec;
  u32 first;
  u32 group;
  u32 pad;
};

// Output bytes of one round (256 slices) that g_emit_lanes stages in LDS
// before writing them out in 16-byte stores; rounds with more output write
// the output buffer directly.
constexpr u32 kOutStage = 15104;

struct LaneEmitShared {
  DecodeTables tables;
  Stage stage;
  u16 codes[320];
  BlockRec rec;
  u64 first, chunk_end, round_lo, round_hi;
  u64 carry;  // the state of the byte before the next round (kLastInherit: not known)
  u32 count, next_g, need, unit_end, unit_group, any_lead;
  u64 red[2][kEmitThreads / 64];
  __align__(16) u8 ostage[kOutStage + 16];  // a whole number of 16-byte lines
  // block_header interface
  u64 pos, d0, end, size;
  u32 type, final_block, status, nl, nd, build_status;
};

// Sets bits [start, start + n) of a bitmap: atomic OR on the two end words
// (shared with neighbouring ranges), plain stores on the words between.
__device__ __forceinline__ void bits_set_range(u32* bits, u64 start, u32 n) {
  if (!n) return;
  const u64 end = start + n;
  const u64 w0 = start >> 5, w1 = (end - 1) >> 5;
  const u32 lo = ~0u << (start & 31), hi = ~0u >> (31 - ((end - 1) & 31));
  if (w0 == w1) {
    atomicOr(bits + w0, lo & hi);
    return;
  }
  atomicOr(bits + w0, lo);
  for (u64 w = w0 + 1; w < w1; ++w) bits[w] = ~0u;
  atomicOr(bits + w1, hi);
}

// Where a slice's output bytes go.  GlobalBytes writes the output buffer (and
// with kAdler adds every byte to the thread's Adler-32 sums); StagedBytes
// writes a workgroup's LDS stage that holds output positions [base, ...),
// copied out (and summed) once the round is done.  zero() fills bytes whose
// value a later resolve round provides.
template <bool kAdler>
struct GlobalBytes {
  u8* out;
  AdlerAcc* acc;
  u64 end;
  __device__ __forceinline__ u8 get(u64 p) const { return out[p]; }
  __device__ __forceinline__ void put(u64 p, u8 v) const {
    out[p] = v;
    if (kAdler) acc->add_byte(v, end - p);
  }
  __device__ __forceinline__ void fill(u64 p, u32 n, u8 v) const {
    for (u32 j = 0; j < n; ++j) put(p + j, v);
  }
  __device__ __forceinline__ void zero(u64, u32) const {}
};

struct StagedBytes {
  u8* lds;
  u64 base;
  __device__ __forceinline__ u8 get(u64 p) const { return lds[p - base]; }
  __device__ __forceinline__ void put(u64 p, u8 v) const { lds[p - base] = v; }
  __device__ __forceinline__ void zero(u64 p, u32 n) const {
    for (u32 j = 0; j < n; ++j) lds[p - base + j] = 0;
  }
};

// A round's output: positions [base, base + kOutStage) in the LDS stage
// (copied out and summed when the round is done), later ones straight to
// the output buffer (summed as they are written).  The stage is all zero
// when a round starts (the copy-out clears what it read), so the bytes a
// resolve round provides are zero without a store each.
// Byte pointers into LDS and into global memory, typed with their address
// spaces so that the compiler issues LDS or global instructions: a flat one
// (what a pointer chosen between the two becomes) counts against both wait
// counters, so every LDS wait after it would also wait for pending stores.
typedef __attribute__((address_space(3))) u8 lds_byte;
typedef __attribute__((address_space(1))) u8 global_byte;
typedef __attribute__((address_space(3))) u32 lds_word;
typedef __attribute__((address_space(1))) u32 global_word;

struct RoundBytes {
  lds_byte* lds;
  u64 base, split;  // split = base + stage bytes
  global_byte* out;
  u64 end;
  // Sums of the bytes written straight to the output, held in the sink (not
  // behind a pointer to the caller's sums, which kept those in scratch
  // memory); the caller adds them after the slice.
  mutable AdlerAcc acc;
  __device__ __forceinline__ RoundBytes(u8* stage, u64 base_, u64 split_, u8* out_, u64 end_)
      : lds((lds_byte*)stage), base(base_), split(split_), out((global_byte*)out_), end(end_) {}
  __device__ __forceinline__ u8 get(u64 p) const {
    if (p < split) return lds[u32(p - base)];
    return out[p];
  }
  __device__ __forceinline__ void put(u64 p, u8 v) const {
    if (p < split) {
      lds[u32(p - base)] = v;
    } else {
      out[p] = v;
      acc.add_byte_unfolded(v, end - p);  // folded once per round (at most 2^18 bytes a thread)
    }
  }
  // out[p, p + n) = v (a run of the byte before it), 16 bytes a store.
  __device__ __forceinline__ void fill(u64 p, u32 n, u8 v) const {
    const u32 v4 = 0x01010101u * v;
    const u32 in_stage = p < split ? u32(min<u64>(split - p, n)) : 0u;
    if (in_stage) {  // the stage's byte 0 lies on a 16-byte boundary
      const u32 k0 = u32(p - base);
      u32 i = 0;
      for (; i < in_stage && ((k0 + i) & 15); ++i) lds[k0 + i] = v;
      for (; i + 16 <= in_stage; i += 16) {
        lds_word* w = (lds_word*)(lds + k0 + i);
        w[0] = w[1] = w[2] = w[3] = v4;
      }
      for (; i < in_stage; ++i) lds[k0 + i] = v;
    }
    if (in_stage == n) return;
    const u64 a = p + in_stage;
    const u64 m = n - in_stage;
    // The bytes weigh end - a down to end - a - m + 1.
    acc.s += u64(v) * m;
    acc.w += u64(v) * (m * (end - a) - m * (m - 1) / 2);
    global_byte* d = out + a;
    u32 i = 0;
    for (; i < m && (reinterpret_cast<uintptr_t>((u8*)(d + i)) & 15); ++i) d[i] = v;
    for (; i + 16 <= m; i += 16) {
      global_word* w = (global_word*)(d + i);
      w[0] = w[1] = w[2] = w[3] = v4;
    }
    for (; i < m; ++i) d[i] = v;
  }
  __device__ __forceinline__ void zero(u64, u32) const {}
};

// roots[dst + j] = root + j * step for j < n, four roots a store where the
// positions are 16-byte aligned (a run's positions are its own: no other
// thread writes them).
__device__ __forceinline__ void roots_fill(u32* roots, u64 dst, u32 n, u32 root, u32 step) {
  u32 j = 0;
  for (; j < n && ((dst + j) & 3u); ++j) roots[dst + j] = root + j * step;
  for (; j + 4 <= n; j += 4) {
    const u32 r = root + j * step;
    *reinterpret_cast<uint4*>(roots + dst + j) = make_uint4(r, r + step, r + 2 * step, r + 3 * step);
  }
  for (; j < n; ++j) roots[dst + j] = root + j * step;
}

// out[dst + j] = out[src0 + j] for j < length where src0 + distance = dst:
// an overlapping copy repeats the first `distance` bytes, so every byte is
// read from [src0, dst), never from this copy's own stores.
template <class Sink>
__device__ __forceinline__ void copy_periodic(const Sink& out, u64 dst, u64 src0, u32 distance,
                                              u32 length) {
  if (distance >= 8) {
    u32 k = 0;  // source index of byte j, j mod distance
    for (u32 j = 0; j < length; j += 8) {
      u8 v[8];
#pragma unroll
      for (u32 i = 0; i < 8; ++i) {
        const u32 kk = k + i >= distance ? k + i - distance : k + i;
        v[i] = j + i < length ? out.get(src0 + kk) : u8(0);
      }
#pragma unroll
      for (u32 i = 0; i < 8; ++i)
        if (j + i < length) out.put(dst + j + i, v[i]);
      k = k + 8 >= distance ? k + 8 - distance : k + 8;
    }
  } else {
    u64 pattern = 0;
    for (u32 i = 0; i < distance; ++i) pattern |= u64(out.get(src0 + i)) << (8 * i);
    u32 k = 0;
    for (u32 j = 0; j < length; ++j) {
      out.put(dst + j, u8(pattern >> (8 * k)));
      k = k + 1 == distance ? 0u : k + 1;
    }
  }
}

// One match of a slice whose output starts at dst0: bytes copied from before
// dst0 (and, once the slice has an unresolved byte, every byte it copies from
// its own output) are marked unresolved with their root; the rest are copied.  `nunres` counts the slice's
// unresolved bytes so far.  tail_at / tail_root: the slice offset just past
// the last match handled, and the root of that match's last byte (kNone when
// it is resolved): the byte before a match is that byte or a literal.
// With kDefer, a run of the byte before the slice at the slice's start (its
// leading run, `lead` bytes) is left unwritten and unmarked: once the round
// is decoded, the workgroup learns that byte's value or root from the slice
// before (emit_lead).  A match that reads the leading run marks it first.
template <bool kDefer, class Sink>
__device__ __forceinline__ void emit_match(const Sink& out, u64 dst0, u64 dst, u32 distance,
                                           u32 length, u32* roots, u32* unres, u32& nunres,
                                           u32& tail_at, u32& tail_root, u32& lead) {
  const u64 src0 = dst - distance;
  const u32 at = u32(dst - dst0);
  const bool extend = kDefer && distance == 1 && (at == 0 || (lead && at == lead && tail_at == lead));
  if (kDefer && !extend && lead && src0 < dst0 + lead && src0 + length > dst0) {
    roots_fill(roots, dst0, lead, u32(dst0 - 1), 0);
    bits_set_range(unres, dst0, lead);
    nunres += lead;
    if (tail_at == lead) tail_root = u32(dst0 - 1);
    lead = 0;
  }
  if (extend) {
    lead = at + length;  // the leading run, begun or extended
    tail_root = kNone;   // not read while the tail is the leading run
  } else if (src0 + length <= dst0) {
    // Every source precedes the slice: unresolved, rooted at the source.
    roots_fill(roots, dst, length, u32(src0), 1);
    bits_set_range(unres, dst, length);
    out.zero(dst, length);
    nunres += length;
    tail_root = u32(src0) + length - 1;
  } else if (distance == 1) {
    // A run of the byte before: one root for the whole run when that byte
    // precedes the slice or ends an unresolved match, else resolved.
    const u64 p = dst - 1;
    const bool before = p < dst0;
    if (before || (at == tail_at && tail_root != kNone)) {
      const u32 root = before ? u32(p) : tail_root;
      roots_fill(roots, dst, length, root, 0);
      bits_set_range(unres, dst, length);
      out.zero(dst, length);
      nunres += length;
      tail_root = root;
    } else {
      out.fill(dst, length, out.get(p));
      tail_root = kNone;
    }
  } else if (!nunres && src0 >= dst0) {
    // Every source is this slice's own resolved output.
    copy_periodic(out, dst, src0, distance, length);
    tail_root = kNone;
  } else {
    u32 last = kNone;
    for (u32 j = 0; j < length; ++j) {
      const u64 d = dst + j, src = d - distance;
      // Once the slice has an unresolved byte, a byte copied from its own
      // output is rooted at its source without checking whether that is
      // resolved: a load of the bitmap (or of the source's root) here would
      // wait for every store the wave has pending.  A resolved source only
      // costs the resolve rounds one link.
      if (src < dst0 || nunres) {
        roots[d] = last = u32(src);
        bit_set(unres, d);
        out.zero(d, 1);
        ++nunres;
      } else {
        out.put(d, out.get(src));
        last = kNone;
      }
    }
    tail_root = last;
  }
  tail_at = at + length;
}

// The state of a slice's last byte as the slice after it sees it: the slice
// ended in its leading run (the state of the byte before the slice), or in a
// resolved byte, or in an unresolved byte with a root.
constexpr u64 kLastInherit = 0;
constexpr u64 kLastValue = 1ull << 32;
constexpr u64 kLastRoot = 2ull << 32;

// Matches a slice decode holds back: literals are written as they are
// decoded, matches queue here (in order) and are copied when a lane of the
// wave has kMatchQueue of them and when the slice ends, so that the lanes of
// a wave copy together rather than each literal step waiting for the copies
// of the few lanes that met a match.  A match only reads bytes before its own
// position, which are literals (already written) or earlier matches (copied
// first), so the output is the same as copying each match at once.
constexpr u32 kMatchQueue = 4;
struct MatchQueue {
  u32 at[kMatchQueue] = {};    // output offset from the slice start
  u32 code[kMatchQueue] = {};  // length | distance << 9
  u32 n = 0;
  __device__ __forceinline__ void push(u32 offset, u32 length, u32 distance) {
#pragma unroll
    for (u32 k = 0; k < kMatchQueue; ++k) {
      at[k] = n == k ? offset : at[k];
      code[k] = n == k ? (length | (distance << 9)) : code[k];
    }
    ++n;
  }
  // Copies the queued matches in order (the head, then the rest moves up).
  template <bool kDefer, class Sink>
  __device__ __forceinline__ void flush(const Sink& out, u64 dst0, u32* roots, u32* unres,
                                        u32& nunres, u32& tail_at, u32& tail_root, u32& lead) {
    for (; n; --n) {
      emit_match<kDefer>(out, dst0, dst0 + at[0], code[0] >> 9, code[0] & 511u, roots, unres,
                         nunres, tail_at, tail_root, lead);
#pragma unroll
      for (u32 k = 0; k + 1 < kMatchQueue; ++k) {
        at[k] = at[k + 1];
        code[k] = code[k + 1];
      }
    }
  }
};

// Decode one slice [entry, stop) into out[dst0 ..], within the block's output
// [.., block_end) of a stream whose output starts at out[floor]; adds the
// slice's unresolved bytes to `unres_total`.  Returns 0 or an error.  `sh`
// holds the block's tables and the staged bits.  With `cross` (a run of
// fixed blocks), an EOB before `stop` is followed by the next block's fixed
// header, and decoding goes on after it.
// With kDefer, `lead` returns the slice's deferred leading run and `last` the
// state of its last byte for the slices after it (emit_lead).
template <bool kChecked, bool kDefer, class Shared, class Sink>
__device__ u32 emit_slice(Shared& sh, u32 blim, u32 entry, u32 stop, u64 dst0, u64 block_end,
                          u32 window, const Sink& out, u32* roots, u32* unres, u64& unres_total,
                          u64 floor, bool cross, u32& lead, u64& last, u8* marks) {
  Win4<kChecked> r;
  r.words = sh.stage.words;
  r.limit = blim;
  r.seek(entry);
  u64 dst = dst0;
  u32 nunres = 0, err = 0;  // unresolved bytes of this slice
  MatchQueue q;
  u32 tail_at = 0, tail_root = kNone;  // see emit_match
  lead = 0;
  bool live = true;
  for (;;) {
    // One copy site for queued matches: when a lane's queue is full, and
    // once every lane of the wave has finished decoding.
    const bool any_live = __ballot(live) != 0;
    if (live) {
      u32 length = 0, x = 0, x2 = 0, x3 = 0;  // x: the literal (length 1) or the distance
      u32 got = 1;                            // tokens taken (2, 3: literals x, x2, x3)
      u32 l1, l12;
      if (r.pos() >= stop) {
        live = false;
      } else if (!(got = quick_triple<kChecked>(sh.tables.ll, sh.tables.dd, r, stop, length, x, x2,
                                                x3, l1, l12))) {
        u32 lit, distance;
        if (window_token<kChecked>(sh.tables.ll, sh.tables.dd, r, lit, length, distance)) {
          err = kExtent;
          live = false;
        } else if (!length) {
          live = false;
          if (cross && r.pos() < stop) {
            // The run's next block: a non-final or final fixed header.
            if (r.avail() < 3 || ((r.bits32() >> 1) & 3u) != 1u) {
              err = kExtent;
            } else {
              r.advance(3);
              live = true;
              got = 0;  // no token to emit this step
            }
          }
        } else {
          x = length == 1 ? lit : distance;
          got = 1;
        }
      }
      if (live && got && length + got - 1 > block_end - dst) {
        err = kExtent;
        live = false;
      }
      if (live && got) {
        if (length == 1) {
          out.put(dst++, u8(x));
          if (got >= 2) out.put(dst++, u8(x2));
          if (got == 3) out.put(dst++, u8(x3));
        } else if (x > window || x > dst - floor) {
          err = kBadDistance;
          live = false;
        } else {
          q.push(u32(dst - dst0), length, x);
          dst += length;
        }
      }
    }
    if (!any_live || __ballot(q.n == kMatchQueue))
      q.template flush<kDefer>(out, dst0, roots, unres, nunres, tail_at, tail_root, lead);
    if (!any_live) break;
  }
  unres_total += nunres;
  if (nunres) mark_groups(marks, dst0, dst - dst0);
  if (kDefer) {
    const u32 n = u32(dst - dst0);
    if (!n || lead == n) last = kLastInherit;
    else if (tail_at == n && tail_root != kNone) last = kLastRoot | tail_root;
    else last = kLastValue | out.get(dst - 1);
  }
  return err;
}
}  // namespace

// One 256-thread workgroup per accepted segment with block records: stored
// blocks are copied by the workgroup; fixed/dynamic blocks decode their
// described slices in parallel, one slice per thread, with the tables that
// describe stored (or rebuilt from the header), writing output in place.  A
// byte copied from before its slice's output start is queued as unresolved
// (root = source position).  A run of fixed blocks (kRecFixedRun) decodes its
// slices across the run's block headers.
__global__ __launch_bounds__(kEmitThreads) __attribute__((amdgpu_waves_per_eu(4))) void g_emit_lanes(
    const u8* body, u64 len, State* st, const Segment* acc, const BlockRec* recs,
    const u64* slice_entry, const u32* slice_off, const u32* group_link,
    const BlockTables* tables, u8* out, u32* roots, u32* unres, u64 out_end, u64* parts,
    EmitUnit* units, u64 unit_capacity, u32 unit_pass, u8* marks) {
  __shared__ LaneEmitShared sh;
  if (st->status) return;
  const u32 t = threadIdx.x;
  const u64 items = unit_pass ? min<u64>(st->emit_units, unit_capacity) : st->accepted;
  const bool segments_few = st->accepted < kSpreadSegments;
  const u32 window = st->window;
  const u64 floor = st->floor;
  u64 unres_total = 0;  // this thread's unresolved bytes, counted once per wave at the end
  AdlerAcc sums;        // Adler-32 sums of the bytes this thread writes
  // The output stage starts all zero (ordered before the first round by the
  // barrier of its segment's set-up).
  for (u32 k = t; 16 * k < sizeof(sh.ostage); k += kEmitThreads)
    *reinterpret_cast<uint4*>(sh.ostage + 16 * k) = make_uint4(0, 0, 0, 0);
  for (u64 si = blockIdx.x; si < items; si += gridDim.x) {
    u32 ri, first = 0, unit_group = kNone;
    u64 block_out;
    if (unit_pass) {
      const EmitUnit u = units[si];
      ri = u.rec;
      block_out = u.block_out;
      first = u.first;
      unit_group = u.group;
    } else {
      const Segment seg = acc[si];
      ri = seg.rec_first;
      block_out = seg.prefix;
    }
    if (ri == kNone) continue;
    u32 error = 0;
    if (!t) {
      sh.stage.count = 0;
      sh.stage.bit0 = 0;
      sh.carry = kLastInherit;
    }
    __syncthreads();
    while (ri != kNone) {
      if (!t) {
        sh.rec = recs[ri];
        sh.pos = sh.rec.start;
      }
      __syncthreads();
      const BlockRec rec = sh.rec;
      if (unit_pass && (rec.type == 0 || first >= rec.lanes)) {
        error = kExtent;  // never queued: units are rounds of coded blocks
        break;
      }
      if (rec.type == 0) {
        copy_bytes(out + block_out, body + (rec.data >> 3), rec.size, body + len, t, kEmitThreads,
                   &sums, out_end - block_out);
        if (!t && rec.size) sh.carry = kLastValue | body[(rec.data >> 3) + rec.size - 1];
      } else {
        const bool cross = (rec.pad & kRecFixedRun) != 0;
        if (!t) {
          // The slices this workgroup emits: in the unit pass, its unit's
          // round.  In the segment pass, a fixed run's rounds, and when the
          // segments are too few to fill the grid every block's rounds, are
          // queued as units so that they spread over the grid (with the
          // queue full, emitted here); other blocks are emitted here, round
          // after round with the tables loaded once.  A round's four slice
          // groups are consecutive and its last links to the next round's
          // first (a fixed run's groups are all consecutive).
          u32 end = rec.lanes, g0 = rec.group;
          if (unit_pass) {
            end = min(first + kEmitThreads, rec.lanes);
            g0 = unit_group;
          } else if (rec.lanes && (cross || segments_few)) {
            end = 0;
            const u32 rounds = (rec.lanes + kEmitThreads - 1) / kEmitThreads;
            const u64 q =
                atomicAdd(reinterpret_cast<unsigned long long*>(&st->emit_units), u64(rounds));
            if (q + rounds <= unit_capacity) {
              u32 g = rec.group;
              for (u32 r = 0; r < rounds; ++r) {
                EmitUnit u;
                u.block_out = block_out;
                u.rec = ri;
                u.first = r * kEmitThreads;
                u.group = g;
                u.pad = 0;
                units[q + r] = u;
                if (r + 1 < rounds) g = cross ? g + kEmitThreads / 64 : group_link[g + 3];
              }
            } else {
              for (u64 r = q; r < unit_capacity && r < q + rounds; ++r) units[r].rec = kNone;
              end = rec.lanes;
            }
          }
          sh.unit_end = end;
          sh.unit_group = g0;
        }
        __syncthreads();
        const u32 unit_end = sh.unit_end;
        u32 g = sh.unit_group;
        u32 done = first;
        bool tables_pending = false;
        if (done < unit_end) {  // uniform
          if (rec.table == kNone) {
            block_header<true, true, false>(body, len, ~0ull, sh);
            if (sh.status || sh.type != rec.type || sh.d0 != rec.data) { error = kExtent; break; }
          }
          tables_pending = rec.table != kNone;
        }
        while (g != kNone && done < unit_end) {
          // One describe round: up to 256 slices in consecutive groups.  The
          // round's slice entries and offsets, and in the first round the
          // block's tables, load together (one memory latency).
          const u32 count = rec.lanes - done < kEmitThreads ? rec.lanes - done : kEmitThreads;
          u64 entry = 0, stop = 0;
          u32 off = 0;
          if (t < count) {
            entry = slice_entry[u64(g) * 64 + t];
            off = slice_off[u64(g) * 64 + t];
            if (t + 1 < count) stop = slice_entry[u64(g) * 64 + t + 1];
          }
          if (tables_pending) {
            const u32* src_ll = reinterpret_cast<const u32*>(&tables[rec.table].ll);
            const u32* src_dd = reinterpret_cast<const u32*>(&tables[rec.table].dd);
            u32* dst_ll = reinterpret_cast<u32*>(&sh.tables.ll);
            u32* dst_dd = reinterpret_cast<u32*>(&sh.tables.dd);
            copy_tables<kEmitThreads>(dst_ll, dst_dd, src_ll, src_dd, t);
            tables_pending = false;
          }
          if (!t) {
            // The next round's first group and first entry only when one
            // follows (a block of at most 256 slices has a single round).
            const bool more = done + count < rec.lanes;
            const u32 next_g = more ? group_link[g + (count + 63) / 64 - 1] : kNone;
            sh.next_g = next_g;
            sh.first = entry;
            sh.chunk_end = next_g != kNone ? slice_entry[u64(next_g) * 64] : rec.end;
            sh.need = !staged_covers(sh.stage, body, len, entry, sh.chunk_end);
            sh.any_lead = 0;
            // The round's output: from its first slice to the next round's.
            sh.round_lo = block_out + off;
            sh.round_hi = block_out + (next_g != kNone ? slice_off[u64(next_g) * 64] : rec.size);
          }
          __syncthreads();
          if (sh.need) {
            stage_range(body, len, sh.first, sh.chunk_end, sh.stage);
            __syncthreads();
          }
          // The round's output goes through the LDS stage, whose byte 0 is
          // the output position `lo16` (16-byte aligned in memory), as far
          // as the stage reaches; any rest goes straight to the output.
          const u64 lo = sh.round_lo, hi = sh.round_hi;
          const u64 skew = (reinterpret_cast<uintptr_t>(out) + lo) & 15u;
          const u64 lo16 = lo - skew;
          const u64 split = min<u64>(hi, lo16 + kOutStage);
          u32 lerr = 0, lead = 0;
          u64 last = kLastInherit;
          if (t < count) {
            if (t + 1 >= count) stop = sh.chunk_end;
            const u64 dst0 = block_out + off;
            const u32 blim = stage_limit(sh.stage, len);
            const u32 e_rel = u32(entry - sh.stage.bit0), s_rel = u32(stop - sh.stage.bit0);
            // Writes stay inside the round: a slice that would pass its end
            // is an extent error.
            const u64 rend = min(block_out + rec.size, hi);
            const RoundBytes sink(sh.ostage, lo16, split, out, out_end);
            // Unchecked decoding when the slice and a token of overshoot lie
            // before the body end.
            if (dst0 < lo || dst0 > rend || stop < entry || stop - entry > kMaxEmitSlice)
              lerr = kExtent;  // never from a consistent describe or walk
            else if (stop + 64 <= len * 8)
              lerr = emit_slice<false, true>(sh, blim, e_rel, s_rel, dst0, rend, window, sink,
                                             roots, unres, unres_total, floor, cross, lead, last,
                                             marks);
            else
              lerr = emit_slice<true, true>(sh, blim, e_rel, s_rel, dst0, rend, window, sink,
                                            roots, unres, unres_total, floor, cross, lead, last,
                                            marks);
            sums.s += sink.acc.s;
            sums.w += sink.acc.w;
            if (lead) sh.any_lead = 1;
          }
          if (lerr) atomicMax(&st->emit_status, lerr);
          __syncthreads();
          if (sh.any_lead) {  // uniform
            // Leading runs: each slice learns the state of the byte before it
            // by a scan over the round's slices (the last state that is not
            // "inherit" before it; before slice 0, the carry of the round
            // before), then writes its run or marks it unresolved.  The stage
            // words hold the scan: this round's bits are decoded.
            u64* scan = reinterpret_cast<u64*>(sh.stage.words);
            scan[t] = last;
            __syncthreads();
            for (u32 d = 1; d < kEmitThreads; d <<= 1) {
              const u64 own = scan[t], left = t >= d ? scan[t - d] : kLastInherit;
              __syncthreads();
              if (own == kLastInherit) scan[t] = left;
              __syncthreads();
            }
            if (lead && !lerr) {
              const u64 dst0 = block_out + off;
              const u64 before = t ? scan[t - 1] : sh.carry;
              if (before >> 32 == kLastValue >> 32) {
                const RoundBytes sink(sh.ostage, lo16, split, out, out_end);
                sink.fill(dst0, lead, u8(before));
                sums.s += sink.acc.s;
                sums.w += sink.acc.w;
              } else {
                const u32 root = before >> 32 == kLastRoot >> 32 ? u32(before) : u32(dst0 - 1);
                roots_fill(roots, dst0, lead, root, 0);
                bits_set_range(unres, dst0, lead);
                mark_groups(marks, dst0, lead);
                unres_total += lead;
              }
            }
            __syncthreads();
            if (!t) {
              if (scan[count - 1] != kLastInherit) sh.carry = scan[count - 1];
              sh.stage.count = 0;
            }
          } else if (t + 1 == count) {
            sh.carry = last;
          }
          // The staged part in whole 16-byte lines (bytes of the neighbouring
          // round in its first line one by one), summed on the way.
          const u64 span = split - lo16;
          for (u64 k = t; 16 * k < span; k += kEmitThreads) {
            const u64 r0 = 16 * k, a = lo16 + r0;
            if (r0 >= skew && r0 + 16 <= span) {
              const uint4 q = *reinterpret_cast<const uint4*>(sh.ostage + r0);
              *reinterpret_cast<uint4*>(out + a) = q;
              sums.add16(q, out_end - a);
            } else {
              for (u32 j = 0; j < 16; ++j) {
                if (r0 + j < skew || r0 + j >= span) continue;
                const u8 v = sh.ostage[r0 + j];
                out[a + j] = v;
                sums.add_byte(v, out_end - (a + j));
              }
            }
            *reinterpret_cast<uint4*>(sh.ostage + r0) = make_uint4(0, 0, 0, 0);  // for the next round
          }
          done += count;
          g = sh.next_g;
          sums.fold();
          __syncthreads();
        }
      }
      block_out += rec.size;
      ri = unit_pass ? kNone : rec.next;
      __syncthreads();
    }
    if (!t && error) atomicMax(&st->emit_status, error);
    __syncthreads();
  }
  for (u32 off = 32; off; off >>= 1) unres_total += __shfl_down(unres_total, off, 64);
  if (lane_id() == 0 && unres_total)
    atomicAdd(reinterpret_cast<unsigned long long*>(&st->unresolved[0]), unres_total);
  // The workgroup's Adler-32 partial pair.
  u64 ps = sums.s % kAdlerMod, pw = sums.w % kAdlerMod;
  for (u32 off = 32; off; off >>= 1) {
    ps += __shfl_down(ps, off, 64);
    pw += __shfl_down(pw, off, 64);
  }
  if (lane_id() == 0) {
    sh.red[0][t >> 6] = ps;
    sh.red[1][t >> 6] = pw;
  }
  __syncthreads();
  if (!t) {
    u64 a = 0, b = 0;
    for (u32 w = 0; w < kEmitThreads / 64; ++w) {
      a += sh.red[0][w];
      b += sh.red[1][w];
    }
    const u32 slot = blockIdx.x % kAdlerSlots;
    if (a | b) {  // workgroups that wrote nothing add nothing
      atomicAdd(reinterpret_cast<unsigned long long*>(&parts[2 * slot]), a % kAdlerMod);
      atomicAdd(reinterpret_cast<unsigned long long*>(&parts[2 * slot + 1]), b % kAdlerMod);
    }
  }
}

// Large files of a batch: one 256-thread workgroup per file decodes its
// blocks in turn: a stored block by a copy, a fixed or dynamic block by
// describe's parallel slices and then one slice per thread, as g_emit_lanes
// does.  Copies that reach before their slice are left to g_resolve over the
// batch output.  A file whose decode meets anything unusual (any status, an
// exhausted slice-group pool, a bad encoded row) is flagged in `redo` for
// the serial per-file decoder, which restates the reference's statuses.
__global__ __launch_bounds__(kDescThreads) void g_batch_wide(
    const u8* in, u8* out, const BatchFile* files, const u32* list, u32 n, const u32* encoded,
    u32 max_blocks, State* st, u64* slice_entry, u32* slice_off, u32* group_link,
    u64 group_capacity, u32* roots, u32* unres, u32* redo, u32* wanted) {
  __shared__ DescShared sh;
  __shared__ u64 e_first, e_chunk_end;
  __shared__ u32 e_count, e_next, e_need, bad, window;
  const u32 t = threadIdx.x;
  u64 unres_total = 0;
  for (u32 i = blockIdx.x; i < n; i += gridDim.x) {
    const u32 f = list[i];
    const BatchFile file = files[f];
    if (!t) {
      u64 in_size = file.in_size;
      u32 b = 0;
      if (encoded) {
        b = encoded[2 * u64(f) + 1] != 0 || encoded[2 * u64(f)] > file.in_size;
        in_size = encoded[2 * u64(f)];
      }
      u32 w = 0, want = 0;
      if (!b) b = check_framing(in + file.in_offset, in_size, w, want) != kOk;
      bad = b;
      window = w;
      wanted[i] = want;
      e_first = in_size;  // the stream length, until the block loop starts
      sh.pos = 0;
      sh.stage.count = 0;
      sh.stage.bit0 = 0;
    }
    __syncthreads();
    const u64 in_size = e_first;
    const u8* body = in + file.in_offset + 2;
    const u64 len = bad ? 0 : in_size - 6;
    const u64 base = file.out_offset, out_size = file.out_size;
    u64 produced = 0;
    u32 blocks = 0;
    __syncthreads();
    while (!bad) {
      block_header<true, true>(body, len, out_size - produced, sh);
      if (sh.status || ++blocks > max_blocks) {  // uniform
        if (!t) bad = 1;
        break;
      }
      if (sh.type == 0) {
        copy_bytes(out + base + produced, body + (sh.d0 >> 3), sh.size, body + len, t,
                   kDescThreads);
      } else {
        if (!t) {
          sh.hint = len * 8;
          sh.group = kNone;
          sh.lanes = 0;
          sh.table = kNone;
        }
        __syncthreads();
        describe_tokens(body, len, out_size - produced, sh, st, slice_entry, slice_off, group_link,
                        group_capacity);
        // A block that ends past the file's output (describe checks the
        // limit only between rounds) is never emitted.
        if (sh.status || sh.group == kNone || sh.size > out_size - produced) {  // uniform
          if (!t) bad = 1;
          break;
        }
        // The block's slices, one per thread, a describe round at a time.
        const u64 block_out = base + produced, block_end = block_out + sh.size;
        u32 g = sh.group, done = 0;
        const u32 lanes = sh.lanes;
        while (g != kNone && done < lanes) {
          if (!t) {
            const u32 count = lanes - done < kDescThreads ? lanes - done : kDescThreads;
            const u32 ng = (count + 63) / 64;
            const u32 next_g = group_link[g + ng - 1];
            e_count = count;
            e_next = next_g;
            e_first = slice_entry[u64(g) * 64];
            e_chunk_end = next_g != kNone && done + count < lanes ? slice_entry[u64(next_g) * 64]
                                                                   : sh.end;
            e_need = !staged_covers(sh.stage, body, len, e_first, e_chunk_end);
          }
          __syncthreads();
          const u32 count = e_count;
          if (e_need) {
            stage_range(body, len, e_first, e_chunk_end, sh.stage);
            __syncthreads();
          }
          if (t < count) {
            const u64 entry = slice_entry[u64(g) * 64 + t];
            const u64 stop = t + 1 < count ? slice_entry[u64(g) * 64 + t + 1] : e_chunk_end;
            const u64 dst0 = block_out + slice_off[u64(g) * 64 + t];
            const u32 blim = stage_limit(sh.stage, len);
            const u32 e_rel = u32(entry - sh.stage.bit0), s_rel = u32(stop - sh.stage.bit0);
            u32 lerr;
            u32 no_lead;  // a batch file decodes without deferred leading runs
            u64 no_last;
            if (stop + 64 <= len * 8)
              lerr = emit_slice<false, false>(sh, blim, e_rel, s_rel, dst0, block_end, window,
                                       GlobalBytes<false>{out, nullptr, 0}, roots,
                                       unres, unres_total, base, false, no_lead, no_last,
                                       nullptr);
            else
              lerr = emit_slice<true, false>(sh, blim, e_rel, s_rel, dst0, block_end, window,
                                      GlobalBytes<false>{out, nullptr, 0}, roots,
                                      unres, unres_total, base, false, no_lead, no_last,
                                      nullptr);
            if (lerr) bad = 1;
          }
          done += count;
          g = e_next;
          __syncthreads();
        }
        if (done < lanes) bad = 1;
      }
      produced += sh.size;
      if (!t) sh.pos = sh.end;
      __syncthreads();
      if (bad || sh.final_block) break;
    }
    __syncthreads();
    if (!t) {
      const bool ok = !bad && !sh.status && sh.final_block && produced == out_size &&
                      (sh.end + 7) / 8 == len;
      redo[f] = ok ? 0u : 1u;
    }
    __syncthreads();
  }
  for (u32 off = 32; off; off >>= 1) unres_total += __shfl_down(unres_total, off, 64);
  if (lane_id() == 0 && unres_total)
    atomicAdd(reinterpret_cast<unsigned long long*>(&st->unresolved[0]), unres_total);
}

// Large batch files after resolution: Adler-32 of each decoded file against
// its trailer; [0, 0] when it matches, else the file is flagged for the
// serial decoder (so are all of them if a chain stayed unresolved).
__global__ __launch_bounds__(256) void g_batch_wide_finish(const BatchFile* files, const u32* list,
                                                           u32 n, const u8* out, const State* st,
                                                           const u32* wanted, u32* redo,
                                                           u32* meta) {
  __shared__ u64 red[2][4];
  const u32 t = threadIdx.x, lane = lane_id(), wave = t >> 6;
  for (u32 i = blockIdx.x; i < n; i += gridDim.x) {
    const u32 f = list[i];
    if (redo[f]) continue;  // uniform
    const BatchFile file = files[f];
    const u8* o = out + file.out_offset;
    const u64 len = file.out_size;
    // Bytes before the first 16-byte boundary and after the last one singly,
    // the rest as 16-byte loads (byte k weighs len - k).
    const u64 lead = (16 - (reinterpret_cast<uintptr_t>(o) & 15)) & 15;
    const u64 head = lead < len ? lead : len;
    const u64 mid = (len - head) & ~u64(15);
    u64 s = 0, w = 0;
    if (t < head + (len - head - mid)) {  // at most 15 + 15 single bytes
      const u64 k = t < head ? t : head + mid + (t - head);
      const u64 v = o[k];
      s = v;
      w = (len - k) * v;
    }
    const uint4* q = reinterpret_cast<const uint4*>(o + head);
    for (u64 g = t; g < mid / 16; g += 256) {
      const uint4 x = q[g];
      u32 bs = 0, bw = 0;  // sum of the 16 bytes, and of each times its index
      auto take = [&](u32 word, u32 j0) {
#pragma unroll
        for (u32 j = 0; j < 4; ++j) {
          const u32 b = (word >> (8 * j)) & 255u;
          bs += b;
          bw += (j0 + j) * b;
        }
      };
      take(x.x, 0);
      take(x.y, 4);
      take(x.z, 8);
      take(x.w, 12);
      s += bs;
      w += (len - head - 16 * g) * bs - bw;
      if (w >> 62) w %= kAdlerMod;
    }
    s %= kAdlerMod;
    w %= kAdlerMod;
    for (u32 off = 32; off; off >>= 1) {
      s += __shfl_down(s, off, 64);
      w += __shfl_down(w, off, 64);
    }
    if (!lane) {
      red[0][wave] = s;
      red[1][wave] = w;
    }
    __syncthreads();
    if (!t) {
      const u32 a = u32((red[0][0] + red[0][1] + red[0][2] + red[0][3] + 1) % kAdlerMod);
      const u64 w_all = red[1][0] + red[1][1] + red[1][2] + red[1][3] + len % kAdlerMod;
      const u32 b = u32(w_all % kAdlerMod);
      if (((b << 16) | a) == wanted[i] && !st->unresolved[1]) {
        meta[2 * u64(f)] = 0;
        meta[2 * u64(f) + 1] = 0;
      } else {
        redo[f] = 1;
      }
    }
    __syncthreads();
  }
}

// Chain links a position follows in resolve round r: 2, 4, and in the last
// round as many as its chain has (a root always precedes its position, so
// every chain ends).  Early rounds see nearly every unresolved byte, and a
// wave waits for its longest chain, so they take few links (measured on 64 MiB
// of text: 2, 8, 32 took the rounds 6 % longer); each round leaves every
// position's root as far along its chain as it got, so after two rounds a
// chain of n links is n / 8 roots long.  Schedules of 2, 8 / 4, 16 / 4, 8, 16
// links before the last round took as long within 3 %.
constexpr u32 kResolveRounds = 3;
constexpr u32 kXcds = 8;  // MI355X: 8 accelerator complex dies of 32 CUs
__host__ __device__ constexpr u32 resolve_links(u32 round) {
  return round == 0 ? 2u : round == 1 ? 4u : 0xffffffffu;
}
inline u32 resolve_rounds(u64) { return kResolveRounds; }

// One resolution round: round r scans the unresolved bits of buffer (r & 1)
// (round 0: the bits set by emission; counts[r] unresolved positions,
// zero-filled before the first round) and writes every word of the other
// buffer with the positions still unresolved, counted in counts[r + 1].  A
// position follows up to resolve_links(round) links of its root chain through this
// round's snapshot (roots: any root read is an earlier byte of the same
// chain, so concurrent updates are harmless); at a resolved byte it takes
// that byte, else it keeps the root reached.  Round r thus covers
// the product of resolve_links over rounds 0..r.  Only bytes written by earlier launches are
// read.  The last round leaves its count in st->unresolved[1] (status 20 in
// g_finish).
// With `parts`, every resolved byte is added to this workgroup's Adler-32
// pair parts[2b], parts[2b + 1] (a byte at position p weighs out_end - p).
__global__ __launch_bounds__(256) void g_resolve(State* st, u8* out, u32* roots, u32* bits0,
                                                 u32* bits1, u64* counts, u32 round,
                                                 u32 max_rounds, u64 words, u64 out_end,
                                                 u64* parts, u8* marks0, u8* marks1) {
  __shared__ u64 red[2][16];
  if (st->status || st->emit_status) return;
  const u64 n_in = round ? counts[round] : st->unresolved[0];
  if (!n_in) return;
  u64 as = 0, aw = 0;
  const u32* bits = round & 1 ? bits1 : bits0;
  u32* next_bits = round & 1 ? bits0 : bits1;
  u64* next_count = round + 1 == max_rounds ? &st->unresolved[1] : &counts[round + 1];
  const u32 lane = lane_id();
  u32 kept = 0;
  // A wave takes a group of 64 bitmap words at a time and lists the group's
  // unresolved positions in LDS (a prefix sum over the words' bit counts);
  // its lanes then follow the root chains of the list's entries, 64 at a
  // time, so that sparse and dense groups alike keep every lane busy.  The
  // entries still unresolved are gathered into the group's next words in LDS.
  // With group marks (marks0 for rounds 0, 2, ..., marks1 for the others), a
  // round reads only the marked groups of its bitmap and marks those it
  // leaves unresolved bytes in for the next round; the other groups' words
  // of the next bitmap are never read.
  __shared__ u16 list[256 / 64][64 * 32];
  __shared__ u32 left_words[256 / 64][64];
  const u32 wave = threadIdx.x >> 6;
  const u8* marks = round & 1 ? marks1 : marks0;
  u8* next_marks = round & 1 ? marks0 : marks1;
  const u32 links = resolve_links(round);
  // Workgroups are dealt to the 8 XCDs in turn (workgroup b to XCD b mod 8),
  // each with its own L2.  XCD x takes the x-th eighth of the groups, its
  // waves consecutive groups, so that the chains a wave follows back into
  // the previous 32 KiB mostly read lines its own XCD's waves loaded.
  const u64 ngroups = (words + 63) / 64;
  // Follows the chain of entry e of group g; a byte left unresolved sets its
  // bit in `left` (the group's next words).  The lane's stores (the byte, or
  // the root reached) wait in `pend` until its next entry's loads have
  // returned: a load waits for every store issued before it, so each entry's
  // chain would otherwise wait for the previous entry's stores.
  u32 pend_u = 0, pend_v = 0, pend_kind = 0;  // kind 1: out[u] = v; 2: roots[u] = v
  const auto commit = [&]() {
    if (pend_kind == 1) out[pend_u] = u8(pend_v);
    else if (pend_kind == 2)
      __hip_atomic_store(roots + pend_u, pend_v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    pend_kind = 0;
  };
  const auto chase = [&](u64 g, u32 e, u32* left) {
    const u32 u = u32(g * 2048 + e);
    u32 r = roots[u];
    bool unres = (bits[r >> 5] >> (r & 31)) & 1u;
    for (u32 k = 0; unres && k < links; ++k) {
      r = __hip_atomic_load(roots + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      unres = (bits[r >> 5] >> (r & 31)) & 1u;
    }
    const u32 v = unres ? r : u32(out[r]);
    commit();
    pend_u = u;
    pend_v = v;
    pend_kind = unres ? 2u : 1u;
    if (!unres) {
      as += v;
      aw += (out_end - u) * v;
      if (aw >> 62) aw %= kAdlerMod;
    } else {
      atomicOr(&left[e >> 5], 1u << (e & 31));
    }
  };
  // The group's unresolved positions into the wave's list (a prefix sum over
  // the words' bit counts); returns their number.
  const auto list_group = [&](u64 g, u32 m) {
    const u32 cnt = __popc(m);
    u32 incl = cnt;
#pragma unroll
    for (u32 off = 1; off < 64; off <<= 1) {
      const u32 y = __shfl_up(incl, off, 64);
      if (lane >= off) incl += y;
    }
    for (u32 k = incl - cnt; m; m &= m - 1, ++k) list[wave][k] = u16(lane * 32 + __builtin_ctz(m));
    return __shfl(incl, 63, 64);
  };
  if (ngroups <= gridDim.x) {  // uniform
    // Few groups (a small output): a workgroup per group, its four waves
    // chasing every fourth batch of 64 entries, so that a group's chains are
    // followed four times as fast.  Each wave lists the group itself.
    for (u64 g = blockIdx.x; g < ngroups; g += gridDim.x) {
      if (marks && !marks[g]) {  // uniform
        if (!threadIdx.x) next_marks[g] = 0;
        continue;
      }
      const u64 w = g * 64 + lane;
      const u32 total = list_group(g, w < words ? bits[w] : 0u);
      if (!total) {  // uniform
        if (!wave && w < words) next_bits[w] = 0;
        if (marks && !threadIdx.x) next_marks[g] = 0;
        continue;
      }
      if (!wave) left_words[0][lane] = 0;
      __syncthreads();
      for (u32 i = wave * 64 + lane; i < total; i += 256) chase(g, list[wave][i], left_words[0]);
      commit();
      __syncthreads();
      if (!wave) {
        const u32 nb = left_words[0][lane];
        if (w < words) next_bits[w] = nb;
        kept += __popc(nb);
        const bool left = __ballot(nb != 0) != 0;
        if (marks && !lane) next_marks[g] = left ? 1 : 0;
      }
      __syncthreads();  // the list and words are rewritten for the next group
    }
  } else {
    // Workgroups are dealt to the 8 XCDs in turn (workgroup b to XCD b mod
    // 8), each with its own L2.  XCD x takes the x-th eighth of the groups,
    // its waves consecutive groups, so that the chains a wave follows back
    // into the previous 32 KiB mostly read lines its own XCD's waves loaded.
    const u32 xcds = gridDim.x < kXcds ? gridDim.x : kXcds;
    const u32 xcd = blockIdx.x % xcds, xcd_block = blockIdx.x / xcds;
    const u64 xcd_waves =
        u64(gridDim.x / xcds + (xcd < gridDim.x % xcds ? 1u : 0u)) * (blockDim.x / 64);
    const u64 g_end = ngroups * (xcd + 1) / xcds;
    for (u64 g = ngroups * xcd / xcds + u64(xcd_block) * (blockDim.x / 64) + wave; g < g_end;
         g += xcd_waves) {
      if (marks && !marks[g]) {  // uniform
        if (!lane) next_marks[g] = 0;
        continue;
      }
      const u64 w = g * 64 + lane;
      const u32 total = list_group(g, w < words ? bits[w] : 0u);
      if (!total) {  // uniform
        if (w < words) next_bits[w] = 0;
        if (marks && !lane) next_marks[g] = 0;
        continue;
      }
      left_words[wave][lane] = 0;
      wave_sync();
      for (u32 i = lane; i < total; i += 64) chase(g, list[wave][i], left_words[wave]);
      commit();
      wave_sync();
      const u32 nb = left_words[wave][lane];
      if (w < words) next_bits[w] = nb;
      kept += __popc(nb);
      const bool left = __ballot(nb != 0) != 0;
      if (marks && !lane) next_marks[g] = left ? 1 : 0;
      wave_sync();  // the list and words are rewritten for the next group
    }
  }
  for (u32 off = 32; off; off >>= 1) kept += __shfl_down(kept, off, 64);
  if (lane_id() == 0 && kept) atomicAdd(reinterpret_cast<unsigned long long*>(next_count), u64(kept));
  if (parts) {  // uniform
    adler_block_sum(as, aw, red);
    if (!threadIdx.x) {
      const u32 slot = blockIdx.x % kAdlerSlots;
      atomicAdd(reinterpret_cast<unsigned long long*>(&parts[2 * slot]), as);
      atomicAdd(reinterpret_cast<unsigned long long*>(&parts[2 * slot + 1]), aw);
    }
  }
}

constexpr u32 kCrcTile = 16384;  // output bytes per CRC-32 tile (256 threads x 64)

// CRC-32 registers (computed from 0, no inversions) of the 16 KiB tiles of
// out[0..n), one workgroup per tile (grid-stride).  The last tile is read
// right-aligned behind zero bytes: leading zeros leave a register that starts
// at 0 unchanged, so every thread's 64-byte piece has full length and the
// pieces join with one factor per tree level (x^(8 * 64 * 2^l)).
__global__ __launch_bounds__(256) void g_crc_tiles(const State* st, const u8* out, u64 n,
                                                   u64* parts, u64 tiles, u32 open) {
  __shared__ u32 table[256];
  __shared__ u32 factor[8];
  __shared__ u32 red[256];
  if (st->status || st->emit_status) return;
  if (open) {  // an open-ended decode's output is the bytes its path produced
    n = min(n, st->produced);
    tiles = (n + kCrcTile - 1) / kCrcTile;
  }
  const u32 t = threadIdx.x;
  table[t] = crc_byte_update(0, t);
  if (t < 8) factor[t] = crc_shift_bytes(u64(64) << t);
  __syncthreads();
  for (u64 tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const u64 begin = tile * kCrcTile;
    const u64 m = min<u64>(kCrcTile, n - begin);
    const u64 pad = kCrcTile - m;
    const u64 lo = u64(t) * 64;  // this thread's piece in the padded tile
    u32 c = 0;
    const u8* src = out + begin + lo;
    if (!pad && (reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
      const uint4* v = reinterpret_cast<const uint4*>(src);
      uint4 q[4] = {v[0], v[1], v[2], v[3]};
      const u32* w = reinterpret_cast<const u32*>(q);
      for (u32 j = 0; j < 16; ++j)
        for (u32 k = 0; k < 4; ++k) c = table[(c ^ (w[j] >> (8 * k))) & 0xffu] ^ (c >> 8);
    } else {
      for (u32 j = 0; j < 64; ++j) {
        const u64 p = lo + j;
        const u32 b = p >= pad ? out[begin + p - pad] : 0u;
        c = table[(c ^ b) & 0xffu] ^ (c >> 8);
      }
    }
    red[t] = c;
    __syncthreads();
    for (u32 l = 0; l < 8; ++l) {
      const u32 w = 1u << l;
      if ((t & (2 * w - 1)) == 0) red[t] = crc_mul(red[t], factor[l]) ^ red[t + w];
      __syncthreads();
    }
    if (!t) parts[tile] = red[0];
    __syncthreads();
  }
}

// CRC-32 of out[0..n) from g_crc_tiles' registers, by one 256-thread
// workgroup: each thread joins a run of tiles, then the runs join pairwise.
// Valid in thread 0.
__device__ u32 crc_from_tiles(const u64* parts, u64 n) {
  __shared__ u32 reg[256];
  __shared__ u64 len[256];
  const u32 t = threadIdx.x;
  const u64 tiles = (n + kCrcTile - 1) / kCrcTile;
  const u64 per = (tiles + 255) / 256;
  const u64 lo = min<u64>(tiles, t * per), hi = min<u64>(tiles, lo + per);
  const u32 full = crc_shift_bytes(kCrcTile);
  u32 c = 0;
  u64 bytes = 0;
  for (u64 k = lo; k < hi; ++k) {
    const u64 m = min<u64>(kCrcTile, n - k * kCrcTile);
    c = crc_mul(c, m == kCrcTile ? full : crc_shift_bytes(m)) ^ u32(parts[k]);
    bytes += m;
  }
  reg[t] = c;
  len[t] = bytes;
  __syncthreads();
  for (u32 w = 1; w < 256; w <<= 1) {
    if ((t & (2 * w - 1)) == 0) {
      reg[t] = crc_mul(reg[t], crc_shift_bytes(len[t + w])) ^ reg[t + w];
      len[t] += len[t + w];
    }
    __syncthreads();
  }
  return crc_finish(reg[0], n);
}

// Final status and the output on failure, over a grid of 256-thread
// workgroups.  The status before the trailer check (the first error of the
// decode, or unresolved references) is read by every workgroup: on a decode
// error each zeroes its grid-stride share of out[0..n).  Workgroup 0 then
// checks the trailer (`check`): Adler-32 from the `nparts` pairs the emitters
// and resolve rounds accumulated (every output byte is summed once, by
// whichever kernel wrote it), CRC-32 and size from g_crc_tiles' tile
// registers, or nothing, and writes the metadata.  A trailer mismatch keeps
// the output.
// Open-ended decode (`open.open`, one member of a concatenation): n is the
// output's capacity, the member's size is what its path produced, and its
// trailer is read after its last block in `body`; the output is left as it
// is (the caller clears it on failure), and report[0..2] gets the status, the
// member's input bytes (body_off + body bytes + trailer) and its output bytes.
__global__ __launch_bounds__(256) void g_finish(State* st, u64 n, u32* meta, const u64* parts,
                                                u32 nparts, u32 check, u8* out, OpenEnd open,
                                                const u8* body, u64 body_off, u64* report) {
  __shared__ u64 red[2][4];
  const u32 t = threadIdx.x, lane = lane_id(), wave = t >> 6;
  u32 status = st->status;
  if (!status) status = st->emit_status;
  // References still unresolved after every round.
  if (!status && st->unresolved[1]) status = kReferenceDepth;
  if (status && !open.open) {  // uniform; st->status never holds a trailer mismatch here
    const u64 stride = u64(gridDim.x) * blockDim.x;
    for (u64 i = u64(blockIdx.x) * blockDim.x + t; i < n; i += stride) out[i] = 0;
  }
  if (blockIdx.x) return;
  // Adler-32 weights were taken against the capacity's end: W = sum (cap - i) x_i.
  const u64 cap = n;
  u32 wanted = st->wanted, isize = st->isize;
  u64 end_byte = 0;
  if (open.open) {
    n = status ? 0 : st->produced;
    end_byte = (st->stream_end + 7) / 8;
    const u8* tr = body + end_byte;  // inside the input: the walk checked that it fits
    if (!status && check == kCheckAdler)
      wanted = (u32(tr[0]) << 24) | (u32(tr[1]) << 16) | (u32(tr[2]) << 8) | u32(tr[3]);
    if (!status && check == kCheckCrc) {
      wanted = u32(tr[0]) | (u32(tr[1]) << 8) | (u32(tr[2]) << 16) | (u32(tr[3]) << 24);
      isize = u32(tr[4]) | (u32(tr[5]) << 8) | (u32(tr[6]) << 16) | (u32(tr[7]) << 24);
    }
  }
  if (!status && check == kCheckCrc) {  // uniform
    const u32 got = crc_from_tiles(parts, n);
    if (!t && (got != wanted || u32(n) != isize)) status = kGzipCheckMismatch;
  }
  if (!status && check == kCheckAdler) {  // uniform: every emitter and round wrote its pair
    u64 s = 0, w = 0;
    for (u32 i = t; i < nparts; i += 256) {
      s += parts[2 * i] % kAdlerMod;
      w += parts[2 * i + 1] % kAdlerMod;
    }
    for (u32 off = 32; off; off >>= 1) {
      s += __shfl_down(s, off, 64);
      w += __shfl_down(w, off, 64);
    }
    if (!lane) {
      red[0][wave] = s;
      red[1][wave] = w;
    }
    __syncthreads();
    const u64 s_all = (red[0][0] + red[0][1] + red[0][2] + red[0][3]) % kAdlerMod;
    const u32 a = u32((s_all + 1) % kAdlerMod);
    // sum (n - i) x_i = W - (cap - n) * S (mod 65521).
    const u64 shift = ((cap - n) % kAdlerMod) * s_all % kAdlerMod;
    const u32 b = u32((red[1][0] + red[1][1] + red[1][2] + red[1][3] + kAdlerMod - shift +
                       n % kAdlerMod) %
                      kAdlerMod);
    if (((b << 16) | a) != wanted) status = kAdlerMismatch;
  }
  if (!t) {
    meta[0] = status;
    meta[1] = 0;
    if (open.open) {
      report[0] = status;
      report[1] = body_off + end_byte + open.trailer;
      report[2] = n;
    }
  }
}

namespace {
u32 clamp_grid(u64 want, u32 cap) { return u32(want < 1 ? 1 : (want > cap ? cap : want)); }

#define HZ_TRY(expr)                          \
  do {                                        \
    hipError_t _e = (expr);                   \
    if (_e != hipSuccess) return _e;          \
  } while (0)
}  // namespace

hipError_t run_inflate_general(hipStream_t stream, Scratch& scratch, const u8* in, u64 in_size,
                               u8* out, u64 out_size, u32 max_candidates, u32 max_blocks,
                               u32* meta, const StreamFormat& fmt) {
  // The body as the launches see it: after the wrapper's fixed fields and
  // before its trailer; g_frame finds where the first block starts inside it.
  const u64 body_off = fmt.format == kFormatGzip ? 10 : fmt.format == kFormatRaw ? 0 : 2;
  const u64 trailer = fmt.format == kFormatGzip ? 8 : fmt.format == kFormatRaw ? 0 : 4;
  const u8* body = in + body_off;
  // An open-ended decode's body runs to the input's end: its trailer (and any
  // later member) lies somewhere inside.
  const u64 len = in_size - body_off - (fmt.open ? 0 : trailer);
  const OpenEnd open{fmt.open ? 1u : 0u, u32(trailer), fmt.windowed ? 1u : 0u};
  const u32 check = fmt.format == kFormatGzip ? kCheckCrc
                    : fmt.format == kFormatRaw ? kCheckNone : kCheckAdler;
  // The stream's output starts `out_base` bytes into `out` (dictionary history).
  const u64 out_base = fmt.out_base, out_total = out_base + out_size;
  u8* stream_out = out + out_base;
  State* st = nullptr;
  HZ_TRY(scratch.alloc(&st, 1));
  // Emission and resolution scratch sizes.  A resolve chain hops back across
  // slices (or serially emitted segments), so its length is bounded by the
  // number of slices plus segments.
  const u64 group_capacity = (len * 8) / 8192 + 65536;
  const u64 words = (out_total + 31) / 32 + 1;
  const u32 rounds = resolve_rounds(group_capacity * 64 + u64(max_blocks));
  // Fixed-run tiles of the body and their bitmap (zeroed with the rest).
  const u64 tiles = (len * 8 + kFixTileBits - 1) / kFixTileBits;
  const u64 need_words = tiles / 32 + 1;
  // Adler-32 partial pairs: kAdlerSlots each for the lane emitter, the
  // serial emitter and the resolve rounds (workgroups add theirs, so they
  // start at zero), summed by g_finish.  The pairs, the round counts and the
  // first unresolved bitmap are zeroed by g_frame.
  u8* zeroed = nullptr;
  const u64 zero_u64 = 2 * u64(3 * kAdlerSlots) + rounds + 1;
  // Resolve group marks (emission marks groups in marks0).
  const u64 mark_groups_n = (words + 63) / 64;
  const u64 zero_bytes = 8 * zero_u64 + 4 * words + 4 * need_words + (mark_groups_n + 3) / 4 * 4;
  HZ_TRY(scratch.alloc(&zeroed, zero_bytes));
  HZ_LAUNCH(g_frame, dim3(clamp_grid((zero_bytes / 4 + 255) / 256, 2048)), dim3(256), 0, stream,
            in, in_size, fmt.format, fmt.dict, fmt.dict_len, body_off, out_base, st,
            reinterpret_cast<u32*>(zeroed), zero_bytes / 4);
  HZ_TRY(hipGetLastError());

  // Discovery.
  const u64 groups = len ? (len + kDiscRange - 1) / kDiscRange : 1;
  const u64 pre_capacity = groups * kDiscCap + u64(max_candidates) + 1;
  const u64 pre_blocks = (pre_capacity + kDiscThreads - 1) / kDiscThreads;
  // Valid counts per kValPerWave pre-candidates; the launch has a wave for
  // every val_chunk(n) of them (n <= pre_capacity).
  const u64 val_ranges = (pre_capacity + kValPerWave - 1) / kValPerWave;
  const u64 val_waves = std::max(val_ranges, std::min(pre_capacity, kValResident));
  u32 *wg_count = nullptr, *wave_valid = nullptr;
  u64 *wg_list = nullptr, *pre = nullptr, *cand = nullptr;
  HZ_TRY(scratch.alloc(&wg_count, groups));
  HZ_TRY(scratch.alloc(&wg_list, groups * kDiscCap));
  HZ_TRY(scratch.alloc(&pre, pre_capacity));
  HZ_TRY(scratch.alloc(&wave_valid, val_ranges));
  const u64 cand_capacity = u64(max_candidates) + 1;
  HZ_TRY(scratch.alloc(&cand, cand_capacity));
  // Each discovery workgroup takes per_block consecutive ranges.
  const u64 per_block = (groups + 8191) / 8192;
  const u64 blocks = (groups + per_block - 1) / per_block;
  u32* dense = nullptr;
  u32* block_total = nullptr;
  u64* block_base = nullptr;
  HZ_TRY(scratch.alloc(&dense, groups));
  HZ_TRY(scratch.alloc(&block_total, blocks));
  HZ_TRY(scratch.alloc(&block_base, blocks));
  HZ_LAUNCH(g_discover, dim3(u32(blocks)), dim3(kDiscThreads), 0, stream, body, len, st, wg_count,
            wg_list, dense, block_total, groups, per_block);
  HZ_TRY(hipGetLastError());
  HZ_LAUNCH(g_discover_scan, dim3(1), dim3(1024), 0, stream, st, block_total, block_base, blocks,
            pre_capacity, wave_valid);
  HZ_TRY(hipGetLastError());
  HZ_LAUNCH(g_discover_gather, dim3(u32((groups + kDiscThreads / 64 - 1) / (kDiscThreads / 64))),
            dim3(kDiscThreads), 0, stream, st, wg_count, wg_list, block_base, pre, groups,
            per_block);
  HZ_TRY(hipGetLastError());
  HZ_LAUNCH(g_discover_dense, dim3(64), dim3(kDiscThreads), 0, stream, body, len, st, dense,
            wg_count, block_base, pre, per_block);
  HZ_TRY(hipGetLastError());
  HZ_LAUNCH(g_validate, dim3(u32(val_waves)), dim3(64), 0, stream, body, len, st, pre,
            wave_valid);
  HZ_TRY(hipGetLastError());
  HZ_LAUNCH(g_valid_scatter, dim3(u32(pre_blocks)), dim3(kDiscThreads), 0, stream, st, pre,
            wave_valid, cand, cand_capacity, u64(max_candidates));
  HZ_TRY(hipGetLastError());

  // Describe every candidate's segment.
  u64 *seg_end = nullptr, *seg_size = nullptr;
  u32 *seg_blocks = nullptr, *seg_next = nullptr, *seg_flags = nullptr, *exit_node = nullptr;
  u32* seg_rec = nullptr;
  HZ_TRY(scratch.alloc(&seg_end, cand_capacity));
  HZ_TRY(scratch.alloc(&seg_size, cand_capacity));
  HZ_TRY(scratch.alloc(&seg_blocks, cand_capacity));
  HZ_TRY(scratch.alloc(&seg_next, cand_capacity));
  HZ_TRY(scratch.alloc(&seg_flags, cand_capacity));
  HZ_TRY(scratch.alloc(&seg_rec, cand_capacity));
  HZ_TRY(scratch.alloc(&exit_node, cand_capacity));
  // Block records and slice groups; running out only sends a segment to the
  // serial emitter.
  const u64 rec_capacity = u64(max_blocks) + cand_capacity + 1024;
  BlockRec* recs = nullptr;
  u64* slice_entry = nullptr;
  u32 *slice_off = nullptr, *group_link = nullptr;
  HZ_TRY(scratch.alloc(&recs, rec_capacity));
  const u64 table_capacity = std::min<u64>(rec_capacity, len / 8192 + 1024);
  BlockTables* tables = nullptr;
  u64* hdr_d0 = nullptr;
  u32* hdr_info = nullptr;
  HZ_TRY(scratch.alloc(&tables, table_capacity));
  HZ_TRY(scratch.alloc(&hdr_d0, table_capacity));
  HZ_TRY(scratch.alloc(&hdr_info, table_capacity));
  // Grid-stride kernels over candidates, segments or units launch at most one
  // workgroup per 64 body bytes (at least 256): a small stream has few of
  // them, and idle workgroups of a 4096-wide launch cost their dispatch.
  const u64 items_cap = std::max<u64>(256, len / 64);
  HZ_LAUNCH(g_headers, dim3(clamp_grid(std::min(table_capacity, 2 * items_cap), 8192)), dim3(kWave), 0, stream, body, len, st,
            cand, tables, table_capacity, hdr_d0, hdr_info);
  HZ_TRY(hipGetLastError());
  HZ_TRY(scratch.alloc(&slice_entry, group_capacity * 64));
  HZ_TRY(scratch.alloc(&slice_off, group_capacity * 64));
  HZ_TRY(scratch.alloc(&group_link, group_capacity));
  u32 *seg_last = nullptr, *region_cand = nullptr;
  HZ_TRY(scratch.alloc(&seg_last, cand_capacity));
  HZ_TRY(scratch.alloc(&region_cand, cand_capacity));
  u32* fix_need = reinterpret_cast<u32*>(zeroed + 8 * zero_u64 + 4 * words);
  HZ_LAUNCH(g_describe, dim3(clamp_grid(std::min(cand_capacity, items_cap), 4096)), dim3(kDescThreads), 0, stream, body, len,
            cand, st, out_size, seg_end, seg_size, seg_blocks, seg_next, seg_flags, seg_rec, recs,
            rec_capacity, slice_entry, slice_off, group_link, group_capacity, tables,
            table_capacity, hdr_d0, hdr_info, seg_last, region_cand);
  HZ_TRY(hipGetLastError());
  HZ_LAUNCH(g_fix_mark, dim3(1), dim3(256), 0, stream, st, cand, len, seg_end, seg_flags,
            region_cand, fix_need, tiles);
  HZ_TRY(hipGetLastError());

  // Long fixed-Huffman runs deferred by describe (each launch returns at once
  // when there are none).
  FixSummary* fix_sum = nullptr;
  FixRun* fix_runs = nullptr;
  FixTile* fix_rt = nullptr;
  const u64 run_capacity = cand_capacity + 1024;
  const u64 rt_capacity = tiles + 64 * 4096;
  FixTask* fix_tasks = nullptr;
  const u64 task_capacity = 4 * tiles + 4096;  // beyond it, g_fix_sum decodes the rests itself
  HZ_TRY(scratch.alloc(&fix_sum, (tiles ? tiles : 1) * kFixEntries));
  HZ_TRY(scratch.alloc(&fix_tasks, task_capacity));
  HZ_TRY(scratch.alloc(&fix_runs, run_capacity));
  HZ_TRY(scratch.alloc(&fix_rt, rt_capacity));
  HZ_LAUNCH(g_fix_sum, dim3(clamp_grid((tiles + 7) / 8, 2048)), dim3(256), 0, stream, body, len,
            st, fix_need, fix_sum, tiles, fix_tasks, task_capacity);
  HZ_TRY(hipGetLastError());
  HZ_LAUNCH(g_fix_rem, dim3(clamp_grid((task_capacity + 255) / 256, 2048)), dim3(256), 0, stream,
            body, len, st, fix_tasks, task_capacity, fix_sum);
  HZ_TRY(hipGetLastError());
  FixGroupSum* fix_groups = nullptr;
  const u64 fix_group_count = tiles / kFixGroupTiles;
  HZ_TRY(scratch.alloc(&fix_groups, (fix_group_count ? fix_group_count : 1) * 64));
  HZ_LAUNCH(g_fix_groups, dim3(clamp_grid((fix_group_count * 64 + 255) / 256, 2048)), dim3(256), 0,
            stream, st, fix_need, fix_sum, tiles, fix_groups);
  HZ_TRY(hipGetLastError());
  HZ_LAUNCH(g_fix_walk, dim3(clamp_grid(std::min(cand_capacity, items_cap), 2048)), dim3(kWave), 0, stream, body, len, st,
            cand, fix_need, fix_sum, tiles, seg_end, seg_size, seg_blocks, seg_next, seg_flags,
            seg_rec, seg_last, region_cand, recs, rec_capacity, fix_runs, run_capacity, fix_rt,
            rt_capacity, group_link, group_capacity, out_size, fix_groups);
  HZ_TRY(hipGetLastError());
  HZ_LAUNCH(g_fix_slices, dim3(clamp_grid((rt_capacity * kFixGroupTiles + 255) / 256, 2048)),
            dim3(256), 0, stream, body, len, st, fix_rt, rt_capacity, fix_runs, run_capacity,
            fix_sum, slice_entry, slice_off);
  HZ_TRY(hipGetLastError());

  // Chain selection, then the exact walk if the fast chain declined.
  Segment* acc = nullptr;
  HZ_TRY(scratch.alloc(&acc, u64(max_blocks) + 1));
  HZ_LAUNCH(g_chain, dim3(1), dim3(1024), 0, stream, st, cand, seg_end, seg_size, seg_blocks,
            seg_next, seg_flags, seg_rec, exit_node, len, out_size, max_blocks, acc, out_base,
            open);
  HZ_TRY(hipGetLastError());
  HZ_LAUNCH(g_exact_walk, dim3(1), dim3(kWave), 0, stream, body, len, st, out_size, max_blocks,
            acc, out_base, open);
  HZ_TRY(hipGetLastError());

  // Emission and cross-segment resolution.
  const u32 emit_grid = clamp_grid(std::min<u64>(max_blocks, items_cap), 4096);
  // A workgroup per group of 64 words while there are at most 2048 groups
  // (g_resolve then shares each group among its waves), else 2048.
  const u32 resolve_grid = clamp_grid((words + 63) / 64, 2048);
  u64* adler_parts = reinterpret_cast<u64*>(zeroed);
  u64* counts = adler_parts + 2 * u64(3 * kAdlerSlots);
  u32* bits0 = reinterpret_cast<u32*>(counts + rounds + 1);
  u32 *roots = nullptr, *bits1 = nullptr;
  HZ_TRY(scratch.alloc(&roots, out_total ? out_total : 1));
  HZ_TRY(scratch.alloc(&bits1, words));
  u8* marks0 = zeroed + 8 * zero_u64 + 4 * words + 4 * need_words;
  u8* marks1 = nullptr;
  HZ_TRY(scratch.alloc(&marks1, mark_groups_n));
  const u64 out_end = out_total;  // a byte at position p is stream byte n - (out_end - p)
  // Emission by segments, then the queued units of long fixed runs.
  EmitUnit* units = nullptr;
  const u64 unit_capacity = group_capacity + 64;  // a round holds at least one slice group
  HZ_TRY(scratch.alloc(&units, unit_capacity));
  for (u32 pass = 0; pass < 2; ++pass) {
    HZ_LAUNCH(g_emit_lanes, dim3(emit_grid), dim3(kEmitThreads), 0, stream, body, len, st, acc,
              recs, slice_entry, slice_off, group_link, tables, out, roots, bits0, out_end,
              adler_parts, units, unit_capacity, pass, marks0);
    HZ_TRY(hipGetLastError());
  }
  HZ_LAUNCH(g_emit_serial, dim3(emit_grid), dim3(kWave), 0, stream, body, len, st, acc, out,
            roots, bits0, out_end, adler_parts + 2 * kAdlerSlots, marks0);
  HZ_TRY(hipGetLastError());
  for (u32 round = 0; round < rounds; ++round) {
    HZ_LAUNCH(g_resolve, dim3(resolve_grid), dim3(256), 0, stream, st, out, roots, bits0, bits1,
              counts, round, rounds, words, out_end, adler_parts + 4 * kAdlerSlots, marks0, marks1);
    HZ_TRY(hipGetLastError());
  }
  u64* parts = nullptr;
  u32 nparts = 0;
  const u32 finish_grid = clamp_grid((out_size + 255) / 256, 4096);
  if (check == kCheckAdler) {
    // The pairs of the emitters, then those of the resolve rounds.
    HZ_LAUNCH(g_finish, dim3(finish_grid), dim3(256), 0, stream, st, out_size, meta, adler_parts,
              3 * kAdlerSlots, check, stream_out, open, body, body_off, fmt.report);
    return hipGetLastError();
  }
  if (check == kCheckCrc) {
    const u64 tiles = (out_size + kCrcTile - 1) / kCrcTile;
    HZ_TRY(scratch.alloc(&parts, tiles ? tiles : 1));
    if (tiles) {
      HZ_LAUNCH(g_crc_tiles, dim3(clamp_grid(tiles, 4096)), dim3(256), 0, stream, st, stream_out,
                out_size, parts, tiles, open.open);
      HZ_TRY(hipGetLastError());
    }
  }
  HZ_LAUNCH(g_finish, dim3(finish_grid), dim3(256), 0, stream, st, out_size, meta, parts, nparts,
            check, stream_out, open, body, body_off, fmt.report);
  return hipGetLastError();
}


hipError_t run_inflate_batch_wide(hipStream_t stream, Scratch& scratch, const u8* in, u8* out,
                                  u64 out_total, const BatchFile* files, const u32* list,
                                  u32 n, u64 in_bits, const u32* encoded, u32 max_blocks,
                                  u32* redo, u32* meta) {
  if (!n) return hipSuccess;
  // Slice groups: at most one per 64 slices of >= kDescMinSlice bits, plus
  // the partly filled last group of every describe round.
  const u64 group_capacity = in_bits / (u64(kDescMinSlice) * 64) +
                             in_bits / (u64(kDescThreads) * kDescMinSlice) + 8 * u64(n) + 64;
  const u32 rounds = resolve_rounds(group_capacity * 64 + u64(max_blocks));
  const u64 words = (out_total + 31) / 32 + 1;
  // The state, the resolve counts and the first bitmap start zeroed: one
  // allocation, cleared by one fill.
  const u64 st_bytes = scratch_round(sizeof(State));
  const u64 counts_bytes = scratch_round((rounds + 1) * sizeof(u64));
  u8* zeroed = nullptr;
  HZ_TRY(scratch.alloc(&zeroed, st_bytes + counts_bytes + words * 4));
  HZ_TRY(launch_fill(stream, zeroed, 0, st_bytes + counts_bytes + words * 4));
  State* st = reinterpret_cast<State*>(zeroed);
  u64* counts = reinterpret_cast<u64*>(zeroed + st_bytes);
  u32* bits0 = reinterpret_cast<u32*>(zeroed + st_bytes + counts_bytes);
  u64* slice_entry = nullptr;
  u32 *slice_off = nullptr, *group_link = nullptr, *wanted = nullptr;
  HZ_TRY(scratch.alloc(&slice_entry, group_capacity * 64));
  HZ_TRY(scratch.alloc(&slice_off, group_capacity * 64));
  HZ_TRY(scratch.alloc(&group_link, group_capacity));
  HZ_TRY(scratch.alloc(&wanted, u64(n) + 1));
  u32 *roots = nullptr, *bits1 = nullptr;
  HZ_TRY(scratch.alloc(&roots, out_total ? out_total : 1));
  HZ_TRY(scratch.alloc(&bits1, words));
  HZ_LAUNCH(g_batch_wide, dim3(n), dim3(kDescThreads), 0, stream, in, out, files, list, n,
            encoded, max_blocks, st, slice_entry, slice_off, group_link, group_capacity, roots,
            bits0, redo, wanted);
  HZ_TRY(hipGetLastError());
  for (u32 round = 0; round < rounds; ++round) {
    HZ_LAUNCH(g_resolve, dim3(u32(clamp_grid((words + 255) / 256, 2048))), dim3(256), 0, stream,
              st, out, roots, bits0, bits1, counts, round, rounds, words, 0ull, nullptr, nullptr,
              nullptr);
    HZ_TRY(hipGetLastError());
  }
  HZ_LAUNCH(g_batch_wide_finish, dim3(n), dim3(256), 0, stream, files, list, n, out, st, wanted,
            redo, meta);
  return hipGetLastError();
}

}  // namespace hz
