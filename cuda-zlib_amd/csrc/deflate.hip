// Chunked zlib encoder (default 32 KiB chunks).
//
// Stream layout (the reference's compress path, native/codec_ffi.cu:551-612,
// encoder E:283-418): header 78 01; every chunk is one block of the cheapest
// type (stored, fixed or dynamic Huffman); a non-final fixed/dynamic block is
// followed by an empty stored block so every chunk ends byte aligned and
// chunks concatenate at byte granularity; Adler-32 trailer, big endian.  The
// worst chunk costs len + 5 bytes, so a stream always fits in
// n + 5 * chunks + 6 bytes.
//
// Unlike the reference, a chunk's LZ77 window includes up to 32 KiB of the
// same input before it (the decoder has already produced those bytes), which
// keeps the ratio below whole-stream zlib level 1.  The independent mode
// (run_deflate with `independent`) limits every window to its own chunk, as
// the reference's per-chunk encoder does.
//
// e_parse, one 1024-thread workgroup per chunk; the LDS holds the window and
// the hash table.  For chunks up to about 35 KiB two workgroups share a CU
// (80 KiB each, up to 11 KiB of history for 32 KiB chunks), so that one
// runs while the other waits at a barrier; larger chunks take a whole CU:
//   stage    window (history + chunk) into LDS as aligned dwords; Adler-32
//            partial sums of the chunk bytes
//   history  every history position enters the hash table
//   parse    steps of 1024 positions, one per thread: 4-byte hash into 8192
//            one-way buckets; candidates = the bucket plus the previous
//            position of the same wave when its hash is equal; longest
//            match (ties: nearest); one-step lazy rule (a position yields to a
//            longer match at the next position).  With f(j) = j + max(1, L_j)
//            the greedy token starts are the orbit of 0 under f: every wave
//            finds the first orbit point past itself from each of its
//            positions (pointer doubling by shuffles), wave 0 chains the 16
//            waves' entries, and each wave walks its orbit from its entry over
//            its match lanes (or marks it by doubling when matches are dense).
//            Tokens go to a global list, histograms by LDS atomics; the step's
//            positions enter the table by atomicMax, so the newest position
//            wins independently of execution order.
// e_tree, one two-wave workgroup per chunk (eight per CU):
//   huffman  optimal code lengths limited to 15/7 bits (leaves sorted by a
//            bitonic network, package-merge with each level merged along
//            merge paths); wave-parallel code-length RLE and canonical codes
//   choose   exact bit costs of stored / fixed / dynamic, hence the chunk's
//            compressed extent
// e_scan places every chunk from the extents; then e_emit, one 256-thread
// workgroup per chunk (eight per CU): 4 tokens per thread per round, bit
// lengths, block-wide exclusive scan, atomicOr into an LDS bit ring whose
// complete 16-byte lines go straight to the chunk's place in the output.
// Then per-file wrapper and metadata, all on device (no host
// synchronisation).
#include <algorithm>
#include <vector>

#include "deflate_common.h"
#include "kernels.h"

namespace hz {
namespace {

constexpr u32 kParseThreads = 1024;
constexpr u32 kParseWaves = kParseThreads / 64;
static_assert(kParseWaves <= 16, "the wave-count scan covers one 16-lane DPP row");
constexpr u32 kStep = kParseThreads;  // parse positions per step
constexpr u32 kHashBits = 13;
constexpr u32 kBuckets = 1u << kHashBits;
constexpr u32 kWays = 1;
constexpr u32 kNear = 1;
constexpr u32 kWalkMatches = 4;  // waves with at most this many match lanes walk their orbit
constexpr u32 kMaxDist = 32768;
constexpr u32 kHistory = 32768;
constexpr u32 kMaxSteps = 65536 / 1024 + 1;  // parse steps of the largest chunk
// LDS of a CU, and of each of two parse workgroups sharing one.  Two
// workgroups per CU fill each other's barrier waits (the chain of wave
// entries and the slowest wave's lookups); they need 8 waves per SIMD, so
// the parse kernel keeps to 64 VGPRs.
constexpr u32 kLdsBudget = 160 * 1024;
constexpr u32 kPairBudget = kLdsBudget / 2;
constexpr u32 kPairMinHistory = 8192;  // least history that keeps the paired layout
constexpr u32 kEmitThreads = 256;
constexpr u32 kEmitWaves = kEmitThreads / 64;
constexpr u32 kTokensPerThread = 4;
constexpr u32 kTreeThreads = 128;

struct ChunkDesc {
  u64 in_off;    // absolute input offset of the chunk
  u64 file_off;  // chunk offset inside its file
  u64 file_len;  // length of the chunk's file
  u32 len;       // chunk bytes
  u32 hist;      // history bytes staged before the chunk (same file)
  u32 file;
  u32 last;      // last chunk of its file
};

struct FileDesc {
  u64 in_off, in_len;     // input range
  u64 out_off, capacity;  // padded output slot
  u32 first_chunk, chunks;
};

// Parse results of one chunk, consumed by e_emit.
struct ChunkStats {
  u32 freq_ll[288];
  u32 freq_d[32];
  u32 ntok;
  u32 extra_bits;  // length and distance extra bits of all matches
  u64 sum_s;       // sum of the chunk bytes
  u64 sum_l;       // sum of (offset in chunk) * byte
};

struct ChunkResult {
  u32 extent;   // compressed bytes of the chunk
  u32 status;   // 0 or kCompressionOverflow
  u64 adler_s;  // sum of bytes mod 65521
  u64 adler_b;  // sum of (file_len - i) * byte over the chunk, mod 65521
};

struct ParseShared {
  u32 table[kBuckets * kWays];  // position + 1 per way, 0 = empty
  u16 exitv[kStep];             // first orbit point past the position's wave
  u16 went[kParseWaves];        // orbit entry of each wave (0xffff: none)
  u8 wave_match[kParseWaves];   // the wave has a match in the current step
  u8 mark[kStep];               // token starts of waves that mark by doubling
  u32 freq_ll[288];
  u32 freq_d[32];
  u32 wave_count[2][kParseWaves];  // token counts of the last two steps, by step parity
  u32 adv;                      // step advance: first orbit point at or past the step's end
  u32 extra_bits;
  u64 red_s[kParseWaves], red_l[kParseWaves];
  // Positions a step skipped (inside a match past the step's end), which the
  // parse never hashed: [skip_lo, skip_hi) per range, window-relative.
  u32 skip_lo[kMaxSteps], skip_hi[kMaxSteps];
  u32 nskip;
};

constexpr u32 kParseShared = (sizeof(ParseShared) + 15) & ~u32(15);

// LDS of one parse workgroup for chunks of `chunk` bytes: half a CU when
// that leaves at least kPairMinHistory bytes of history, else the whole CU.
constexpr u32 parse_budget(u32 chunk) {
  return kParseShared + chunk + 32 + kPairMinHistory <= kPairBudget ? kPairBudget : kLdsBudget;
}

// Largest history that fits the parse budget next to a chunk of `chunk` bytes.
constexpr u32 history_limit(u32 chunk) {
  return parse_budget(chunk) - kParseShared - chunk - 32 < kHistory
             ? parse_budget(chunk) - kParseShared - chunk - 32
             : kHistory;
}
static_assert(kParseShared + 65535 + 32 + 16384 < kLdsBudget, "parse LDS layout exceeds the budget");
static_assert(parse_budget(32768) == kPairBudget, "32 KiB chunks parse two workgroups per CU");

// Package-merge scratch of one tree of at most N symbols (one wave).
template <u32 N>
struct HuffScratchT {
  static constexpr u32 kItems = 2 * N;           // items of one level (< 2 * symbols)
  static constexpr u32 kWords = (kItems + 31) / 32;
  u16 list[N];
  u16 sorted[N];
  u32 leaf[N];                   // leaf weights in sorted order
  u32 items[2][kItems];          // item weights of two consecutive levels
  u32 leafbits[16][kWords];      // per level: which items are leaves
};
using HuffScratchLL = HuffScratchT<320>;  // literal/length tree (286), then code lengths (19)
using HuffScratchD = HuffScratchT<32>;    // distance tree (30)

// A chunk's block coding, from e_tree to e_emit: code lengths, canonical
// codes (bit-reversed), the code-length RLE and the chosen block.
struct alignas(16) CodeTables {
  u8 len_ll[288];
  u8 len_d[32];
  u8 len_cl[20];
  u16 code_ll[288];
  u16 code_d[32];
  u16 code_cl[20];
  u16 rle[320];  // code-length RLE: symbol | extra << 5
  u32 nrle, hlit, hdist, hclen, mode, extent, hdr_bits;
};
static_assert(sizeof(CodeTables) % 16 == 0, "code tables copy as uint4");

// e_tree LDS.
struct TreeShared {
  u32 freq_ll[288];
  u32 freq_d[32];
  u32 freq_cl[20];
  CodeTables tab;
  HuffScratchLL hs_ll;
  HuffScratchD hs_d;
};

// e_emit LDS; the bit buffer follows it.
struct EmitShared {
  CodeTables tab;
  u32 scan[kEmitWaves];
  u32 status;
};


// e_emit's bit buffer is a ring: word w of the chunk's output lines lives at
// ring[w % kRingWords].  A round of 1024 tokens writes at most 1536 words,
// and the lines below a round's first bit leave for the output during the
// next round, so the live words always fit.
constexpr u32 kRingWords = 4096;
constexpr u32 kRingMask = kRingWords - 1;
static_assert(2 * (kEmitThreads * kTokensPerThread * 48 / 32) + 8 < kRingWords,
              "two rounds of the longest tokens fit the ring");

__device__ __forceinline__ u32 win_u32(const u32* win, u32 q) {
  return __builtin_amdgcn_alignbyte(win[(q >> 2) + 1], win[q >> 2], q & 3);
}

__device__ __forceinline__ u32 win_byte(const u32* win, u32 q) {
  return (win[q >> 2] >> (8 * (q & 3))) & 0xff;
}

__device__ __forceinline__ u32 hash4(u32 v) { return (v * 2654435761u) >> (32 - kHashBits); }

// Length of the common prefix of window positions a < b, at most maxlen.
// One dword first (most candidates end there), then sixteen bytes a round
// (five dwords of each side in flight); bytes read past the window's end are
// ignored by the clamp to maxlen (the LDS allocation holds 32 bytes past the
// largest window).
__device__ __forceinline__ u32 match_len(const u32* win, u32 a, u32 b, u32 maxlen) {
  {
    const u32 x = win_u32(win, a) ^ win_u32(win, b);
    if (x) return min(maxlen, u32(__builtin_ctz(x)) >> 3);
  }
  const u32 sa = a & 3, sb = b & 3;
  const u32* pa = win + (a >> 2) + 1;
  const u32* pb = win + (b >> 2) + 1;
  for (u32 m = 4; m < maxlen; m += 16, pa += 4, pb += 4) {
    u32 da[5], db[5];
#pragma unroll
    for (u32 k = 0; k < 5; ++k) {
      da[k] = pa[k];
      db[k] = pb[k];
    }
#pragma unroll
    for (u32 k = 0; k < 4; ++k) {
      const u32 x = __builtin_amdgcn_alignbyte(da[k + 1], da[k], sa) ^
                    __builtin_amdgcn_alignbyte(db[k + 1], db[k], sb);
      if (x) return min(maxlen, m + 4 * k + (u32(__builtin_ctz(x)) >> 3));
    }
  }
  return maxlen;
}

// RFC 1951 length code (257..285) and extra bits for a match length 3..258.
__device__ __forceinline__ void length_code(u32 len, u32& sym, u32& nbits, u32& extra) {
  if (len == 258) { sym = 285; nbits = 0; extra = 0; return; }
  if (len < 11) { sym = 254 + len; nbits = 0; extra = 0; return; }
  const u32 l = len - 3;
  const u32 k = 31 - __builtin_clz(l);  // 3..7
  sym = 257 + 4 * (k - 1) + ((l >> (k - 2)) & 3);
  nbits = k - 2;
  extra = l & ((1u << (k - 2)) - 1);
}

// Distance code (0..29) and extra bits for a distance 1..32768.
__device__ __forceinline__ void dist_code(u32 d, u32& sym, u32& nbits, u32& extra) {
  if (d <= 4) { sym = d - 1; nbits = 0; extra = 0; return; }
  const u32 x = d - 1;
  const u32 k = 31 - __builtin_clz(x);  // 2..14
  sym = 2 * k + ((x >> (k - 1)) & 1);
  nbits = k - 1;
  extra = x & ((1u << (k - 1)) - 1);
}

__device__ __forceinline__ u32 fixed_len(u32 s) {
  return s < 144 ? 8u : s < 256 ? 9u : s < 280 ? 7u : 8u;
}

// Bitonic sort of the m leaf keys (weight << 9 | symbol) over 64 * kRegs
// slots, m <= 64 * kRegs, into hs.sorted / hs.leaf: slot r * 64 + lane in
// register r; partners within a lane swap registers, partners across lanes
// exchange by shuffles.  Padding keys sort last, so every width that holds
// the m keys gives the same order.
template <u32 kRegs, class HS>
__device__ void sort_leaves(HS& hs, const u32* freq, u32 m, u32 lane) {
  u32 key[kRegs];
#pragma unroll
  for (u32 r = 0; r < kRegs; ++r) {
    const u32 i = r * 64 + lane;
    if (i < m) {
      const u32 s = hs.list[i];
      key[r] = ((freq[s] ? freq[s] : 1u) << 9) | s;
    } else {
      key[r] = 0xffffffffu;
    }
  }
#pragma clang loop unroll(full)
  for (u32 k = 2; k <= 64 * kRegs; k <<= 1) {
#pragma clang loop unroll(full)
    for (u32 j = k >> 1; j; j >>= 1) {
      if (j >= 64) {
        const u32 rj = j >> 6;
#pragma clang loop unroll(full)
        for (u32 r = 0; r < kRegs; ++r) {
          if (r & rj) continue;
          const u32 e = r * 64 + lane;
          const bool up = (e & k) == 0;
          const u32 a = key[r], b = key[r | rj];
          const bool swap = up ? a > b : a < b;
          key[r] = swap ? b : a;
          key[r | rj] = swap ? a : b;
        }
      } else {
#pragma clang loop unroll(full)
        for (u32 r = 0; r < kRegs; ++r) {
          const u32 e = r * 64 + lane;
          const u32 other = __shfl_xor(key[r], j, 64);
          const bool up = (e & k) == 0, lower = (lane & j) == 0;
          // The lower slot keeps the smaller key in an ascending run.
          const bool take_min = up == lower;
          key[r] = take_min ? min(key[r], other) : max(key[r], other);
        }
      }
    }
  }
#pragma unroll
  for (u32 r = 0; r < kRegs; ++r) {
    const u32 i = r * 64 + lane;
    if (i < m) {
      hs.sorted[i] = u16(key[r] & 511);
      hs.leaf[i] = key[r] >> 9;
    }
  }
}

// Optimal length-limited code lengths by package-merge (one wave; every lane
// calls).  Leaves are sorted by (frequency, symbol) with a bitonic network.  Level
// `limit` holds the sorted leaves; level j merges the leaves with the
// packages of level j + 1 (sums of its consecutive item pairs), each lane
// merging one stretch of the output along the merge path (leaves before
// packages of equal weight).  The first 2m - 2 items of level 1 are taken;
// a taken package takes its two children, so the taken items of every level
// are a prefix, and a leaf's length is the number of levels whose taken
// prefix holds it.  Unused symbols get length 0 (at least two symbols get a
// code).  64 * kRegs slots hold at least n leaves.
template <u32 kRegs, class HS>
__device__ void huffman_lengths(HS& hs, const u32* freq, u32 n, u32 limit, u8* len) {
  const u32 lane = lane_id();
  u32 m = 0;
  for (u32 base = 0; base < n; base += 64) {
    const u32 s = base + lane;
    const bool used = s < n && freq[s] != 0;
    if (s < n) len[s] = 0;
    const u64 bal = __ballot(used);
    if (used) hs.list[m + __popcll(bal & lanemask_lt())] = u16(s);
    m += __popcll(bal);
  }
  if (m < 2) {
    for (u32 s = 0; m < 2 && s < n; ++s)
      if (!freq[s]) {
        if (!lane) hs.list[m] = u16(s);
        ++m;
      }
  }
  wave_sync();
  // The narrowest sort that holds the m leaves (short chunks use few symbols).
  if (kRegs >= 8 && m > 256) sort_leaves<(kRegs >= 8 ? 8u : 1u)>(hs, freq, m, lane);
  else if (kRegs >= 4 && m > 128) sort_leaves<(kRegs >= 4 ? 4u : 1u)>(hs, freq, m, lane);
  else if (kRegs >= 2 && m > 64) sort_leaves<(kRegs >= 2 ? 2u : 1u)>(hs, freq, m, lane);
  else sort_leaves<1>(hs, freq, m, lane);
  for (u32 i = lane; i < 16 * HS::kWords; i += 64) (&hs.leafbits[0][0])[i] = 0;
  wave_sync();
  // Level `limit`: the leaves.
  u32* prev = hs.items[0];
  for (u32 i = lane; i < m; i += 64) prev[i] = hs.leaf[i];
  for (u32 i = lane; i < m; i += 64) atomicOr(&hs.leafbits[limit][i >> 5], 1u << (i & 31));
  u32 size = m;
  wave_sync();
  for (u32 j = limit - 1; j >= 1; --j) {
    u32* next = hs.items[(limit - j) & 1];
    const u32 np = size / 2, total = m + np;
    // Output stretch [d0, d1) of this lane; its split point along the merge
    // path: a leaves and d0 - a packages precede it.
    const u32 d0 = u32(u64(total) * lane / 64), d1 = u32(u64(total) * (lane + 1) / 64);
    u32 lo = d0 > np ? d0 - np : 0u, hi = d0 < m ? d0 : m;
    while (lo < hi) {  // least a such that leaf a comes after package d0 - 1 - a
      const u32 a = (lo + hi) / 2, b = d0 - 1 - a;
      const u32 pk = prev[2 * b] + prev[2 * b + 1];
      if (hs.leaf[a] <= pk) lo = a + 1;
      else hi = a;
    }
    u32 a = lo, b = d0 - lo;
    for (u32 d = d0; d < d1; ++d) {
      const u32 pk = b < np ? prev[2 * b] + prev[2 * b + 1] : 0xffffffffu;
      if (a < m && (b >= np || hs.leaf[a] <= pk)) {
        next[d] = hs.leaf[a++];
        atomicOr(&hs.leafbits[j][d >> 5], 1u << (d & 31));
      } else {
        next[d] = pk;
        ++b;
      }
    }
    size = total;
    prev = next;
    wave_sync();
  }
  // Taken prefixes from level 1 down: taken_j items, of which c_j leaves.
  // (Levels are unrolled so that c[] stays in registers.)
  u32 taken = 2 * m - 2;
  u32 c[16];
#pragma unroll
  for (u32 j = 0; j < 16; ++j) c[j] = 0;
#pragma unroll
  for (u32 j = 1; j <= 15; ++j) {
    if (j > limit) break;
    u32 leaves = 0;
    for (u32 w = lane; w * 32 < taken; w += 64) {
      u32 bits = hs.leafbits[j][w];
      if ((w + 1) * 32 > taken) bits &= (1u << (taken & 31)) - 1u;
      leaves += __builtin_popcount(bits);
    }
    for (u32 off = 32; off; off >>= 1) leaves += __shfl_xor(leaves, off, 64);
    c[j] = leaves;
    taken = 2 * (taken - leaves);
  }
  for (u32 i = lane; i < m; i += 64) {
    u32 l = 0;
#pragma unroll
    for (u32 j = 1; j <= 15; ++j) l += i < c[j] ? 1u : 0u;
    len[hs.sorted[i]] = u8(l);
  }
  wave_sync();
}

// Canonical codes (bit-reversed) from lengths, one wave: length counts by
// ballots, then each symbol's rank among the earlier symbols of its length.
__device__ void canonical_codes_wave(const u8* len, u32 n, u16* code) {
  const u32 lane = lane_id();
  u32 cnt[16];
#pragma unroll
  for (u32 l = 0; l < 16; ++l) cnt[l] = 0;
  for (u32 base = 0; base < n; base += 64) {
    const u32 s = base + lane;
    const u32 l = s < n ? len[s] : 0u;
#pragma unroll
    for (u32 k = 1; k < 16; ++k) cnt[k] += __popcll(__ballot(l == k));
  }
  u32 start[16];
  u32 c = 0;
  start[0] = 0;
#pragma unroll
  for (u32 k = 1; k < 16; ++k) {
    c = (c + (k > 1 ? cnt[k - 1] : 0u)) << 1;
    start[k] = c;
  }
  for (u32 base = 0; base < n; base += 64) {
    const u32 s = base + lane;
    const u32 l = s < n ? len[s] : 0u;
    u32 mine = 0;
#pragma unroll
    for (u32 k = 1; k < 16; ++k) {
      const u64 b = __ballot(l == k);
      if (l == k) mine = start[k] + __popcll(b & lanemask_lt());
      start[k] += __popcll(b);
    }
    if (l) code[s] = u16(bit_reverse(mine, l));
  }
}

// One past the last nonzero length in len[0, n), at least `floor` (one wave).
__device__ __forceinline__ u32 used_extent(const u8* len, u32 n, u32 floor) {
  const u32 lane = lane_id();
  u32 last = 0;
  for (u32 base = 0; base < n; base += 64) {
    const u32 s = base + lane;
    const u64 b = __ballot(s < n && len[s] != 0);
    if (b) last = base + 64 - __builtin_clzll(b);
  }
  return last > floor ? last : floor;
}

// The RLE symbols of a run of `run` equal lengths `v` (zlib's scheme: 18/17
// for zeros, 16 for repeats of a nonzero length after one literal copy);
// emit(symbol | extra << 5) for each.
template <class F>
__device__ __forceinline__ void rle_run(u32 v, u32 run, F&& emit) {
  if (!v) {
    u32 r = run;
    while (r >= 11) {
      const u32 t = r < 138 ? r : 138;
      emit(18u | ((t - 11) << 5));
      r -= t;
    }
    if (r >= 3) {
      emit(17u | ((r - 3) << 5));
      r = 0;
    }
    while (r--) emit(0u);
  } else {
    emit(v);
    u32 r = run - 1;
    while (r >= 3) {
      const u32 t = r < 6 ? r : 6;
      emit(16u | ((t - 3) << 5));
      r -= t;
    }
    while (r--) emit(v);
  }
}

// Code-length RLE of the literal/length and distance lengths, one wave: the
// same symbols as a serial left-to-right pass.  Each lane owns the runs that
// start at its positions; run ends come from the start ballots, outputs from
// a scan of per-run symbol counts.
__device__ void rle_lengths_wave(TreeShared& sh) {
  CodeTables& tab = sh.tab;
  const u32 lane = lane_id();
  const u32 total = tab.hlit + tab.hdist;  // <= 316: five ballot words
  auto at = [&](u32 k) -> u32 { return k < tab.hlit ? tab.len_ll[k] : tab.len_d[k - tab.hlit]; };
  if (lane < 20) sh.freq_cl[lane] = 0;
  u64 starts[5];
#pragma unroll
  for (u32 c = 0; c < 5; ++c) {
    const u32 i = c * 64 + lane;
    const bool st = i < total && (i == 0 || at(i) != at(i - 1));
    starts[c] = __ballot(st);
  }
  // Run of each start this lane owns, and its symbol count.
  u32 v[5], run[5], cnt[5];
#pragma unroll
  for (u32 c = 0; c < 5; ++c) {
    const u32 i = c * 64 + lane;
    v[c] = run[c] = cnt[c] = 0;
    if ((starts[c] >> lane) & 1) {
      u32 end = total;
      u64 rest = lane == 63 ? 0ull : starts[c] & (~0ull << (lane + 1));
      if (rest) end = c * 64 + __builtin_ctzll(rest);
      else
        for (u32 k = c + 1; k < 5; ++k)
          if (starts[k]) { end = k * 64 + __builtin_ctzll(starts[k]); break; }
      v[c] = at(i);
      run[c] = end - i;
      u32 nsym = 0;
      rle_run(v[c], run[c], [&](u32) { ++nsym; });
      cnt[c] = nsym;
    }
  }
  wave_sync();
  u32 carry = 0;
#pragma unroll
  for (u32 c = 0; c < 5; ++c) {
    u32 x = cnt[c];
    for (u32 off = 1; off < 64; off <<= 1) {
      const u32 y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    u32 at_sym = carry + x - cnt[c];
    carry += __shfl(x, 63, 64);
    if (cnt[c])
      rle_run(v[c], run[c], [&](u32 sym) {
        tab.rle[at_sym++] = u16(sym);
        atomicAdd(&sh.freq_cl[sym & 31], 1u);
      });
  }
  if (!lane) tab.nrle = carry;
  wave_sync();
}

// Serial LSB-first writer into the LDS bit buffer (header and block tail);
// ORs into words that the caller has cleared.
struct StageWriter {
  u32* ring;
  u32 pos;
  __device__ __forceinline__ void put(u32 v, u32 n) {
    if (!n) return;
    const u32 w = pos >> 5, s = pos & 31;
    const u64 x = u64(v) << s;
    ring[w & kRingMask] |= u32(x);
    if (s + n > 32) ring[(w + 1) & kRingMask] |= u32(x >> 32);
    pos += n;
  }
};

__device__ __forceinline__ void or_bits(u32* ring, u32 pos, u64 v) {
  const u32 w = pos >> 5, s = pos & 31;
  const u64 lo = v << s;
  const u32 hi = s ? u32(v >> (64 - s)) : 0u;
  if (u32(lo)) atomicOr(&ring[w & kRingMask], u32(lo));
  if (u32(lo >> 32)) atomicOr(&ring[(w + 1) & kRingMask], u32(lo >> 32));
  if (hi) atomicOr(&ring[(w + 2) & kRingMask], hi);
}

// Block-wide exclusive scan of one u32 per thread of e_emit; returns the
// prefix and writes the total.  Contains barriers: every thread must call it.
__device__ __forceinline__ u32 block_scan(u32* scan, u32 v, u32& total) {
  const u32 lane = lane_id(), wave = threadIdx.x >> 6;
  u32 x = v;
  for (u32 off = 1; off < 64; off <<= 1) {
    const u32 y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) scan[wave] = x;
  lds_barrier();
  u32 before = 0;
  total = 0;
  for (u32 w = 0; w < kEmitWaves; ++w) {
    const u32 s = scan[w];
    if (w < wave) before += s;
    total += s;
  }
  lds_barrier();
  return before + x - v;
}

// Code bits of one token (LSB first) and their count.
__device__ __forceinline__ u32 token_bits(const CodeTables& sh, u32 tk, u64& bits) {
  if (!(tk >> 31)) {
    bits = sh.code_ll[tk];
    return sh.len_ll[tk];
  }
  const u32 ml = ((tk >> 16) & 0xff) + 3, md = (tk & 0xffff) + 1;
  u32 ls, lb, lx, ds, db, dx;
  length_code(ml, ls, lb, lx);
  dist_code(md, ds, db, dx);
  u32 n = sh.len_ll[ls];
  bits = sh.code_ll[ls];
  bits |= u64(lx) << n;
  n += lb;
  bits |= u64(sh.code_d[ds]) << n;
  n += sh.len_d[ds];
  bits |= u64(dx) << n;
  return n + db;
}

}  // namespace

// Single-stream chunk and file descriptors.
__global__ void e_single_descs(u64 n, u32 chunk, u32 chunks, u32 hist_max, u64 capacity,
                               ChunkDesc* descs, FileDesc* file) {
  const u64 tid = u64(blockIdx.x) * blockDim.x + threadIdx.x;
  const u64 stride = u64(gridDim.x) * blockDim.x;
  for (u64 c = tid; c < chunks; c += stride) {
    ChunkDesc d;
    d.in_off = c * chunk;
    d.file_off = d.in_off;
    d.file_len = n;
    d.len = u32(min<u64>(chunk, n - min<u64>(n, d.in_off)));
    d.hist = u32(min<u64>(hist_max, d.in_off));
    d.file = 0;
    d.last = c + 1 == chunks;
    descs[c] = d;
  }
  if (!tid) {
    file->in_off = 0;
    file->in_len = n;
    file->out_off = 0;
    file->capacity = capacity;
    file->first_chunk = 0;
    file->chunks = chunks;
  }
}

// LZ77 parse of consecutive chunks per workgroup.  Dynamic LDS: ParseShared
// + window.
//
// A chunk that continues the workgroup's previous chunk in the same file
// keeps the hash table: its entries move down by the window's shift and
// those that leave the window are cleared.  The table then holds exactly
// what hashing every history position into an empty table gives (a bucket
// keeps the largest position that hashed to it), once the positions the
// previous parse never hashed are added: its last three (their four bytes
// reach into this chunk) and those its steps skipped inside matches.
__global__ __launch_bounds__(kParseThreads) __attribute__((amdgpu_waves_per_eu(8))) void e_parse(
    const u8* in, const ChunkDesc* descs, u32 chunks, const u32* runs, u32* tokens,
    ChunkStats* stats) {
  extern __shared__ __align__(16) u8 dyn[];
  ParseShared& sh = *reinterpret_cast<ParseShared*>(dyn);
  u32* win = reinterpret_cast<u32*>(dyn + kParseShared);
  const u32 t = threadIdx.x, lane = lane_id(), wave = t >> 6;
  // This workgroup's run of consecutive chunks: [runs[b], runs[b + 1]), or
  // an equal share of the chunks.
  const u32 per = (chunks + gridDim.x - 1) / gridDim.x;
  const u32 c0 = runs ? runs[blockIdx.x] : blockIdx.x * per;
  const u32 c1 = runs ? runs[blockIdx.x + 1] : min(chunks, c0 + per);
  u64 prev_in = 0, prev_start = 0;  // previous chunk: input offset, window start
  u32 prev_len = 0, prev_file = 0;
  bool have_prev = false;
  ChunkDesc d = c0 < c1 ? descs[c0] : ChunkDesc{};
  for (u32 c = c0; c < c1; ++c) {
    const ChunkDesc nd = c + 1 < c1 ? descs[c + 1] : ChunkDesc{};
    const u32 hist = d.hist, end = d.hist + d.len;
    // This window starts `shift` bytes into the previous one.
    const bool carry = have_prev && hist && d.file == prev_file && d.in_off == prev_in + prev_len;
    const u32 shift = carry ? u32(d.in_off - hist - prev_start) : 0u;
    const u32 prev_skips = sh.nskip;  // read before thread 0 resets it (after a barrier)
    if (carry) {
      for (u32 i = t; i < kBuckets * kWays; i += kParseThreads) {
        const u32 e = sh.table[i];
        sh.table[i] = e > shift ? e - shift : 0u;
      }
    } else {
      for (u32 i = t; i < kBuckets * kWays; i += kParseThreads) sh.table[i] = 0;
    }

    // ---- stage the window as aligned dwords; Adler partials of the chunk ----
    {
      const uintptr_t addr = reinterpret_cast<uintptr_t>(in + d.in_off - hist);
      const u32 a = u32(addr & 3);
      const u32* g = reinterpret_cast<const u32*>(addr - a);
      const u32 nw = (end + 3) / 4;
      u64 s = 0, l = 0;
      // A thread's dwords are loaded kStageBatch at a time, all loads in
      // flight before the first is used (one memory latency per batch; the
      // CU's other parse workgroup runs meanwhile).
      constexpr u32 kStageBatch = 4;
      for (u32 k0 = t; k0 < nw; k0 += kStageBatch * kParseThreads) {
        u32 lo[kStageBatch], hi[kStageBatch];
#pragma unroll
        for (u32 j = 0; j < kStageBatch; ++j) {
          // Source dword k holds window byte 4k; dword k+1 is read only when
          // it holds a window byte, so no dword outside the input is touched.
          const u32 k = k0 + j * kParseThreads;
          lo[j] = k < nw ? g[k] : 0u;
          hi[j] = (k < nw && a && 4 * (k + 1) < a + end) ? g[k + 1] : 0u;
        }
#pragma unroll
        for (u32 j = 0; j < kStageBatch; ++j) {
          const u32 k = k0 + j * kParseThreads;
          if (k >= nw) break;
          u32 v = a ? __builtin_amdgcn_alignbyte(hi[j], lo[j], a) : lo[j];
          if (4 * k + 4 > end) v &= (1u << (8 * (end - 4 * k))) - 1;
          win[k] = v;
          if (4 * k + 4 > hist) {
            // Chunk bytes of this dword (v is zero past the end): byte sum
            // and position-weighted sum by dot products.
            const u32 lo_q = 4 * k;
            const u32 mask = lo_q >= hist ? ~0u : ~0u << (8 * (hist - lo_q));
            const u32 b = v & mask;
            const u32 sum = __builtin_amdgcn_udot4(b, 0x01010101u, 0u, false);
            const u32 wsum = __builtin_amdgcn_udot4(b, 0x03020100u, 0u, false);
            s += sum;
            // (lo_q - hist) may be negative here: bytes before hist are
            // masked out, so the sum over the dword's chunk bytes stays exact
            // mod 2^64.
            l += u64(i64(lo_q) - i64(hist)) * sum + wsum;
          }
        }
      }
      for (u32 k = nw + t; k < nw + 4; k += kParseThreads) win[k] = 0;
      for (u32 off = 32; off; off >>= 1) {
        s += __shfl_down(s, off, 64);
        l += __shfl_down(l, off, 64);
      }
      if (!lane) {
        sh.red_s[wave] = s;
        sh.red_l[wave] = l;
      }
    }
    for (u32 i = t; i < 288; i += kParseThreads) sh.freq_ll[i] = 0;
    if (t < 32) sh.freq_d[t] = 0;
    if (!t) sh.extra_bits = 0;
    lds_barrier();

    // ---- history positions enter the table ----
    if (carry) {
      // The previous chunk's skipped ranges and last three positions.
      // In the previous window's positions; those before `shift` left.
      const u32 n = prev_skips, prev_end = shift + hist;
      for (u32 k = 0; k <= n; ++k) {
        const u32 lo_p = k < n ? sh.skip_lo[k] : (prev_end > 3 ? prev_end - 3 : 0u);
        const u32 hi_p = k < n ? sh.skip_hi[k] : prev_end;
        const u32 lo = max(lo_p, shift) - shift, hi = hi_p > shift ? hi_p - shift : 0u;
        for (u32 q = lo + t; q < hi; q += kParseThreads)
          if (q + 4 <= end) atomicMax(&sh.table[hash4(win_u32(win, q))], q + 1);
      }
    } else {
#pragma unroll 4
      for (u32 base = 0; base < hist; base += kStep) {
        const u32 q = base + t;
        if (q < hist && q + 4 <= end) atomicMax(&sh.table[hash4(win_u32(win, q))], q + 1);
      }
    }
    lds_barrier();
    if (!t) sh.nskip = 0;  // every thread read it before the barrier above

    // ---- parse ----
    u32* tok = tokens + d.in_off;
    u32 ntok = 0, extra = 0;
    // A step's tokens are stored during the next step, once every wave's
    // count is in LDS (no barrier of its own): pend_tok is this lane's token,
    // pend_bal the wave's token lanes, pend_buf the counts' buffer.
    u32 pend_tok = 0, pend_buf = 0, cur_buf = 0;
    u64 pend_bal = 0;
    bool pending = false;
    const auto flush = [&]() {
      // Tokens of the earlier waves and of the step: an inclusive scan of the
      // wave counts over lanes 0-15 (DPP row shifts stay inside one row).
      u32 inc = lane < kParseWaves ? sh.wave_count[pend_buf][lane] : 0u;
      inc += u32(__builtin_amdgcn_update_dpp(0, int(inc), 0x111, 0xf, 0xf, false));
      inc += u32(__builtin_amdgcn_update_dpp(0, int(inc), 0x112, 0xf, 0xf, false));
      inc += u32(__builtin_amdgcn_update_dpp(0, int(inc), 0x114, 0xf, 0xf, false));
      inc += u32(__builtin_amdgcn_update_dpp(0, int(inc), 0x118, 0xf, 0xf, false));
      const u32 w = u32(__builtin_amdgcn_readfirstlane(int(wave)));
      const u32 before = w ? u32(__builtin_amdgcn_readlane(int(inc), int(w - 1))) : 0u;
      if ((pend_bal >> lane) & 1) tok[ntok + before + __popcll(pend_bal & lanemask_lt())] = pend_tok;
      ntok += u32(__builtin_amdgcn_readlane(int(inc), int(kParseWaves - 1)));
    };
    for (u32 p = hist; p < end;) {
      const u32 q = p + t;
      const bool hashable = q + 4 <= end;
      const u32 v = hashable ? win_u32(win, q) : 0u;
      const u32 h = hashable ? hash4(v) : kBuckets + t;  // unique stand-in: never a bucket
      // Nearest earlier position of the wave with the same hash (1..kNear
      // back): the hash shifted up the wave one lane at a time (DPP
      // wave_shr:1; lane 0 receives ~0u, which matches no hash).
      u32 near = 0;
      {
        u32 hk = h;
#pragma unroll
        for (u32 k = 1; k <= kNear; ++k) {
          hk = u32(__builtin_amdgcn_update_dpp(-1, int(hk), 0x138, 0xf, 0xf, false));
          if (!near && hk == h) near = k;
        }
      }
      u32 best_len = 0, best_dist = 0;
      if (hashable) {
        const u32 maxlen = min(258u, end - q);  // >= 4
        static_assert(kWays == 1, "one read holds a bucket");
        const u32 ent[kWays] = {sh.table[h]};
        // Candidates by distance (0: none): the ways, then the near position.
        u32 dist[kWays + 1];
#pragma unroll
        for (u32 k = 0; k < kWays; ++k) {
          const u32 cand = ent[k] - 1;
          dist[k] = ent[k] && cand < q && q - cand <= kMaxDist ? q - cand : 0u;
        }
        dist[kWays] = near;
        // The first dword decides most candidates: fewer than three equal
        // bytes is no match, three is a match of 3; only four equal bytes
        // continue the comparison.  All first dwords are read at once (an
        // absent candidate reads the position itself).
        u32 x0[kWays + 1];
#pragma unroll
        for (u32 k = 0; k <= kWays; ++k) x0[k] = win_u32(win, q - dist[k]) ^ v;
#pragma unroll
        for (u32 k = 0; k <= kWays; ++k) {
          const u32 x = x0[k];
          if (!dist[k] || (x & 0xffffffu)) continue;
          const u32 m = x ? 3u : 4u + match_len(win, q - dist[k] + 4, q + 4, maxlen - 4);
          if (m > best_len || (m == best_len && dist[k] < best_dist)) {
            best_len = m;
            best_dist = dist[k];
          }
        }
      }
      // Lazy rule; f(t) = end of a token starting at t.  The next position's
      // match length comes from the next lane (DPP wave_shl:1); a wave's last
      // lane has no lookahead and takes its match greedily, so the step needs
      // no barrier here.
      const u32 lim = min(kStep, end - p);
      const u32 cur_ml = best_len >= 3 ? best_len : 0u;
      const u32 next_ml = u32(__builtin_amdgcn_update_dpp(0, int(cur_ml), 0x130, 0xf, 0xf, false));
      const u32 L = (cur_ml && next_ml <= cur_ml) ? cur_ml : 0u;
      const u32 f = t + (L ? L : 1u);
      // Token starts = orbit of 0 under f.  Each wave finds, for each of its
      // 64 positions, the first orbit point past the wave (pointer doubling
      // by shuffles; J[k] = f^(2^k) while inside the wave); wave 0 chains the
      // waves' entries; each wave then finds its orbit from its entry.
      const u32 w0 = wave * 64, wend = w0 + 64;
      const u64 matches = __ballot(L != 0);
      u32 J[6];
      u32 x = f;
      if (matches) {
#pragma unroll
        for (u32 k = 0; k < 6; ++k) {
          J[k] = x;
          const u32 y = __shfl(x, int((x - w0) & 63), 64);
          x = x < wend ? y : x;
        }
      } else {
        x = wend;  // all literals: every orbit in the wave leaves it at its end
      }
      sh.exitv[t] = u16(x);
      if (!lane) sh.wave_match[wave] = matches != 0;
      lds_barrier();
      // Every lookup of the step is done: its positions enter the table.
      if (hashable) atomicMax(&sh.table[h], q + 1);
      // The previous step's tokens: waves 1-15 now, while wave 0 chains;
      // wave 0 after the chain.
      if (pending && wave != 0) flush();
      if (wave == 0) {
        // The chain of wave entries, by wave 0 from registers (one wave only:
        // the hops are scalar work, and the scalar unit is shared by the
        // CU): lane l holds the exits of position l of every wave; each hop
        // leaves its wave, so wave w is entered at most once, at iteration w.
        if (!__ballot(lane < kParseWaves && sh.wave_match[lane])) {
          // No match in the step: every wave is entered at its first position.
          if (lane < kParseWaves) sh.went[lane] = u16(lane * 64 < lim ? lane * 64 : 0xffffu);
          if (!lane) sh.adv = (lim + 63) & ~63u;
        } else {
          u32 ex[kParseWaves];
#pragma unroll
          for (u32 w = 0; w < kParseWaves; ++w) ex[w] = sh.exitv[w * 64 + lane];
          u32 e = 0, went = 0xffffu;  // e is uniform; lane w keeps wave w's entry
#pragma unroll
          for (u32 w = 0; w < kParseWaves; ++w) {
            if (e < lim && (e >> 6) == w) {
              went = lane == w ? e : went;
              e = u32(__builtin_amdgcn_readlane(int(ex[w]), int(e & 63)));
            }
          }
          if (lane < kParseWaves) sh.went[lane] = u16(went);
          if (!lane) sh.adv = e;
        }
      }
      lds_barrier();
      if (pending && wave == 0) flush();
      const u32 entry = u32(__builtin_amdgcn_readfirstlane(int(sh.went[wave])));
      const u32 adv = sh.adv;
      // The wave's orbit from its entry.  With few match lanes it is walked
      // over them (a literal's successor is the next lane): every lane from
      // the current point up to the next match lane starts a token, and the
      // walk resumes past that match, in scalar registers.  Otherwise marks
      // are pushed from the entry, 2^k hops in round k.
      u64 starts = 0;
      if (__popcll(matches) > kWalkMatches) {
        sh.mark[t] = t == entry;
        wave_sync();
#pragma unroll
        for (u32 k = 0; k < 6; ++k) {
          if (sh.mark[t] && J[k] < wend) sh.mark[J[k]] = 1;
          wave_sync();
        }
        starts = __ballot(sh.mark[t]);
      } else {
        u32 e = entry == 0xffffu ? 64u : entry - w0;
        while (e < 64) {
          const u64 from = ~0ull << e;
          const u64 m = matches & from;
          if (!m) {
            starts |= from;
            break;
          }
          const u32 s = u32(__builtin_ctzll(m));
          starts |= from & (~0ull >> (63 - s));
          e = s + u32(__builtin_amdgcn_readlane(int(L), int(s)));
        }
      }
      const bool start = t < lim && ((starts >> lane) & 1);
      const u64 bal = __ballot(start);
      if (!lane) sh.wave_count[cur_buf][wave] = __popcll(bal);
      if (start) {
        if (L) {
          u32 ls, lb, lx, ds, db, dx;
          length_code(L, ls, lb, lx);
          dist_code(best_dist, ds, db, dx);
          atomicAdd(&sh.freq_ll[ls], 1u);
          atomicAdd(&sh.freq_d[ds], 1u);
          extra += lb + db;
          pend_tok = 0x80000000u | ((L - 3) << 16) | (best_dist - 1);
        } else {
          const u32 lit = hashable ? (v & 0xff) : win_byte(win, q);
          atomicAdd(&sh.freq_ll[lit], 1u);
          pend_tok = lit;
        }
      }
      pend_bal = bal;
      pend_buf = cur_buf;
      cur_buf ^= 1u;
      pending = true;
      if (!t && adv > lim && p + lim < end && sh.nskip < kMaxSteps) {
        // Positions [p + lim, p + adv) were skipped.
        sh.skip_lo[sh.nskip] = p + lim;
        sh.skip_hi[sh.nskip] = min(p + adv, end);
        ++sh.nskip;
      }
      p += adv;
      // No barrier here: the next step writes exitv before its first
      // barrier, and went, adv, mark and the other count buffer after it;
      // this step read exitv, went and mark before its last barrier, and adv
      // right after it; its counts are read during the next step, before
      // that step's second barrier; its table entries went in before its
      // last barrier, after every lookup of the step.
    }
    lds_barrier();
    if (pending) flush();
    if (extra) atomicAdd(&sh.extra_bits, extra);
    lds_barrier();
    ChunkStats& st = stats[c];
    for (u32 i = t; i < 288; i += kParseThreads) st.freq_ll[i] = sh.freq_ll[i] + (i == 256);
    if (t < 32) st.freq_d[t] = sh.freq_d[t];
    if (!t) {
      st.ntok = ntok;
      st.extra_bits = sh.extra_bits;
      u64 s = 0, l = 0;
      for (u32 w = 0; w < kParseWaves; ++w) {
        s += sh.red_s[w];
        l += sh.red_l[w];
      }
      st.sum_s = s;
      st.sum_l = l;
    }
    prev_in = d.in_off;
    prev_start = d.in_off - hist;
    prev_len = d.len;
    prev_file = d.file;
    have_prev = true;
    d = nd;
    lds_barrier();
  }
}

// Block coding of one chunk per workgroup of two waves (grid-stride): code
// lengths (literal/length tree on wave 0, distance tree on wave 1), the
// code-length RLE and its tree, exact costs and the block type (wave 0),
// canonical codes; the tables go to the chunk's CodeTables.  The trees are
// chains of dependent LDS accesses, so many small workgroups per CU hide
// their latency (about 13 KiB of LDS each).
__global__ __launch_bounds__(kTreeThreads) __attribute__((amdgpu_waves_per_eu(4))) void e_tree(const ChunkDesc* descs, u32 chunks,
                                                       const ChunkStats* stats,
                                                       CodeTables* tables,
                                                       ChunkResult* results) {
  __shared__ TreeShared sh;
  CodeTables& tab = sh.tab;
  const u32 t = threadIdx.x, lane = lane_id(), wave = t >> 6;
  for (u32 c = blockIdx.x; c < chunks; c += gridDim.x) {
    const ChunkDesc d = descs[c];
    const ChunkStats& st = stats[c];
    for (u32 i = t; i < 288; i += kTreeThreads) sh.freq_ll[i] = i < 286 ? st.freq_ll[i] : 0u;
    if (t < 32) sh.freq_d[t] = t < 30 ? st.freq_d[t] : 0u;
    lds_barrier();
    if (wave == 0) huffman_lengths<8>(sh.hs_ll, sh.freq_ll, 286, 15, tab.len_ll);
    else huffman_lengths<1>(sh.hs_d, sh.freq_d, 30, 15, tab.len_d);
    lds_barrier();
    if (wave == 0) {
      tab.hlit = used_extent(tab.len_ll, 286, 257);
      tab.hdist = used_extent(tab.len_d, 30, 1);
      wave_sync();
      rle_lengths_wave(sh);
      huffman_lengths<1>(sh.hs_ll, sh.freq_cl, 19, 7, tab.len_cl);
      u32 dyn_bits = 0, fix_bits = 0, hdr = 0;
      for (u32 sy = lane; sy < 286; sy += 64) {
        dyn_bits += sh.freq_ll[sy] * tab.len_ll[sy];
        fix_bits += sh.freq_ll[sy] * fixed_len(sy);
      }
      if (lane < 30) {
        dyn_bits += sh.freq_d[lane] * tab.len_d[lane];
        fix_bits += sh.freq_d[lane] * 5;
      }
      for (u32 i = lane; i < tab.nrle; i += 64) {
        const u32 sy = tab.rle[i] & 31;
        hdr += tab.len_cl[sy] + (sy == 16 ? 2 : sy == 17 ? 3 : sy == 18 ? 7 : 0);
      }
      for (u32 off = 32; off; off >>= 1) {
        dyn_bits += __shfl_down(dyn_bits, off, 64);
        fix_bits += __shfl_down(fix_bits, off, 64);
        hdr += __shfl_down(hdr, off, 64);
      }
      // HCLEN: one past the last nonzero code-length length in RFC order.
      const u64 cl_used = __ballot(lane < 19 && tab.len_cl[cl_order(lane)] != 0);
      if (!lane) {
        const u32 last = cl_used ? 64 - __builtin_clzll(cl_used) : 0u;
        const u32 hc = last > 4 ? last : 4u;
        tab.hclen = hc;
        hdr += 3 + 14 + 3 * hc;
        const u64 dyn_total = u64(hdr) + dyn_bits + st.extra_bits;
        const u64 fix_total = 3ull + fix_bits + st.extra_bits;
        auto extent = [&](u64 bits) -> u64 {
          return d.last ? (bits + 7) / 8 : (bits + 3 + 7) / 8 + 4;
        };
        const u64 e_stored = u64(d.len) + 5, e_fixed = extent(fix_total), e_dyn = extent(dyn_total);
        // Ties keep stored before fixed before dynamic (the reference's order, E:312-356).
        u32 mode = 0;
        u64 best = e_stored;
        if (e_fixed < best) { mode = 1; best = e_fixed; }
        if (e_dyn < best) { mode = 2; best = e_dyn; }
        tab.mode = mode;
        tab.extent = u32(best);
        tab.hdr_bits = mode == 2 ? hdr : 3u;
        results[c].extent = u32(best);
        results[c].status = 0;
        const u64 S = st.sum_s % kAdlerMod, L = st.sum_l % kAdlerMod;
        results[c].adler_s = S;
        results[c].adler_b =
            (((d.file_len - d.file_off) % kAdlerMod) * S + kAdlerMod - L) % kAdlerMod;
      }
    }
    lds_barrier();
    const u32 mode = tab.mode;
    if (mode == 1) {
      for (u32 i = t; i < 288; i += kTreeThreads) tab.len_ll[i] = u8(fixed_len(i));
      if (t < 30) tab.len_d[t] = 5;
      lds_barrier();
    }
    if (mode) {
      if (wave == 0) {
        canonical_codes_wave(tab.len_ll, mode == 1 ? 288 : 286, tab.code_ll);
      } else {
        canonical_codes_wave(tab.len_d, 30, tab.code_d);
        if (mode == 2) canonical_codes_wave(tab.len_cl, 19, tab.code_cl);
      }
    }
    lds_barrier();
    uint4* dst = reinterpret_cast<uint4*>(tables + c);
    const uint4* src = reinterpret_cast<const uint4*>(&tab);
    for (u32 i = t; i < sizeof(CodeTables) / 16; i += kTreeThreads) dst[i] = src[i];
    lds_barrier();
  }
}

// Bit emission of one chunk per workgroup (grid-stride) with the chunk's
// CodeTables, straight into the chunk's place in the output stream (after
// its file's 2-byte header and the earlier chunks, from the extent scan).
// The bits go through an LDS bit ring (18 KiB of LDS in all, so eight
// workgroups share a CU) that starts at the chunk's byte offset inside an
// aligned 16-byte line: ring line k is output line k.  After each round's
// scan the lines below the round's first bit are complete and are stored
// (whole lines as 16-byte stores, the chunk's partial first and last lines
// byte by byte, so that neighbouring chunks' bytes are never written) and
// cleared for reuse.  A chunk whose bits do not match its extent (an
// internal inconsistency) marks its file failed; nothing is written past
// the extent.
__global__ __launch_bounds__(kEmitThreads) __attribute__((amdgpu_waves_per_eu(8))) void e_emit(
    const u8* in, const ChunkDesc* descs, const FileDesc* files, u32 chunks, const u32* tokens,
    const ChunkStats* stats, const CodeTables* tables, const u64* sums, u8* out,
    u32* file_bad) {
  __shared__ EmitShared es;
  __shared__ __align__(16) u32 stage[kRingWords];
  CodeTables& sh = es.tab;
  const u32 t = threadIdx.x;
  for (u32 c = blockIdx.x; c < chunks; c += gridDim.x) {
    const ChunkDesc d = descs[c];
    const FileDesc f = files[d.file];
    u8* dst = out + f.out_off + 2 + (sums[4 * u64(c)] - sums[4 * u64(f.first_chunk)]);
    {
      const uint4* src = reinterpret_cast<const uint4*>(tables + c);
      uint4* dst4 = reinterpret_cast<uint4*>(&sh);
      for (u32 i = t; i < sizeof(CodeTables) / 16; i += kEmitThreads) dst4[i] = src[i];
      if (!t) es.status = 0;
    }
    lds_barrier();

    // ---- emission ----
    const u32 mode = sh.mode;
    if (mode == 0) {
      if (!t) {
        dst[0] = u8(d.last ? 1 : 0);
        dst[1] = u8(d.len & 0xff);
        dst[2] = u8(d.len >> 8);
        dst[3] = u8(~d.len & 0xff);
        dst[4] = u8((~d.len >> 8) & 0xff);
      }
      const u8* src = in + d.in_off;
      copy_bytes(dst + 5, src, d.len, src + d.len, t, kEmitThreads);
    } else {
      uint4* ring4 = reinterpret_cast<uint4*>(stage);
      for (u32 i = t; i < kRingWords / 4; i += kEmitThreads) ring4[i] = uint4{0u, 0u, 0u, 0u};
      // Output line k is bytes [16k, 16k + 16) from `line0`; the chunk's
      // bytes are [lead, lead + extent) of them.
      const u32 lead = u32(reinterpret_cast<uintptr_t>(dst) & 15);
      u8* line0 = dst - lead;
      const u32 last_byte = lead + sh.extent;
      u32 stored = 0;  // output lines stored and cleared (uniform)
      const auto store_lines = [&](u32 upto) {  // lines [stored, upto) are complete
        for (u32 k = stored + t; k < upto; k += kEmitThreads) {
          uint4& r = ring4[k & (kRingMask / 4)];
          const u32 lo = max(16 * k, lead), hi = min(16 * k + 16, last_byte);
          if (lo == 16 * k && hi == 16 * k + 16) {
            *reinterpret_cast<uint4*>(line0 + 16 * k) = r;
          } else {
            for (u32 b = lo; b < hi; ++b) {
              const u32 q = (b >> 2) & 3;
              const u32 word = q == 0 ? r.x : q == 1 ? r.y : q == 2 ? r.z : r.w;
              line0[b] = u8(word >> (8 * (b & 3)));
            }
          }
          r = uint4{0u, 0u, 0u, 0u};
        }
        if (upto > stored) stored = upto;
      };
      lds_barrier();
      // Header: the fixed fields by thread 0 (before the scan's barriers),
      // then the code-length RLE symbols, two per thread, placed by a scan.
      const u32 nrle = mode == 2 ? sh.nrle : 0u;
      const u32 fixed_bits = mode == 2 ? 17 + 3 * sh.hclen : 3u;
      const u32 bit0 = 8 * lead;
      if (!t) {
        StageWriter out = {stage, bit0};
        out.put(d.last ? 1u : 0u, 1);
        out.put(mode == 1 ? 1u : 2u, 2);
        if (mode == 2) {
          out.put(sh.hlit - 257, 5);
          out.put(sh.hdist - 1, 5);
          out.put(sh.hclen - 4, 4);
          for (u32 i = 0; i < sh.hclen; ++i) out.put(sh.len_cl[cl_order(i)], 3);
        }
      }
      u64 hb[2];
      u32 hn[2], hmine = 0;
#pragma unroll
      for (u32 k = 0; k < 2; ++k) {
        const u32 i = 2 * t + k;
        hn[k] = 0;
        hb[k] = 0;
        if (i < nrle) {
          const u32 sy = sh.rle[i] & 31, x = sh.rle[i] >> 5;
          const u32 cl = sh.len_cl[sy];
          hb[k] = u64(sh.code_cl[sy]) | (u64(x) << cl);
          hn[k] = cl + (sy == 16 ? 2u : sy == 17 ? 3u : sy == 18 ? 7u : 0u);
        }
        hmine += hn[k];
      }
      u32 htotal;
      u32 hoff = bit0 + fixed_bits + block_scan(es.scan, hmine, htotal);
#pragma unroll
      for (u32 k = 0; k < 2; ++k) {
        if (hn[k]) or_bits(stage, hoff, hb[k]);
        hoff += hn[k];
      }
      if (!t && fixed_bits + htotal != sh.hdr_bits) es.status = kCompressionOverflow;
      lds_barrier();
      const u32* tok = tokens + d.in_off;
      const u32 ntokens = stats[c].ntok;
      u32 pos = bit0 + sh.hdr_bits;
      // The tokens of the next round are loaded (one 16-byte load per
      // thread) while the current round is coded, so the global-memory
      // latency overlaps the scan's barriers.
      static_assert(kTokensPerThread == 4, "one uint4 of tokens per thread and round");
      constexpr u32 kRound = kEmitThreads * kTokensPerThread;
      // (A batch file's chunk may start at any byte, so its token list is
      // only 4-byte aligned: then the four tokens load one by one.)
      const bool aligned16 = (reinterpret_cast<uintptr_t>(tok) & 15) == 0;
      const auto load4 = [&](u32 first) -> uint4 {
        if (aligned16 && first + 4 <= ntokens) return *reinterpret_cast<const uint4*>(tok + first);
        uint4 r = {0u, 0u, 0u, 0u};
        if (first < ntokens) r.x = tok[first];
        if (first + 1 < ntokens) r.y = tok[first + 1];
        if (first + 2 < ntokens) r.z = tok[first + 2];
        if (first + 3 < ntokens) r.w = tok[first + 3];
        return r;
      };
      uint4 next = load4(t * kTokensPerThread);
      for (u32 base = 0; base < ntokens; base += kRound) {
        const u32 first = base + t * kTokensPerThread;
        const uint4 cur = next;
        next = load4(first + kRound);
        const u32 tk[4] = {cur.x, cur.y, cur.z, cur.w};
        u64 bits[kTokensPerThread];
        u32 nbits[kTokensPerThread];
        u32 mine = 0;
#pragma unroll
        for (u32 k = 0; k < kTokensPerThread; ++k) {
          nbits[k] = first + k < ntokens ? token_bits(sh, tk[k], bits[k]) : 0u;
          mine += nbits[k];
        }
        u32 total;
        u32 off = pos + block_scan(es.scan, mine, total);
        // Every earlier round's bits are in the ring (the scan's barriers).
        store_lines(min(pos / 128, last_byte / 16));
#pragma unroll
        for (u32 k = 0; k < kTokensPerThread; ++k) {
          if (nbits[k]) or_bits(stage, off, bits[k]);
          off += nbits[k];
        }
        pos += total;
      }
      lds_barrier();
      if (!t) {
        StageWriter out = {stage, pos};
        out.put(sh.code_ll[256], sh.len_ll[256]);
        if (!d.last) {
          out.put(0, 3);
          if (out.pos & 7) out.pos += 8 - (out.pos & 7);
          out.put(0, 16);
          out.put(0xffff, 16);
        }
        const u32 bytes = (out.pos + 7) / 8 - lead;
        if (bytes != sh.extent) es.status = kCompressionOverflow;
      }
      lds_barrier();
      store_lines((last_byte + 15) / 16);
      if (!t && es.status) atomicOr(&file_bad[d.file], 1u);
    }
    lds_barrier();
  }
}

// One workgroup: exclusive scans of chunk extents, Adler partial sums and
// failed-chunk counts; sums[4 * i + k] holds the prefix before chunk i.
// Also clears the files' failure flags, which e_emit sets.
__global__ __launch_bounds__(1024) void e_scan(const ChunkResult* results, u32 chunks, u64* sums,
                                               u32* file_bad, u32 file_count) {
  __shared__ u64 part[4][1024];
  const u32 t = threadIdx.x;
  for (u32 fi = t; fi < file_count; fi += 1024) file_bad[fi] = 0;
  const u64 per = (u64(chunks) + 1023) / 1024;
  const u64 lo = min<u64>(chunks, t * per), hi = min<u64>(chunks, lo + per);
  u64 acc[4] = {0, 0, 0, 0};
  for (u64 i = lo; i < hi; ++i) {
    acc[0] += results[i].extent;
    acc[1] += results[i].adler_s;
    acc[2] += results[i].adler_b;
    acc[3] += results[i].status != 0;
  }
  for (u32 k = 0; k < 4; ++k) part[k][t] = acc[k];
  __syncthreads();
  for (u32 off = 1; off < 1024; off <<= 1) {
    u64 x[4];
    for (u32 k = 0; k < 4; ++k) x[k] = t >= off ? part[k][t - off] : 0;
    __syncthreads();
    for (u32 k = 0; k < 4; ++k) part[k][t] += x[k];
    __syncthreads();
  }
  u64 run[4];
  for (u32 k = 0; k < 4; ++k) run[k] = part[k][t] - acc[k];
  for (u64 i = lo; i < hi; ++i) {
    for (u32 k = 0; k < 4; ++k) sums[4 * i + k] = run[k];
    run[0] += results[i].extent;
    run[1] += results[i].adler_s;
    run[2] += results[i].adler_b;
    run[3] += results[i].status != 0;
  }
  if (t == 1023)
    for (u32 k = 0; k < 4; ++k) sums[4 * u64(chunks) + k] = run[k];
}

// Per file: status, wrapper and metadata [length, status].
// Zeroes out[from, capacity) with every thread of the grid: bytes up to the
// first 16-byte boundary of memory at or after out + from and after the last
// one before out + capacity one by one, 16-byte stores between (out may have
// any alignment).
__device__ void zero_tail(u8* out, u64 capacity, u64 from) {
  from = min<u64>(from, capacity);
  const uintptr_t base = reinterpret_cast<uintptr_t>(out);
  const u64 first16 = from + ((16 - ((base + from) & 15)) & 15);
  const u64 end16 = capacity - ((base + capacity) & 15);
  const u64 tid = u64(blockIdx.x) * blockDim.x + threadIdx.x, stride = u64(gridDim.x) * blockDim.x;
  if (first16 >= end16) {
    for (u64 i = from + tid; i < capacity; i += stride) out[i] = 0;
    return;
  }
  for (u64 i = from + tid; i < first16; i += stride) out[i] = 0;
  for (u64 i = end16 + tid; i < capacity; i += stride) out[i] = 0;
  uint4* o = reinterpret_cast<uint4*>(out + first16);
  const u64 n16 = (end16 - first16) / 16;
  for (u64 i = tid; i < n16; i += stride) o[i] = uint4{0u, 0u, 0u, 0u};
}


// File fi's status and stream length (total) from the chunk scans.
__device__ __forceinline__ u32 wrap_status(const FileDesc& f, u32 fi, const u64* sums,
                                           const u32* file_bad, u64& total) {
  const u64 a0 = f.first_chunk, a1 = f.first_chunk + f.chunks;
  u32 status = sums[4 * a1 + 3] != sums[4 * a0 + 3] || file_bad[fi] ? kCompressionOverflow : 0u;
  total = sums[4 * a1] - sums[4 * a0] + 6;
  if (total > f.capacity) status = kCompressionOverflow;
  return status;
}

// The zlib header and Adler-32 trailer of every file, its metadata row and
// its ok flag.  With `tail` (a single stream, count 1), the whole grid also
// zeroes the slot after the stream, [total, tail), or all of it when the
// stream failed.
__global__ void e_wrap(const FileDesc* files, u32 count, const u64* sums, u8* out, u32* meta,
                       u32* file_ok, const u32* file_bad, u64 tail) {
  const u32 tid = blockIdx.x * blockDim.x + threadIdx.x;
  if (tail) {
    u64 total = 0;
    const u32 status = wrap_status(files[0], 0, sums, file_bad, total);
    zero_tail(out, tail, status ? 0 : total);
  }
  for (u32 fi = tid; fi < count; fi += gridDim.x * blockDim.x) {
    const FileDesc f = files[fi];
    const u64 a0 = f.first_chunk, a1 = f.first_chunk + f.chunks;
    u64 total = 0;
    const u32 status = wrap_status(f, fi, sums, file_bad, total);
    file_ok[fi] = status ? 0u : 1u;
    if (status) {
      meta[2 * u64(fi)] = 0;
      meta[2 * u64(fi) + 1] = status;
      continue;
    }
    const u64 S = (sums[4 * a1 + 1] - sums[4 * a0 + 1]) % kAdlerMod;
    const u64 B = (sums[4 * a1 + 2] - sums[4 * a0 + 2] + f.in_len) % kAdlerMod;
    const u32 adler = u32((B << 16) | ((S + 1) % kAdlerMod));
    u8* o = out + f.out_off;
    o[0] = 0x78;
    o[1] = 0x01;
    o[total - 4] = u8(adler >> 24);
    o[total - 3] = u8(adler >> 16);
    o[total - 2] = u8(adler >> 8);
    o[total - 1] = u8(adler);
    meta[2 * u64(fi)] = u32(total);
    meta[2 * u64(fi) + 1] = 0;
  }
}

// Zeroes the output slot of every failed file of a batch (e_emit has already
// written its chunks); one workgroup per file, grid-stride.
__global__ __launch_bounds__(256) void e_clear_failed(const FileDesc* files, u32 count,
                                                      const u32* file_ok, u8* out) {
  for (u32 fi = blockIdx.x; fi < count; fi += gridDim.x) {
    if (file_ok[fi]) continue;
    const FileDesc f = files[fi];
    for (u64 i = threadIdx.x; i < f.capacity; i += blockDim.x) out[f.out_off + i] = 0;
  }
}

namespace {

#define HZ_TRY(expr)                 \
  do {                               \
    hipError_t _e = (expr);          \
    if (_e != hipSuccess) return _e; \
  } while (0)


// Scratch of one encode call.  Every buffer is carved before the first
// launch, so that a call which cannot get its scratch enqueues nothing.
struct ChunkBuffers {
  ChunkDesc* descs = nullptr;
  u32* runs = nullptr;  // optional: e_parse workgroup b takes chunks [runs[b], runs[b + 1])
  u32 run_count = 0;    // workgroups (runs) that `runs` describes
  FileDesc* files = nullptr;
  u32* tokens = nullptr;
  ChunkStats* stats = nullptr;
  CodeTables* tables = nullptr;
  ChunkResult* results = nullptr;
  u64* sums = nullptr;
  u32* file_ok = nullptr;
  u32* file_bad = nullptr;
};

hipError_t alloc_chunks(Scratch& scratch, u64 chunks, u32 file_count, u64 in_total,
                        ChunkBuffers& b) {
  HZ_TRY(scratch.alloc(&b.descs, chunks));
  HZ_TRY(scratch.alloc(&b.files, file_count));
  HZ_TRY(scratch.alloc(&b.tokens, in_total ? in_total : 1));
  HZ_TRY(scratch.alloc(&b.stats, chunks));
  HZ_TRY(scratch.alloc(&b.tables, chunks));
  HZ_TRY(scratch.alloc(&b.results, chunks));
  HZ_TRY(scratch.alloc(&b.sums, 4 * (chunks + 1)));
  HZ_TRY(scratch.alloc(&b.file_ok, file_count));
  HZ_TRY(scratch.alloc(&b.file_bad, file_count));
  return hipSuccess;
}

// Parse workgroups for `chunks` chunks: one or two per CU (as many as their
// LDS allows), each taking a run of consecutive chunks.  Batches launch
// kBatchParseRuns times as many shorter runs, so that workgroups that finish
// early take further runs.
constexpr u64 kBatchParseRuns = 2;
hipError_t parse_grid_size(u64 chunks, u32 chunk_bytes, u32* grid) {
  int device = 0, cus = 0;
  HZ_TRY(hipGetDevice(&device));
  HZ_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
  const u64 per_cu = kLdsBudget / parse_budget(chunk_bytes);
  *grid = u32(std::min<u64>(chunks, per_cu * u64(cus > 0 ? cus : 1)));
  return hipSuccess;
}

hipError_t run_chunks(hipStream_t stream, const ChunkBuffers& b, const u8* in, u64 chunks,
                      u32 file_count, u8* out, u32 chunk_bytes, u32* meta, bool clear_failed,
                      u64 tail = 0) {
  const u32 parse_lds = kParseShared + history_limit(chunk_bytes) + chunk_bytes + 32;

  HZ_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(e_parse),
                             hipFuncAttributeMaxDynamicSharedMemorySize, int(parse_lds)));
  const u32 grid = u32(chunks < 65536 ? chunks : 65536);
  u32 parse_grid = 0;
  HZ_TRY(parse_grid_size(chunks, chunk_bytes, &parse_grid));
  if (b.runs) parse_grid = b.run_count;
  HZ_LAUNCH(e_parse, dim3(parse_grid), dim3(kParseThreads), parse_lds, stream, in, b.descs,
            u32(chunks), b.runs, b.tokens, b.stats);
  HZ_TRY(hipGetLastError());
  HZ_LAUNCH(e_tree, dim3(grid), dim3(kTreeThreads), 0, stream, b.descs, u32(chunks), b.stats,
            b.tables, b.results);
  HZ_TRY(hipGetLastError());
  // The extents are known from the trees: their scan places every chunk
  // before any is emitted.
  HZ_LAUNCH(e_scan, dim3(1), dim3(1024), 0, stream, b.results, u32(chunks), b.sums, b.file_bad,
            file_count);
  HZ_TRY(hipGetLastError());
  HZ_LAUNCH(e_emit, dim3(grid), dim3(kEmitThreads), 0, stream, in, b.descs, b.files, u32(chunks),
            b.tokens, b.stats, b.tables, b.sums, out, b.file_bad);
  HZ_TRY(hipGetLastError());
  // A single stream's slot after the stream is zeroed by the same launch.
  const u32 wrap_grid = tail ? u32(std::min<u64>(1024, (tail / 16 + 255) / 256 + 1))
                             : (file_count + 255) / 256;
  HZ_LAUNCH(e_wrap, dim3(wrap_grid), dim3(256), 0, stream, b.files, file_count, b.sums, out, meta,
            b.file_ok, b.file_bad, tail);
  HZ_TRY(hipGetLastError());
  if (clear_failed) {
    HZ_LAUNCH(e_clear_failed, dim3(std::min<u32>(file_count, 65536)), dim3(256), 0, stream,
              b.files, file_count, b.file_ok, out);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t run_deflate(hipStream_t stream, Scratch& scratch, const u8* in, u64 in_size, u8* out,
                       u64 capacity, u32 chunk_bytes, u32* meta, bool independent) {
  const u64 chunks = in_size ? (in_size + chunk_bytes - 1) / chunk_bytes : 1;
  ChunkBuffers b;
  HZ_TRY(alloc_chunks(scratch, chunks, 1, in_size, b));
  HZ_LAUNCH(e_single_descs, dim3(u32(std::min<u64>(1024, (chunks + 255) / 256))), dim3(256), 0,
            stream, in_size, chunk_bytes, u32(chunks), independent ? 0u : history_limit(chunk_bytes),
            capacity, b.descs, b.files);
  HZ_TRY(hipGetLastError());
  return run_chunks(stream, b, in, chunks, 1, out, chunk_bytes, meta, false, capacity);
}

u64 deflate_scratch_bytes(u64 in_size, u32 chunk_bytes) {
  struct Sizing final : Scratch {
    u64 total = 0;
    hipError_t alloc_bytes(void** p, u64 bytes) override {
      *p = nullptr;
      total += scratch_round(bytes);
      return hipSuccess;
    }
  } sizing;
  const u64 chunks = in_size ? (in_size + chunk_bytes - 1) / chunk_bytes : 1;
  ChunkBuffers b;
  (void)alloc_chunks(sizing, chunks, 1, in_size, b);
  return sizing.total;
}

hipError_t run_deflate_batch(hipStream_t stream, Scratch& scratch, const u8* in, u64 in_total,
                             const BatchFile* files_host, u32 count, u8* out, u64 out_total,
                             u32 chunk_bytes, u32* meta) {
  (void)out_total;
  std::vector<ChunkDesc> descs;
  std::vector<FileDesc> files(count);
  const u32 hist_max = history_limit(chunk_bytes);
  for (u32 f = 0; f < count; ++f) {
    const BatchFile& bf = files_host[f];
    const u64 n = bf.in_size;
    const u64 k = n ? (n + chunk_bytes - 1) / chunk_bytes : 1;
    files[f] = {bf.in_offset, n, bf.out_offset, bf.out_size, u32(descs.size()), u32(k)};
    for (u64 j = 0; j < k; ++j) {
      ChunkDesc d;
      d.in_off = bf.in_offset + j * chunk_bytes;
      d.file_off = j * chunk_bytes;
      d.file_len = n;
      d.len = u32(std::min<u64>(chunk_bytes, n - std::min<u64>(n, j * chunk_bytes)));
      d.hist = u32(std::min<u64>(hist_max, j * chunk_bytes));
      d.file = f;
      d.last = j + 1 == k;
      descs.push_back(d);
    }
  }
  ChunkBuffers b;
  HZ_TRY(alloc_chunks(scratch, descs.size(), count, in_total, b));
  // Parse runs of about equal work (bytes plus a fixed cost per chunk) rather
  // than of equal chunk counts: a batch's chunks range from a few bytes to a
  // full chunk, and a run that collects many full chunks would finish last.
  u32 parse_grid = 0;
  HZ_TRY(parse_grid_size(descs.size(), chunk_bytes, &parse_grid));
  parse_grid = u32(std::min<u64>(descs.size(), u64(parse_grid) * kBatchParseRuns));
  constexpr u64 kChunkCost = 4096;
  std::vector<u32> runs(u64(parse_grid) + 1, u32(descs.size()));
  u64 work = 0, done = 0;
  for (const ChunkDesc& d : descs) work += d.len + kChunkCost;
  runs[0] = 0;
  u32 next = 1;
  for (u64 c = 0; c < descs.size(); ++c) {
    done += descs[c].len + kChunkCost;
    while (next < parse_grid && done * parse_grid >= work * next) runs[next++] = u32(c + 1);
  }
  HZ_TRY(scratch.alloc(&b.runs, runs.size()));
  b.run_count = parse_grid;
  HZ_TRY(upload_to_device(stream, b.runs, runs.data(), runs.size() * sizeof(u32)));
  HZ_TRY(upload_to_device(stream, b.descs, descs.data(), descs.size() * sizeof(ChunkDesc)));
  HZ_TRY(upload_to_device(stream, b.files, files.data(), count * sizeof(FileDesc)));
  return run_chunks(stream, b, in, descs.size(), count, out, chunk_bytes, meta, true);
}

}  // namespace hz
