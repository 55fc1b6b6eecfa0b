/* CPU oracle for the zlib/DEFLATE codec -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference codec's decode semantics, used by the
 * tests, smoke() and bench.py's cpu_baseline leg to check results against.
 * Nothing in the product links or calls this file.
 *
 * What it restates (reference file:line, paths under src/cuda_zlib/):
 *   - zlib framing and its precedence: native/codec_ffi.cu:304-329, _codec.py:97-112
 *   - canonical Huffman build/decode incl. error rules: _decode_kernels.py:135-232
 *   - dynamic/fixed table construction: _decode_kernels.py:240-296
 *   - serial small-stream route (stream-order statuses, partial output):
 *     native/batch_decode.cuh:123-296 (DecodeOneFile)
 *   - general route: candidate discovery count (_decode_kernels.py:998-1140),
 *     exact chain walk (select_chain, _decode_kernels.py:1226-1408), emission
 *     history/window checks (parse_block<Emit>, 683-781), verification
 *     (native/codec_ffi.cu:344-360, 467-483)
 *   - route selection and bounds: native/codec_ffi.cu:662-707
 *   - Adler-32 (RFC 1950 s.9; zlib.adler32 is the closed-form check)
 *
 * Pinned by tests/test_oracle.py against zlib.decompress / zlib.adler32, the
 * status-pinned fixtures of the reference's tests (rewritten in
 * tests/deflate_writer.py), libdeflate, and brute force on tiny codes.
 * Known approximation: the reference walks long fixed-Huffman regions through
 * 2048-byte tile summaries; here every non-initial fixed block is parsed with
 * the remaining output as its bound.  Success results are identical; only the
 * precedence between an overflow and a later error inside one fixed region can
 * differ (no reference fixture covers it).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef uint8_t u8;
typedef uint16_t u16;
typedef uint32_t u32;
typedef uint64_t u64;

#define MAX_BYTES 0xffffffffull
#define MAX_CANDIDATES 262144u
#define MAX_BLOCKS 262144u

enum {
  ST_OK = 0, ST_TRUNC = 1, ST_RESERVED = 2, ST_TREE = 3, ST_SYMBOL = 4, ST_REPEAT = 5,
  ST_DISTANCE = 6, ST_OVERFLOW = 7, ST_BLOCKS = 9, ST_UNDISCOVERED = 10, ST_SIZE = 11,
  ST_EXTENT = 12, ST_ZTRUNC = 14, ST_HEADER = 15, ST_GZIP = 16, ST_DICT = 17,
  ST_CANDIDATES = 18, ST_ADLER = 21, ST_BOUNDS = 23
};

/* ---- bits: LSB-first reader over [data, data + bytes) ---------------------- */
typedef struct {
  const u8* data;
  u64 total; /* bits */
  u64 pos;
} Bits;

static u64 avail(const Bits* b) { return b->pos <= b->total ? b->total - b->pos : 0; }

/* Bits [pos, pos + 57) as a word; bytes past the range read as zero. */
static u64 peek_word(const Bits* b) {
  const u64 byte = b->pos >> 3, nbytes = (b->total + 7) >> 3;
  u64 v = 0;
  if (byte + 8 <= nbytes) {
    memcpy(&v, b->data + byte, 8);
  } else {
    for (u64 i = 0; byte + i < nbytes && i < 8; ++i) v |= (u64)b->data[byte + i] << (8 * i);
  }
  return v >> (b->pos & 7);
}

/* take(n), n <= 32: 0 on truncation (the reference's sticky error 1). */
static int take(Bits* b, unsigned n, u32* v) {
  if ((u64)n > avail(b)) return 0;
  *v = n ? (u32)(peek_word(b) & ((1ull << n) - 1)) : 0;
  b->pos += n;
  return 1;
}

/* ---- canonical Huffman (RFC 1951 3.2.2) ------------------------------------ */
typedef struct {
  u16 count[16];
  u16 symbol[288];
  unsigned maximum;
} Huff;

static unsigned huff_build(Huff* h, const u8* lens, unsigned n, int empty_ok, int single_ok,
                           unsigned limit) {
  memset(h->count, 0, sizeof h->count);
  h->maximum = 0;
  for (unsigned i = 0; i < n; ++i) {
    if (lens[i] > limit) return ST_TREE;
    h->count[lens[i]]++;
    if (lens[i] > h->maximum) h->maximum = lens[i];
  }
  if (!h->maximum) return empty_ok ? ST_OK : ST_TREE;
  int left = 1;
  for (unsigned l = 1; l <= limit; ++l) {
    left = (left << 1) - h->count[l];
    if (left < 0) return ST_TREE;
  }
  if (left && !(single_ok && h->maximum == 1 && h->count[1] == 1)) return ST_TREE;
  u16 offs[16];
  offs[1] = 0;
  for (unsigned l = 1; l < 15; ++l) offs[l + 1] = offs[l] + h->count[l];
  for (unsigned i = 0; i < n; ++i)
    if (lens[i]) h->symbol[offs[lens[i]]++] = (u16)i;
  return ST_OK;
}

/* Canonical bit-serial decode: truncation -> 1, no code within maximum -> 4. */
static int huff_decode(Bits* b, const Huff* h, unsigned* err) {
  const u64 bits = peek_word(b), left = avail(b);
  u32 code = 0, first = 0, index = 0;
  for (unsigned len = 1; len <= h->maximum; ++len) {
    if (len > left) { *err = ST_TRUNC; return -1; }
    code |= (u32)(bits >> (len - 1)) & 1u;
    u32 count = h->count[len];
    if (code < first + count) {
      b->pos += len;
      return h->symbol[index + code - first];
    }
    index += count;
    first = (first + count) << 1;
    code <<= 1;
  }
  *err = ST_SYMBOL;
  return -1;
}

typedef struct {
  Huff ll, dd, cl;
} Tables;

static unsigned fixed_tables(Tables* t) {
  u8 lens[288];
  for (unsigned i = 0; i < 288; ++i) lens[i] = i < 144 ? 8 : i < 256 ? 9 : i < 280 ? 7 : 8;
  unsigned err = huff_build(&t->ll, lens, 288, 0, 1, 15);
  if (err) return err;
  for (unsigned i = 0; i < 32; ++i) lens[i] = 5;
  return huff_build(&t->dd, lens, 32, 0, 1, 15);
}

static unsigned dynamic_tables(Bits* b, Tables* t) {
  static const u8 order[19] = {16, 17, 18, 0, 8, 7, 9, 6, 10, 5, 11, 4, 12, 3, 13, 2, 14, 1, 15};
  u32 hlit, hdist, hclen;
  if (!take(b, 5, &hlit) || !take(b, 5, &hdist) || !take(b, 4, &hclen)) return ST_TRUNC;
  unsigned nl = hlit + 257, nd = hdist + 1, nc = hclen + 4;
  if (nl > 286) return ST_TREE;
  u8 clens[19] = {0};
  for (unsigned i = 0; i < nc; ++i) {
    u32 v;
    if (!take(b, 3, &v)) return ST_TRUNC;
    clens[order[i]] = (u8)v;
  }
  unsigned err = huff_build(&t->cl, clens, 19, 0, 0, 7);
  if (err) return err;
  u8 lens[320];
  unsigned i = 0;
  while (i < nl + nd) {
    int sym = huff_decode(b, &t->cl, &err);
    if (sym < 0) return err;
    if (sym < 16) { lens[i++] = (u8)sym; continue; }
    u32 repeat, value, x;
    if (sym == 16) {
      if (!i) return ST_REPEAT;
      if (!take(b, 2, &x)) return ST_TRUNC;
      repeat = x + 3;
      value = lens[i - 1];
    } else if (sym == 17) {
      if (!take(b, 3, &x)) return ST_TRUNC;
      repeat = x + 3;
      value = 0;
    } else {
      if (!take(b, 7, &x)) return ST_TRUNC;
      repeat = x + 11;
      value = 0;
    }
    if (repeat > nl + nd - i) return ST_REPEAT;
    for (u32 j = 0; j < repeat; ++j) lens[i++] = (u8)value;
  }
  if (!lens[256]) return ST_TREE;
  err = huff_build(&t->ll, lens, nl, 0, 1, 15);
  if (err) return err;
  return huff_build(&t->dd, lens + nl, nd, 1, 1, 15);
}

/* RFC 1951 3.2.5 tables. */
static const u16 LBASE[29] = {3,  4,  5,  6,  7,  8,  9,  10, 11,  13,  15,  17,  19,  23, 27,
                              31, 35, 43, 51, 59, 67, 83, 99, 115, 131, 163, 195, 227, 258};
static const u8 LEXTRA[29] = {0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 2, 2, 2,
                              2, 3, 3, 3, 3, 4, 4, 4, 4, 5, 5, 5, 5, 0};
static const u16 DBASE[30] = {1,   2,   3,   4,   5,   7,    9,    13,   17,   25,
                              33,  49,  65,  97,  129, 193,  257,  385,  513,  769,
                              1025, 1537, 2049, 3073, 4097, 6145, 8193, 12289, 16385, 24577};
static const u8 DEXTRA[30] = {0, 0, 0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 5, 5, 6,
                              6, 7, 7, 8, 8, 9, 9, 10, 10, 11, 11, 12, 12, 13, 13};

/* One token.  Returns status; *length 0 = EOB, *distance 0 = literal.
 * Check order follows the reference's fixed_token (_decode_kernels.py:393-420). */
static unsigned token(Bits* b, Tables* t, u32 window, u32* lit, u32* length, u32* distance) {
  unsigned err = 0;
  *length = 0;
  *distance = 0;
  int sym = huff_decode(b, &t->ll, &err);
  if (sym < 0) return err;
  if (sym < 256) { *lit = (u32)sym; *length = 1; return ST_OK; }
  if (sym == 256) return ST_OK;
  if (sym > 285) return ST_SYMBOL;
  u32 x;
  if (!take(b, LEXTRA[sym - 257], &x)) return ST_TRUNC;
  *length = LBASE[sym - 257] + x;
  int ds = huff_decode(b, &t->dd, &err);
  if (ds < 0) return err;
  if (ds > 29) return ST_SYMBOL;
  if (!take(b, DEXTRA[ds], &x)) return ST_TRUNC;
  *distance = DBASE[ds] + x;
  if (*distance > window) return ST_DISTANCE;
  return ST_OK;
}

uint32_t oracle_adler32(const uint8_t* data, uint64_t n) {
  u64 a = 1, b = 0;
  while (n) {
    u64 chunk = n < 5552 ? n : 5552; /* largest run without u32 overflow in zlib's form */
    n -= chunk;
    while (chunk--) {
      a += *data++;
      b += a;
    }
    a %= 65521;
    b %= 65521;
  }
  return (u32)((b << 16) | a);
}

static unsigned framing(const u8* in, u64 size, u32* window, u32* wanted) {
  *window = 0;
  *wanted = 0;
  if (size < 8) return ST_ZTRUNC;
  u32 cmf = in[0], flg = in[1];
  if (cmf == 0x1f && flg == 0x8b) return ST_GZIP;
  if ((cmf & 15) != 8 || (cmf >> 4) > 7 || (cmf * 256 + flg) % 31) return ST_HEADER;
  if (flg & 32) return ST_DICT;
  *window = 1u << ((cmf >> 4) + 8);
  *wanted = ((u32)in[size - 4] << 24) | ((u32)in[size - 3] << 16) | ((u32)in[size - 2] << 8) |
            in[size - 1];
  return ST_OK;
}

/* ---- serial route: native/batch_decode.cuh:123-296 ------------------------- */
uint32_t oracle_inflate_serial(const uint8_t* in, uint64_t in_size, uint8_t* out,
                               uint64_t out_size, uint32_t max_blocks) {
  if (in_size > MAX_BYTES || out_size > MAX_BYTES || !max_blocks || max_blocks > MAX_BLOCKS)
    return ST_BOUNDS;
  memset(out, 0, out_size);
  u32 window, wanted;
  unsigned st = framing(in, in_size, &window, &wanted);
  if (st) return st;
  const u64 body = in_size - 6;
  Bits b = {in + 2, body * 8, 0};
  Tables t;
  u64 produced = 0;
  u32 blocks = 0;
  for (;;) {
    if (blocks >= max_blocks) return ST_BLOCKS;
    ++blocks;
    u32 final, type;
    if (!take(&b, 1, &final) || !take(&b, 2, &type)) return ST_TRUNC;
    if (type == 3) return ST_RESERVED;
    if (type == 0) {
      b.pos = (b.pos + 7) & ~(u64)7;
      u32 n, comp;
      if (!take(&b, 16, &n) || !take(&b, 16, &comp)) return ST_TRUNC;
      if ((n ^ comp) != 0xffffu) return ST_SYMBOL;
      if (n > out_size - produced) return ST_OVERFLOW;
      if ((u64)n * 8 > avail(&b)) return ST_TRUNC;
      memcpy(out + produced, in + 2 + (b.pos >> 3), n);
      produced += n;
      b.pos += (u64)n * 8;
    } else {
      st = type == 1 ? fixed_tables(&t) : dynamic_tables(&b, &t);
      if (st) return st;
      for (;;) {
        u32 lit = 0, length, distance;
        st = token(&b, &t, window, &lit, &length, &distance);
        if (st) return st;
        if (!length) break;
        if (length > out_size - produced) return ST_OVERFLOW;
        if (!distance) { out[produced++] = (u8)lit; continue; }
        if (distance > produced) return ST_DISTANCE;
        for (u32 j = 0; j < length; ++j) out[produced + j] = out[produced + j - distance];
        produced += length;
      }
    }
    if (final) break;
  }
  if (produced != out_size) return ST_SIZE;
  if ((b.pos + 7) / 8 != body) return ST_EXTENT;
  if (oracle_adler32(out, out_size) != wanted) return ST_ADLER;
  return ST_OK;
}

/* ---- general route ---------------------------------------------------------- */

/* A valid dynamic header at bit `start` (BTYPE == 2 and a table build that
 * succeeds): the reference's dynamic_prefix_window + dynamic_valid. */
static int dynamic_candidate(const u8* body, u64 len, u64 start) {
  Bits b = {body, len * 8, start + 1};
  u32 type;
  if (!take(&b, 2, &type) || type != 2) return 0;
  Tables t;
  return dynamic_tables(&b, &t) == ST_OK;
}

/* Stored-block endpoint seeds announcing a following fixed block
 * (_decode_kernels.py:1019-1038): one per detection, duplicates included. */
static int stored_seed(const u8* body, u64 len, u64 byte) {
  if (!byte || len - byte < 5) return 0;
  u32 n = body[byte] | ((u32)body[byte + 1] << 8);
  u32 comp = body[byte + 2] | ((u32)body[byte + 3] << 8);
  if ((n ^ comp) != 0xffffu || (u64)n + 4 >= len - byte) return 0;
  u32 before = (u32)body[byte - 1] << 8;
  if (byte >= 2) before |= body[byte - 2];
  int possible = 0;
  for (u32 gap = 3; gap <= 10; ++gap)
    if (byte * 8 >= gap && ((before >> (17 - gap)) & 3u) == 0) possible = 1;
  u64 endpoint = byte + 4 + n;
  return possible && ((body[endpoint] >> 1) & 3u) == 1;
}

/* Cheap necessary conditions checked first: BTYPE == 2, HLIT <= 29 and a
 * complete code-length code (Kraft sum of the HCLEN 3-bit lengths == 128).
 * dynamic_tables() is the exact test; this only skips hopeless offsets. */
static int dynamic_prefix(const u8* body, u64 len, u64 start) {
  Bits b = {body, len * 8, start};
  if (avail(&b) < 17) return 0;
  u64 w = peek_word(&b);
  if (((w >> 1) & 3) != 2 || ((w >> 3) & 31) > 29) return 0;
  u32 nc = (u32)((w >> 13) & 15) + 4;
  if (avail(&b) < 17 + 3 * (u64)nc) return 0;
  b.pos += 17;
  u64 lens = peek_word(&b);
  if (nc > 19) return 0;
  u32 kraft = 0;
  for (u32 i = 0; i < nc; ++i) {
    u32 l = (u32)((i < 19 && 3 * i < 57) ? (lens >> (3 * i)) & 7 : 0);
    if (3 * i >= 54) { /* beyond the peeked word: read directly */
      Bits c = {body, len * 8, start + 17 + 3 * i};
      u32 v;
      take(&c, 3, &v);
      l = v;
    }
    if (l) kraft += 128u >> l;
    if (kraft > 128) return 0;
  }
  return kraft == 128;
}

uint64_t oracle_candidate_count(const uint8_t* body, uint64_t len) {
  u64 count = 1; /* bit 0 is always a candidate */
  for (u64 byte = 0; byte < len; ++byte) {
    count += (u64)stored_seed(body, len, byte);
    for (u32 bit = 0; bit < 8; ++bit) {
      u64 s = byte * 8 + bit;
      if (s && dynamic_prefix(body, len, s) && dynamic_candidate(body, len, s)) ++count;
    }
  }
  return count;
}

/* parse_block semantics (_decode_kernels.py:683-781).  emit: write output and
 * apply the history/window checks of emission; prefix = output offset. */
static unsigned parse_block(const u8* body, u64 len, u64 start, u64 limit, u32 window, int emit,
                            u8* out, u64 prefix, u64* end, u64* size, u32* final) {
  Bits b = {body, len * 8, start};
  Tables t;
  u32 type;
  *size = 0;
  *end = start;
  *final = 0;
  if (!take(&b, 1, final) || !take(&b, 2, &type)) return ST_TRUNC;
  if (type == 3) return ST_RESERVED;
  u64 produced = 0;
  unsigned st = ST_OK;
  if (type == 0) {
    b.pos = (b.pos + 7) & ~(u64)7;
    u32 n, comp;
    if (!take(&b, 16, &n) || !take(&b, 16, &comp)) return ST_TRUNC;
    if ((n ^ comp) != 0xffffu) return ST_SYMBOL;
    if (n > limit) return ST_OVERFLOW;
    if ((u64)n * 8 > avail(&b)) return ST_TRUNC;
    if (emit) memcpy(out + prefix, body + (b.pos >> 3), n);
    produced = n;
    b.pos += (u64)n * 8;
  } else {
    st = type == 1 ? fixed_tables(&t) : dynamic_tables(&b, &t);
    if (st) return st;
    for (;;) {
      u32 lit = 0, length, distance;
      st = token(&b, &t, emit ? window : 32768u, &lit, &length, &distance);
      if (st) break;
      if (!length) break;
      if (!distance) {
        if (produced >= limit) { st = ST_OVERFLOW; break; }
        if (emit) out[prefix + produced] = (u8)lit;
        ++produced;
        continue;
      }
      if (length > limit - produced) { st = ST_OVERFLOW; break; }
      if (emit) {
        if (distance > prefix + produced) { st = ST_DISTANCE; break; }
        u64 d = prefix + produced;
        for (u32 j = 0; j < length; ++j) out[d + j] = out[d + j - distance];
      }
      produced += length;
    }
  }
  *end = b.pos;
  *size = produced;
  return st;
}

typedef struct {
  u64 start, end, size, prefix;
} Accepted;

uint32_t oracle_inflate_general(const uint8_t* in, uint64_t in_size, uint8_t* out,
                                uint64_t out_size, uint64_t max_candidates, uint32_t max_blocks) {
  memset(out, 0, out_size);
  u32 window, wanted;
  unsigned st = framing(in, in_size, &window, &wanted);
  if (st) return st;
  const u8* body = in + 2;
  const u64 len = in_size - 6;
  if (oracle_candidate_count(body, len) > max_candidates) return ST_CANDIDATES;

  /* Exact chain from bit 0 (select_chain, _decode_kernels.py:1226-1408). */
  u64 cap = 1024, n = 0;
  Accepted* blocks = (Accepted*)malloc(cap * sizeof(Accepted));
  u64 next = 0, output = 0;
  st = ST_OK;
  for (;;) {
    if (n >= max_blocks) { st = ST_BLOCKS; break; }
    Bits h = {body, len * 8, next};
    u32 final, type;
    if (!take(&h, 1, &final) || !take(&h, 2, &type)) { st = ST_TRUNC; break; }
    if (type == 3) { st = ST_RESERVED; break; }
    u64 end, size;
    u32 fin;
    if (next == 0 || type == 2) {
      if (next && !dynamic_candidate(body, len, next)) { st = ST_UNDISCOVERED; break; }
      st = parse_block(body, len, next, out_size, 32768u, 0, NULL, 0, &end, &size, &fin);
    } else {
      st = parse_block(body, len, next, out_size - output, 32768u, 0, NULL, 0, &end, &size, &fin);
    }
    if (st) break;
    if (end <= next || end > len * 8) { st = ST_EXTENT; break; }
    if (size > out_size - output) { st = ST_OVERFLOW; break; }
    if (n >= max_blocks) { st = ST_BLOCKS; break; }
    if (n == cap) {
      cap *= 2;
      blocks = (Accepted*)realloc(blocks, cap * sizeof(Accepted));
    }
    blocks[n].start = next;
    blocks[n].end = end;
    blocks[n].size = size;
    blocks[n].prefix = output;
    ++n;
    output += size;
    next = end;
    if (fin) {
      if (output != out_size) st = ST_SIZE;
      else if ((next + 7) / 8 != len) st = ST_EXTENT;
      break;
    }
  }
  if (!st) {
    /* Emission with the declared window and the accepted prefix as history. */
    for (u64 i = 0; i < n && !st; ++i) {
      u64 end, size;
      u32 fin;
      st = parse_block(body, len, blocks[i].start, blocks[i].size, window, 1, out,
                       blocks[i].prefix, &end, &size, &fin);
    }
  }
  free(blocks);
  if (st) {
    memset(out, 0, out_size);
    return st;
  }
  if (oracle_adler32(out, out_size) != wanted) return ST_ADLER;
  return ST_OK;
}

/* Route selection and bounds (native/codec_ffi.cu:662-707). */
uint32_t oracle_decompress(const uint8_t* in, uint64_t in_size, uint8_t* out, uint64_t out_size,
                           int64_t max_candidates, int64_t max_blocks) {
  if (out_size > MAX_BYTES) return ST_BOUNDS;
  if (in_size > MAX_BYTES || max_candidates < 1 || max_candidates > MAX_CANDIDATES ||
      max_blocks < 1 || max_blocks > MAX_BLOCKS) {
    memset(out, 0, out_size);
    return ST_BOUNDS;
  }
  if (in_size < 8) {
    memset(out, 0, out_size);
    return ST_ZTRUNC;
  }
  if (max_candidates == MAX_CANDIDATES && max_blocks == MAX_BLOCKS && out_size <= 65536 &&
      in_size <= 131072)
    return oracle_inflate_serial(in, in_size, out, out_size, (u32)max_blocks);
  return oracle_inflate_general(in, in_size, out, out_size, (u64)max_candidates, (u32)max_blocks);
}

/* Tree-validity classification of a code-length vector, for brute-force tests. */
uint32_t oracle_huff_build_status(const uint8_t* lens, uint32_t n, int empty_ok, int single_ok,
                                  uint32_t limit) {
  Huff h;
  if (n > 288) return ST_TREE;
  return huff_build(&h, lens, n, empty_ok, single_ok, limit);
}
