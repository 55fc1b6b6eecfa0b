// CPU bounds check of the codec's device readers, compiled for the host.
//
// The decode kernels read compressed bytes through BitIn (global memory),
// WordBits over LDS-staged words, and copy stored payloads with copy_bytes;
// wrappers are parsed by parse_frame.  Here the same code (deflate_common.h,
// built with hipcc --offload-host-only) reads buffers that end exactly at a
// PROT_NONE page, so a read past the end is a SIGSEGV instead of a silent
// garbage value -- the check that cannot be made on the GPU without faulting
// it.  Every truncation of every input is decoded; the statuses are printed
// for the Python side to compare.
//
// Usage: guarded_readers <mode> <file>...
//   walk   decode each zlib stream (and every truncation) with BitIn
//   staged the same body decoded with WordBits/fast_token over guarded words
//   copy   copy_bytes over every length/alignment pair up to 96 bytes
//   frame  parse_frame on every truncation, in each format
//   pairs  quick_pair (literal pairs) and quick_triple (three literals)
//          against quick_token over guarded words
//   window window_token (one token from the Win4 registers) against
//          fast_token over WordBits at every bit of every block body, at the
//          body end and at a varying nearer limit
//   longcodes  long_code (per-length bounds) against a bit-by-bit canonical
//          walk on random complete, single-code and empty tables, every
//          15-bit prefix the primary LUT misses and every bit budget
//   guard  reads one byte past a guarded buffer (must crash: checks the guard)
#include <sys/mman.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "deflate_common.h"

using namespace hz;

namespace {

// `n` bytes that end where an inaccessible page begins.
struct Guarded {
  u8* map = nullptr;
  size_t length = 0;
  u8* data = nullptr;
  Guarded(const u8* src, size_t n) {
    const size_t page = size_t(sysconf(_SC_PAGESIZE));
    const size_t body = (n + page - 1) / page * page + page;  // a mapped page before the data too
    length = body + page;
    map = static_cast<u8*>(mmap(nullptr, length, PROT_READ | PROT_WRITE,
                                MAP_PRIVATE | MAP_ANONYMOUS, -1, 0));
    if (map == MAP_FAILED) { perror("mmap"); exit(2); }
    if (mprotect(map + body, page, PROT_NONE)) { perror("mprotect"); exit(2); }
    data = map + body - n;
    if (n) memcpy(data, src, n);
  }
  ~Guarded() { munmap(map, length); }
};

std::vector<u8> read_file(const char* path) {
  FILE* f = fopen(path, "rb");
  if (!f) { perror(path); exit(2); }
  std::vector<u8> v;
  u8 buf[65536];
  size_t k;
  while ((k = fread(buf, 1, sizeof buf, f)) > 0) v.insert(v.end(), buf, buf + k);
  fclose(f);
  return v;
}

// Serial inflate of a raw DEFLATE body with the product's BitIn and table
// builders; output into a guarded buffer of `limit` bytes.  Returns a status.
u32 inflate_body(const u8* body, u64 len, u8* out, u64 limit, u64& produced) {
  static DecodeTables t;
  BitIn r;
  r.init(body, len, 0);
  produced = 0;
  for (u32 blocks = 0; blocks < 100000; ++blocks) {
    u32 final_block, type;
    if (!r.take(1, final_block) || !r.take(2, type)) return kTruncated;
    if (type == 3) return kReservedBlock;
    if (type == 0) {
      r.seek((r.pos + 7) & ~u64(7));
      u32 n, comp;
      if (!r.take(16, n) || !r.take(16, comp)) return kTruncated;
      if ((n ^ comp) != 0xffffu) return kBadSymbol;
      if (n > limit - produced) return kOutputOverflow;
      if (u64(n) * 8 > r.avail()) return kTruncated;
      copy_bytes(out + produced, body + (r.pos >> 3), n, body + len, 0, 1);
      produced += n;
      r.seek(r.pos + u64(n) * 8);
    } else {
      const u32 err = type == 1 ? build_fixed_tables(t) : build_dynamic_tables(t, r);
      if (err) return err;
      for (;;) {
        u32 lit, length, distance;
        const u32 e = decode_token(t, r, 32768u, lit, length, distance);
        if (e) return e;
        if (!length) break;
        if (length > limit - produced) return kOutputOverflow;
        if (!distance) {
          out[produced++] = u8(lit);
          continue;
        }
        if (distance > produced) return kBadDistance;
        for (u32 j = 0; j < length; ++j, ++produced) out[produced] = out[produced - distance];
      }
    }
    if (final_block) return (r.pos + 7) / 8 == len ? kOk : kExtent;
  }
  return kBlockCapacity;
}

// The same body through WordBits and fast_token over staged words, the way
// the describe and emission kernels read their LDS stage: the words hold the
// body plus a margin of zero words (what stage_range leaves past the body
// end), and the checked reader stops at the body's last bit.
u32 staged_body(const u8* body, u64 len, u64& produced) {
  static DecodeTables t;
  const u32 margin_words = 16;
  const u64 words = (len + 3) / 4 + margin_words;
  std::vector<u32> host(words, 0u);
  memcpy(host.data(), body, len);
  Guarded g(reinterpret_cast<const u8*>(host.data()), words * 4);
  const u32* w = reinterpret_cast<const u32*>(g.data);
  BitIn hdr;
  hdr.init(body, len, 0);
  produced = 0;
  for (u32 blocks = 0; blocks < 100000; ++blocks) {
    u32 final_block, type;
    if (!hdr.take(1, final_block) || !hdr.take(2, type)) return kTruncated;
    if (type == 3) return kReservedBlock;
    if (type == 0) {
      hdr.seek((hdr.pos + 7) & ~u64(7));
      u32 n, comp;
      if (!hdr.take(16, n) || !hdr.take(16, comp)) return kTruncated;
      if ((n ^ comp) != 0xffffu) return kBadSymbol;
      if (u64(n) * 8 > hdr.avail()) return kTruncated;
      produced += n;
      hdr.seek(hdr.pos + u64(n) * 8);
    } else {
      u32 err = type == 1 ? build_fixed_tables(t) : build_dynamic_tables(t, hdr);
      if (err) return err;
      fast_format(t.ll, true, 0, 1);
      fast_format(t.dd, false, 0, 1);
      WordBits<true> q;
      q.words = w;
      q.limit = u32(len * 8);
      q.seek(u32(hdr.pos));
      for (;;) {
        u32 lit, length, distance;
        err = fast_token(t.ll, t.dd, q, lit, length, distance);
        if (err) return err;
        if (!length) break;
        produced += length;
      }
      hdr.seek(q.pos());
    }
    if (final_block) return (hdr.pos + 7) / 8 == len ? kOk : kExtent;
  }
  return kBlockCapacity;
}

// The same body decoded three times over guarded staged words in slices of
// `slice_bits`: A with quick_token (one token at a time), B with quick_pair
// (literal pairs), C with quick_triple (up to three literals); all fall back
// to fast_token.  Each slice decodes the tokens that start before its stop,
// so after every slice A, B and C must stand at the same position, and their
// outputs must agree byte for byte.  Returns a status (kExtent when they
// disagree); `out` is B's output.
u32 pairs_body(const u8* body, u64 len, u32 slice_bits, std::vector<u8>& out) {
  static DecodeTables t;
  const u32 margin_words = 16;
  const u64 words = (len + 3) / 4 + margin_words;
  std::vector<u32> host(words, 0u);
  memcpy(host.data(), body, len);
  Guarded g(reinterpret_cast<const u8*>(host.data()), words * 4);
  const u32* w = reinterpret_cast<const u32*>(g.data);
  BitIn hdr;
  hdr.init(body, len, 0);
  out.clear();
  std::vector<u8> other;
  for (u32 blocks = 0; blocks < 100000; ++blocks) {
    u32 final_block, type;
    if (!hdr.take(1, final_block) || !hdr.take(2, type)) return kTruncated;
    if (type == 3) return kReservedBlock;
    if (type == 0) {
      hdr.seek((hdr.pos + 7) & ~u64(7));
      u32 n, comp;
      if (!hdr.take(16, n) || !hdr.take(16, comp)) return kTruncated;
      if ((n ^ comp) != 0xffffu) return kBadSymbol;
      if (u64(n) * 8 > hdr.avail()) return kTruncated;
      for (u32 i = 0; i < n; ++i) out.push_back(body[(hdr.pos >> 3) + i]);
      hdr.seek(hdr.pos + u64(n) * 8);
      if (final_block) return (hdr.pos + 7) / 8 == len ? kOk : kExtent;
      continue;
    }
    u32 err = type == 1 ? build_fixed_tables(t) : build_dynamic_tables(t, hdr);
    if (err) return err;
    fast_format(t.ll, true, 0, 1);
    fast_format(t.dd, false, 0, 1);
    other = out;
    std::vector<u8> third = out;
    std::vector<u8> starts(len * 8 + 64, 0);  // token starts A met
    Win4<true> a, b, c;
    a.words = b.words = c.words = w;
    a.limit = b.limit = c.limit = u32(len * 8);
    a.seek(u32(hdr.pos));
    b.seek(u32(hdr.pos));
    c.seek(u32(hdr.pos));
    bool ended = false;
    while (!ended) {
      const u32 stop = a.pos() + slice_bits;
      // A: one token at a time.
      while (!ended && a.pos() < stop) {
        starts[a.pos()] = 1;
        u32 length, x;
        if (!quick_token<true>(t.ll, t.dd, a, length, x)) {
          WordBits<true> q;
          q.words = w;
          q.limit = a.limit;
          q.seek(a.pos());
          u32 lit, distance;
          err = fast_token(t.ll, t.dd, q, lit, length, distance);
          if (err) return err;
          a.seek(q.pos());
          if (!length) { ended = true; break; }
          x = length == 1 ? lit : distance;
        }
        if (length == 1) { other.push_back(u8(x)); continue; }
        if (x > other.size()) return kBadDistance;
        for (u32 j = 0; j < length; ++j) other.push_back(other[other.size() - x]);
      }
      // B: literal pairs, the same stop.
      bool b_ended = false;
      while (!b_ended && b.pos() < stop) {
        u32 length, x, x2, l1;
        const u32 start = b.pos();
        const u32 got = quick_pair<true>(t.ll, t.dd, b, stop, length, x, x2, l1);
        // The second literal starts l1 bits in, at one of A's token starts.
        if (got == 2 && (start + l1 >= stop || !starts[start + l1])) return kExtent;
        if (!got) {
          WordBits<true> q;
          q.words = w;
          q.limit = b.limit;
          q.seek(b.pos());
          u32 lit, distance;
          err = fast_token(t.ll, t.dd, q, lit, length, distance);
          if (err) return err;
          b.seek(q.pos());
          if (!length) { b_ended = true; break; }
          x = length == 1 ? lit : distance;
        }
        if (length == 1) {
          out.push_back(u8(x));
          if (got == 2) out.push_back(u8(x2));
          continue;
        }
        if (x > out.size()) return kBadDistance;
        for (u32 j = 0; j < length; ++j) out.push_back(out[out.size() - x]);
      }
      // C: up to three literals a step, the same stop; every step ends at
      // one of A's token starts or at or past the stop.
      bool c_ended = false;
      while (!c_ended && c.pos() < stop) {
        u32 length, x, x2, x3, l1, l12;
        const u32 start = c.pos();
        const u32 got = quick_triple<true>(t.ll, t.dd, c, stop, length, x, x2, x3, l1, l12);
        if (got >= 2 && c.pos() < stop && !starts[c.pos()]) return kExtent;
        // The second and third literals start at A's token starts before the stop.
        if (got >= 2 && (start + l1 >= stop || !starts[start + l1])) return kExtent;
        if (got == 3 && (start + l12 >= stop || !starts[start + l12])) return kExtent;
        if (!got) {
          WordBits<true> q;
          q.words = w;
          q.limit = c.limit;
          q.seek(c.pos());
          u32 lit, distance;
          err = fast_token(t.ll, t.dd, q, lit, length, distance);
          if (err) return err;
          c.seek(q.pos());
          if (!length) { c_ended = true; break; }
          x = length == 1 ? lit : distance;
        }
        if (length == 1) {
          third.push_back(u8(x));
          if (got >= 2) third.push_back(u8(x2));
          if (got == 3) third.push_back(u8(x3));
          continue;
        }
        if (x > third.size()) return kBadDistance;
        for (u32 j = 0; j < length; ++j) third.push_back(third[third.size() - x]);
      }
      if (a.pos() != b.pos() || ended != b_ended || out.size() != other.size()) return kExtent;
      if (a.pos() != c.pos() || ended != c_ended || third.size() != other.size()) return kExtent;
    }
    if (out != other || third != other) return kExtent;
    hdr.seek(b.pos());
    if (final_block) return (hdr.pos + 7) / 8 == len ? kOk : kExtent;
  }
  return kBlockCapacity;
}

int mode_pairs(int argc, char** argv) {
  for (int i = 0; i < argc; ++i) {
    const std::vector<u8> s = read_file(argv[i]);
    printf("%s", argv[i]);
    for (u32 slice : {29u, 97u, 512u}) {
      Frame f;
      std::vector<u8> out;
      u32 st = parse_frame(s.data(), s.size(), kFormatZlib, false, f);
      if (!st) st = pairs_body(s.data() + f.body, f.body_len, slice, out);
      u32 a = 1, b = 0;
      for (u8 c : out) {
        a = (a + c) % 65521;
        b = (b + a) % 65521;
      }
      printf(" s%u=%u bytes%u=%zu adler%u=%u", slice, st, slice, out.size(), slice, (b << 16) | a);
    }
    printf("\n");
  }
  return 0;
}

int mode_walk(int argc, char** argv, bool staged) {
  for (int i = 0; i < argc; ++i) {
    const std::vector<u8> s = read_file(argv[i]);
    // The output bound is what the whole stream decodes to (at most 4 MiB):
    // the guarded output buffer ends there, so no truncation may write past it.
    u64 bound = 4u << 20;
    {
      std::vector<u8> big(bound);
      Frame f;
      u64 produced = 0;
      if (!parse_frame(s.data(), s.size(), kFormatZlib, false, f))
        inflate_body(s.data() + f.body, f.body_len, big.data(), bound, produced);
      bound = produced;
    }
    std::vector<u8> zeros(bound, 0);
    Guarded out(zeros.data(), bound);
    printf("%s", argv[i]);
    u64 sum = 0;
    for (u64 n = 0; n <= s.size(); ++n) {
      Guarded in(s.data(), n);
      Frame f;
      u32 st = parse_frame(in.data, n, kFormatZlib, false, f);
      u64 produced = 0;
      if (!st) {
        if (staged) st = staged_body(in.data + f.body, f.body_len, produced);
        else st = inflate_body(in.data + f.body, f.body_len, out.data, bound, produced);
      }
      sum = sum * 31 + st;
      if (n == s.size()) printf(" full=%u bytes=%llu", st, (unsigned long long)produced);
    }
    printf(" digest=%llu\n", (unsigned long long)sum);
  }
  return 0;
}

int mode_copy() {
  u8 src[256], expect[256];
  for (u32 i = 0; i < 256; ++i) src[i] = u8(i * 7 + 3);
  u32 cases = 0;
  for (u32 n = 0; n <= 96; ++n)
    for (u32 sa = 0; sa < 16; ++sa)
      for (u32 da = 0; da < 16; ++da) {
        // Source ends at the guard; the destination buffer is guarded too.
        Guarded s(src + sa, n);
        std::vector<u8> zeros(n + da, 0);
        Guarded d(zeros.data(), n + da);
        AdlerAcc acc;
        copy_bytes(d.data + da, s.data, n, s.data + n, 0, 1, &acc, n);
        memcpy(expect, src + sa, n);
        if (memcmp(d.data + da, expect, n)) {
          printf("copy mismatch n=%u sa=%u da=%u\n", n, sa, da);
          return 1;
        }
        u64 s1 = 0, w1 = 0;
        for (u32 j = 0; j < n; ++j) {
          s1 += expect[j];
          w1 += u64(n - j) * expect[j];
        }
        if (acc.s != s1 || acc.w % kAdlerMod != w1 % kAdlerMod) {
          printf("copy sums n=%u sa=%u da=%u\n", n, sa, da);
          return 1;
        }
        ++cases;
      }
  printf("copy cases=%u\n", cases);
  return 0;
}

int mode_frame(int argc, char** argv) {
  for (int i = 0; i < argc; ++i) {
    const std::vector<u8> s = read_file(argv[i]);
    printf("%s", argv[i]);
    for (u32 format = 0; format < 3; ++format) {
      u64 sum = 0;
      for (u64 n = 0; n <= s.size(); ++n) {
        Guarded in(s.data(), n);
        Frame f;
        const u32 st = parse_frame(in.data, n, format, false, f);
        sum = sum * 31 + st + (st ? 0 : f.body * 7 + f.body_len);
        if (n == s.size()) printf(" f%u=%u", format, st);
      }
      printf(" d%u=%llu", format, (unsigned long long)sum);
    }
    printf("\n");
  }
  return 0;
}

// window_token against fast_token at every bit position of each dynamic or
// fixed block's body (and past it, into the next header and garbage), with
// the body end as the limit and with a nearer limit that varies with the
// position: the status, the token and, on success, the end position must
// agree.  Prints "window <file> positions=<n> bad=<k>".
int mode_window(int argc, char** argv) {
  static DecodeTables t;
  int rc = 0;
  for (int i = 0; i < argc; ++i) {
    const std::vector<u8> s = read_file(argv[i]);
    Frame f;
    if (parse_frame(s.data(), s.size(), kFormatZlib, false, f) || !f.body_len) continue;
    const u8* body = s.data() + f.body;
    const u64 len = f.body_len;
    const u64 words = (len + 3) / 4 + 16;
    std::vector<u32> host(words, 0u);
    memcpy(host.data(), body, len);
    Guarded g(reinterpret_cast<const u8*>(host.data()), words * 4);
    const u32* w = reinterpret_cast<const u32*>(g.data);
    BitIn hdr;
    hdr.init(body, len, 0);
    u64 positions = 0, bad = 0;
    for (u32 blocks = 0; blocks < 1000; ++blocks) {
      u32 final_block, type;
      if (!hdr.take(1, final_block) || !hdr.take(2, type) || type == 0 || type == 3) break;
      const u32 err = type == 1 ? build_fixed_tables(t) : build_dynamic_tables(t, hdr);
      if (err) break;
      fast_format(t.ll, true, 0, 1);
      fast_format(t.dd, false, 0, 1);
      const u32 from = u32(hdr.pos);
      const u32 end = u32(len * 8);
      u32 next = end;
      for (u32 p = from; p < end; ++p) {
        for (u32 near = 0; near < 2; ++near) {
          const u32 limit = near ? p + (p * 7 + 3) % 53 : end;
          if (limit > end) continue;
          WordBits<true> q;
          q.words = w;
          q.limit = limit;
          q.seek(p);
          Win4<true> r;
          r.words = w;
          r.limit = limit;
          r.seek(p);
          u32 lit1 = 0, len1 = 0, d1 = 0, lit2 = 0, len2 = 0, d2 = 0;
          const u32 e1 = fast_token(t.ll, t.dd, q, lit1, len1, d1);
          const u32 e2 = window_token<true>(t.ll, t.dd, r, lit2, len2, d2);
          bool same = e1 == e2;
          if (same && !e1) {
            same = len1 == len2 && q.pos() == r.pos() && (len1 != 1 || lit1 == lit2) &&
                   (len1 < 3 || d1 == d2);
            if (!near && !len1 && next == end) next = q.pos();  // first EOB
          }
          if (!same) {
            if (bad < 5)
              printf("mismatch %s p=%u limit=%u: fast %u/%u/%u/%u@%u window %u/%u/%u/%u@%u\n",
                     argv[i], p, limit, e1, len1, lit1, d1, q.pos(), e2, len2, lit2, d2, r.pos());
            ++bad;
          }
          ++positions;
        }
      }
      // The next block: follow the true parse to this block's end.
      Win4<true> r;
      r.words = w;
      r.limit = end;
      r.seek(from);
      for (;;) {
        u32 lit, length, distance;
        if (window_token<true>(t.ll, t.dd, r, lit, length, distance)) { final_block = 1; break; }
        if (!length) break;
      }
      hdr.seek(r.pos());
      if (final_block) break;
    }
    printf("window %s positions=%llu bad=%llu\n", argv[i], (unsigned long long)positions,
           (unsigned long long)bad);
    if (bad) rc = 1;
  }
  return rc;
}

// Bit-by-bit canonical decode (RFC 1951 3.2.2 order): the code value grows
// one bit at a time and is compared with the length's code range.
template <int N, int P>
i32 walk_code(const HuffTable<N, P>& t, u32 b, u32 avail, u32& len_out, u32& err) {
  u32 code = 0, first = 0, index = 0;
  for (u32 len = 1; len <= t.maximum; ++len) {
    if (len > avail) { err = kTruncated; return -1; }
    code |= (b >> (len - 1)) & 1u;
    const u32 c = t.count[len];
    if (code < first + c) {
      len_out = len;
      return i32(t.symbols[index + code - first]);
    }
    index += c;
    first = (first + c) << 1;
    code <<= 1;
  }
  err = kBadSymbol;
  return -1;
}

u64 rng_state = 0x9e3779b97f4a7c15ull;
u32 rnd(u32 n) {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 7;
  rng_state ^= rng_state << 17;
  return u32((rng_state >> 11) % n);
}

// Lengths of a random complete code over `used` of n symbols (leaves split
// until there are `used`; `deep` favours splitting the deepest leaf, which
// makes codes up to 15 bits), or one length-1 code, or none.
void random_lengths(u8* lens, u32 n, u32 kind) {
  for (u32 i = 0; i < n; ++i) lens[i] = 0;
  if (kind == 1) { lens[rnd(n)] = 1; return; }
  if (kind == 2) return;
  const u32 used = 2 + rnd(n - 1);
  std::vector<u32> depth(1, 0);
  const bool deep = rnd(2);
  while (depth.size() < used) {
    u32 pick = rnd(u32(depth.size()));
    if (deep && rnd(4)) {
      for (u32 i = 0; i < depth.size(); ++i)
        if (depth[i] > depth[pick] && depth[i] < 15) pick = i;
    }
    if (depth[pick] >= 15) {
      bool any = false;
      for (u32 i = 0; i < depth.size(); ++i)
        if (depth[i] < 15) { pick = i; any = true; break; }
      if (!any) break;
    }
    const u32 d = depth[pick] + 1;
    depth[pick] = d;
    depth.push_back(d);
  }
  std::vector<u32> syms(n);
  for (u32 i = 0; i < n; ++i) syms[i] = i;
  for (u32 i = n - 1; i > 0; --i) std::swap(syms[i], syms[rnd(i + 1)]);
  for (u32 i = 0; i < depth.size(); ++i) lens[syms[i]] = u8(depth[i]);
}

template <int N, int P>
u64 check_long_codes(u32 trials, u32& bad) {
  static HuffTable<N, P> t;
  u8 lens[N];
  u64 checked = 0;
  for (u32 trial = 0; trial < trials; ++trial) {
    const u32 kind = trial % 16 == 1 ? 1u : trial % 16 == 2 ? 2u : 0u;
    random_lengths(lens, N, kind);
    if (huff_build(t, lens, N, true, true, 15)) { ++bad; continue; }
    // The wave build's per-lane bounds: inclusive weighted sums of the counts.
    u32 wsum = 0, csum = 0;
    for (u32 l = 1; l < 16; ++l) {
      const u32 c = t.count[l];
      wsum += c << (15 - l);
      csum += c;
      const u32 first = (wsum - (c << (15 - l))) >> (15 - l);
      if (t.limit[l] != u16(wsum) || t.base[l] != u16(csum - c - first)) ++bad;
    }
    for (u32 v = 0; v < (1u << 15); ++v) {
      const u32 b = bit_reverse(v, 15) | (rnd(1u << 17) << 15);  // bits past 15: noise
      if (t.primary[b & ((1u << P) - 1)] & 15u) continue;
      for (u32 avail = 0; avail <= 17; ++avail) {
        const u32 a = avail == 17 ? 0xffffffffu : avail;
        u32 l1 = 99, l2 = 99, e1 = 0, e2 = 0;
        const i32 s1 = walk_code(t, b, a, l1, e1);
        const i32 s2 = long_code(t, b, a, l2, e2);
        if (s1 != s2 || (s1 >= 0 ? l1 != l2 : e1 != e2)) {
          if (bad < 10)
            printf("mismatch N=%d trial=%u v=%u avail=%u: walk %d/%u/%u long %d/%u/%u\n", N,
                   trial, v, a, s1, l1, e1, s2, l2, e2);
          ++bad;
        }
        ++checked;
      }
    }
  }
  return checked;
}

int mode_long_codes() {
  u32 bad = 0;
  const u64 a = check_long_codes<288, 10>(400, bad);
  const u64 b = check_long_codes<32, 8>(400, bad);
  const u64 c = check_long_codes<19, 7>(100, bad);
  printf("longcodes checked=%llu bad=%u\n", (unsigned long long)(a + b + c), bad);
  return bad ? 1 : 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  const char* mode = argv[1];
  if (!strcmp(mode, "walk")) return mode_walk(argc - 2, argv + 2, false);
  if (!strcmp(mode, "staged")) return mode_walk(argc - 2, argv + 2, true);
  if (!strcmp(mode, "copy")) return mode_copy();
  if (!strcmp(mode, "frame")) return mode_frame(argc - 2, argv + 2);
  if (!strcmp(mode, "pairs")) return mode_pairs(argc - 2, argv + 2);
  if (!strcmp(mode, "longcodes")) return mode_long_codes();
  if (!strcmp(mode, "window")) return mode_window(argc - 2, argv + 2);
  if (!strcmp(mode, "guard")) {
    const u8 byte = 1;
    Guarded g(&byte, 1);
    volatile const u8* p = g.data;
    printf("%u\n", unsigned(p[1]));  // the first byte of the inaccessible page
    return 0;
  }
  return 2;
}
