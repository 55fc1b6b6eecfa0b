"""Independent RFC 1950/1951 stream writer for hand-built test streams.

Builds streams zlib cannot emit (every header alignment, maximum-length codes,
reserved symbols, bad repeats, over-window distances, stored decoys) so the
decoder's parity tests reach the edge cases the reference's own tests pin.
The cases in ``pinned_cases()`` carry the statuses those tests assert
(reference tests/test_decode.py, test_stored_fast_decode.py, test_batch.py,
test_literal_lookahead.py, test_small_shared_decode.py, test_regressions.py).
"""

import random
import struct
import zlib

FIXED_LL = [8] * 144 + [9] * 112 + [7] * 24 + [8] * 8
FIXED_D = [5] * 32
CL_ORDER = (16, 17, 18, 0, 8, 7, 9, 6, 10, 5, 11, 4, 12, 3, 13, 2, 14, 1, 15)
LENGTH_BASE = (3, 4, 5, 6, 7, 8, 9, 10, 11, 13, 15, 17, 19, 23, 27, 31, 35, 43, 51, 59,
               67, 83, 99, 115, 131, 163, 195, 227, 258)
LENGTH_EXTRA = (0,) * 8 + tuple(e for e in range(1, 6) for _ in range(4)) + (0,)
DIST_BASE = (1, 2, 3, 4, 5, 7, 9, 13, 17, 25, 33, 49, 65, 97, 129, 193, 257, 385, 513, 769,
             1025, 1537, 2049, 3073, 4097, 6145, 8193, 12289, 16385, 24577)
DIST_EXTRA = (0,) * 4 + tuple(e for e in range(1, 14) for _ in range(2))


def canonical(lengths):
    """Canonical Huffman codes (RFC 1951 3.2.2): symbol -> (code, length)."""
    counts = [0] * 16
    for n in lengths:
        if n:
            counts[n] += 1
    next_code, code = [0] * 16, 0
    for bits in range(1, 16):
        code = (code + counts[bits - 1]) << 1 if bits > 1 else 0
        next_code[bits] = code
    codes = {}
    for symbol, n in enumerate(lengths):
        if n:
            codes[symbol] = (next_code[n], n)
            next_code[n] += 1
    return codes


class BitWriter:
    """LSB-first bit packer; Huffman codes are written most-significant bit first."""

    def __init__(self):
        self.data = bytearray()
        self.pending = 0   # bits not yet flushed to `data`
        self.width = 0     # number of pending bits (< 8 between calls)

    @property
    def nbits(self):
        return len(self.data) * 8 + self.width

    def put(self, value, width):
        assert 0 <= value < (1 << width) or (width == 0 and value == 0)
        self.pending |= value << self.width
        self.width += width
        while self.width >= 8:
            self.data.append(self.pending & 255)
            self.pending >>= 8
            self.width -= 8
        return self

    def code(self, entry):
        code, length = entry
        self.put(int(format(code, "0%db" % length)[::-1], 2), length)
        return self

    def align(self):
        if self.width:
            self.put(0, 8 - self.width)
        return self

    def raw(self, data):
        self.align()
        self.data.extend(data)
        return self

    def drop_last_bit(self):
        if self.width:
            self.width -= 1
            self.pending &= (1 << self.width) - 1
        else:
            last = self.data.pop()
            self.pending, self.width = last & 0x7F, 7
        return self

    def getvalue(self):
        return bytes(self.data) + (bytes((self.pending,)) if self.width else b"")


def header(cmf=0x78, flags=0):
    return bytes((cmf, flags | (-(cmf * 256 + flags) % 31)))


def wrap(body, raw, cmf=0x78, flags=0):
    return header(cmf, flags) + body + struct.pack(">I", zlib.adler32(raw))


def stored(raw, final=True):
    assert len(raw) <= 65535
    return bytes((int(final),)) + struct.pack("<HH", len(raw), len(raw) ^ 0xFFFF) + raw


def compressed(raw, level=6, strategy=zlib.Z_DEFAULT_STRATEGY, wbits=15, flush=zlib.Z_FINISH):
    c = zlib.compressobj(level, zlib.DEFLATED, wbits, 8, strategy)
    return c.compress(raw) + c.flush(flush)


class Block:
    """Writes tokens of one fixed or dynamic block into a BitWriter."""

    def __init__(self, writer, final, ll_lengths=None, d_lengths=None, cl_lengths=None,
                 hclen=None):
        self.w = writer
        if ll_lengths is None:
            writer.put(int(final), 1).put(1, 2)
            self.ll, self.d = canonical(FIXED_LL), canonical(FIXED_D)
            return
        writer.put(int(final), 1).put(2, 2)
        writer.put(len(ll_lengths) - 257, 5).put(len(d_lengths) - 1, 5)
        if cl_lengths is None:
            cl_lengths = _complete_cl(set(ll_lengths) | set(d_lengths))
        count = hclen or max(4, max(CL_ORDER.index(s) + 1 for s, n in enumerate(cl_lengths) if n))
        writer.put(count - 4, 4)
        for s in CL_ORDER[:count]:
            writer.put(cl_lengths[s], 3)
        cl = canonical(cl_lengths)
        for n in list(ll_lengths) + list(d_lengths):
            writer.code(cl[n])
        self.ll, self.d = canonical(ll_lengths), canonical(d_lengths)

    def literal(self, byte):
        self.w.code(self.ll[byte])
        return self

    def literals(self, data):
        for b in data:
            self.w.code(self.ll[b])
        return self

    def symbol(self, s):
        self.w.code(self.ll[s])
        return self

    def match(self, length, distance):
        li = max(i for i, base in enumerate(LENGTH_BASE) if base <= length)
        if length == 258:
            li = 28
        self.w.code(self.ll[257 + li])
        self.w.put(length - LENGTH_BASE[li], LENGTH_EXTRA[li])
        di = max(i for i, base in enumerate(DIST_BASE) if base <= distance)
        self.w.code(self.d[di])
        self.w.put(distance - DIST_BASE[di], DIST_EXTRA[di])
        return self

    def end(self):
        self.w.code(self.ll[256])
        return self.w


def _complete_cl(used):
    """A complete code-length code covering every length symbol in `used`."""
    used = sorted(set(used) | {0})
    lengths = [0] * 19
    if len(used) == 1:
        used.append(1 if used[0] != 1 else 2)
    k = len(used)
    # Complete tree with k leaves: (2**depth - k) leaves at depth-1, the rest at depth.
    depth = max(1, (k - 1).bit_length())
    short = 2 ** depth - k
    for i, s in enumerate(used):
        lengths[s] = depth - 1 if i < short else depth
    return lengths


def literal_only_block(w, data, final=True, long_codes=False, single_eob=False):
    """Dynamic literal-only block with a hand-chosen tree and no distance codes."""
    ll = [0] * 257
    if long_codes:
        for s in range(14):
            ll[s] = s + 1
        ll[14] = ll[256] = 15
    else:
        ll[256] = 1
        if not single_eob:
            ll[65] = 1
    cl = [0] * 19
    if long_codes:
        cl[:16] = [4] * 16
    else:
        cl[0] = cl[1] = 1
    blk = Block(w, final, ll, [0], cl)
    return blk.literals(data).end()


def _deep_lengths(rng, count):
    """Lengths of a complete code over `count` symbols with codes of up to 15
    bits: leaves are split (often the deepest one that can still grow) until
    there are `count`, so many codes are 11-15 bits long."""
    depth = [0]
    while len(depth) < count:
        growable = [i for i, d in enumerate(depth) if d < 15]
        if rng.random() < 0.4:
            pick = max(growable, key=lambda i: (depth[i], i))
        else:
            pick = rng.choice(growable)
        depth[pick] += 1
        depth.append(depth[pick])
    rng.shuffle(depth)
    return depth


def long_code_mix_stream(blocks=3, tokens=12000, seed=5150):
    """Dynamic blocks whose literal/length and distance codes run up to 15 bits
    (literal/length codes of most lengths from 9 to 15), with tokens drawn
    uniformly over the symbols, so that most literals, lengths and distances
    take codes longer than a decoder's primary table."""
    rng = random.Random(seed)
    w = BitWriter()
    out = bytearray()
    for b in range(blocks):
        ll = _deep_lengths(rng, 286)
        d = _deep_lengths(rng, 30)
        assert max(ll) == 15 and max(d) >= 12
        blk = Block(w, b == blocks - 1, ll, d)
        for _ in range(tokens):
            if len(out) < 64 or rng.random() < 0.6:
                byte = rng.randrange(256)
                blk.literal(byte)
                out.append(byte)
                continue
            li = rng.randrange(29)
            length = LENGTH_BASE[li] + rng.randrange(1 << LENGTH_EXTRA[li])
            if li == 28:
                length = 258
            top = min(len(out), 32768)
            di = rng.randrange(max(i for i, base in enumerate(DIST_BASE) if base <= top) + 1)
            span = min(DIST_BASE[di] + (1 << DIST_EXTRA[di]) - 1, top) - DIST_BASE[di] + 1
            distance = DIST_BASE[di] + rng.randrange(span)
            blk.match(length, distance)
            for _ in range(length):
                out.append(out[-distance])
        blk.end()
    return wrap(w.getvalue(), bytes(out)), bytes(out)


def literal_only_stream(data, **kwargs):
    w = BitWriter()
    literal_only_block(w, data, **kwargs)
    return wrap(w.getvalue(), data)


def fixed_stream(data, final=True):
    w = BitWriter()
    Block(w, final).literals(data).end()
    return wrap(w.getvalue(), data)


# ---- pinned fixtures ----------------------------------------------------------

def alignment_stream(prefix_count):
    """Fixed 9-bit literals shift a following dynamic block to every bit alignment."""
    w = BitWriter()
    Block(w, False).literals(b"\x90" * prefix_count).end()
    suffix = b"A" * 37
    literal_only_block(w, suffix)
    raw = b"\x90" * prefix_count + suffix
    return wrap(w.getvalue(), raw), raw


def many_dynamic_stream(empty, count=128):
    w = BitWriter()
    parts = []
    for i in range(count):
        raw = b"" if empty else b"A" * (i % 3)
        parts.append(raw)
        literal_only_block(w, raw, final=i == count - 1)
    raw = b"".join(parts)
    return wrap(w.getvalue(), raw), raw


def embedded_candidate_stream():
    """Valid dynamic headers hidden inside stored literal data (decoys)."""
    def piece(data, single_eob=False, corrupt=False):
        w = BitWriter()
        literal_only_block(w, data, single_eob=single_eob)
        if corrupt:
            w.drop_last_bit()  # replace the 1-bit EOB with the tree's unused code
            w.put(1, 1)
        return w.getvalue()
    decoys = (b"candidate-boundary\x00" + piece(b"", single_eob=True) + piece(b"A")
              + piece(b"", single_eob=True, corrupt=True)) * 16
    w = BitWriter()
    w.raw(stored(decoys, final=False))
    suffix = b"A" * 2048
    literal_only_block(w, suffix)
    raw = decoys + suffix
    return wrap(w.getvalue(), raw), raw


def distance_window_stream(prefix_bytes=0):
    """Stored history then a fixed match at distance 257; CINFO=0 variant breaks the window."""
    prefix = random.Random(prefix_bytes).randbytes(prefix_bytes) if prefix_bytes else b""
    seed = bytes(range(256)) * 2
    w = BitWriter()
    history = prefix + seed
    for i in range(0, len(history), 65535):
        w.raw(stored(history[i:i + 65535], final=False))
    Block(w, True).match(3, 257).end()
    raw = history + history[-257:-254]
    payload = wrap(w.getvalue(), raw)
    return payload, header(cmf=0x08) + payload[2:], raw


def medium_compound_stream(history_error=False, window_error=False, reserved=False):
    """70000 bytes of 'A' from one fixed block of 258-byte matches."""
    w = BitWriter()
    blk = Block(w, True)
    if history_error:
        blk.match(258, 1)
        produced = 258
    else:
        blk.literal(65)
        produced = 1
    matches, literals = divmod(70000 - produced, 258)
    for _ in range(matches):
        blk.match(258, 1)
    blk.literals(b"A" * literals)
    raw = b"A" * 70000
    if window_error:
        blk.match(258, 257)
        raw += b"A" * 258
    blk.symbol(286 if reserved else 256)
    payload = wrap(w.getvalue(), raw)
    if window_error:
        payload = header(cmf=0x08) + payload[2:]
    return payload, raw


def fixed_summary_stream(invalid=False):
    prefix, literals = b"A" * 17, bytes(range(256)) * 4
    w = BitWriter()
    literal_only_block(w, prefix, final=False)
    blk = Block(w, True).literals(literals)
    if invalid:
        blk.symbol(286)
    blk.symbol(256)
    raw = prefix + literals
    return wrap(w.getvalue(), raw), raw


def invalid_repeat_stream(kind):
    symbol = 16 if kind == "repeat-before-length" else 18
    cl = [0] * 19
    cl[0] = cl[symbol] = 1
    w = BitWriter()
    w.put(1, 1).put(2, 2).put(0, 5).put(0, 5)
    count = max(4, CL_ORDER.index(symbol) + 1, CL_ORDER.index(0) + 1)
    w.put(count - 4, 4)
    for s in CL_ORDER[:count]:
        w.put(cl[s], 3)
    code = canonical(cl)[symbol]
    if symbol == 16:
        w.code(code).put(0, 2)
    else:
        w.code(code).put(127, 7).code(code).put(127, 7)
    return wrap(w.getvalue(), b"")


def dense_prefix_stored_stream(size=2 * 1024 ** 2):
    marker = invalid_repeat_stream("repeat-before-length")[2:-4]
    raw = (marker * ((size + len(marker) - 1) // len(marker)))[:size]
    chunks = [raw[i:i + 65535] for i in range(0, len(raw), 65535)]
    body = b"".join(stored(c, final=i == len(chunks) - 1) for i, c in enumerate(chunks))
    return wrap(body, raw), raw


def stored_stream(lengths, raw=None, padding=False):
    size = sum(lengths)
    if raw is None:
        raw = (bytes(range(251)) * ((size + 250) // 251))[:size]
    blocks, offset = [], 0
    for i, n in enumerate(lengths):
        block = stored(raw[offset:offset + n], i == len(lengths) - 1)
        if padding:
            block = bytes((block[0] | 0xF8,)) + block[1:]
        blocks.append(block)
        offset += n
    return wrap(b"".join(blocks), raw), raw


def deep_reference_stream(match_blocks):
    seed = bytes(range(256)) + b"\x00\x01"
    w = BitWriter()
    w.raw(stored(seed, final=False))
    for i in range(match_blocks):
        Block(w, i + 1 == match_blocks).match(258, 258).end()
    raw = seed * (match_blocks + 1)
    return wrap(w.getvalue(), raw), raw


def reserved_ending_stream(data, ending):
    """Fixed literals then a reserved LL symbol (286) or a reserved distance (30)."""
    w = BitWriter()
    blk = Block(w, True).literals(data)
    if ending == "reserved-ll":
        blk.symbol(286)
    else:
        blk.symbol(257)
        w.code(canonical(FIXED_D)[30])
    blk.symbol(256)
    return wrap(w.getvalue(), data)


def truncated_fixed_stream(data):
    """Fixed literals with the EOB and final header missing: bits run out."""
    w = BitWriter()
    Block(w, True).literals(data)
    return wrap(w.getvalue(), data)


def pinned_cases():
    """(name, payload, expected_size, max_candidates, max_blocks, status, output-or-None).

    `status` None means only "nonzero" is pinned.  Output None means unpinned.
    """
    M = 262144
    cases = []
    add = cases.append
    empty_payload = literal_only_stream(b"", single_eob=True)
    # test_decode.py:1063-1095 (limits and recovery)
    embedded, embedded_raw = embedded_candidate_stream()
    many, _ = many_dynamic_stream(True)
    add(("limit-candidates-0", empty_payload, 0, 0, 256, 23, b""))
    add(("limit-blocks-0", empty_payload, 0, 4096, 0, 23, b""))
    add(("limit-candidates-max", empty_payload, 0, 262145, 256, 23, b""))
    add(("limit-blocks-max", empty_payload, 0, 4096, 262145, 23, b""))
    add(("limit-empty-input", b"", 0, 4096, 256, 14, b""))
    add(("limit-bad-header", b"\x00" + empty_payload[1:], 0, 4096, 256, 15, b""))
    add(("limit-missing-final", wrap(stored(b"A", final=False), b"A"), 1, 4096, 256, 1, b"\x00"))
    add(("limit-candidate-overflow", embedded, len(embedded_raw), 1, 256, 18,
         bytes(len(embedded_raw))))
    add(("limit-block-cap", many, 0, 4096, 127, 9, b""))
    add(("limit-recovery", empty_payload, 0, 4096, 256, 0, b""))
    # test_decode.py:822-852 (framing precedence and window; both routes of discovery)
    for prefix_bytes in (65537, 1048577):
        payload, small_window, raw = distance_window_stream(prefix_bytes)
        damaged = b"\x07" + payload[3:-1] + bytes((payload[-1] ^ 1,))
        n = len(raw)
        add(("frame-window-%d" % prefix_bytes, header(cmf=0x88) + damaged, n, M, M, 15, bytes(n)))
        add(("frame-check-%d" % prefix_bytes, payload[:1] + bytes((payload[1] ^ 1,)) + damaged,
             n, M, M, 15, bytes(n)))
        add(("frame-gzip-%d" % prefix_bytes, b"\x1f\x8b" + damaged, n, M, M, 16, bytes(n)))
        add(("frame-dict-%d" % prefix_bytes, header(flags=0x20) + damaged, n, M, M, 17, bytes(n)))
        add(("frame-small-window-%d" % prefix_bytes, small_window, n, M, M, 6, bytes(n)))
        add(("frame-valid-%d" % prefix_bytes, payload, n, M, M, 0, raw))
    # test_decode.py:910-948 (medium compound precedence)
    payload, raw = medium_compound_stream()
    hist_res, _ = medium_compound_stream(history_error=True, reserved=True)
    win_res, win_raw = medium_compound_stream(window_error=True, reserved=True)
    window, _ = medium_compound_stream(window_error=True)
    add(("compound-valid", payload, len(raw), M, M, 0, raw))
    add(("compound-history-reserved", hist_res, len(raw), M, M, 4, bytes(len(raw))))
    add(("compound-window-reserved", win_res, len(win_raw), M, M, 4, bytes(len(win_raw))))
    add(("compound-window-overflow", window, len(win_raw) - 1, M, M, 7, bytes(len(win_raw) - 1)))
    add(("compound-adler", payload[:-1] + bytes((payload[-1] ^ 1,)), len(raw), M, M, 21, raw))
    # test_decode.py:1098-1118 (fixed region after an unaligned dynamic block)
    payload, raw = fixed_summary_stream()
    invalid, _ = fixed_summary_stream(invalid=True)
    add(("fixed-region-valid", payload, len(raw), 4096, 256, 0, raw))
    add(("fixed-region-reserved", invalid, len(raw), 4096, 256, 4, bytes(len(raw))))
    # test_decode.py:951-971 (medium repetition vs declared window)
    period = random.Random(91577).randbytes(257)
    raw = (period * ((262144 + 256) // 257))[:262144]
    payload = compressed(raw)
    add(("period-valid", payload, len(raw), M, M, 0, raw))
    add(("period-small-window", header(cmf=0x08) + payload[2:], len(raw), M, M, 6, bytes(len(raw))))
    # test_decode.py:882-907 (medium zeros, checksum)
    for size in (65536, 65537, 262144, 1048577):
        raw = bytes(size)
        payload = compressed(raw)
        add(("zeros-%d" % size, payload, size, M, M, 0, raw))
        add(("zeros-adler-%d" % size, payload[:-1] + bytes((payload[-1] ^ 1,)), size, M, M, 21,
             raw))
    # test_decode.py:781-819 (large stored stream errors)
    for size in (65537, 1048577):
        raw = random.Random(size).randbytes(size)
        payload = compressed(raw, level=0)
        add(("stored-%d-header" % size, b"\x00" + payload[1:], size, M, M, 15, bytes(size)))
        add(("stored-%d-adler" % size, payload[:-1] + bytes((payload[-1] ^ 1,)), size, M, M, 21,
             raw))
        bad = bytearray(payload)
        bad[2] = (bad[2] & 0xF8) | 7
        add(("stored-%d-reserved" % size, bytes(bad), size, M, M, None, bytes(size)))
        add(("stored-%d-short" % size, payload, size - 1, M, M, None, None))
        add(("stored-%d-long" % size, payload, size + 1, M, M, None, None))
    # test_stored_fast_decode.py:64-98 (stored stream statuses)
    payload, raw = stored_stream((32768, 32769))
    n = len(raw)
    bad_length = bytearray(payload)
    bad_length[5] ^= 1
    combined = bytes(bad_length[:-1]) + bytes((bad_length[-1] ^ 1,))
    missing_final = bytearray(payload)
    missing_final[2 + 5 + 32768] &= ~1
    add(("stored-length", bytes(bad_length), n, M, M, 4, bytes(n)))
    add(("stored-length-and-adler", combined, n, M, M, 4, bytes(n)))
    add(("stored-truncated-body", payload[:-5] + payload[-4:], n, M, M, 1, bytes(n)))
    add(("stored-extra-body", payload[:-4] + b"\0" * 5 + payload[-4:], n, M, M, 12, bytes(n)))
    add(("stored-header-and-body", b"\0" + combined[1:], n, M, M, 15, bytes(n)))
    add(("stored-dictionary-and-body", header(flags=0x20) + combined[2:], n, M, M, 17, bytes(n)))
    add(("stored-adler", payload[:-1] + bytes((payload[-1] ^ 1,)), n, M, M, 21, raw))
    add(("stored-short-output", payload, n - 5, M, M, 7, None))
    add(("stored-long-output", payload, n + 5, M, M, 11, bytes(n + 5)))
    add(("stored-missing-final", bytes(missing_final), n, M, M, 1, bytes(n)))
    marker = literal_only_stream(b"", single_eob=True)[2:-4]
    raw = (marker * ((65537 + len(marker) - 1) // len(marker)))[:65537]
    payload, _ = stored_stream((65535, 2), raw)
    add(("stored-candidate-overflow", payload, len(raw), 1, 256, 18, bytes(len(raw))))
    recovery, recovery_raw = stored_stream((65535, 2), b"\0" * 65537)
    add(("stored-candidate-recovery", recovery, len(recovery_raw), 1, 256, 0, recovery_raw))
    payload, raw = stored_stream((65535, 2))
    add(("stored-block-cap", payload, len(raw), 4096, 1, 9, bytes(len(raw))))
    add(("stored-block-recovery", compressed(bytes(len(raw))), len(raw), 4096, 1, 0,
         bytes(len(raw))))
    # test_stored_fast_decode.py:213-235 (26215 empty stored blocks, general route)
    payload, raw = stored_stream((0,) * 26215)
    add(("stored-empty-chain", payload, 0, M, M, 0, b""))
    add(("stored-empty-chain-adler", payload[:-1] + bytes((payload[-1] ^ 1,)), 0, M, M, 21, b""))
    # test_literal_lookahead.py:104-137 and test_small_shared_decode.py:108-137
    text = bytes((i * 7 + 32) % 95 + 32 for i in range(80))
    for ending in ("reserved-ll", "reserved-distance"):
        add(("small-%s" % ending, reserved_ending_stream(text, ending), len(text) + 3, M, M, 4,
             text + bytes(3)))
    add(("small-truncated", truncated_fixed_stream(text), len(text) + 3, M, M, 1, text + bytes(3)))
    good = fixed_stream(text)
    add(("small-checksum", good[:-1] + bytes((good[-1] ^ 1,)), len(text), M, M, 21, text))
    add(("small-bounds", good, 37, M, M, 7, text[:37]))
    add(("small-hex-reserved-ll", bytes.fromhex("789c731c030000000001"), 32, M, M, 4,
         b"A" + bytes(31)))
    add(("small-hex-reserved-distance", bytes.fromhex("789c73043e00000001"), 32, M, M, 4,
         b"A" + bytes(31)))
    # test_decode.py:641-657 (two dynamic blocks whose first match lacks history)
    ll = [0] * 258
    ll[256] = ll[257] = 1
    cl = [0] * 19
    cl[0] = cl[1] = 1
    w = BitWriter()
    for final in (False, True):
        Block(w, final, ll, [1], cl).match(3, 1).end()
    add(("history-first-block", wrap(w.getvalue(), b"A" * 6), 6, M, M, 6, bytes(6)))
    # test_decode.py:669-676 (declared window on the small route)
    payload, small_window, raw = distance_window_stream()
    add(("window-valid", payload, len(raw), M, M, 0, raw))
    add(("window-small", small_window, len(raw), M, M, 6, None))
    # test_decode.py:620-666 (wrapper/body mutations: nonzero only)
    raw = b"a checked fresh compressed stream\x00" * 128
    payload = compressed(raw)
    add(("mut-too-small", payload, len(raw) - 1, M, M, None, None))
    add(("mut-too-large", payload, len(raw) + 1, M, M, None, None))
    add(("mut-truncated-trailer", payload[:-1], len(raw), M, M, None, None))
    add(("mut-truncated-body", payload[:-6] + payload[-4:], len(raw), M, M, None, None))
    add(("mut-trailing-byte", payload + b"\x00", len(raw), M, M, None, None))
    add(("mut-concatenated", payload + payload, len(raw), M, M, None, None))
    add(("mut-reserved-block", wrap(b"\x07\x00", raw), len(raw), M, M, None, None))
    body = bytearray(stored(raw[:4000]))
    body[3] ^= 1
    add(("mut-stored-length", wrap(bytes(body), raw[:4000]), 4000, M, M, None, None))
    add(("mut-distance-before-history", wrap(b"\x03\x02\x00", b"AAA"), 3, M, M, None, None))
    for kind in ("repeat-before-length", "repeat-overflow"):
        add(("mut-" + kind, invalid_repeat_stream(kind), 0, M, M, None, None))
    return cases


def valid_streams():
    """(name, payload, raw) streams zlib accepts, covering block types and edge layouts."""
    out = []
    rng = random.Random(87123)
    dyn = bytes(rng.choices(range(16), weights=range(1, 17), k=32768))
    out.append(("stored-l0", compressed(bytes(range(256)) * 512, level=0), bytes(range(256)) * 512))
    text = b"fixed Huffman, overlapping history\x00" * 256
    out.append(("fixed", compressed(text, strategy=zlib.Z_FIXED), text))
    out.append(("dynamic", compressed(dyn), dyn))
    for raw in (b"", b"A" * 65536, bytes(range(251)) * 256):
        out.append(("fixed-%d" % len(raw), compressed(raw, strategy=zlib.Z_FIXED), raw))
    for i in range(8):
        p, r = alignment_stream(i)
        out.append(("alignment-%d" % i, p, r))
    for empty in (True, False):
        p, r = many_dynamic_stream(empty)
        out.append(("many-dynamic-%s" % empty, p, r))
    p, r = embedded_candidate_stream()
    out.append(("embedded", p, r))
    raw = bytes((14,)) * 65536
    out.append(("long-codes", literal_only_stream(raw, long_codes=True), raw))
    p, r = long_code_mix_stream()
    out.append(("long-code-mix", p, r))
    for blocks in (257, 1050):
        p, r = deep_reference_stream(blocks)
        out.append(("deep-%d" % blocks, p, r))
    for prefix in (65537, 1048577):
        p, _, r = distance_window_stream(prefix)
        out.append(("prefixed-window-%d" % prefix, p, r))
    p, r = dense_prefix_stored_stream()
    out.append(("dense-prefix-stored", p, r))
    out.append(("padded-final", _padded_final(), b"A"))
    for distance in (8192, 32768):
        first = random.Random(11219 + distance).randbytes(distance)
        c = zlib.compressobj()
        prefix = c.compress(first) + c.flush(zlib.Z_SYNC_FLUSH)
        repeat = first if distance < 32768 else first[1024:]
        out.append(("sync-history-%d" % distance, prefix + c.compress(repeat) + c.flush(),
                    first + repeat))
    return out


def _padded_final():
    w = BitWriter()
    Block(w, True).literal(65).end()
    body = bytearray(w.getvalue())
    body[-1] |= 0xFC
    return wrap(bytes(body), b"A")
