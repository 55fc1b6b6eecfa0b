"""Pins the CPU oracle before the GPU decoder's results are checked against it.

Checks: zlib.decompress / zlib.adler32 on valid streams (closed-form oracle),
the statuses and failed outputs the reference's own tests pin, brute-force
tree classification on tiny alphabets, an independent Python candidate scan,
and a mutation sweep where every disagreement with strict zlib must be one of
the reference's documented deviations.
"""

import itertools
import random
import zlib

import pytest

import deflate_writer as dw
from oracle import oracle


def strict_zlib(payload):
    d = zlib.decompressobj()
    raw = d.decompress(payload) + d.flush()
    if not d.eof or d.unused_data or d.unconsumed_tail:
        raise zlib.error("incomplete or trailing data")
    return raw


@pytest.mark.parametrize("size", [0, 1, 5551, 5552, 5553, 100000, 1 << 20])
def test_adler32_matches_zlib(size):
    data = random.Random(size).randbytes(size)
    assert oracle.adler32(data) == zlib.adler32(data)
    assert oracle.adler32(b"\xff" * size) == zlib.adler32(b"\xff" * size)


@pytest.mark.parametrize("name,payload,raw", dw.valid_streams(), ids=lambda v: v if isinstance(v, str) else "")
def test_valid_fixture_streams(name, payload, raw):
    assert strict_zlib(payload) == raw
    assert oracle.decompress(payload, len(raw)) == (raw, 0)
    assert oracle.inflate_general(payload, len(raw)) == (raw, 0)
    assert oracle.inflate_serial(payload, len(raw)) == (raw, 0)


@pytest.mark.parametrize("case", dw.pinned_cases(), ids=lambda c: c[0])
def test_pinned_statuses(case):
    name, payload, expected, max_candidates, max_blocks, status, output = case
    got, st = oracle.decompress(payload, expected, max_candidates, max_blocks)
    if status is None:
        assert st != 0
    else:
        assert st == status
    if output is not None:
        assert got == output


def test_writer_fixtures_agree_with_zlib():
    for kind in ("repeat-before-length", "repeat-overflow"):
        with pytest.raises(zlib.error):
            zlib.decompress(dw.invalid_repeat_stream(kind))
    payload, small, raw = dw.distance_window_stream()
    assert zlib.decompress(payload) == raw
    assert zlib.decompress(small) == raw  # zlib ignores CINFO; the codec enforces it
    with pytest.raises(zlib.error):
        zlib.decompress(dw.fixed_summary_stream(invalid=True)[0])
    for ending in ("reserved-ll", "reserved-distance"):
        with pytest.raises(zlib.error):
            zlib.decompress(dw.reserved_ending_stream(b"abc", ending))


def _kraft_class(lengths, empty_ok, single_ok, limit=15):
    """Independent classification: 0 valid, 3 invalid (RFC 1951 3.2.2 + the codec's rules)."""
    if any(n > limit for n in lengths):
        return 3
    used = [n for n in lengths if n]
    if not used:
        return 0 if empty_ok else 3
    total = sum(2 ** (limit - n) for n in used)
    if total > 2 ** limit:
        return 3
    if total < 2 ** limit and not (single_ok and used == [1]):
        return 3
    return 0


def test_tree_classification_brute_force():
    for n in range(1, 5):
        for lengths in itertools.product(range(0, 5), repeat=n):
            for empty_ok, single_ok in ((0, 0), (0, 1), (1, 1)):
                want = _kraft_class(lengths, empty_ok, single_ok, limit=4)
                assert oracle.huff_build_status(lengths, empty_ok, single_ok, limit=4) == want


def _huffman_lengths(weights):
    """Code lengths of a Huffman tree over `weights` (heap construction)."""
    import heapq
    heap = [(w, i, (i,)) for i, w in enumerate(weights)]
    heapq.heapify(heap)
    depth = [0] * len(weights)
    tick = len(weights)
    while len(heap) > 1:
        w1, _, a = heapq.heappop(heap)
        w2, _, b = heapq.heappop(heap)
        for s in a + b:
            depth[s] += 1
        heapq.heappush(heap, (w1 + w2, tick, a + b))
        tick += 1
    return depth


def test_tiny_random_trees_decode_like_zlib():
    rng = random.Random(5)
    checked = 0
    while checked < 200:
        k = rng.randint(1, 40)
        symbols = rng.sample(range(256), k)
        depth = _huffman_lengths([rng.randint(1, 1000) for _ in range(k + 1)])
        if max(depth) > 15:
            continue
        ll = [0] * 257
        for s, n in zip(symbols + [256], depth):
            ll[s] = n
        data = bytes(rng.choice(symbols) for _ in range(rng.randint(0, 300)))
        w = dw.BitWriter()
        dw.Block(w, True, ll, [0]).literals(data).end()
        payload = dw.wrap(w.getvalue(), data)
        assert strict_zlib(payload) == data
        assert oracle.decompress(payload, len(data)) == (data, 0)
        assert oracle.inflate_general(payload, len(data)) == (data, 0)
        checked += 1


def _py_dynamic_valid(body, start):
    """Independent Python check of a dynamic header at `start` (RFC 1951 3.2.7)."""
    nbits = len(body) * 8
    pos = start

    def take(n):
        nonlocal pos
        if pos + n > nbits:
            raise EOFError
        v = 0
        for i in range(n):
            v |= ((body[(pos + i) >> 3] >> ((pos + i) & 7)) & 1) << i
        pos += n
        return v

    def decoder(lengths):
        codes = dw.canonical(lengths)
        return {(c, n): s for s, (c, n) in codes.items()}, max(lengths)

    def decode(table):
        mapping, maximum = table
        code = 0
        for n in range(1, maximum + 1):
            code = (code << 1) | take(1)
            if (code, n) in mapping:
                return mapping[(code, n)]
        raise ValueError

    try:
        take(1)
        if take(2) != 2:
            return False
        nl, nd, nc = take(5) + 257, take(5) + 1, take(4) + 4
        if nl > 286:
            return False
        cl = [0] * 19
        for i in range(nc):
            cl[dw.CL_ORDER[i]] = take(3)
        if _kraft_class(cl, 0, 0, 7):
            return False
        table = decoder(cl)
        lengths = []
        while len(lengths) < nl + nd:
            s = decode(table)
            if s < 16:
                lengths.append(s)
            elif s == 16:
                if not lengths:
                    return False
                lengths += [lengths[-1]] * (take(2) + 3)
            elif s == 17:
                lengths += [0] * (take(3) + 3)
            else:
                lengths += [0] * (take(7) + 11)
            if len(lengths) > nl + nd:
                return False
        if not lengths[256]:
            return False
        return (_kraft_class(lengths[:nl], 0, 1) == 0
                and _kraft_class(lengths[nl:], 1, 1) == 0)
    except (EOFError, ValueError):
        return False


def test_candidate_count_matches_independent_scan():
    streams = [dw.alignment_stream(3)[0], dw.many_dynamic_stream(False, count=12)[0],
               dw.compressed(bytes(random.Random(1).choices(b"abcdefgh", k=3000)))]
    payload, _ = dw.embedded_candidate_stream()
    streams.append(payload[:1500] + payload[-6:])
    for payload in streams:
        body = payload[2:-4]
        count = 1 + sum(_py_dynamic_valid(body, s) for s in range(1, len(body) * 8))
        seeds = oracle.candidate_count(body) - count
        assert seeds >= 0
        assert oracle.candidate_count(body) == count + seeds
        # Independent seed count.
        py_seeds = 0
        for byte in range(1, len(body)):
            if len(body) - byte < 5:
                continue
            n = body[byte] | body[byte + 1] << 8
            comp = body[byte + 2] | body[byte + 3] << 8
            if n ^ comp != 0xFFFF or n + 4 >= len(body) - byte:
                continue
            before = body[byte - 1] << 8 | (body[byte - 2] if byte >= 2 else 0)
            possible = any(byte * 8 >= gap and (before >> (17 - gap)) & 3 == 0
                           for gap in range(3, 11))
            if possible and (body[byte + 4 + n] >> 1) & 3 == 1:
                py_seeds += 1
        assert seeds == py_seeds


@pytest.mark.parametrize("seed", range(6))
def test_mutations_agree_with_strict_zlib(seed):
    rng = random.Random(seed)
    sources = [dw.compressed(bytes(rng.choices(b"abcd \n", k=3000)), level) for level in (1, 6, 9)]
    sources.append(dw.compressed(rng.randbytes(2000), 0))
    sources.append(dw.compressed(b"xyz" * 500, 6, zlib.Z_FIXED))
    disagreements = 0
    for _ in range(300):
        src = rng.choice(sources)
        raw = zlib.decompress(src)
        data = bytearray(src)
        for _ in range(rng.randint(1, 3)):
            i = rng.randrange(2, len(data) - 4)
            data[i] ^= 1 << rng.randrange(8)
        payload = bytes(data[:-4]) + zlib.adler32(b"").to_bytes(4, "big")
        try:
            want = strict_zlib(payload)
        except zlib.error:
            want = None
        size = len(want) if want is not None else len(raw)
        payload = payload[:-4] + zlib.adler32(want if want is not None else raw).to_bytes(4, "big")
        try:
            want = strict_zlib(payload)
        except zlib.error:
            want = None
        for route in (oracle.inflate_serial, oracle.inflate_general):
            got, status = route(payload, size)
            if want is not None and len(want) == size:
                assert (got, status) == (want, 0)
            elif status == 0:
                disagreements += 1
                assert _hdist_over_30(payload), "oracle accepted a stream zlib rejects"
    assert disagreements < 30


def _hdist_over_30(payload):
    """True if some dynamic block declares HDIST > 29 (the reference accepts it)."""
    body = payload[2:-4]
    for start in range(len(body) * 8 - 17):
        b = int.from_bytes(body[start // 8:start // 8 + 4].ljust(4, b"\0"), "little") >> (start % 8)
        if (b >> 1) & 3 == 2 and ((b >> 8) & 31) >= 30:
            return True
    return False
