"""Frame-vector adapter: CPU checks of its rules, GPU decode of zlib frame vectors.

The adapter follows the reference's PyCBC integration
(integrations/pycbc/gwf_deflate_jax.py:22-55): codec errors become frame errors
(a preset dictionary counts as a malformed frame), a missing backend or an
unsupported vector becomes ``GWFDeflateUnavailable``, and decoded bytes are
reinterpreted as the vector's samples.  Expected samples come from NumPy on
the CPU, so the GPU result is checked against an independent reading of the
same bytes.
"""

import zlib

import numpy as np
import pytest

import workloads


def _vector(samples, type_code, little=True, diff=False):
    from cuda_zlib import gwf
    dtype = gwf.SAMPLE_TYPES[type_code]
    values = np.ascontiguousarray(samples, dtype=dtype)
    if diff:
        values = np.diff(values, prepend=values.dtype.type(0)).astype(dtype)
    if not little:
        values = values.astype(dtype.newbyteorder(">"))
    method = gwf.CompressionKind.DIFF_GZIP if diff else gwf.CompressionKind.GZIP
    compress = int(method) | (gwf.LITTLE_ENDIAN_FLAG if little else 0)
    return gwf.FrVect(compress, type_code, values.size, zlib.compress(values.tobytes(), 6))


def test_vector_fields():
    from cuda_zlib import gwf
    v = gwf.FrVect(0x101, 3, 10, b"")
    assert v.kind is gwf.CompressionKind.GZIP and v.little_endian
    assert v.dtype == np.dtype("<f4") and v.nbytes == 40
    assert gwf.FrVect(3, 1, 4, b"").kind is gwf.CompressionKind.DIFF_GZIP
    assert not gwf.FrVect(3, 1, 4, b"").little_endian
    with pytest.raises(gwf.GWFDeflateUnavailable):
        gwf.FrVect(0x105, 1, 4, b"").kind  # zero suppression is not zlib
    with pytest.raises(gwf.GWFDeflateUnavailable):
        gwf.FrVect(0x101, 8, 4, b"").dtype  # strings have no numeric samples


@pytest.mark.parametrize("raised,payload,expected", [
    ("CodecError", b"x", "GWFFormatError"),
    ("UnsupportedStream", b"\x78\x01", "GWFDeflateUnavailable"),
    ("UnsupportedStream", b"\x78\x20", "GWFFormatError"),  # preset-dictionary flag
    ("BackendUnavailable", b"x", "GWFDeflateUnavailable"),
])
def test_codec_errors_map_to_frame_errors(monkeypatch, raised, payload, expected):
    import cuda_zlib
    from cuda_zlib import _codec, gwf

    def failing(*args, **kwargs):
        raise getattr(cuda_zlib, raised)("injected")

    monkeypatch.setattr(_codec, "decompress_zlib", failing)
    with pytest.raises(getattr(gwf, expected)):
        gwf.decompress_zlib(payload, 0)


def test_unsupported_vectors_are_refused_before_decoding(monkeypatch):
    from cuda_zlib import _codec, gwf
    monkeypatch.setattr(_codec, "decompress_zlib",
                        lambda *a, **k: pytest.fail("decoder called for an unsupported vector"))
    with pytest.raises(gwf.GWFDeflateUnavailable):
        gwf.decode_fr_vect_deflate(gwf.FrVect(0x101, 8, 3, b""))
    with pytest.raises(gwf.GWFDeflateUnavailable):
        gwf.decode_fr_vect_deflate(gwf.FrVect(0x100, 3, 3, b""))  # raw, not compressed


def _strain(n):
    return np.frombuffer(workloads.strain(n, 11), dtype="<f4")


CASES = [
    ("float32-strain-le", lambda: _strain(200000), 3, True, False),
    ("float32-strain-be", lambda: _strain(70001), 3, False, False),
    ("float64-be", lambda: _strain(30000).astype(np.float64), 2, False, False),
    ("int16-le", lambda: (np.arange(100000) % 2000 - 1000).astype(np.int16), 1, True, False),
    ("int16-diff-be", lambda: (np.cumsum(np.random.default_rng(1).integers(-3, 4, 150000)) % 30000)
     .astype(np.int16), 1, False, True),
    ("int32-diff-le", lambda: np.random.default_rng(2).integers(-2**31, 2**31, 50000)
     .astype(np.int32), 4, True, True),
    ("uint8", lambda: np.frombuffer(workloads.text_like(90000, np.random.default_rng(3)), np.uint8),
     12, True, False),
    ("complex64-be", lambda: (_strain(20000) + 1j * _strain(20000)[::-1]).astype(np.complex64),
     6, False, False),
    ("empty", lambda: np.zeros(0, np.float32), 3, True, False),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_gpu_decode_matches_numpy(gpu, no_cpu_codec, case):
    from cuda_zlib import gwf
    _, make, type_code, little, diff = case
    samples = make()
    vector = _vector(samples, type_code, little, diff)
    with no_cpu_codec:
        decoded = gwf.decode_fr_vect_deflate(vector, 0)
    got = decoded.cpu().numpy()
    assert got.dtype == gwf.SAMPLE_TYPES[type_code].newbyteorder("=")
    np.testing.assert_array_equal(got, np.asarray(samples, dtype=got.dtype))


@pytest.mark.gpu
def test_gpu_encoded_vector_round_trips_through_zlib_and_the_gpu(gpu):
    from cuda_zlib import gwf
    samples = _strain(300000)
    vector = gwf.encode_fr_vect_deflate(samples, 3, little_endian=False)
    assert zlib.decompress(vector.payload) == samples.astype(">f4").tobytes()
    np.testing.assert_array_equal(gwf.decode_fr_vect_deflate(vector, 0).cpu().numpy(), samples)
    ints = (np.arange(80000) * 7 % 1000).astype(np.int32)
    diffed = gwf.encode_fr_vect_deflate(ints, 4, difference=True)
    np.testing.assert_array_equal(gwf.decode_fr_vect_deflate(diffed, 0).cpu().numpy(), ints)


@pytest.mark.gpu
def test_gpu_corrupt_payload_is_a_format_error(gpu):
    from cuda_zlib import gwf
    vector = _vector(_strain(50000), 3)
    bad = gwf.FrVect(vector.compress, vector.type_code, vector.n_data,
                     vector.payload[:-1] + bytes([vector.payload[-1] ^ 0x40]))
    with pytest.raises(gwf.GWFFormatError):
        gwf.decode_fr_vect_deflate(bad, 0)
    short = gwf.FrVect(vector.compress, vector.type_code, vector.n_data + 1, vector.payload)
    with pytest.raises(gwf.GWFFormatError):
        gwf.decode_fr_vect_deflate(short, 0)
