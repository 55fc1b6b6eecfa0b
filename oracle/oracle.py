"""ctypes wrapper over the CPU oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, to check results against.  The product never imports it.
"""

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "liboracle.so")
MAX_CANDIDATES = 262144
MAX_BLOCKS = 262144
_lib = None


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            import importlib.util
            spec = importlib.util.spec_from_file_location("oracle_build", os.path.join(HERE, "build.py"))
            module = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(module)
            module.build()
        lib = ctypes.CDLL(LIBRARY)
        p, u64, u32, i64 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int64
        lib.oracle_adler32.argtypes = [p, u64]
        lib.oracle_adler32.restype = u32
        lib.oracle_inflate_serial.argtypes = [p, u64, p, u64, u32]
        lib.oracle_inflate_serial.restype = u32
        lib.oracle_inflate_general.argtypes = [p, u64, p, u64, u64, u32]
        lib.oracle_inflate_general.restype = u32
        lib.oracle_decompress.argtypes = [p, u64, p, u64, i64, i64]
        lib.oracle_decompress.restype = u32
        lib.oracle_candidate_count.argtypes = [p, u64]
        lib.oracle_candidate_count.restype = u64
        lib.oracle_huff_build_status.argtypes = [p, u32, ctypes.c_int, ctypes.c_int, u32]
        lib.oracle_huff_build_status.restype = u32
        _lib = lib
    return _lib


def _in(data):
    return ctypes.c_char_p(bytes(data)) if len(data) else None


def adler32(data):
    return _load().oracle_adler32(_in(data), len(data))


def _run(fn, payload, expected, *extra):
    out = ctypes.create_string_buffer(max(1, expected))
    status = fn(_in(payload), len(payload), out, expected, *extra)
    return out.raw[:expected], int(status)


def decompress(payload, expected, max_candidates=MAX_CANDIDATES, max_blocks=MAX_BLOCKS):
    """(output, status) with the codec's route selection and semantics."""
    return _run(_load().oracle_decompress, payload, expected, max_candidates, max_blocks)


def inflate_serial(payload, expected, max_blocks=MAX_BLOCKS):
    return _run(_load().oracle_inflate_serial, payload, expected, max_blocks)


def inflate_general(payload, expected, max_candidates=MAX_CANDIDATES, max_blocks=MAX_BLOCKS):
    return _run(_load().oracle_inflate_general, payload, expected, max_candidates, max_blocks)


def candidate_count(body):
    return int(_load().oracle_candidate_count(_in(body), len(body)))


def huff_build_status(lengths, empty_ok, single_ok, limit=15):
    data = bytes(lengths)
    return int(_load().oracle_huff_build_status(_in(data), len(data), int(empty_ok),
                                                int(single_ok), limit))
