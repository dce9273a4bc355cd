"""ORACLE: test infrastructure, never the product.

CPU restatements of the reference's algorithms on the serve path, each function citing the reference file:line it
follows, used for comparison by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg only. The product path
(tierstream_amd) never imports, links or calls anything here.

Contents:
  xxh64_oracle.c      XXH64 and the verify checkpoint layout (liboracle.so)
  synth.py            the synthetic byte generator (numpy): the words the product's device generator must give
  fixtures.py         small synthetic models (source file + desc-v1 JSON), engine checksums, route streams
  score_profile.py    TSSCPRF1 score-profile writer (hashlib SHA-256)
  ref.py              ctypes driver of _ref/libtsref_harness.so: the reference's CPU backend through its C ABI, and its
                      DgCore on an immediate transport (placement oracle) or a memcpy transport (the CPU baseline)
  ref_harness.cpp     the C++ side of that driver (compiled against the reference's sources, never copied)
  _ref/ (built)       libtsref.so and libtsref_harness.so: the reference's own CPU library compiled from its sources by
                      the Makefile (target `ref`), and the harness linked with it
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libtsref.so"

_olib = None


def olib() -> C.CDLL:
    global _olib
    if _olib is None:
        if not LIB.exists():
            raise RuntimeError(f"{LIB} is not built (make -C oracle)")
        _olib = C.CDLL(str(LIB))
        u64 = C.c_uint64
        _olib.oracle_xxh64.restype = u64
        _olib.oracle_xxh64.argtypes = [C.c_void_p, C.c_size_t]
        _olib.oracle_xxh64_extents.restype = u64
        _olib.oracle_xxh64_extents.argtypes = [C.POINTER(C.c_void_p), C.POINTER(u64), C.c_uint32]
        _olib.oracle_checkpoints.restype = u64
        _olib.oracle_checkpoints.argtypes = [C.POINTER(C.c_void_p), C.POINTER(u64), C.c_uint32, u64,
                                             C.POINTER(u64), u64, C.POINTER(u64)]
    return _olib


def xxh64(data) -> int:
    """XXH64 seed 0 of a bytes-like / numpy array (reference src/xxh64.cpp:106-110)."""
    import numpy as np
    a = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8) if isinstance(data, (bytes, bytearray))
                             else data).view(np.uint8)
    return int(olib().oracle_xxh64(a.ctypes.data_as(C.c_void_p), a.nbytes))


def xxh64_extents(arrays) -> int:
    import numpy as np
    arrs = [np.ascontiguousarray(a).view(np.uint8) for a in arrays]
    ptrs = (C.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
    sizes = (C.c_uint64 * len(arrs))(*[a.nbytes for a in arrs])
    return int(olib().oracle_xxh64_extents(ptrs, sizes, len(arrs)))


def checkpoints(arrays, seg: int):
    """(states uint64[4k], digest) of arrays back to back, per the tsa.h checkpoint layout."""
    import numpy as np
    arrs = [np.ascontiguousarray(a).view(np.uint8) for a in arrays]
    ptrs = (C.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
    sizes = (C.c_uint64 * len(arrs))(*[a.nbytes for a in arrs])
    cap = sum(a.nbytes // seg + 2 for a in arrs) + 1
    states = np.zeros(4 * cap, dtype=np.uint64)
    dig = C.c_uint64(0)
    k = olib().oracle_checkpoints(ptrs, sizes, len(arrs), seg, states.ctypes.data_as(C.POINTER(C.c_uint64)), cap,
                                  C.byref(dig))
    if k == 0:
        raise ValueError("invalid checkpoint layout")
    return states[: 4 * k], int(dig.value)
