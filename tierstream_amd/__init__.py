"""tierstream_amd: the MI355X build of tierstream's serve path.

The product is the native library libtierstream_amd.so (the ss_* / ts_* C ABI of strix-stream plus the tsa_* device
byte-path extensions). This module is the host-side mirror the tests and the benchmark use: ctypes declarations of the
C ABI (same names, argument meanings and status codes as reference include/strix_stream/ss.h), thin helpers, and
errors raised as SsError(status, message) the way the reference C tests CHECK_OK a status.

Loading fails loudly when the library has not been built (python -m tierstream_amd.build, or __graft_entry__.build()):
there is no Python or CPU fallback for any call.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libtierstream_amd.so"
ENGINE_PATH = PKG / "libtsa_engine.so"

# ss_status
SS_OK, SS_E_INVALID, SS_E_DESC, SS_E_IO, SS_E_NOMEM, SS_E_BACKEND, SS_E_CAPACITY, SS_E_HASH, SS_E_UNSUPPORTED = range(9)
STATUS_NAMES = {0: "SS_OK", 1: "SS_E_INVALID", 2: "SS_E_DESC", 3: "SS_E_IO", 4: "SS_E_NOMEM", 5: "SS_E_BACKEND",
                6: "SS_E_CAPACITY", 7: "SS_E_HASH", 8: "SS_E_UNSUPPORTED", 9: "SS_E_RECIPE"}
SS_TIER_RESIDENT, SS_TIER_PINNED, SS_TIER_DISK, SS_TIER_PAIR, SS_TIER_RESIDENT_BACKED = range(5)
SS_BACKEND_CPU, SS_BACKEND_CUDA, SS_BACKEND_HIP = range(3)
SS_FORWARD_HOST, SS_FORWARD_DEVICE_GATED = 0, 1
TSA_MAX_EXTENTS = 4
TSA_SCATTER_BLOCK_BYTES = 16384


class SsError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status
        self.message = message


class TsaExtent(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("bytes", C.c_uint64)]


class TsaUnit(C.Structure):
    _fields_ = [("ext", TsaExtent * TSA_MAX_EXTENTS), ("n_ext", C.c_uint32), ("reserved", C.c_uint32)]


class TsaVerifyUnit(C.Structure):
    _fields_ = [("ext", TsaExtent * TSA_MAX_EXTENTS), ("n_ext", C.c_uint32), ("reserved", C.c_uint32),
                ("seg_first", C.c_uint64), ("states", C.c_void_p), ("digest", C.c_uint64), ("total", C.c_uint64)]


class TsaArenaVerify(C.Structure):
    _fields_ = [("arena", C.c_void_p * TSA_MAX_EXTENTS), ("part_bytes", C.c_uint64 * TSA_MAX_EXTENTS),
                ("n_parts", C.c_uint32), ("reserved", C.c_uint32), ("seg_bytes", C.c_uint64),
                ("states_dev", C.c_void_p), ("digests_dev", C.c_void_p)]


class TsaScatterJob(C.Structure):
    _fields_ = [("src", C.c_void_p), ("dst", C.c_void_p * TSA_MAX_EXTENTS), ("bytes", C.c_uint64 * TSA_MAX_EXTENTS),
                ("n_parts", C.c_uint32), ("reserved", C.c_uint32), ("block_first", C.c_uint64)]


_lib = None


def lib() -> C.CDLL:
    """The product library (loaded once). Raises if it is not built: nothing falls back to Python."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run python -m tierstream_amd.build (no fallback exists)")
        _lib = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        _declare(_lib)
    return _lib


def _declare(L: C.CDLL) -> None:
    st = C.c_int
    vp, u32, u64, i32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int32
    sigs = {
        "ss_last_error": (C.c_char_p, []),
        "ss_abi_version": (C.c_int, []),
        "tsa_xxh64_digest": (st, [vp, u32, vp, vp]),
        "tsa_xxh64_host": (u64, [vp, u64]),
        "tsa_checkpoint_count": (u64, [C.POINTER(u64), u32, u64]),
        "tsa_xxh64_checkpoints": (st, [C.POINTER(TsaUnit), u64, C.POINTER(u64), u64, C.POINTER(u64)]),
        "tsa_xxh64_verify": (st, [vp, u32, u64, u64, vp, vp]),
        "tsa_xxh64_verify_slots": (st, [vp, C.POINTER(u32), C.POINTER(i32), u32, vp, vp]),
        "tsa_xxh64_scatter_verify_slots": (st, [vp, C.POINTER(u32), C.POINTER(i32), u32, vp, vp, vp]),
        "tsa_scatter_blocks": (u64, [C.POINTER(u64), u32]),
        "tsa_scatter": (st, [vp, u32, u64, vp]),
        "tsa_synth": (st, [vp, u64, u64, u64, u64, u32, C.c_float, vp]),
        "tsa_device_count": (st, [C.POINTER(C.c_int)]),
        "tsa_set_device": (st, [C.c_int]),
        "tsa_malloc": (st, [C.POINTER(vp), u64]),
        "tsa_free": (st, [vp]),
        "tsa_host_alloc": (st, [C.POINTER(vp), u64]),
        "tsa_host_free": (st, [vp]),
        "tsa_memcpy": (st, [vp, vp, u64, C.c_int, vp]),
        "tsa_memset": (st, [vp, C.c_int, u64, vp]),
        "tsa_stream_create": (st, [C.POINTER(vp)]),
        "tsa_stream_destroy": (st, [vp]),
        "tsa_stream_sync": (st, [vp]),
        "tsa_device_sync": (st, []),
        "tsa_event_create": (st, [C.POINTER(vp)]),
        "tsa_event_destroy": (st, [vp]),
        "tsa_event_record": (st, [vp, vp]),
        "tsa_event_sync": (st, [vp]),
        "tsa_event_elapsed_ms": (st, [vp, vp, C.POINTER(C.c_float)]),
    }
    for name, (res, args) in sigs.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _ = i32


def check(status: int) -> None:
    if status != SS_OK:
        msg = lib().ss_last_error()
        raise SsError(status, msg.decode() if msg else "")


# ---- device memory plumbing (numpy <-> HBM) -------------------------------------------------------------------------
class DeviceBuffer:
    """hipMalloc'd bytes, freed on close / garbage collection."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().tsa_malloc(C.byref(p), self.nbytes))
        self.ptr = p.value

    def close(self) -> None:
        if self.ptr:
            lib().tsa_free(C.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def upload(self, arr, offset: int = 0, stream=None) -> None:
        import numpy as np
        a = np.ascontiguousarray(arr)
        assert offset + a.nbytes <= self.nbytes
        check(lib().tsa_memcpy(C.c_void_p(self.ptr + offset), a.ctypes.data_as(C.c_void_p), a.nbytes, 0, stream))
        check(lib().tsa_stream_sync(stream))

    def download(self, nbytes: int | None = None, offset: int = 0, dtype="uint8", stream=None):
        import numpy as np
        n = self.nbytes - offset if nbytes is None else int(nbytes)
        out = np.empty(n, dtype=np.uint8)
        check(lib().tsa_memcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr + offset), n, 1, stream))
        check(lib().tsa_stream_sync(stream))
        return out.view(dtype)


def gpu_count() -> int:
    n = C.c_int(0)
    st = lib().tsa_device_count(C.byref(n))
    return n.value if st == SS_OK else 0


# ---- device byte path helpers ----------------------------------------------------------------------------------------
def make_unit(extents) -> TsaUnit:
    """extents: [(ptr, bytes), ...] (1..4)."""
    u = TsaUnit()
    assert 1 <= len(extents) <= TSA_MAX_EXTENTS
    for i, (p, b) in enumerate(extents):
        u.ext[i].ptr = p
        u.ext[i].bytes = b
    u.n_ext = len(extents)
    return u


def upload_struct_array(structs) -> DeviceBuffer:
    import numpy as np
    n = len(structs)
    size = C.sizeof(type(structs[0])) if n else 8
    raw = (C.c_char * (size * max(n, 1)))()
    for i, s in enumerate(structs):
        C.memmove(C.addressof(raw) + i * size, C.addressof(s), size)
    buf = DeviceBuffer(size * max(n, 1))
    buf.upload(np.frombuffer(raw, dtype=np.uint8))
    return buf


def device_digests(units) -> list[int]:
    """XXH64 of each unit (TsaUnit over device memory), computed by the device kernel."""
    import numpy as np
    n = len(units)
    table = upload_struct_array(units)
    out = DeviceBuffer(8 * max(n, 1))
    check(lib().tsa_xxh64_digest(C.c_void_p(table.ptr), n, C.c_void_p(out.ptr), None))
    check(lib().tsa_stream_sync(None))
    return [int(x) for x in out.download(8 * n).view(np.uint64)]


def checkpoint_count(extent_bytes, seg_bytes: int) -> int:
    arr = (C.c_uint64 * len(extent_bytes))(*extent_bytes)
    return int(lib().tsa_checkpoint_count(arr, len(extent_bytes), seg_bytes))


def host_checkpoints(host_arrays, seg_bytes: int):
    """Checkpoints + digest of host numpy arrays laid out as extents (the library's host side of verify)."""
    import numpy as np
    u = make_unit([(a.ctypes.data, a.nbytes) for a in host_arrays])
    n = checkpoint_count([a.nbytes for a in host_arrays], seg_bytes)
    states = np.zeros(4 * max(n, 1), dtype=np.uint64)
    dig = C.c_uint64(0)
    check(lib().tsa_xxh64_checkpoints(C.byref(u), seg_bytes, states.ctypes.data_as(C.POINTER(C.c_uint64)), n,
                                      C.byref(dig)))
    return states[: 4 * n], int(dig.value)
