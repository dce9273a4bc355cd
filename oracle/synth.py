"""ORACLE: the synthetic byte generator restated in numpy (test infrastructure only).

Word i of stream `sid` under `seed` is mix64(key + (i + 1) * 0x9E3779B97F4A7C15) with key = mix64(seed ^ sid *
0xD1B54A32D192ED03) and mix64 the splitmix64 finalizer; kind 0 stores each word little-endian (uniform bytes). The
product's device generator (tsa_synth) must give the same bytes for kind 0 (integer arithmetic, bit-exact). Kind 1
(bf16 N(0, sigma), Box-Muller in float32) is restated for distribution checks only: the device's logf / sincosf may
differ from numpy's in the last ulp, so its bytes are not compared bit for bit. Kind 2 (Q4 blocks: an fp16 scale and
16 bytes of 4-bit values per 18 bytes) is integer arithmetic and compared bit for bit.

Byte-level fixture helpers (the closed form the reference's own tests use, tests/fixture.hpp:16-22) live here too.
"""
from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15
SID_ODD = 0xD1B54A32D192ED03


def mix64_scalar(z: int) -> int:
    z &= M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def key(seed: int, sid: int) -> int:
    seed, sid = int(seed), int(sid)
    return mix64_scalar((seed ^ ((sid * SID_ODD) & M64)) & M64)


def _mix64(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def words(seed: int, sid: int, first: int, n: int) -> np.ndarray:
    k = np.uint64(key(seed, sid))
    i = np.arange(first + 1, first + 1 + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix64(k + i * np.uint64(GOLDEN))


def uniform_bytes(seed: int, sid: int, offset: int, nbytes: int) -> np.ndarray:
    """kind 0: nbytes (a multiple of 8) starting at byte `offset` (a multiple of 8) of the stream."""
    assert nbytes % 8 == 0 and offset % 8 == 0
    return words(seed, sid, offset // 8, nbytes // 8).astype("<u8").view(np.uint8)


def bf16_normal(seed: int, sid: int, offset: int, nbytes: int, sigma: float) -> np.ndarray:
    """kind 1 in numpy float32 (distribution checks only)."""
    assert nbytes % 8 == 0 and offset % 8 == 0
    n_out = nbytes // 8
    w = words(seed, sid, 2 * (offset // 8), 2 * n_out)
    u1 = ((w >> np.uint64(32)).astype(np.float32) + np.float32(0.5)) * np.float32(2.3283064365386963e-10)
    u2 = ((w & np.uint64(0xFFFFFFFF)).astype(np.float32) + np.float32(0.5)) * np.float32(2.3283064365386963e-10)
    r = np.float32(sigma) * np.sqrt(np.float32(-2.0) * np.log(u1))
    ang = np.float32(6.283185307179586) * u2
    z = np.stack([r * np.cos(ang), r * np.sin(ang)], axis=1).astype(np.float32).reshape(-1)
    x = z.view(np.uint32)
    rne = ((x + np.uint32(0x7FFF) + ((x >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    return rne.view(np.uint8)


def q4_blocks(seed: int, sid: int, offset: int, nbytes: int) -> np.ndarray:
    """kind 2: Q4 blocks of 18 bytes from the stream's byte 0: block b = the fp16 scale 0x2000 | (word 3b & 0x3FF)
    little-endian, then the 16 bytes of words 3b + 1 and 3b + 2 little-endian. Integer arithmetic: bit-exact."""
    j = np.arange(offset, offset + nbytes, dtype=np.uint64)
    b = j // np.uint64(18)
    o = (j - b * np.uint64(18)).astype(np.int64)
    b0 = int(b[0]) if nbytes else 0
    nb = (int(b[-1]) - b0 + 1) if nbytes else 0
    w = words(seed, sid, 3 * b0, 3 * nb).reshape(nb, 3) if nb else np.zeros((0, 3), np.uint64)
    scale = (np.uint64(0x2000) | (w[:, 0] & np.uint64(0x3FF))).astype("<u2").view(np.uint8).reshape(nb, 2)
    block = np.concatenate([scale, w[:, 1:].astype("<u8").view(np.uint8).reshape(nb, 16)], axis=1)  # [nb][18]
    return block[(b - np.uint64(b0)).astype(np.int64), o]


def fixture_byte_at(L: int, u: int, part: int, i: np.ndarray) -> np.ndarray:
    """Closed-form test bytes (the shape of the reference's tests/fixture.hpp:16-22): a byte of (layer, unit, part,
    offset) that differs between neighbours, so a unit served from the wrong place never checksums right."""
    i = np.asarray(i, dtype=np.uint64)
    h = (i * np.uint64(2654435761) + np.uint64(L * 1000003 + u * 7919 + part * 104729 + 17)) & np.uint64(0xFFFFFFFF)
    return ((h ^ (h >> np.uint64(13))) & np.uint64(0xFF)).astype(np.uint8)
