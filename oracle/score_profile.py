"""Test infrastructure: TSSCPRF1 score profiles written from their published format (reference src/dg_score.hpp:4-8,
include/strix_stream/ss.h:739-744; writer reference src/dg_score.cpp:103-120, identity :45-62), with Python's hashlib
as the SHA-256. Only tests use it: it makes the profiles a context loads and the broken ones it must refuse.

Layout, little endian: "TSSCPRF1", u32 version 1, u32 n_gated, u32 units[n_gated], identity[32], u32 prov_len,
prov, per gated layer units^2 u32 counts row-major [previous unit][unit], then the SHA-256 of every byte before it.
identity = SHA-256 of u32 n_gated, then per gated layer: u32 model layer index, u32 units, u64 unit_bytes, the
per-unit xxh64 list."""
from __future__ import annotations

import hashlib
import struct


def identity(layers) -> bytes:
    """layers: [(model layer index, units, unit_bytes, [xxh64 per unit])] of the gated layers in order."""
    b = struct.pack("<I", len(layers))
    for index, units, unit_bytes, hashes in layers:
        assert len(hashes) == units
        b += struct.pack("<IIQ", index, units, unit_bytes)
        b += b"".join(struct.pack("<Q", h) for h in hashes)
    return hashlib.sha256(b).digest()


def model_identity(m) -> bytes:
    """The identity of a fixtures.Model (every layer gated, layer index = position)."""
    return identity([(L, m.units, m.unit_bytes, m.hashes[L * m.units:(L + 1) * m.units]) for L in range(m.layers)])


def write(units, ident: bytes, prov: bytes, cells) -> bytes:
    """cells: per gated layer a flat list of units^2 counts (row-major)."""
    assert len(ident) == 32 and len(cells) == len(units)
    b = b"TSSCPRF1" + struct.pack("<II", 1, len(units)) + b"".join(struct.pack("<I", u) for u in units)
    b += ident + struct.pack("<I", len(prov)) + prov
    for u, c in zip(units, cells):
        assert len(c) == u * u
        b += struct.pack(f"<{u * u}I", *c)
    return b + hashlib.sha256(b).digest()
