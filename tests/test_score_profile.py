"""Scored eviction's TSSCPRF1 profiles on the CPU: this library's SHA-256 against Python's hashlib (FIPS 180-4 padding
edges included), and its profile checks against the reference's own (dg_profile_check, compiled from its sources in
oracle/_ref): a profile written from the published format passes both with its provenance, and every broken rule
(size, magic, version, layer count, units, provenance length, identity, checksum, a flipped count) is refused by both.
The reference's rules: src/dg_score.cpp:82-101."""
import ctypes as C
import hashlib
import struct

import numpy as np
import pytest

from oracle import ref, score_profile
from tierstream_amd import ss

u32 = C.c_uint32
SS_E_INVALID = 1


def _ours(data: bytes, units, ident: bytes):
    L = ss._declare()
    arr = (u32 * max(len(units), 1))(*units)
    prov = C.create_string_buffer(4097)
    st = L.tsa_test_score_profile_check(data, len(data), arr, len(units), ident, prov, 4097)
    return st, prov.value


def _theirs(data: bytes, units, ident: bytes):
    arr = (u32 * max(len(units), 1))(*units)
    return ref.lib().refdg_profile_check(data, len(data), arr, len(units), ident)


@pytest.mark.parametrize("n", [0, 1, 3, 55, 56, 57, 63, 64, 65, 119, 120, 127, 128, 129, 1000, 4099])
def test_sha256_matches_hashlib(n):
    rng = np.random.default_rng(n)
    d = rng.integers(0, 256, size=n, dtype=np.uint8).tobytes()
    out = C.create_string_buffer(32)
    assert ss._declare().tsa_test_sha256(d, n, out) == 0
    assert out.raw == hashlib.sha256(d).digest()


def test_sha256_known_answers():
    """FIPS 180-2 appendix B: one block and two blocks."""
    out = C.create_string_buffer(32)
    L = ss._declare()
    assert L.tsa_test_sha256(b"abc", 3, out) == 0
    assert out.raw.hex() == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    m = b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq"
    assert L.tsa_test_sha256(m, len(m), out) == 0
    assert out.raw.hex() == "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"


def _profile(units, prov=b"fit: 1000 tokens"):
    rng = np.random.default_rng(sum(units))
    ident = hashlib.sha256(bytes(units)).digest()
    cells = [[int(v) for v in rng.integers(0, 1 << 32, size=u * u, dtype=np.uint64)] for u in units]
    return score_profile.write(units, ident, prov, cells), ident


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref (the reference) is not built")
def test_valid_profile_passes_both():
    units = [8, 5, 16]
    data, ident = _profile(units)
    st, prov = _ours(data, units, ident)
    assert st == 0 and prov == b"fit: 1000 tokens"
    assert _theirs(data, units, ident) == 0
    data, ident = _profile(units, prov=b"")
    assert _ours(data, units, ident)[0] == 0 and _theirs(data, units, ident) == 0


def _broken(units):
    data, ident = _profile(units)
    G = len(units)
    at_id = 16 + 4 * G
    out = {
        "truncated header": data[:at_id + 20],
        "empty": b"",
        "bad magic": b"TSSCPRF2" + data[8:],
        "version 2": data[:8] + struct.pack("<I", 2) + data[12:],
        "n_gated": data[:12] + struct.pack("<I", G + 1) + data[16:],
        "units": data[:16] + struct.pack("<I", units[0] + 1) + data[20:],
        "one byte short": data[:-1],
        "one byte long": data + b"\0",
        "identity": data[:at_id] + bytes(32) + data[at_id + 32:],
        "checksum": data[:-1] + bytes([data[-1] ^ 1]),
        "a count flipped": data[:at_id + 40 + 16 + 5] + bytes([data[at_id + 40 + 16 + 5] ^ 0x10]) +
                           data[at_id + 40 + 16 + 6:],
    }
    # a provenance above 4096 bytes (with a matching size and checksum, so only that rule fails)
    out["provenance > 4096"] = score_profile.write(units, ident, b"x" * 4097, _cells(units))
    return out, ident


def _cells(units):
    return [[1] * (u * u) for u in units]


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref (the reference) is not built")
def test_broken_profiles_are_refused_by_both():
    units = [8, 5, 16]
    cases, ident = _broken(units)
    for name, data in cases.items():
        st, _ = _ours(data, units, ident)
        assert st == SS_E_INVALID, name
        assert _theirs(data, units, ident) == 1, name


def test_units_above_65536_are_refused():
    units = [65537]
    ident = bytes(32)
    st, _ = _ours(b"\0" * 64, units, ident)
    assert st == SS_E_INVALID


def test_identity_binds_layer_index_units_bytes_and_hashes():
    """The identity changes with each of its inputs (a profile from another model, layer set or descriptor fails)."""
    base = [(0, 4, 4096, [1, 2, 3, 4]), (2, 4, 4096, [5, 6, 7, 8])]
    i0 = score_profile.identity(base)
    assert len(i0) == 32
    for j, alt in enumerate([
        [(1, 4, 4096, [1, 2, 3, 4]), base[1]],
        [(0, 4, 8192, [1, 2, 3, 4]), base[1]],
        [(0, 4, 4096, [1, 2, 3, 5]), base[1]],
        [base[0]],
    ]):
        assert score_profile.identity(alt) != i0, j


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref (the reference) is not built")
def test_identity_matches_reference():
    """The test writer's identity is the reference's (dg_score_identity), so a profile it writes binds as the
    reference's would."""
    rng = np.random.default_rng(4)
    layers = [(int(i), int(u), int(b), [int(h) for h in rng.integers(0, 1 << 63, size=int(u), dtype=np.uint64)])
              for i, u, b in [(0, 8, 4096), (3, 5, 12288), (7, 16, 786432)]]
    G = len(layers)
    idx = (u32 * G)(*[x[0] for x in layers])
    un = (u32 * G)(*[x[1] for x in layers])
    ub = (C.c_uint64 * G)(*[x[2] for x in layers])
    hs = [h for x in layers for h in x[3]]
    ha = (C.c_uint64 * len(hs))(*hs)
    out = C.create_string_buffer(32)
    assert ref.lib().refdg_score_identity(G, idx, un, ub, ha, out) == 0
    assert out.raw == score_profile.identity(layers)
