"""The XXH64 oracle pinned before it is trusted (CPU only).

Pins: the reference's own known answers (tests/test_core.cpp:64-82), the independent python-xxhash library (3.8.1,
the published XXH64) on every length class 0..300 and on large random buffers, streaming == one shot, and the
checkpoint layout reproducing the digest. A dropped term, a wrong rotation or a transposed lane fails the KATs and the
library comparison; an off-by-one in the tail handling fails the length sweep.
"""
import numpy as np
import pytest
import xxhash

import oracle
from oracle import synth

KATS = [(b"", 0xEF46DB3751D8E999), (b"a", 0xD24EC4F1A98C6E5B), (b"abc", 0x44BC2CF5AD770999),
        (b"Nobody inspects the spammish repetition", 0xFBCEA83C8A378BF1)]


@pytest.mark.parametrize("data,want", KATS)
def test_reference_known_answers(data, want):
    assert oracle.xxh64(data) == want


def test_against_python_xxhash_every_length():
    rng = np.random.default_rng(7)
    for n in range(0, 301):
        a = rng.integers(0, 256, n, dtype=np.uint8)
        assert oracle.xxh64(a) == xxhash.xxh64_intdigest(a.tobytes()), n


@pytest.mark.parametrize("n", [4096, 1 << 20, (1 << 20) + 13, 3 * (1 << 20) + 31])
def test_against_python_xxhash_large(n):
    a = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8)
    assert oracle.xxh64(a) == xxhash.xxh64_intdigest(a.tobytes())


def test_streaming_equals_one_shot():
    big = (np.arange(10007, dtype=np.uint64) * 131 + 7).astype(np.uint8)
    # extents of uneven sizes (every one a multiple of 32 except the last) give the one-shot digest
    parts = [big[:32 * 7], big[32 * 7:32 * 100], big[32 * 100:]]
    assert oracle.xxh64_extents(parts) == oracle.xxh64(big)


@pytest.mark.parametrize("sizes,seg", [([1 << 16], 4096), ([4096, 8192, 100], 1024), ([31], 32), ([0], 64),
                                       ([64, 64, 64, 65], 64), ([1 << 20, 1 << 20, (1 << 20) + 7], 65536)])
def test_checkpoints_reproduce_digest(sizes, seg):
    rng = np.random.default_rng(sum(sizes) + seg)
    arrs = [rng.integers(0, 256, s, dtype=np.uint8) for s in sizes]
    states, dig = oracle.checkpoints(arrs, seg)
    assert dig == xxhash.xxh64_intdigest(b"".join(a.tobytes() for a in arrs))
    # the first checkpoint is the seed state
    assert [int(x) for x in states[:4]] == [(0x9E3779B185EBCA87 + 0xC2B2AE3D27D4EB4F) & ((1 << 64) - 1),
                                            0xC2B2AE3D27D4EB4F, 0, (1 << 64) - 0x9E3779B185EBCA87]


def test_synth_uniform_words_are_splitmix():
    # word 0 of stream 3 under seed 11, by the scalar formula
    k = synth.key(11, 3)
    w0 = synth.mix64_scalar(k + synth.GOLDEN)
    got = synth.uniform_bytes(11, 3, 0, 16).view("<u8")
    assert int(got[0]) == w0
    assert int(got[1]) == synth.mix64_scalar(k + 2 * synth.GOLDEN)
    # an offset continues the same stream
    assert np.array_equal(synth.uniform_bytes(11, 3, 8, 8), synth.uniform_bytes(11, 3, 0, 16)[8:])


def test_bf16_normal_distribution():
    b = synth.bf16_normal(5, 1, 0, 1 << 20, 0.02).view(np.uint16).astype(np.uint32) << 16
    x = b.view(np.float32)
    assert abs(float(x.mean())) < 1e-3 and abs(float(x.std()) - 0.02) < 1e-3


def test_q4_blocks_layout():
    """Q4 block b of a stream, by the scalar formula: the fp16 scale 0x2000 | (word 3b & 0x3FF) little-endian (a
    positive fp16 with exponent field 8: [2^-7, 2^-6)), then words 3b + 1 and 3b + 2 little-endian; an offset inside
    a block continues the same stream."""
    k = synth.key(7, 3)
    word = [synth.mix64_scalar(k + (i + 1) * synth.GOLDEN) for i in range(9)]
    got = synth.q4_blocks(7, 3, 0, 54).reshape(3, 18)
    for b in range(3):
        scale = int(got[b, 0]) | int(got[b, 1]) << 8
        assert scale == 0x2000 | (word[3 * b] & 0x3FF)
        assert 2.0 ** -7 <= float(np.array([scale], dtype="<u2").view(np.float16)[0]) < 2.0 ** -6
        assert bytes(got[b, 2:]) == word[3 * b + 1].to_bytes(8, "little") + word[3 * b + 2].to_bytes(8, "little")
    assert np.array_equal(synth.q4_blocks(7, 3, 13, 40), synth.q4_blocks(7, 3, 0, 54)[13:53])
