"""The CPU baseline the benchmark reports (the reference DgCore on a synchronous memcpy transport over host memory):
every landed unit's bytes hash to the descriptor's XXH64 through fetches, evictions and write-backs, and its cache
counters equal the reference core's on the immediate transport for the same placement and tokens."""
import numpy as np
import pytest

from oracle import fixtures, ref

pytestmark = pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built (needs the reference sources)")

KiB = 1024


@pytest.mark.parametrize("wb_defer,inclusive,policy", [(1, 0, 0), (0, 0, 0), (1, 3, 0), (1, 0, 1), (0, 3, 1)])
def test_cpu_baseline_moves_the_right_bytes(tmp_path, wb_defer, inclusive, policy):
    layers, units, parts, n_ids = 4, 8, [16 * KiB, 16 * KiB, 32 * KiB], 2
    m = fixtures.write_model(tmp_path, layers, units, parts, top_k=n_ids, seed=7)
    keys = layers * units
    residents = list(range(10))                      # layer 0 and two units of layer 1
    D = 3
    P, Q = keys - len(residents), 6
    order = residents + list(range(keys))
    rng = np.random.default_rng(3)
    tokens = 20
    ids = np.stack([np.stack([rng.choice(units, size=n_ids, replace=False) for _ in range(layers)])
                    for _ in range(tokens)]).astype(np.uint32)
    offsets = [g * m.stride for g in range(keys)]
    warm = 5  # replayed untimed: the timed tokens start from the placement after them
    ms, got = ref.cpu_baseline([units] * layers, len(residents) + D, n_ids, P + Q, D, parts, m.stride, order, m.path,
                               offsets, m.hashes, ids, wb_defer=wb_defer, inclusive=inclusive, setup_threads=2,
                               warm=warm, policy=policy)
    assert ms.shape == (tokens - warm,) and np.all(ms > 0)
    assert got["hash_mismatches"] == 0
    assert got["misses"] > 0 and got["evicted"] > 0
    assert got["copied_bytes"] == got["misses"] * m.unit_bytes
    eager = ref.RefDg([units] * layers, len(residents) + D, n_ids, P + Q, D, parts, order, wb_defer=wb_defer,
                      inclusive=inclusive, score=dict(policy=policy) if policy else None)
    try:
        for t in range(tokens):
            _, want = eager.token(ids[t])
            if t == warm - 1:
                before = dict(want)
    finally:
        eager.close()
    # the eager core's counters over the same timed tokens (after the same warmup)
    for k in ("misses", "fetched", "evicted", "writebacks_done", "score_layers", "score_candidates"):
        assert got[k] == want[k] - before[k], k
    if policy:
        assert want["scored_victims"] > 0 and got["score_layers"] > 0 and got["score_candidates"] > 0
    if inclusive == 0:
        assert got["writebacks_done"] > 0                # exclusive: evictions write units back, and they re-land intact


@pytest.mark.parametrize("clean_evict", [0, 1])
def test_cpu_baseline_three_tier(tmp_path, clean_evict):
    """Three tiers: the file-tier units are read from the source file into staging buffers on a miss (two source
    files: the first two layers in one, the rest in the other) and every landed unit hashes right; the counters equal
    the immediate-transport core's."""
    layers, units, parts, n_ids = 4, 8, [16 * KiB, 16 * KiB, 32 * KiB], 2
    m = fixtures.write_model(tmp_path, layers, units, parts, top_k=n_ids, seed=7)
    keys = layers * units
    residents = list(range(10))
    tiers = [0] * 10 + [1] * 12 + [2] * 10
    flags = [1 if t == 2 else 0 for t in tiers]
    D, P, Q = 3, 12, 4
    order = residents + list(range(keys))
    # the same bytes split over two files (layers 0-1, layers 2-3)
    with open(m.path, "rb") as f:
        raw = f.read()
    half = 2 * units * m.stride
    paths = [tmp_path / "a.bin", tmp_path / "b.bin"]
    paths[0].write_bytes(raw[:half])
    paths[1].write_bytes(raw[half:])
    path_of = [0 if g < 2 * units else 1 for g in range(keys)]
    offsets = [(g if g < 2 * units else g - 2 * units) * m.stride for g in range(keys)]
    rng = np.random.default_rng(5)
    tokens = 24
    ids = np.stack([np.stack([rng.choice(units, size=n_ids, replace=False) for _ in range(layers)])
                    for _ in range(tokens)]).astype(np.uint32)
    ms, got = ref.cpu_baseline_disk([units] * layers, len(residents) + D, n_ids, P + Q, D, parts, m.stride, order,
                                    paths, path_of, offsets, m.hashes, ids, flags, P, 3, clean_evict=clean_evict,
                                    setup_threads=2)
    assert ms.shape == (tokens,) and got["hash_mismatches"] == 0
    assert got["disk_reads"] > 0 and got["copied_bytes"] == got["misses"] * m.unit_bytes
    eager = ref.RefDg([units] * layers, len(residents) + D, n_ids, P + Q, D, parts, order,
                      disk=dict(flags=flags, home_blocks=P, disk_staging=3, clean_evict=clean_evict))
    try:
        for t in range(tokens):
            _, want = eager.token(ids[t])
    finally:
        eager.close()
    for k in ("misses", "fetched", "evicted", "writebacks_done", "disk_reads", "disk_drops"):
        assert got[k] == want[k], k

