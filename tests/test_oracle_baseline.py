"""The CPU baseline the benchmark reports (the reference DgCore on a synchronous memcpy transport over host memory):
every landed unit's bytes hash to the descriptor's XXH64 through fetches, evictions and write-backs, and its cache
counters equal the reference core's on the immediate transport for the same placement and tokens."""
import numpy as np
import pytest

from oracle import fixtures, ref

pytestmark = pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built (needs the reference sources)")

KiB = 1024


@pytest.mark.parametrize("wb_defer,inclusive", [(1, 0), (0, 0), (1, 3)])
def test_cpu_baseline_moves_the_right_bytes(tmp_path, wb_defer, inclusive):
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
    ms, got = ref.cpu_baseline([units] * layers, len(residents) + D, n_ids, P + Q, D, parts, m.stride, order, m.path,
                               offsets, m.hashes, ids, wb_defer=wb_defer, inclusive=inclusive, setup_threads=2)
    assert ms.shape == (tokens,) and np.all(ms > 0)
    assert got["hash_mismatches"] == 0
    assert got["misses"] > 0 and got["evicted"] > 0
    assert got["copied_bytes"] == got["misses"] * m.unit_bytes
    eager = ref.RefDg([units] * layers, len(residents) + D, n_ids, P + Q, D, parts, order, wb_defer=wb_defer,
                      inclusive=inclusive)
    try:
        for t in range(tokens):
            _, want = eager.token(ids[t])
    finally:
        eager.close()
    for k in ("misses", "fetched", "evicted", "writebacks_done"):
        assert got[k] == want[k], k
    if inclusive == 0:
        assert got["writebacks_done"] > 0                # exclusive: evictions write units back, and they re-land intact
