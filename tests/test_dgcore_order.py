"""Copy order of the device-gated core on the CPU (tsa_test_dgcore_check_order): the product's core on a transport that
keeps its copies as a device would run them - each stream in order, streams ordered only by the waits the core asks
for - and fails at the first file read, copy in or copy out whose memory a copy not ordered before it may still use.

The regression case is the three-tier shape of the GPU parity cases (tests/test_gpu_dg_parity.py::
test_three_tier_matches_reference with big staged parts and dg_bank_keep 1): at a boundary a victim's write-back is
queued into a pinned block and copied at once (prestaged); the next token routes the victim again, which drops the
queued write-back and frees the block; a bank-served file miss later reads into that block. The read must wait for
the prestaged copy (on the MI355X the device check caught the unit whose bytes the late copy overwrote)."""
import numpy as np
import pytest

from test_dgcore_parity import OurCore, _lib

KiB = 1024
BIG_PARTS = [8454144, 64 * KiB, 4 * 1024 * KiB]


def _routes(layers, units, n_ids, tokens, seed):
    """The GPU parity cases' route stream (Zipf(1.1) over a per-layer permutation)."""
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, units + 1) ** 1.1
    p /= p.sum()
    perms = [np.random.default_rng(seed + L).permutation(units) for L in range(layers)]
    out = np.zeros((tokens, layers, n_ids), dtype=np.int32)
    for t in range(tokens):
        for L in range(layers):
            out[t, L] = perms[L][rng.choice(units, size=n_ids, replace=False, p=p)]
    return out


def _three_tier_core(bank_keep, clean_evict):
    layers, units, n_ids, staging, spares = 4, 8, 2, 4, 6
    tiers = [0] * 12 + [1] * 10 + [2] * 10
    D = 3  # one spare slot for each gated layer with a non-resident unit (layers 1-3)
    core = OurCore([units] * layers, 12 + D, n_ids, 10 + spares, D, BIG_PARTS, list(range(12)) + list(range(32)),
                   wb_defer=1, inclusive=0,
                   disk=dict(flags=[1 if t == 2 else 0 for t in tiers], home_blocks=10, disk_staging=staging,
                             clean_evict=clean_evict, bank_keep=bank_keep))
    _, L = _lib()
    core.tsa.check(L.tsa_test_dgcore_check_order(core.h, 1))
    return core


@pytest.mark.parametrize("bank_keep,clean_evict", [(1, 0), (1, 1), (0, 0), (2, 0)])
def test_a_dropped_prestaged_write_back_orders_its_block(bank_keep, clean_evict):
    core = _three_tier_core(bank_keep, clean_evict)
    try:
        routes = _routes(4, 8, 2, 24, seed=9)
        for t in range(routes.shape[0]):
            _, counts = core.token(routes[t])
        if bank_keep:
            assert counts["wb_cancelled"] > 0 and counts["bank_kept"] > 0, counts  # (the sequence above occurs)
    finally:
        core.close()
