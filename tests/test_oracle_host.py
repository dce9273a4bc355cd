"""The host-contract parity cases on the reference CPU backend alone (oracle/_ref, no GPU): the cases the GPU tests
compare against are not vacuous."""
import pytest

from oracle import fixtures, ref

pytestmark = pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built (needs the reference sources)")

KiB = 1024


def test_scored_cases_differ_from_lru(tmp_path):
    """The host-contract SCORED parity cases are not vacuous: on the reference CPU backend the same routes give other
    tables under SCORED than under LRU (the policy decides some evictions)."""
    from tierstream_amd import ss
    m = fixtures.write_model(tmp_path, 4, 8, [32 * KiB, 32 * KiB, 16 * KiB], top_k=2, seed=7)
    routes = fixtures.uniform_routes(4, 8, 2, 24, seed=11)
    st = (m.unit_bytes + 255) // 256 * 256
    host = 32 * ((m.unit_bytes + 4095) // 4096 * 4096) + (64 << 20)
    bkw = dict(device_bytes=8 * st + 16 * st + 2 * 4 * st + st // 2, host_pinned_bytes=host,
               dynamic_slots_per_layer=2, ring_slots=16)
    lru = ref.host_run(m.desc_json(), ss.budget(**bkw), ss.options(pin_planned=0), routes, 0)
    scored = ref.host_run(m.desc_json(), ss.budget(**bkw), ss.options(pin_planned=0, policy=1, score_window=6),
                          routes, 0)
    assert any(a["tables"] != b["tables"] for a, b in zip(lru, scored))
