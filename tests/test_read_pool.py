"""The three-tier read pool's scheduling on the CPU (tsa_test_read_pool: the product's pool with a reader that blocks
each unit behind a gate the scenario opens). The rules are the reference's read pool's (src/dg_load.hpp:211-222 and
its tests, tests/test_dg_load.cpp:463-1120): demand reads start before queued landing reads whatever the submission
order; at most dg_landing_max_queued landing pieces run and one reader stays free of them; a landing read dropped
before it starts is cancelled with nothing read, one dropped part-way loses its queued pieces (aborted bytes) and is
never finished (no hash check); a claimed landing read runs as a demand read ahead of the landing queue and drain waits
for it; a landing read's failure is kept until a claim finds it Failed, a claimed one's is reported; a landing read
part-way yields its reader to a demand read when more demand pieces wait than idle readers could take, and not when
idle readers take them (src/dg_load.cpp:746-750); whole landing reads (dg_landing_chunk 0xFFFFFFFF) start only while fewer
than the cap pieces of any kind run; stop drops unclaimed landing reads; a word's second read waits for its first."""
import ctypes as C

import pytest

SCENARIOS = ["demand_first", "cap", "reserve", "drop", "claim", "failures", "yields", "whole", "stop_drops",
             "word_order", "no_yield_with_idle_readers"]


@pytest.mark.parametrize("i", range(len(SCENARIOS)), ids=SCENARIOS)
def test_read_pool_scenario(i):
    import tierstream_amd as tsa
    L = tsa.lib()
    L.tsa_test_read_pool.argtypes = [C.c_uint32, C.c_char_p, C.c_uint32]
    L.tsa_test_read_pool.restype = C.c_int
    msg = C.create_string_buffer(512)
    st = L.tsa_test_read_pool(i, msg, 512)
    assert st == 0, (SCENARIOS[i], msg.value.decode())


def test_unknown_scenario_is_refused():
    import tierstream_amd as tsa
    L = tsa.lib()
    L.tsa_test_read_pool.argtypes = [C.c_uint32, C.c_char_p, C.c_uint32]
    L.tsa_test_read_pool.restype = C.c_int
    assert L.tsa_test_read_pool(99, None, 0) != 0
