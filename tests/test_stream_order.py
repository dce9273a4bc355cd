"""The host contract's cross-stream wait bookkeeping on the CPU (tsa_test_stream_order: the library's MarkOrder driven
by random event records, waits and stream replacements). The host contract gives a copy stream a wait for an event only
when the stream does not already follow that event's record through an earlier wait (work on one stream completes in
order, so waiting for a stream's later record covers its earlier ones). The check: per stream, a vector clock that
applies every wait must equal one that applies only the waits given; two planted mistakes in the bookkeeping must be
caught. No reference counterpart: the reference gives every wait (src/stream_ctx.cpp); placement and copy contents are
unchanged, which the GPU parity tests check."""
import ctypes as C

import pytest


def _run(seed, n_ops, n_streams, mode):
    import tierstream_amd as tsa
    from tierstream_amd import ss
    counts = (C.c_uint64 * 2)()
    tsa.check(ss._declare().tsa_test_stream_order(seed, n_ops, n_streams, mode, counts))
    return int(counts[0]), int(counts[1])


@pytest.mark.parametrize("n_streams", [2, 3, 5, 8])
def test_skipped_waits_are_implied(n_streams):
    for seed in range(40):
        first_bad, skipped = _run(seed, 4000, n_streams, 0)
        assert first_bad == 0, (seed, n_streams, first_bad)
        assert skipped > 0


@pytest.mark.parametrize("mode", [1, 2], ids=["mark-ignored", "no-forget"])
def test_planted_mistakes_are_caught(mode):
    caught = sum(_run(seed, 4000, 4, mode)[0] > 0 for seed in range(20))
    assert caught == 20


def test_bad_arguments_are_refused():
    import tierstream_amd as tsa
    from tierstream_amd import ss
    counts = (C.c_uint64 * 2)()
    L = ss._declare()
    assert L.tsa_test_stream_order(1, 10, 0, 0, counts) == tsa.SS_E_INVALID
    assert L.tsa_test_stream_order(1, 10, 17, 0, counts) == tsa.SS_E_INVALID
    assert L.tsa_test_stream_order(1, 10, 4, 3, counts) == tsa.SS_E_INVALID
