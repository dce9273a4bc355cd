"""dg_disk_queue_adapt's read-depth controller against the reference's own (DgDepthCtl, compiled from its sources in
oracle/_ref), on the CPU: the same busy periods (reads, bytes, busy ns) give the same depth after every period, the
same counters and the same recent verdicts (their rates compared as doubles, exactly).

The sequences model a drive whose throughput per depth changes over time: phases where depth U is faster, where
depth 1 is faster, where they are within the 3 % margin, where the rate moves inside a calibration (split verdicts)
and where it drifts more than 25 % while held; busy periods of 1-12 reads, so windows close at varying points
(reference docs/design.md 3.17, src/dg_load.cpp:578-672)."""
import ctypes as C

import numpy as np
import pytest

from oracle import ref

u32, u64 = C.c_uint32, C.c_uint64
COUNTERS = ["changes", "calibrations", "windows", "verdicts", "reads_1", "bytes_1", "ns_1", "reads_u", "bytes_u",
            "ns_u", "depth", "bound", "calibrating"]


def _drive(fn, bound, periods):
    n = len(periods)
    r = np.array([p[0] for p in periods], dtype=np.uint64)
    b = np.array([p[1] for p in periods], dtype=np.uint64)
    t = np.array([p[2] for p in periods], dtype=np.uint64)
    depth = np.zeros(max(n, 1), dtype=np.uint32)
    counters = np.zeros(len(COUNTERS), dtype=np.uint64)
    recent = np.zeros(16 * 7, dtype=np.float64)
    nr = u32()
    P = C.POINTER
    st = fn(bound, n, r.ctypes.data_as(P(u64)), b.ctypes.data_as(P(u64)), t.ctypes.data_as(P(u64)),
            depth.ctypes.data_as(P(u32)), counters.ctypes.data_as(P(u64)), recent.ctypes.data_as(P(C.c_double)),
            C.byref(nr))
    assert st == 0
    return depth[:n].tolist(), dict(zip(COUNTERS, counters.tolist())), recent[:7 * nr.value].reshape(-1, 7).tolist()


def _fns():
    import tierstream_amd as tsa
    L = tsa.lib()
    args = [u32, u32, C.POINTER(u64), C.POINTER(u64), C.POINTER(u64), C.POINTER(u32), C.POINTER(u64),
            C.POINTER(C.c_double), C.POINTER(u32)]
    L.tsa_test_depth_ctl.argtypes = args
    L.tsa_test_depth_ctl.restype = C.c_int
    R = ref.lib()
    R.refdg_depth_ctl.argtypes = args
    R.refdg_depth_ctl.restype = C.c_int
    return L.tsa_test_depth_ctl, R.refdg_depth_ctl


def _periods(seed, n=1500):
    """Busy periods whose rate depends on the depth the controller chose - unknown here, so each period's ns is drawn
    from a per-phase (rate at U, rate at 1) pair and a coin picks which applies; the controllers see identical input,
    which is all the parity needs."""
    rng = np.random.default_rng(seed)
    out = []
    phase_left = 0
    ru = r1 = 1.0
    for _ in range(n):
        if phase_left == 0:
            phase_left = int(rng.integers(20, 400))
            kind = rng.integers(0, 4)
            base = float(rng.uniform(0.5, 3.0))  # GB/s
            if kind == 0:
                ru, r1 = base * 1.3, base
            elif kind == 1:
                ru, r1 = base, base * 1.3
            elif kind == 2:
                ru, r1 = base * 1.01, base
            else:
                ru, r1 = base * float(rng.uniform(0.5, 2.0)), base * float(rng.uniform(0.5, 2.0))
        phase_left -= 1
        reads = int(rng.integers(0, 13)) if rng.random() > 0.02 else 0
        bytes_ = reads * int(rng.choice([4096 * 1024, 9 << 20, 336 << 20]))
        rate = ru if rng.random() < 0.5 else r1
        ns = int(bytes_ / rate * float(rng.uniform(0.8, 1.2))) if bytes_ else int(rng.integers(0, 1000))
        out.append((reads, bytes_, ns))
    return out


@pytest.mark.parametrize("bound", [1, 2, 4, 8])
@pytest.mark.parametrize("seed", range(12))
def test_depth_controller_matches_reference(seed, bound):
    if not ref.available():
        pytest.skip("oracle/_ref (the reference) is not built")
    ours, theirs = _fns()
    periods = _periods(seed * 31 + bound)
    d_o, c_o, r_o = _drive(ours, bound, periods)
    d_t, c_t, r_t = _drive(theirs, bound, periods)
    assert d_o == d_t
    assert c_o == c_t
    assert r_o == r_t


def test_depth_controller_cases_reach_every_verdict():
    """The sequences are not vacuous: over the seeds, verdicts of every kind occur (keep U, keep 1, split) and the
    controller recalibrates both on drift and on the re-check count."""
    if not ref.available():
        pytest.skip("oracle/_ref (the reference) is not built")
    ours, _ = _fns()
    why = set()
    cal = 0
    for seed in range(12):
        _, c, r = _drive(ours, 4, _periods(seed * 31 + 4, n=4000))
        why |= {int(v[6]) for v in r}
        cal += c["calibrations"]
    assert {1, 2, 3} <= why, why  # keep U, keep 1, split
    assert cal > 24


def test_single_reader_never_adapts():
    ours, _ = _fns()
    d, c, r = _drive(ours, 1, [(32, 32 << 20, 10 ** 7)] * 10)
    assert d == [1] * 10 and c["windows"] == 0 and r == []
