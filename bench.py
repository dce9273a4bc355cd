#!/usr/bin/env python3
"""Decode-step serve benchmark of libtierstream_amd on one MI355X.

Workload (default): the Mixtral-shape MoE decode. 32 layers x 8 experts, each expert a unit of three bf16 parts
(gate and up 4096 x 14336, down 14336 x 4096: 112 MiB each, 336 MiB per unit), values N(0, 0.02) from the
counter-based generator. Routes are Zipf(1.1) top-2 over a per-layer seeded permutation, batch 1. 40 % of the units
(102) are planned residents in HBM and the other 154 live in hipHostMalloc pinned memory. The context runs
SS_FORWARD_DEVICE_GATED: each token is a hipGraph of begin, then per layer export, wait and the engine's expert
stand-in, then end. The stand-in is a checksum that reads every byte of both routed units through ss_dg_slot.
Every landed unit is re-hashed in HBM by the device XXH64 verify (verify_hash = 2).

A step is one token: ss_begin -> graph launch -> ss_end on the engine thread (the reference's decode-step serve
latency). The timed region is exactly --steps tokens after --warmup untimed ones, bracketed by device
synchronizations. The JSON line's value is the p50 step latency in ms.

Beside it:
  h2d        miss bytes over the wall clock of the timed region, and over the copy engine's busy time (timed events
             around every part copy of the probe tokens after the timed ones: brackets are left out of the timed
             region, whose copies they would delay), against the pinned host-to-device peak measured in the same run
             (2 GiB hipMemcpyAsync from hipHostMalloc memory)
  roofline   the device XXH64 verify kernel (the dominant kernel of the library): unit bytes hashed per launch over
             its mean launch time (timed events on the stream it runs on), against the 8 TB/s HBM peak
  wait       the zero-miss layer wait on the device timeline (wall-clock stamps, 10 ns): the wait kernel's own entry
             to exit, and from the export kernel's end to the layer's compute start with the two kernel dispatch gaps
             either side of the wait; and the miss layers' wait for their copies
  cpu_baseline  the reference DgCore (compiled from the reference sources) on a synchronous memcpy transport over host
             memory with a host XXH64 of every landed unit, one thread, over a bounded sample of the same tokens
Checks at full size: no unit fails its device hash check, and every routed unit's checksum is the same each time it
is routed (a stale or partial copy would change it).
"""
from __future__ import annotations

import argparse
import json
import os
import shutil
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

METRIC = "decode-step serve latency p50/p99; miss H2D GB/s and HBM GB/s vs roofline"
HBM_PEAK_GBPS = 8000.0
TICK_NS = 10.0  # wall_clock64 runs at 100 MHz on gfx950
# HBM bytes one verify launch moves per unit it checks, keyed by unit bytes: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE
# on a launch of one unit of this shape (dg_verify_lds_kernel through tsa_xxh64_verify_slots), each scaled by the
# counter's reading for a copy kernel of known size (FETCH 2.0, WRITE 1.0), 2 KiB checkpoint segments: 349,927.25 KiB
# fetched, nothing written (profiles/dg_verify_lds_kernel_mixtral_unit_pmc.md).
VERIFY_TRAFFIC_PER_UNIT = {352321536: 358325504, 24772608: 25338624}
# The staged units' fused scatter and check (dg_scatter_verify_lds_kernel), keyed by unit bytes: FETCH_SIZE x 2.0 +
# WRITE_SIZE x 1.0 on one launch of one unit of this shape through tsa_xxh64_scatter_verify_slots, 2 KiB segments
# (profiles/dg_scatter_verify_lds_kernel_deepseek_unit_pmc.md).
SCATTER_VERIFY_TRAFFIC_PER_UNIT = {24772608: 50273920}
TRAFFIC_SOURCE = {("verify", 352321536): "profiles/dg_verify_lds_kernel_mixtral_unit_pmc.md",
                  ("verify", 24772608): "profiles/dg_scatter_verify_lds_kernel_deepseek_unit_pmc.md",
                  ("fused", 24772608): "profiles/dg_scatter_verify_lds_kernel_deepseek_unit_pmc.md"}
# The host contract's verify_kernel: HBM bytes fetched per algorithmic byte hashed, keyed by unit bytes, from
# rocprofv3 --pmc FETCH_SIZE over the bench's own timed steps (scaled as above): a full batch of 32 units fetches
# 149,987.63 KiB x 2.0 = 307,174,656 B for 301,989,888 B of units (2 KiB checkpoint segments), nothing written
# (profiles/verify_kernel_qwen3_host_pmc.md).
# dense-prefix: a batch of 2 blobs (469,762,048 B) fetches 232,268.63 KiB x 2.0 = 475,686,144 B
# (profiles/verify_kernel_dense_prefix_host_pmc.md).
HOST_VERIFY_TRAFFIC_RATIO: dict[int, float] = {9437184: 307174656 / 301989888, 234881024: 475686144 / 469762048}
HOST_TRAFFIC_SOURCE = {9437184: "profiles/verify_kernel_qwen3_host_pmc.md",
                       234881024: "profiles/verify_kernel_dense_prefix_host_pmc.md"}


def dg_check_kernel(parts, seg, fused):
    """The kernel the library launches for a device-gated check of this arena shape: the LDS-streamed one for 2 KiB
    segments and 16-byte aligned parts of at least 16 bytes (the arena's parts are separate allocations), the chain
    loop otherwise."""
    lds = seg == 2048 and all(pb % 16 == 0 and pb >= 16 for pb in parts)
    if fused:
        return "dg_scatter_verify_lds_kernel" if lds else "dg_scatter_verify_kernel"
    return "dg_verify_lds_kernel" if lds else "dg_verify_kernel"


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed tokens (default: the workload's: mixtral 256)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="mixtral")
    ap.add_argument("--part-bytes", type=int, default=0, help="scale every part to this size (0 = full size)")
    ap.add_argument("--probe-tokens", type=int, default=32, help="tokens after the timed ones that read the stamps")
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="target CPU time of the baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--workdir", default="", help="where the source file is written (default /dev/shm)")
    ap.add_argument("--layers", type=int, default=0, help="run the workload with this many layers (0 = all)")
    ap.add_argument("--disk-dir", default="",
                    help="three tiers: where the file tier's source file is written (default: the temp directory, "
                         "a drive that takes direct I/O; the other layers' file stays in --workdir)")
    ap.add_argument("--inclusive", type=int, default=0,
                    help="dg_inclusive_blocks (clean copies; 0 = spare slots + banks); spare blocks = this + 4")
    ap.add_argument("--policy", default="lru", choices=["lru", "scored", "auto"],
                    help="device-gated eviction policy (SS_POLICY_LRU / SCORED / SCORED_AUTO; default 700/200/100 "
                         "weights, no profile)")
    ap.add_argument("--bank-keep", type=int, default=0, choices=[0, 1, 2],
                    help="three tiers: dg_bank_keep (bank-served file misses kept in a pinned block)")
    ap.add_argument("--disk-queue", type=int, default=-1,
                    help="three tiers: dg_disk_queue (file reads in flight; -1: the workload's)")
    ap.add_argument("--disk-adapt", action="store_true",
                    help="three tiers: dg_disk_queue SS_DG_DISK_QUEUE_AUTO with dg_disk_queue_adapt")
    ap.add_argument("--predict", type=float, default=0.0,
                    help="device-gated: the engine predicts the next layer's ids (ss_dg_enqueue_predict), each of the "
                         "true ids with this probability and a random unit otherwise (0: no predictions)")
    ap.add_argument("--landing-blocks", type=int, default=0,
                    help="three tiers: dg_landing_blocks (predicted file-homed units read ahead into landing blocks)")
    ap.add_argument("--landing-ttl", type=int, default=0, help="three tiers: dg_landing_ttl")
    ap.add_argument("--landing-max-queued", type=int, default=0, help="three tiers: dg_landing_max_queued")
    ap.add_argument("--landing-chunk", type=int, default=0, help="three tiers: dg_landing_chunk")
    ap.add_argument("--copies", default="hsa", choices=["hsa", "hip"],
                    help="device-gated unit copies: through the HSA runtime's copy engines (the library's default "
                         "where parts are copied whole) or on HIP streams (TSA_DG_COPIES=hip)")
    ap.add_argument("--timeline", default="",
                    help="device-gated: open with dg_diag and write every timed token's per-layer timeline rows "
                         "(ss_dg_timeline_sized) and device stamps to this JSON file (read between tokens: each "
                         "token's latency excludes them, the timed region's wall clock does not)")
    ap.add_argument("--kernels-only", action="store_true",
                    help="only the copy peaks and the library's HBM kernels alone (no serve loop: for counter runs)")
    ap.add_argument("--beside", default="none", choices=["none", "h2d", "d2h"],
                    help="with --kernels-only: time the unit check while pinned copies of this direction run on "
                         "another stream (a landing or a write-back beside a check, as in the serve loop)")
    return ap.parse_args()


def pct(a, q):
    return float(np.percentile(np.asarray(a, dtype=np.float64), q)) if len(a) else None


# ---- peaks measured in the same run ---------------------------------------------------------------------------------
def measure_peaks(tsa, L, C):
    """Pinned H2D peak (2 GiB from hipHostMalloc memory) and an HBM copy (4 GiB device to device: 2 x bytes moved)."""
    out = {}
    n = 2 << 30
    host, dev, dev2, s = C.c_void_p(), C.c_void_p(), C.c_void_p(), C.c_void_p()
    e0, e1 = C.c_void_p(), C.c_void_p()
    tsa.check(L.tsa_host_alloc(C.byref(host), n))
    tsa.check(L.tsa_malloc(C.byref(dev), 2 * n))
    tsa.check(L.tsa_malloc(C.byref(dev2), 2 * n))
    tsa.check(L.tsa_stream_create(C.byref(s)))
    tsa.check(L.tsa_event_create(C.byref(e0)))
    tsa.check(L.tsa_event_create(C.byref(e1)))
    try:
        C.memset(host, 1, n)

        def timed(fn):
            tsa.check(L.tsa_event_record(e0, s))
            fn()
            tsa.check(L.tsa_event_record(e1, s))
            tsa.check(L.tsa_event_sync(e1))
            ms = C.c_float()
            tsa.check(L.tsa_event_elapsed_ms(e0, e1, C.byref(ms)))
            return ms.value / 1e3

        h2d = [n / timed(lambda: tsa.check(L.tsa_memcpy(dev, host, n, 0, s))) / 1e9 for _ in range(6)]
        d2h = [n / timed(lambda: tsa.check(L.tsa_memcpy(host, dev, n, 1, s))) / 1e9 for _ in range(4)]
        d2d = [2 * (2 * n) / timed(lambda: tsa.check(L.tsa_memcpy(dev2, dev, 2 * n, 2, s))) / 1e9 for _ in range(6)]
        # both directions at once (a write-back beside a miss copy): host -> dev on s, dev2 -> host2 on s2
        host2, s2, e2, e3 = C.c_void_p(), C.c_void_p(), C.c_void_p(), C.c_void_p()
        tsa.check(L.tsa_host_alloc(C.byref(host2), n))
        tsa.check(L.tsa_stream_create(C.byref(s2)))
        tsa.check(L.tsa_event_create(C.byref(e2)))
        tsa.check(L.tsa_event_create(C.byref(e3)))
        bidir = []
        try:
            for _ in range(4):
                tsa.check(L.tsa_device_sync())
                tsa.check(L.tsa_event_record(e0, s))
                tsa.check(L.tsa_event_record(e2, s2))
                tsa.check(L.tsa_memcpy(dev, host, n, 0, s))
                tsa.check(L.tsa_memcpy(host2, dev2, n, 1, s2))
                tsa.check(L.tsa_event_record(e1, s))
                tsa.check(L.tsa_event_record(e3, s2))
                tsa.check(L.tsa_event_sync(e1))
                tsa.check(L.tsa_event_sync(e3))
                a, b = C.c_float(), C.c_float()
                tsa.check(L.tsa_event_elapsed_ms(e0, e1, C.byref(a)))
                tsa.check(L.tsa_event_elapsed_ms(e2, e3, C.byref(b)))
                bidir.append((n / (a.value / 1e3) / 1e9, n / (b.value / 1e3) / 1e9))
        finally:
            L.tsa_event_destroy(e2)
            L.tsa_event_destroy(e3)
            L.tsa_stream_destroy(s2)
            L.tsa_host_free(host2)
        bi = max(bidir[1:], key=lambda x: x[0] + x[1])
        out = {"h2d_pinned_GBps": max(h2d[1:]), "h2d_pinned_GBps_median": float(np.median(h2d[1:])),
               "d2h_pinned_GBps": max(d2h[1:]), "bidir_h2d_GBps": bi[0], "bidir_d2h_GBps": bi[1],
               "hbm_copy_GBps": max(d2d[1:]), "pcie_gen5_x16_GBps": 64.0, "hbm_peak_GBps": HBM_PEAK_GBPS}
    finally:
        L.tsa_event_destroy(e0)
        L.tsa_event_destroy(e1)
        L.tsa_stream_destroy(s)
        L.tsa_free(dev)
        L.tsa_free(dev2)
        L.tsa_host_free(host)
    return out


def measure_disk(path, w, n_layers, threads=4, seconds=4.0):
    """Direct-I/O read rate of the file tier's drive: `threads` readers, each reading whole units (every part of a
    unit, one positional read at the unit's 4 KiB-aligned offset) of the file-tier source into its own page-aligned
    buffer, units in a seeded random order, for about `seconds`; and one reader alone (the read depth of
    dg_disk_queue 1). Bytes over wall time."""
    import mmap
    import threading
    n_units = n_layers * w.units
    ub = w.unit_bytes
    out = {}
    try:
        fd = os.open(path, os.O_RDONLY | getattr(os, "O_DIRECT", 0))
    except OSError as e:
        return {"error": f"direct open: {e}"}
    try:
        for nth in sorted({1, threads}):
            order = np.random.default_rng(7 + nth).permutation(n_units)
            nxt = [0]
            lock = threading.Lock()
            done = [0]
            t_end = time.perf_counter() + seconds / 2

            def reader():
                buf = mmap.mmap(-1, ub)
                try:
                    while time.perf_counter() < t_end:
                        with lock:
                            i = nxt[0]
                            nxt[0] += 1
                        if i >= n_units:
                            return
                        got = os.preadv(fd, [buf], int(order[i]) * w.unit_stride_file)
                        with lock:
                            done[0] += got
                finally:
                    buf.close()

            t0 = time.perf_counter()
            th = [threading.Thread(target=reader) for _ in range(nth)]
            for t in th:
                t.start()
            for t in th:
                t.join()
            out[f"readers_{nth}_GBps"] = round(done[0] / (time.perf_counter() - t0) / 1e9, 2)
    finally:
        os.close(fd)
    return out


def verify_seg_bytes(unit_bytes):
    """The device check's checkpoint segment a context uses (the library's rule, tierstream_amd/csrc/dg_ctx.cpp
    verify_seg_bytes): 2 KiB for every unit size."""
    return 2048


def start_copies(tsa, L, C, direction, n=1 << 30, count=24):
    """Queue `count` pinned copies of n bytes in one direction on a stream of their own (about 0.45 s of PCIe work at
    the pinned peak); returns the function that waits for them and frees their buffers."""
    host, dev, s = C.c_void_p(), C.c_void_p(), C.c_void_p()
    tsa.check(L.tsa_host_alloc(C.byref(host), n))
    tsa.check(L.tsa_malloc(C.byref(dev), n))
    tsa.check(L.tsa_stream_create(C.byref(s)))
    C.memset(host, 1, n)
    for _ in range(count):
        if direction == "h2d":
            tsa.check(L.tsa_memcpy(dev, host, n, 0, s))
        else:
            tsa.check(L.tsa_memcpy(host, dev, n, 1, s))

    def done():
        tsa.check(L.tsa_stream_sync(s))
        L.tsa_stream_destroy(s)
        L.tsa_free(dev)
        L.tsa_host_free(host)
    return done


def measure_kernels(tsa, L, C, w, seg=None, reps=10, beside="none"):
    """The library's HBM kernels alone at the workload's unit shape: the device XXH64 verify of one unit (checkpoints
    every `seg` bytes, computed on the host) and the unit scatter used as a plain copy of known size (one part of
    256 MiB: read 256 MiB, write 256 MiB), whose counters calibrate the traffic counters of the others."""
    parts = w.parts
    ub = w.unit_bytes
    seg = seg or verify_seg_bytes(ub)
    bufs = []
    out = {}
    s, e0, e1 = C.c_void_p(), C.c_void_p(), C.c_void_p()
    tsa.check(L.tsa_stream_create(C.byref(s)))
    tsa.check(L.tsa_event_create(C.byref(e0)))
    tsa.check(L.tsa_event_create(C.byref(e1)))

    def dev_alloc(n):
        b = tsa.DeviceBuffer(n)
        bufs.append(b)
        return b

    def timed(fn, n=reps):
        ms = []
        fn()
        tsa.check(L.tsa_stream_sync(s))
        for _ in range(n):
            tsa.check(L.tsa_event_record(e0, s))
            fn()
            tsa.check(L.tsa_event_record(e1, s))
            tsa.check(L.tsa_event_sync(e1))
            t = C.c_float()
            tsa.check(L.tsa_event_elapsed_ms(e0, e1, C.byref(t)))
            ms.append(t.value)
        return float(np.median(ms)) / 1e3

    try:
        # verify: one unit in slot 0 of a one-slot arena (its parts in separate HBM arrays, as in the context), checked
        # by the same kernel the serve loop runs (tsa_xxh64_verify_slots)
        pbufs = [dev_alloc(pb) for pb in parts]
        for p, (b, pb) in enumerate(zip(pbufs, parts)):
            tsa.check(L.tsa_synth(C.c_void_p(b.ptr), pb, 77, p, 0, 1, C.c_float(0.02), None))
        tsa.check(L.tsa_device_sync())
        states, digest = tsa.host_checkpoints([b.download(pb) for b, pb in zip(pbufs, parts)], seg)
        n_ck = states.size // 4
        st_dev = dev_alloc(states.nbytes)
        st_dev.upload(states)
        dg_dev = dev_alloc(8)
        dg_dev.upload(np.array([digest], dtype=np.uint64))
        av = tsa.TsaArenaVerify()
        for p, (b, pb) in enumerate(zip(pbufs, parts)):
            av.arena[p] = b.ptr
            av.part_bytes[p] = pb
        av.n_parts, av.seg_bytes, av.states_dev, av.digests_dev = len(parts), seg, st_dev.ptr, dg_dev.ptr
        keys, slots = (C.c_uint32 * 1)(0), (C.c_int32 * 1)(0)
        fail = dev_alloc(64)
        fail.upload(np.zeros(16, dtype=np.uint32))
        busy = start_copies(tsa, L, C, beside) if beside != "none" else None
        try:
            t = timed(lambda: tsa.check(L.tsa_xxh64_verify_slots(C.byref(av), keys, slots, 1, C.c_void_p(fail.ptr),
                                                                 s)))
        finally:
            if busy:
                busy()
        bad = int(fail.download(4, dtype=np.uint32)[0])
        out["verify"] = {"kernel": dg_check_kernel(parts, seg, False), "unit_bytes": ub, "seg_bytes": seg,
                         "segments": n_ck,
                         "us": round(t * 1e6, 1), "GBps": round(ub / t / 1e9, 1),
                         "frac_of_hbm_peak": round(ub / t / 1e9 / HBM_PEAK_GBPS, 4), "fail_word": bad,
                         "beside": beside}
        if len(parts) > 1 and min(parts) < (8 << 20):  # staged: the scatter and the check in one kernel
            staged = dev_alloc(ub)
            for p, (b, pb) in enumerate(zip(pbufs, parts)):
                tsa.check(L.tsa_memcpy(C.c_void_p(staged.ptr + sum(parts[:p])), C.c_void_p(b.ptr), pb, 2, s))
            tsa.check(L.tsa_stream_sync(s))
            fail.upload(np.zeros(16, dtype=np.uint32))
            t2 = timed(lambda: tsa.check(L.tsa_xxh64_scatter_verify_slots(C.byref(av), keys, slots, 1,
                                                                          C.c_void_p(staged.ptr),
                                                                          C.c_void_p(fail.ptr), s)))
            out["scatter_verify"] = {"kernel": dg_check_kernel(parts, seg, True), "unit_bytes": ub,
                                     "bytes_moved": 2 * ub,
                                     "us": round(t2 * 1e6, 1), "GBps": round(2 * ub / t2 / 1e9, 1),
                                     "frac_of_hbm_peak": round(2 * ub / t2 / 1e9 / HBM_PEAK_GBPS, 4),
                                     "fail_word": int(fail.download(4, dtype=np.uint32)[0])}
        # the scatter kernel as a plain copy: one part of 256 MiB
        n = 256 << 20
        src, dst = dev_alloc(n), dev_alloc(n)
        job = tsa.TsaScatterJob()
        job.src = src.ptr
        job.dst[0] = dst.ptr
        job.bytes[0] = n
        job.n_parts = 1
        job.block_first = 0
        pb_arr = (C.c_uint64 * 1)(n)
        nblk = int(L.tsa_scatter_blocks(pb_arr, 1))
        jdev = dev_alloc(C.sizeof(job))
        jdev.upload(np.frombuffer(bytes(job), dtype=np.uint8))
        t = timed(lambda: tsa.check(L.tsa_scatter(C.c_void_p(jdev.ptr), 1, nblk, s)))
        out["copy_kernel"] = {"kernel": "scatter_kernel (one 256 MiB part)", "bytes_read": n, "bytes_written": n,
                              "us": round(t * 1e6, 1), "GBps": round(2 * n / t / 1e9, 1)}
    finally:
        for b in bufs:
            b.close()
        L.tsa_event_destroy(e0)
        L.tsa_event_destroy(e1)
        L.tsa_stream_destroy(s)
    return out


# ---- the CPU baseline -----------------------------------------------------------------------------------------------
def cpu_baseline(w, shape, files, hashes, routes, start, est_token_s, seconds, policy=0):
    """The reference DgCore on a memcpy transport (oracle/_ref), under the same eviction policy (0 LRU, 1 SCORED,
    2 SCORED_AUTO): tokens 0..start-1 of the same route stream replayed untimed (the warmup: the timed tokens start
    from the placement the device's timed tokens start from), then tokens start.. timed. files: [(path, first layer,
    layers)] as the descriptor's sources."""
    try:
        from oracle import ref
    except Exception as e:  # noqa: BLE001
        return None, f"oracle unavailable: {e}"
    if not ref.available():
        return None, "oracle/_ref is not built"
    from tierstream_amd import workloads as W
    n_tok = int(max(16, min(256, seconds / max(est_token_s, 1e-3))))
    n_tok = min(n_tok, routes.shape[0] - start)
    keys = w.n_units
    residents = list(range(shape.R))
    order = residents + list(range(keys))
    path_of, offsets = [], []
    for i, (_, first, n) in enumerate(files):
        for L in range(first, first + n):
            for u in range(w.units):
                path_of.append(i)
                offsets.append(W.unit_offset(w, L, u, first))
    ids = routes[:start + n_tok].astype(np.uint32)
    hs = (w.unit_bytes + 4095) // 4096 * 4096
    t0 = time.time()
    if shape.F:
        flags = [1 if t == 2 else 0 for t in shape.tiers]
        ms, c = ref.cpu_baseline_disk([w.units] * w.layers, shape.R + shape.D, shape.B, shape.P + shape.Q, shape.D,
                                      w.parts, hs, order, [f[0] for f in files], path_of, offsets, hashes, ids, flags,
                                      shape.P, 8, clean_evict=w.clean_evict, setup_threads=16, warm=start,
                                      policy=policy)
    else:
        ms, c = ref.cpu_baseline([w.units] * w.layers, shape.R + shape.D, shape.B, shape.P + shape.Q, shape.D, w.parts,
                                 hs, order, files[0][0], offsets, hashes, ids, wb_defer=1, inclusive=shape.I,
                                 setup_threads=16, warm=start, policy=policy)
    log(f"cpu baseline: {start} warmup + {n_tok} timed tokens in {time.time() - t0:.1f} s (setup included), "
        f"counters {c}")
    return (ms, c, n_tok), None


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: --gpus {a.gpus}: this benchmark runs on one GPU only (the serve path has no cross-GPU "
              f"exchange; each GPU would open its own context over its share of units)", file=sys.stderr)
        sys.exit(2)
    import ctypes as C

    import tierstream_amd as tsa
    from tierstream_amd import ss
    from tierstream_amd import workloads as W

    L = tsa.lib()
    if tsa.gpu_count() < 1:
        raise SystemExit("bench.py: no HIP device")
    w = W.WORKLOADS[a.workload]
    if a.part_bytes:
        w = W.scaled(w, part_bytes=a.part_bytes)
    if a.layers:
        w = W.scaled(w, layers=a.layers)
    if a.steps is None:
        a.steps = w.steps
    if w.forward != 1:
        return run_host(a, w, tsa, ss, W, L, C)
    if a.inclusive:
        w = W.scaled(w, inclusive_blocks=a.inclusive, spare_units=a.inclusive + 4)
    shape = W.dg_shape(w)
    if a.kernels_only:
        kern = measure_kernels(tsa, L, C, w, beside=a.beside)
        log(f"kernels {kern}")
        peaks = measure_peaks(tsa, L, C)
        print(json.dumps({"kernels_only": True, "workload": w.name, "kernels": kern, "peaks": peaks}), flush=True)
        return
    base = a.workdir or ("/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir())
    work = tempfile.mkdtemp(prefix="tsa_bench_", dir=base)
    path = os.path.join(work, "weights.bin")
    three = shape.F > 0
    cold = shape.cold_first_layer(w)
    cold_work = tempfile.mkdtemp(prefix="tsa_bench_", dir=a.disk_dir or tempfile.gettempdir()) if three else None
    cold_path = os.path.join(cold_work, "weights-file-tier.bin") if three else None
    result = {}
    opened = []  # handles to close in reverse order on every path out (engine, context, plan, descriptor)

    def keep(h):
        opened.append(h)
        return h

    try:
        t0 = time.time()
        log(f"workload {w.name}: {w.layers} x {w.units} units of {w.unit_bytes / 2**20:.1f} MiB, writing "
            f"{W.source_bytes(w, cold) / 1e9:.1f} GB to {path}")
        hashes = W.write_sources_gpu(w, path, n_layers=cold) if cold else []
        files = [(path, 0, cold)] if cold else []
        if three:
            log(f"three tiers: layers {cold}..{w.layers - 1} ({W.source_bytes(w, w.layers - cold) / 1e9:.1f} GB) to "
                f"{cold_path}")
            hashes += W.write_sources_gpu(w, cold_path, first_layer=cold, drop_cache=True)
            files.append((cold_path, cold, w.layers - cold))
        log(f"sources written in {time.time() - t0:.1f} s")
        d = keep(ss.Desc(W.desc_json(w, files, hashes)))
        if three and a.landing_blocks:  # the landing blocks are pinned on top of the plan
            shape.budget["host_pinned_bytes"] += a.landing_blocks * ((w.unit_bytes + 4095) // 4096 * 4096)
        b = ss.budget(**shape.budget)
        plan = keep(ss.Plan(d, b, tiers=shape.tiers) if three else ss.Plan(d, b))
        tiers = plan.tiers()
        n_res = sum(1 for r in tiers for t in r if t == 0)
        n_pin = sum(1 for r in tiers for t in r if t == 1)
        n_file = sum(1 for r in tiers for t in r if t == 2)
        log(f"plan: {n_res} resident units (target {shape.R}), {n_pin} pinned, {n_file} file, D {shape.D}, Q {shape.Q}, "
            f"inclusive {shape.I}, device budget {shape.budget['device_bytes'] / 1e9:.1f} GB, pinned "
            f"{shape.budget['host_pinned_bytes'] / 1e9:.1f} GB")
        disk_peak = measure_disk(cold_path, w, w.layers - cold, threads=max(shape.options.get("dg_disk_queue") or 1, 1)) \
            if three else None
        if disk_peak:
            log(f"file tier drive: {disk_peak}")
        t0 = time.time()
        policy = {"lru": 0, "scored": 1, "auto": 2}[a.policy]
        extra = {}
        if three and a.bank_keep:
            extra["dg_bank_keep"] = a.bank_keep
        if three and a.disk_queue >= 0:
            extra["dg_disk_queue"] = a.disk_queue
        if three and a.disk_adapt:
            extra.update(dg_disk_queue=0xFFFFFFFF, dg_disk_queue_adapt=1)
        if three and a.landing_blocks:
            extra.update(dg_landing_blocks=a.landing_blocks, dg_landing_ttl=a.landing_ttl,
                         dg_landing_max_queued=a.landing_max_queued, dg_landing_chunk=a.landing_chunk)
        opts = {**shape.options, **extra}
        os.environ["TSA_DG_COPIES"] = a.copies  # (read by the open)
        diag = {"dg_diag": 1} if a.timeline else {}
        ctx = keep(ss.Ctx(d, b, plan, ss.options(**opts, verify_hash=2, dg_wait_timeout_ms=20000, policy=policy,
                                                  **diag)))
        os.environ.pop("TSA_DG_COPIES", None)
        copies = "hsa" if ctx.hsa_copies() else "hip"
        open_s = time.time() - t0
        log(f"context open (fill + hash check) in {open_s:.1f} s")
        n_pred = shape.B if a.predict > 0 else 0
        eng = keep(ss.DgEngine(ctx, shape.B, use_graph=True, n_pred=n_pred))
        G = eng.G
        steps, warm, probe = a.steps, a.warmup, a.probe_tokens
        routes = W.route_stream(w, warm + steps + probe)[:, :, :shape.B]
        preds = None
        if n_pred:  # row g: layer g + 1's ids, each kept with probability --predict, else a random unit
            prng = np.random.default_rng(w.seed + 17)
            preds = np.zeros((routes.shape[0], G, n_pred), dtype=np.int32)
            preds[:, :-1] = routes[:, 1:, :n_pred]
            miss = prng.random(preds.shape) >= a.predict
            preds[miss] = prng.integers(0, w.units, size=int(miss.sum()))
            preds[:, -1] = 0
        ck_seen, ck_bad = {}, 0

        def check_cks(t, cks):
            nonlocal ck_bad
            for g in range(G):
                for j in range(shape.B):
                    k = (g, int(routes[t, g, j]))
                    v = int(cks[g, j])
                    if ck_seen.setdefault(k, v) != v:
                        ck_bad += 1

        def pred_of(t):
            return preds[t] if preds is not None else None

        for t in range(warm):
            cks, _ = eng.token(routes[t], preds=pred_of(t))
            check_cks(t, cks)
        # the timed region brackets only the verify launches (their own dispatch stamps: no extra stream work); the
        # copies and write-backs are bracketed in the probe tokens after it
        ctx.profile_enable(ctx.PROF_VERIFY)
        s0 = ctx.dg_stats()
        tsa.check(L.tsa_device_sync())
        lat = np.zeros(steps)
        t_start = time.perf_counter()
        rows = []
        for i in range(steps):
            cks, lat[i] = eng.token(routes[warm + i], preds=pred_of(warm + i))
            check_cks(warm + i, cks)
            if a.timeline:  # (between tokens: outside the token's own latency)
                rows.append({"token": i, "lat_ms": float(lat[i]), "rows": [ctx.dg_timeline(g) for g in range(G)],
                             "stamps": ctx.dg_stamps().astype(np.int64).tolist(),
                             "boundary": ctx.dg_boundary_timeline()})
        if a.timeline:
            with open(a.timeline, "w") as f:
                json.dump(rows, f)
        tsa.check(L.tsa_device_sync())
        wall = time.perf_counter() - t_start
        s1 = ctx.dg_stats()
        prof = ctx.profile_read(wait=True)
        log(f"timed {steps} tokens in {wall:.2f} s: p50 {pct(lat, 50):.2f} ms p99 {pct(lat, 99):.2f} ms; {prof}")
        # the probe tokens: device stamps per layer
        # stamps per gated layer: export end, wait entry, ready seen (0: no miss), wait exit; and the engine's compute
        # start. A zero-miss layer: the wait kernel's own time (entry -> exit), the dispatch gaps either side of it,
        # and export end -> compute start (what the engine sees).
        zero_gap, zero_wait_kernel, gap_in, gap_out, miss_wait = [], [], [], [], []
        ctx.profile_enable(ctx.PROF_COPY | ctx.PROF_WRITEBACK)
        for i in range(probe):
            t = warm + steps + i
            cks, _ = eng.token(routes[t], preds=pred_of(t))
            check_cks(t, cks)
            st = ctx.dg_stamps().astype(np.int64)
            start = eng.stamps().astype(np.int64)
            us = TICK_NS / 1e3
            for g in range(G):
                if st[g, 2] == 0:
                    zero_gap.append((start[g] - st[g, 0]) * us)
                    zero_wait_kernel.append((st[g, 3] - st[g, 1]) * us)
                    gap_in.append((st[g, 1] - st[g, 0]) * us)
                    gap_out.append((start[g] - st[g, 3]) * us)
                else:
                    miss_wait.append((st[g, 2] - st[g, 1]) * TICK_NS / 1e6)
        pprof = ctx.profile_read(wait=True)  # the probe tokens' copy and write-back brackets
        log(f"probe tokens: {pprof}")
        dkeys = ["tokens", "lookups", "misses", "fetched", "evicted", "bank_serves", "writebacks_done",
                 "inclusive_kept", "inclusive_drops", "miss_layers", "wb_forced", "collected_mid", "stalled"]
        if three:
            dkeys += ["disk_reads", "disk_read_bytes", "disk_read_ns", "disk_wait_ns", "disk_stage_waits",
                      "disk_drops", "disk_discards", "clean_drops", "bank_kept"]
        if policy:
            dkeys += ["scored_victims", "score_layers", "score_candidates", "score_ns", "score_fallbacks"]
        if n_pred:
            dkeys += ["predicted", "predicted_true", "prefetched", "prefetch_used"]
        if three and a.landing_blocks:
            dkeys += ["landing_issued", "landing_promoted", "landing_late", "landing_expired", "landing_expired_layer",
                      "landing_dropped_full", "landing_read_bytes", "landing_cancelled", "landing_yields",
                      "landing_aborted_bytes", "landing_wait_ns"]
        dstat = {k: s1[k] - s0[k] for k in dkeys}
        if three:
            dstat["disk_max_in_flight"] = s1["disk_max_in_flight"]
            dstat["disk_queue_resolved"] = s1["disk_queue_resolved"]
            dstat["disk_depth_adapt"] = s1["disk_depth_adapt"]
            dstat["disk_depth_active"] = s1["disk_depth_active"]
            dstat["disk_depth_changes"] = s1["disk_depth_changes"]
            dstat["disk_depth_calibrations"] = s1["disk_depth_calibrations"]
        failures = ctx.verify_failures()
        eng.close()
        ctx.close()
        plan.close()
        d.close()
        peaks = measure_peaks(tsa, L, C)
        log(f"peaks {peaks}")
        kern = measure_kernels(tsa, L, C, w)
        log(f"kernels {kern}")

        copy_gbps = pprof["copy_bytes"] / pprof["copy_ns"] if pprof["copy_ns"] else None
        # units with a part under 8 MiB are staged, and with device verify their scatter is the check
        # (dg_scatter_verify_kernel): each landed unit is read from HBM staging and written to its slot once
        fused = len(w.parts) > 1 and min(w.parts) < (8 << 20)
        ver_bytes = prof["verify_bytes"] * (2 if fused else 1)
        traffic_unit = (SCATTER_VERIFY_TRAFFIC_PER_UNIT if fused else VERIFY_TRAFFIC_PER_UNIT).get(w.unit_bytes)
        ver_gbps = ver_bytes / prof["verify_ns"] if prof["verify_ns"] else None
        miss_bytes = dstat["fetched"] * w.unit_bytes
        result = {
            "metric": METRIC,
            "value": round(pct(lat, 50), 3),
            "unit": "ms",
            "n_gpus": 1,
            "steps": steps,
            "warmup": warm,
            "ms_per_step": round(wall * 1e3 / steps, 3),
            "higher_is_better": False,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "u8",
            "data": (f"synthetic ({'Q4 blocks (fp16 scale + 16 bytes of 4-bit values per 18 bytes)' if w.gen == 2 else 'bf16 N(0, 0.02)'}"
                     f" expert bytes from the counter-based generator; Zipf({w.zipf_s}) routes)"),
            "config": {"workload": f"{w.name}: {w.layers} layers x {w.units} experts, top-{w.top_k}, units "
                                   f"{w.unit_bytes} B (3 parts), {n_res} resident / {n_pin} pinned"
                                   + (f" / {n_file} read from the file tier (direct I/O, "
                                      f"{dstat.get('disk_queue_resolved', 1)} reads in flight)" if three else "")
                                   + ", device-gated hipGraph token, verify_hash 2"
                                   + (f"; {w.layers} of the full model's {W.WORKLOADS[w.name].layers} layers"
                                      if w.layers != W.WORKLOADS[w.name].layers else ""),
                       "policy": a.policy,
                       "copies": copies,
                       "options": {k: v for k, v in extra.items()},
                       "predict": a.predict,
                       "residency": f"{n_res} of {w.n_units} units resident ({100 * n_res / w.n_units:.0f} %); device "
                                    f"arena {shape.R + shape.D + 2 * shape.B + 1} of {w.n_units} unit slots (residents "
                                    f"R {shape.R} + spares D {shape.D} + two banks of {shape.B} + the guard slot)",
                       "layers": w.layers, "experts": w.units, "top_k": w.top_k, "unit_bytes": w.unit_bytes,
                       "resident_units": n_res, "pinned_units": n_pin, "file_units": n_file,
                       "spare_slots": shape.D, "spare_blocks": shape.Q, "inclusive_blocks": shape.I,
                       "device_budget_bytes": shape.budget["device_bytes"],
                       "pinned_budget_bytes": shape.budget["host_pinned_bytes"]},
            "p50_ms": round(pct(lat, 50), 3),
            "p99_ms": round(pct(lat, 99), 3),
            "tokens_per_s": round(steps / wall, 3),
            "misses_per_token": round(dstat["misses"] / steps, 3),
            "h2d": {"miss_bytes": miss_bytes,
                    "busy_GBps": round(copy_gbps, 2) if copy_gbps else None,
                    "busy_sample": f"{pprof['copies']} unit copies of the {probe} probe tokens after the timed ones, "
                                   f"each part bracketed by timed events",
                    "wall_GBps": round(miss_bytes / wall / 1e9, 2),
                    "pinned_peak_GBps": round(peaks["h2d_pinned_GBps"], 2),
                    "frac_of_pinned_peak": round(copy_gbps / peaks["h2d_pinned_GBps"], 3) if copy_gbps else None,
                    "frac_of_pcie_gen5_x16": round(copy_gbps / 64.0, 3) if copy_gbps else None},
            "roofline": {"bound": "hbm",
                         "kernel": dg_check_kernel(w.parts, verify_seg_bytes(w.unit_bytes), fused)
                         + (" (each staged unit into its slot, XXH64-checked on the way)" if fused
                            else " (device XXH64 of every landed unit)"),
                         "achieved": round(ver_gbps, 1) if ver_gbps else None, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(ver_gbps / HBM_PEAK_GBPS, 4) if ver_gbps else None,
                         "traffic": int(traffic_unit * prof["verify_units"] / max(prof["verifies"], 1))
                         if traffic_unit else None,
                         "traffic_source": TRAFFIC_SOURCE.get(("fused" if fused else "verify", w.unit_bytes)),
                         "launches": prof["verifies"], "units": prof["verify_units"],
                         "bytes_per_launch": ver_bytes // max(prof["verifies"], 1),
                         "mean_launch_us": round(prof["verify_ns"] / max(prof["verifies"], 1) / 1e3, 2),
                         "note": "live: each launch checks the units a layer's copies landed, before the layer's ready word "
                                 "(a one-wave dg_publish_kernel behind it writes the slot entries and the ready word; "
                                 "the engine's compute of the layer waits for it); standalone figure under "
                                 "kernels.verify"},
            "kernels": kern,
            "pcie": {k: round(peaks[k], 2) for k in ("h2d_pinned_GBps", "d2h_pinned_GBps", "bidir_h2d_GBps",
                                                    "bidir_d2h_GBps")},
            "hbm_copy_GBps": round(peaks["hbm_copy_GBps"], 1),
            "wait": {"zero_miss_wait_kernel_us_p50": round(pct(zero_wait_kernel, 50), 2) if zero_gap else None,
                     "zero_miss_wait_kernel_us_p99": round(pct(zero_wait_kernel, 99), 2) if zero_gap else None,
                     "zero_miss_layer_us_p50": round(pct(zero_gap, 50), 2) if zero_gap else None,
                     "zero_miss_layer_us_p99": round(pct(zero_gap, 99), 2) if zero_gap else None,
                     "zero_miss_dispatch_gaps_us_p50": [round(pct(gap_in, 50), 2), round(pct(gap_out, 50), 2)]
                     if zero_gap else None,
                     "zero_miss_samples": len(zero_gap),
                     "miss_layer_wait_ms_p50": round(pct(miss_wait, 50), 3) if miss_wait else None,
                     "miss_samples": len(miss_wait)},
            "writeback": {"parts": pprof["writebacks"], "bytes": pprof["writeback_bytes"],
                          "busy_GBps": round(pprof["writeback_bytes"] / pprof["writeback_ns"], 2)
                          if pprof["writeback_ns"] else None,
                          "sample": f"the {probe} probe tokens (part copies to host, issued at each boundary)"},
            "open": {"seconds": round(open_s, 2),
                     "device_bytes": n_res * w.unit_bytes, "pinned_bytes": n_pin * w.unit_bytes,
                     "hashed_bytes": (n_res + n_pin + n_file) * w.unit_bytes,
                     "hashed_GBps": round((n_res + n_pin + n_file) * w.unit_bytes / open_s / 1e9, 2),
                     "device_GBps": round(n_res * w.unit_bytes / open_s / 1e9, 2),
                     "note": "ss_open's fill: every unit read from the source once and hashed on the host (checkpoints "
                             "for the device check), the residents copied into HBM through pinned staging blocks, the "
                             "pinned homes kept in their blocks; 16 worker threads"},
            "stats": dstat,
            "checks": {"verify_failures": failures, "checksum_mismatches": ck_bad,
                       "units_seen": len(ck_seen)},
            "cpu_baseline": None,
        }
        if three:
            rb = dstat["disk_read_bytes"]
            result["file_tier"] = {
                "reads_per_token": round(dstat["disk_reads"] / steps, 3),
                "read_GBps_wall": round(rb / wall / 1e9, 2),
                "read_ms_mean": round(dstat["disk_read_ns"] / max(dstat["disk_reads"], 1) / 1e6, 3),
                "read_GBps_per_reader": round(rb / dstat["disk_read_ns"], 2) if dstat["disk_read_ns"] else None,
                "service_wait_ms_per_token": round(dstat["disk_wait_ns"] / steps / 1e6, 3),
                "reads_in_flight_max": dstat["disk_max_in_flight"],
                "drive_direct_read_GBps": disk_peak,
                "note": "read_GBps_wall: file-tier bytes read over the timed region's wall clock; the reads run on "
                        "reader threads while earlier copies and layers proceed (the service waits only before a "
                        "layer's ready word)"}
        if not a.no_cpu:
            est = float(np.median(lat)) / 1e3 * 20  # a first guess of the CPU's time per token
            got, why = cpu_baseline(w, shape, files, hashes, routes, warm, est, a.cpu_seconds, policy=policy)
            if got:
                ms, c, n_tok = got
                result["cpu_baseline"] = {
                    "value": round(pct(ms, 50), 3), "unit": "ms", "cores": 1, "kind": "reference",
                    "p99_ms": round(pct(ms, 99), 3), "mean_ms": round(float(np.mean(ms)), 3),
                    "copy_GBps": round(c["copied_bytes"] / (float(np.sum(ms)) / 1e3) / 1e9, 2),
                    "sample": f"tokens {warm}..{warm + n_tok - 1} of the same route stream, after tokens 0..{warm - 1} "
                              f"replayed untimed from the open-time placement (so the timed tokens start from the "
                              f"placement the GPU's timed tokens start from): reference DgCore + memcpy transport + "
                              f"host XXH64 of each landed unit"
                              + (", file-tier units read synchronously with direct I/O into staging buffers"
                                 if three else "")
                              + f", 1 thread, policy {a.policy}; misses {c['misses']}, hash mismatches "
                                f"{c['hash_mismatches']}"
                              + (f", file reads {c['disk_reads']}" if three else ""),
                    "cpu": cpu_model(), "nproc": os.cpu_count()}
            else:
                log(f"cpu baseline skipped: {why}")
    finally:
        for h in reversed(opened):  # (close is idempotent: the normal path closed them already)
            h.close()
        shutil.rmtree(work, ignore_errors=True)
        if cold_work:
            shutil.rmtree(cold_work, ignore_errors=True)
    print(json.dumps(result), flush=True)


def run_host(a, w, tsa, ss, W, L, C):
    """The host contract (ss_begin, per layer ss_layer_routes or ss_layer_all, ss_acquire or ss_acquire_groups with
    every group waited for, the engine's read of the routed units through the table, ss_release; ss_end), one step per
    forward, timed on the engine thread (tse_host_run); every landed unit re-hashed in HBM (verify_hash 2)."""
    shape = W.host_shape(w)
    base = a.workdir or ("/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir())
    work = tempfile.mkdtemp(prefix="tsa_bench_", dir=base)
    path = os.path.join(work, "weights.bin")
    result = {}
    opened = []  # handles to close in reverse order on every path out
    try:
        t0 = time.time()
        log(f"workload {w.name}: {w.layers} x {w.units} units of {w.unit_bytes / 2**20:.1f} MiB, writing "
            f"{W.source_bytes(w) / 1e9:.1f} GB to {path}")
        hashes = W.write_sources_gpu(w, path)
        log(f"sources written in {time.time() - t0:.1f} s")
        desc_json = W.desc_json(w, path, hashes)
        d = ss.Desc(desc_json)
        opened.append(d)
        b = ss.budget(**shape.budget)
        plan = ss.Plan(d, b)
        opened.append(plan)
        tiers = plan.tiers()
        n_res = sum(1 for r in tiers for t in r if t == 0)
        t0 = time.time()
        ctx = ss.Ctx(d, b, plan, ss.options(**shape.options))
        opened.append(ctx)
        log(f"context open in {time.time() - t0:.1f} s: {n_res} resident units, mode {shape.mode}, budget {shape.budget}")
        steps, warm = a.steps, a.warmup
        routes = W.route_stream(w, warm + steps)
        if shape.mode == 1:
            routes = np.tile(np.arange(w.units, dtype=np.int32), (warm + steps, w.layers, 1))
        ctx.host_run(routes[:warm], shape.mode, want_tables=False)
        s0 = ctx.stats_total()
        x0 = ctx.exclusive_stats() if w.tier_mode == 1 else None
        ctx.profile_enable(ctx.PROF_VERIFY)  # each check launch bracketed by its dispatch's own begin and end stamps
        tsa.check(L.tsa_device_sync())
        t_start = time.perf_counter()
        cks, _, stats, lat = ctx.host_run(routes[warm:warm + steps], shape.mode, want_tables=False)
        tsa.check(L.tsa_device_sync())
        wall = time.perf_counter() - t_start
        prof = ctx.profile_read(wait=True)
        s1 = ctx.stats_total()
        x1 = ctx.exclusive_stats() if w.tier_mode == 1 else None
        seen, bad = {}, 0
        for t in range(steps):
            for l in range(w.layers):
                for i, u in enumerate(routes[warm + t, l]):
                    if u < 0:
                        continue
                    v = int(cks[t, l, i])
                    if seen.setdefault((l, int(u)), v) != v:
                        bad += 1
        failures = int(ss._declare().tsa_test_verify_failures(ctx.h))
        ctx.close()
        plan.close()
        d.close()
        log(f"timed {steps} steps in {wall:.2f} s: p50 {pct(lat, 50):.2f} ms p99 {pct(lat, 99):.2f} ms")
        peaks = measure_peaks(tsa, L, C)
        kern = measure_kernels(tsa, L, C, w)
        dst = {k: s1[k] - s0[k] for k in s1 if k != "wait_ns"}
        h2d_bytes = dst["bytes_pinned"]
        result = {
            "metric": METRIC, "value": round(pct(lat, 50), 3), "unit": "ms", "n_gpus": 1, "steps": steps,
            "warmup": warm, "ms_per_step": round(wall * 1e3 / steps, 3), "higher_is_better": False, "scaling": "weak",
            "vs_baseline": None, "dtype": "u8",
            "data": f"synthetic ({'bf16 N(0, 0.02)' if w.gen == 1 else 'uniform'} bytes from the counter-based "
                    f"generator; {w.routes} routes)",
            "config": {"workload": f"{w.name}: {w.layers} layers x {w.units} units of {w.unit_bytes} B, "
                                   f"{w.tokens} x top-{w.top_k} per step, {n_res} resident, host contract mode "
                                   f"{shape.mode} ({['ss_acquire', 'ss_layer_all', 'ss_acquire_groups'][shape.mode]}), "
                                   f"{'exclusive' if w.tier_mode == 1 else 'inclusive'}, verify_hash 2",
                       "budget": shape.budget, "options": shape.options},
            "p50_ms": round(pct(lat, 50), 3), "p99_ms": round(pct(lat, 99), 3),
            "h2d": {"bytes_per_step": h2d_bytes // steps, "wall_GBps": round(h2d_bytes / wall / 1e9, 2),
                    "pinned_peak_GBps": round(peaks["h2d_pinned_GBps"], 2),
                    "frac_of_pinned_peak_wall": round(h2d_bytes / wall / 1e9 / peaks["h2d_pinned_GBps"], 3)},
            "roofline": host_roofline(prof, w),
            "kernels": kern,
            "stats": dst,
            "exclusive": {k: x1[k] - x0[k] for k in x1} if x1 else None,
            "checks": {"verify_failures": failures, "checksum_mismatches": bad, "units_seen": len(seen)},
            "cpu_baseline": None,
        }
        if not a.no_cpu:
            try:
                from oracle import ref
                if ref.available():
                    n_tok = int(max(3, min(steps, a.cpu_seconds / max(float(np.median(lat)) / 1e3 * 10, 1e-3))))
                    o = ss.options(**{k: v for k, v in shape.options.items() if k != "verify_hash"}, verify_hash=1)
                    ms, open_s = ref.host_time(desc_json, ss.budget(**shape.budget), o,
                                               routes[warm:warm + n_tok], shape.mode)
                    result["cpu_baseline"] = {
                        "value": round(pct(ms, 50), 3), "unit": "ms", "cores": 3, "kind": "reference",
                        "p99_ms": round(pct(ms, 99), 3),
                        "sample": f"steps {warm}..{warm + n_tok - 1} of the same route stream: the reference CPU "
                                  f"backend (memcpy copies, host XXH64 of what it reads) after its open "
                                  f"({open_s:.1f} s), the engine thread plus its 2 reader threads",
                        "cpu": cpu_model(), "nproc": os.cpu_count()}
            except Exception as e:  # noqa: BLE001
                log(f"cpu baseline skipped: {e}")
    finally:
        for h in reversed(opened):
            h.close()
        shutil.rmtree(work, ignore_errors=True)
    print(json.dumps(result), flush=True)


def host_roofline(prof, w):
    """The host contract's dominant kernel: verify_kernel, the device XXH64 of each batch of landed units (up to 32 per
    launch), live over the timed steps."""
    if not prof["verifies"] or not prof["verify_ns"]:
        return None
    gbps = prof["verify_bytes"] / prof["verify_ns"]
    per_launch = prof["verify_bytes"] / prof["verifies"]
    ratio = HOST_VERIFY_TRAFFIC_RATIO.get(w.unit_bytes)
    return {"bound": "hbm", "kernel": "verify_kernel (device XXH64 of each batch of landed units)",
            "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "traffic": int(ratio * per_launch) if ratio else None,
            "traffic_source": HOST_TRAFFIC_SOURCE.get(w.unit_bytes),
            "launches": prof["verifies"], "units": prof["verify_units"], "bytes_per_launch": int(per_launch),
            "mean_launch_us": round(prof["verify_ns"] / prof["verifies"] / 1e3, 2),
            "note": "live: each launch checks a batch of landed units behind both copy streams while the engine reads "
                    "resident and landed units; bracketed by the dispatch's own begin and end stamps"}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    main()
