"""The serve-path workloads (synthetic models and route streams) at their full sizes and scaled down for tests.

A workload is a desc-v1 model written to one source file (unit-major: every unit's parts back to back at a 4 KiB unit
stride, the layers one after the other), a budget, options and a seeded route stream:

  moe-small    4 layers x 8 experts, 3 parts of 1 MiB uniform bytes, top-2 uniform ids; ranked, VRAM for 50 % of the
               units, the rest pinned (inclusive); 64 decode steps. (host contract)
  dense-prefix 32 blob layers of 4096 x 4096 x 7 bf16 N(0, 0.02); prefix order, 12 of 32 layers resident, the rest
               pinned through the blob ring; ss_layer_all on every layer; 32 forwards. (host contract)
  mixtral      32 layers x 8 experts, parts 4096 x 14336 x 2 (gate, up, down: 112 MiB each) bf16 N(0, 0.02); Zipf(1.1)
               top-2 over a per-layer seeded permutation, batch 1; 40 % of the units resident, the rest pinned;
               device-gated, a hipGraph-captured token; 256 steps. Device-gated mode requires the exclusive tier mode:
               the inclusive intent is kept with dg_inclusive_blocks clean copies.
  qwen3-moe    48 layers x 128 experts, parts 2048 x 768 x 2 (3 MiB each) bf16; 32 tokens x top-8 per step (the route
               union per layer); exclusive with write-backs, ss_acquire_groups hits first; 25 % resident; 128 steps.
  deepseek-q4  58 layers x 256 experts, parts 7168 x 2048 in 18-byte Q4 blocks (8,257,536 bytes each, 24.8 MB per
               unit, 367.8 GB in all); Zipf(1.2) top-8, batch 1; three tiers: VRAM for 54.4 % of the units (200 GB:
               51.2 % residents, 8 spare slots per layer, the banks and the guard), pinned RAM for 17.4 % (64 GB: the
               pinned homes and 24 spare blocks), the rest read from the source file with direct I/O on a miss
               (dg_disk_tier, 4 reads in flight); device-gated, a hipGraph-captured token; 64 steps. The whole model
               needs more host memory than one measurement host holds with its page cache, so the benchmark runs it
               with fewer layers (the same per-layer shape, tier shares and routes).

Bytes come from the counter-based generator (tsa_synth on the GPU, the same words for uniform bytes as
oracle/synth.py); each unit's XXH64 is computed on the host by the library (tsa_xxh64_host).
"""
from __future__ import annotations

import ctypes as C
import json
import math
import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, field, replace
from pathlib import Path

import numpy as np

MiB = 1 << 20
GiB = 1 << 30
UNIT_ALIGN_FILE = 4096


@dataclass
class Workload:
    name: str
    layers: int
    units: int                 # per layer
    parts: list                # part bytes
    kind: str = "moe"          # moe | blob
    top_k: int = 2
    tokens: int = 1            # rows per step (the route union per layer)
    routes: str = "uniform"    # uniform | zipf
    zipf_s: float = 1.1
    gen: int = 0               # tsa_synth kind: 0 uniform bytes, 1 bf16 N(0, sigma)
    sigma: float = 0.02
    resident_fraction: float = 0.5
    order: str = "ranked"
    tier_mode: int = 0         # 0 inclusive, 1 exclusive
    forward: int = 0           # 0 host contract, 1 device-gated
    steps: int = 64
    layer_all: bool = False
    groups: bool = False
    dynamic_slots: int = 0
    ring_slots: int = 0
    spare_units: int = 0
    inclusive_blocks: int = 0
    pinned_fraction: float = 0.0  # three tiers: pinned homes + spare blocks as a share of the units (0: two tiers)
    disk_queue: int = 0        # three tiers: file reads in flight (dg_disk_queue)
    clean_evict: int = 0       # three tiers: dg_clean_evict
    group_units: int = 16      # host contract with groups: units per group (ss_options.group_units)
    seed: int = 1234
    notes: dict = field(default_factory=dict)

    @property
    def unit_bytes(self) -> int:
        return int(sum(self.parts))

    @property
    def n_units(self) -> int:
        return self.layers * self.units

    @property
    def unit_stride_file(self) -> int:
        return (self.unit_bytes + UNIT_ALIGN_FILE - 1) // UNIT_ALIGN_FILE * UNIT_ALIGN_FILE

    @property
    def max_ids(self) -> int:
        return self.units if self.layer_all else min(64, self.tokens * self.top_k) if self.forward else \
            self.tokens * self.top_k


BF16 = 2
WORKLOADS = {
    "moe-small": Workload("moe-small", 4, 8, [MiB] * 3, top_k=2, routes="uniform", gen=0, resident_fraction=0.5,
                          steps=64, ring_slots=0),
    "dense-prefix": Workload("dense-prefix", 32, 1, [4096 * 4096 * 7 * BF16], kind="blob", top_k=1, gen=1,
                             order="prefix", resident_fraction=12 / 32, layer_all=True, steps=32),
    # 36 clean copies in 40 spare blocks: 154 + 40 pinned blocks of 336 MiB (63.7 GiB) stay under the 65 GiB of
    # hipHostMalloc memory one process can hold on the measured MI355X host
    "mixtral": Workload("mixtral", 32, 8, [4096 * 14336 * BF16] * 3, top_k=2, routes="zipf", zipf_s=1.1, gen=1,
                        resident_fraction=0.4, tier_mode=1, forward=1, steps=256, inclusive_blocks=36,
                        spare_units=40),
    "qwen3-moe": Workload("qwen3-moe", 48, 128, [2048 * 768 * BF16] * 3, top_k=8, tokens=32, routes="zipf",
                          zipf_s=1.1, gen=1, resident_fraction=0.25, tier_mode=1, groups=True, steps=128,
                          dynamic_slots=8),
    "deepseek-q4": Workload("deepseek-q4", 58, 256, [7168 * 2048 // 32 * 18] * 3, top_k=8, routes="zipf", zipf_s=1.2,
                            gen=2, resident_fraction=0.512, pinned_fraction=0.174, tier_mode=1, forward=1, steps=64,
                            dynamic_slots=8, spare_units=24, disk_queue=4),
}


def scaled(w: Workload, part_bytes: int | None = None, layers: int | None = None, units: int | None = None,
           steps: int | None = None, **kw) -> Workload:
    """The same shape at a size tests run in seconds."""
    parts = [part_bytes] * len(w.parts) if part_bytes else list(w.parts)
    return replace(w, parts=parts, layers=layers or w.layers, units=units or w.units, steps=steps or w.steps, **kw)


# ---- routes --------------------------------------------------------------------------------------------------------
def route_stream(w: Workload, steps: int | None = None) -> np.ndarray:
    """int32 [steps][layers][max_ids], -1 padded: per step and layer the ids of `tokens` rows x top_k (rows drawn
    without replacement inside a row; for device-gated workloads the flat row-major list, duplicates kept)."""
    steps = w.steps if steps is None else steps
    rng = np.random.default_rng(w.seed)
    perms = [np.random.default_rng(w.seed * 1000 + L).permutation(w.units) for L in range(w.layers)]
    k = min(w.top_k, w.units)
    width = w.tokens * k
    out = np.full((steps, w.layers, max(width, 1)), -1, dtype=np.int32)
    if w.routes == "zipf":
        p = 1.0 / np.power(np.arange(1, w.units + 1, dtype=np.float64), w.zipf_s)
        p /= p.sum()
    else:
        p = np.full(w.units, 1.0 / w.units)
    for s in range(steps):
        for L in range(w.layers):
            rows = []
            for _ in range(w.tokens):
                ranks = rng.choice(w.units, size=k, replace=False, p=p)
                rows.extend(int(perms[L][r]) for r in ranks)
            out[s, L, :len(rows)] = rows
    return out


# ---- sources, descriptor, budget -------------------------------------------------------------------------------------
def unit_offset(w: Workload, L: int, u: int, first_layer: int = 0) -> int:
    """Byte offset of unit (L, u) in the source file that holds layers first_layer.. (unit-major, 4 KiB stride)."""
    return ((L - first_layer) * w.units + u) * w.unit_stride_file


def source_bytes(w: Workload, n_layers: int | None = None) -> int:
    return (w.layers if n_layers is None else n_layers) * w.units * w.unit_stride_file


def write_sources_gpu(w: Workload, path: str | os.PathLike, threads: int = 16, first_layer: int = 0,
                      n_layers: int | None = None, drop_cache: bool = False) -> list:
    """Writes a source file holding layers first_layer .. first_layer + n_layers - 1 (default: every layer) from
    bytes the GPU generates (tsa_synth); returns those units' XXH64 list (model order), computed on the host by the
    library. Each unit's parts are stream ids 4 g + p (g = its global unit index). drop_cache: the file is synced and
    its pages dropped from the page cache afterwards (a direct-I/O reader then reads the device)."""
    import tierstream_amd as tsa
    L = tsa.lib()
    path = str(path)
    n_layers = w.layers - first_layer if n_layers is None else n_layers
    n_units = n_layers * w.units
    g_first = first_layer * w.units
    fd = os.open(path, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o644)
    try:
        os.ftruncate(fd, source_bytes(w, n_layers))
    finally:
        os.close(fd)
    ub = w.unit_bytes
    batch = max(1, min(n_units, (2 * GiB) // max(ub, 1)))  # units per GPU batch
    dev = tsa.DeviceBuffer(batch * w.unit_stride_file)
    host = C.c_void_p()
    tsa.check(L.tsa_host_alloc(C.byref(host), batch * w.unit_stride_file))
    hashes = [0] * n_units
    try:
        fd = os.open(path, os.O_WRONLY)
        with ThreadPoolExecutor(threads) as ex:
            for i0 in range(0, n_units, batch):
                n = min(batch, n_units - i0)
                for i in range(n):
                    off = 0
                    for p, pb in enumerate(w.parts):
                        tsa.check(L.tsa_synth(C.c_void_p(dev.ptr + i * w.unit_stride_file + off), pb, w.seed,
                                              4 * (g_first + i0 + i) + p, 0, w.gen, C.c_float(w.sigma), None))
                        off += pb
                tsa.check(L.tsa_memcpy(host, C.c_void_p(dev.ptr), n * w.unit_stride_file, 1, None))
                tsa.check(L.tsa_stream_sync(None))
                base = host.value

                def one(i):
                    p = base + i * w.unit_stride_file
                    hashes[i0 + i] = int(L.tsa_xxh64_host(C.c_void_p(p), ub))
                    mv = (C.c_char * ub).from_address(p)
                    os.pwrite(fd, mv, (i0 + i) * w.unit_stride_file)

                list(ex.map(one, range(n)))
        if drop_cache:
            os.fsync(fd)
            os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
        os.close(fd)
    finally:
        L.tsa_host_free(host)
        dev.close()
    return hashes


PART_FORMAT = {0: "U8", 1: "BF16", 2: "Q4_0"}


def desc_json(w: Workload, path, hashes: list) -> str:
    """The desc-v1 descriptor. path: one source file holding every layer, or a list of (path, first_layer, n_layers)
    covering the layers in order (each layer's parts read the file that holds it)."""
    files = [(str(path), 0, w.layers)] if isinstance(path, (str, os.PathLike)) else [(str(p), a, n) for p, a, n in path]
    src_of = {}
    for i, (_, a, n) in enumerate(files):
        for L in range(a, a + n):
            src_of[L] = (i, a)
    assert sorted(src_of) == list(range(w.layers)), "the source files must cover every layer once"
    layers = []
    for L in range(w.layers):
        off = 0
        parts = []
        names = ["gate", "up", "down"] if len(w.parts) == 3 else [f"p{i}" for i in range(len(w.parts))]
        src, first = src_of[L]
        for p, pb in enumerate(w.parts):
            parts.append({"name": names[p], "format": PART_FORMAT[w.gen], "source": src,
                          "offset": unit_offset(w, L, 0, first) + off, "stride": w.unit_stride_file, "bytes": pb})
            off += pb
        lay = {"index": L, "kind": w.kind, "n_units": w.units, "unit_bytes": w.unit_bytes, "parts": parts,
               "hash": [f"{h:016x}" for h in hashes[L * w.units:(L + 1) * w.units]]}
        if w.kind == "moe":
            lay["top_k"] = min(w.top_k, w.units)
        layers.append(lay)
    d = {"schema": "strix-stream/desc-v1", "model": w.name, "engine": "tsa-synthetic", "unit_align": 256,
         "order": w.order, "tiers": "pinned|disk" if w.pinned_fraction else "pinned",
         "sources": [{"name": f"weights{i}" if i else "weights", "path": p, "align": 4096}
                     for i, (p, _, _) in enumerate(files)],
         "layers": layers}
    return json.dumps(d)


def unit_stride_dev(w: Workload) -> int:
    return (w.unit_bytes + 255) // 256 * 256


@dataclass
class DgShape:
    """A device-gated workload's cache shape: R planned residents (the first units in model order: equal benefit), D
    spare slots, B ids per layer (2 B + 1 bank and guard slots), P pinned homes, Q spare blocks, I clean copies; three
    tiers: F file-tier units (the last in model order) and the explicit plan tiers (0 resident, 1 pinned, 2 file) in
    model order."""
    R: int
    D: int
    B: int
    P: int
    Q: int
    I: int
    budget: dict
    options: dict
    F: int = 0
    tiers: list | None = None

    def cold_first_layer(self, w: Workload) -> int:
        """The first layer holding a file-tier unit (w.layers with none)."""
        return (self.R + self.P) // w.units if self.F else w.layers


def dg_shape(w: Workload) -> DgShape:
    """The budget and options that give a device-gated workload its resident fraction. Units are ranked with equal
    benefit, so the residents are the first R units in model order. Each layer contributes min(dynamic slots, its
    non-resident units) spare slots; the ring is the 2 B + 1 bank and guard slots. dg_inclusive_blocks covers every unit
    that can be on the device beyond the planned residents (D + 2 B), so evicting one is a drop (the inclusive intent;
    device-gated mode runs the exclusive tier mode), and Q keeps 4 blocks beyond them for write-backs of evicted planned
    residents."""
    st = unit_stride_dev(w)
    hs = (w.unit_bytes + 4095) // 4096 * 4096
    R = int(round(w.resident_fraction * w.n_units))
    B = w.max_ids
    if w.pinned_fraction:
        return _dg_shape_three_tier(w, R, B, st, hs)
    dyn = w.dynamic_slots or 1
    res_in = [min(w.units, max(0, R - L * w.units)) for L in range(w.layers)]
    D = sum(min(dyn, w.units - r) for r in res_in)
    ring = 2 * B + 1
    P = w.n_units - R
    I = w.inclusive_blocks or (D + 2 * B)
    Q = w.spare_units or (I + 4)
    # the planner reserves min(dynamic slots, units) for every layer before it places residents (reference
    # src/plan.cpp:60-64); the spare slots it bills afterwards (D) are what the residents leave
    reserve = w.layers * min(dyn, w.units)
    # the open pins a staging unit, a bounce buffer and its control area on top of the plan's blocks, and admits a
    # budget with four units of startup headroom beyond them
    budget = dict(device_bytes=(R + reserve + ring) * st + st // 2, host_pinned_bytes=(P + Q + 5) * hs + (64 << 20),
                  dynamic_slots_per_layer=dyn, ring_slots=ring, tier_mode=1, host_spare_units=Q)
    options = dict(forward_mode=1, dg_max_ids=B, pin_planned=0, dg_inclusive_blocks=I, dg_wb_defer=1)
    return DgShape(R, D, B, P, Q, I, budget, options)


def _dg_shape_three_tier(w: Workload, R: int, B: int, st: int, hs: int) -> DgShape:
    """Three tiers from explicit plan tiers (a planner spill to the file tier fills the pinned budget and leaves no
    spare block, which device-gated decode needs): the first R units resident, the next P pinned, the last F read from
    their file. Pinned memory holds P homes and Q spare blocks (round(pinned_fraction x units) in all); a device victim
    with no free block drops the least recently homed pinned unit to its file for its block, so Q only absorbs the
    write-backs in flight. No clean copies (inclusive blocks) in three-tier mode."""
    dyn = w.dynamic_slots or 1
    res_in = [min(w.units, max(0, R - L * w.units)) for L in range(w.layers)]
    D = sum(min(dyn, w.units - r) for r in res_in)
    ring = 2 * B + 1
    Q = w.spare_units or (2 * B + 8)
    P = int(round(w.pinned_fraction * w.n_units)) - Q
    F = w.n_units - R - P
    if P < 1 or F < 1:
        raise ValueError(f"{w.name}: three tiers need pinned and file units (R {R}, P {P}, F {F})")
    reserve = w.layers * min(dyn, w.units)
    # the open's own pinned buffers come on top of the plan's: a staging unit, the 8 staging buffers of the file tier,
    # a margin for its control area and a bounce buffer per reader, and four units of startup headroom (landing
    # blocks, when asked for, are added by the caller)
    budget = dict(device_bytes=(R + reserve + ring) * st + st // 2,
                  host_pinned_bytes=(P + Q + 13) * hs + (160 << 20),
                  dynamic_slots_per_layer=dyn, ring_slots=ring, tier_mode=1, host_spare_units=Q)
    options = dict(forward_mode=1, dg_max_ids=B, pin_planned=0, dg_wb_defer=1, dg_disk_tier=1,
                   dg_disk_queue=w.disk_queue, dg_clean_evict=w.clean_evict)
    return DgShape(R, D, B, P, Q, 0, budget, options, F=F, tiers=[0] * R + [1] * P + [2] * F)


@dataclass
class HostShape:
    """A host-contract workload's budget, options and engine mode (0 ss_layer_routes + ss_acquire, 1 ss_layer_all +
    ss_acquire, 2 ss_layer_routes + ss_acquire_groups)."""
    R: int
    budget: dict
    options: dict
    mode: int


def host_shape(w: Workload) -> HostShape:
    """The budget that gives a host-contract workload its resident share. Units are ranked with equal benefit (or in
    prefix order), so the residents are the first R units in model order; the planner reserves the dynamic slots and
    the ring before it places residents (reference src/plan.cpp:60-83), so they are billed on top. Exclusive mode
    bills spare blocks (host_spare_units) for the write-backs of evicted units."""
    st = unit_stride_dev(w)
    hs = (w.unit_bytes + 4095) // 4096 * 4096
    R = int(round(w.resident_fraction * w.n_units))
    dyn = w.dynamic_slots
    ring = w.ring_slots or (2 if w.kind == "blob" else 2 * min(w.units, max(8, w.max_ids // 4)))
    Q = w.spare_units or (dyn * w.layers if w.tier_mode == 1 else 0)
    budget = dict(device_bytes=(R + dyn * w.layers + ring) * st + st // 2,
                  host_pinned_bytes=(w.n_units - R + Q) * hs + hs // 2 + (64 << 20),
                  dynamic_slots_per_layer=dyn, ring_slots=ring, tier_mode=w.tier_mode, host_spare_units=Q)
    options = dict(pin_planned=0 if dyn else 1, verify_hash=2)
    if w.groups:
        options["group_units"] = w.group_units
    mode = 1 if w.layer_all else (2 if w.groups else 0)
    return HostShape(R, budget, options, mode)
