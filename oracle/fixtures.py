"""ORACLE (test infrastructure only): small synthetic models written with numpy, independent of the product.

A model is one source file, unit-major: unit g = (layer L, unit u) at g x stride, its parts back to back; part p of
unit g holds the generator's stream 4 g + p (oracle/synth.py kind 0, the same words the product's device generator
gives). The descriptor carries each unit's XXH64 computed by the oracle. expected() gives a unit's bytes, its digest
and the engine checksum from the file as written.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field

import numpy as np

from . import synth, xxh64

FILE_ALIGN = 4096


@dataclass
class Model:
    path: str
    layers: int
    units: int
    parts: list
    kind: str = "moe"
    top_k: int = 2
    order: str = "ranked"
    seed: int = 99
    hashes: list = field(default_factory=list)
    tiers: str = "pinned"  # the descriptor's tier list ("pinned|disk": the planner spills to the file tier)
    checksums: list = field(default_factory=list)  # engine_checksum of each unit, in unit order (at write time)

    @property
    def unit_bytes(self):
        return int(sum(self.parts))

    @property
    def stride(self):
        return (self.unit_bytes + FILE_ALIGN - 1) // FILE_ALIGN * FILE_ALIGN

    def unit_data(self, L: int, u: int) -> np.ndarray:
        g = L * self.units + u
        return np.concatenate([synth.uniform_bytes(self.seed, 4 * g + p, 0, pb) for p, pb in enumerate(self.parts)])

    def checksum(self, L: int, u: int) -> int:
        """engine_checksum of unit (L, u)'s bytes as written."""
        return self.checksums[L * self.units + u]

    def desc_json(self) -> str:
        layers = []
        for L in range(self.layers):
            off = 0
            parts = []
            for p, pb in enumerate(self.parts):
                parts.append({"name": f"p{p}", "format": "U8", "source": 0,
                              "offset": L * self.units * self.stride + off, "stride": self.stride, "bytes": pb})
                off += pb
            lay = {"index": L, "kind": self.kind, "n_units": self.units, "unit_bytes": self.unit_bytes,
                   "parts": parts, "hash": [f"{h:016x}" for h in self.hashes[L * self.units:(L + 1) * self.units]]}
            if self.kind == "moe":
                lay["top_k"] = self.top_k
            layers.append(lay)
        return json.dumps({"schema": "strix-stream/desc-v1", "model": "oracle-fixture", "engine": "oracle",
                           "unit_align": 256, "order": self.order, "tiers": self.tiers,
                           "sources": [{"name": "w", "path": self.path, "align": 4096}], "layers": layers})


def write_model(directory, layers, units, parts, kind="moe", top_k=2, order="ranked", seed=99,
                tiers="pinned") -> Model:
    m = Model(os.path.join(str(directory), f"weights-{seed}.bin"), layers, units, list(parts), kind, top_k, order, seed,
              tiers=tiers)
    assert all(pb % 8 == 0 for pb in parts)
    with open(m.path, "wb") as f:
        for L in range(layers):
            for u in range(units):
                b = m.unit_data(L, u)
                m.hashes.append(xxh64(b))
                m.checksums.append(engine_checksum(b))
                f.write(b.tobytes())
                f.write(b"\0" * (m.stride - m.unit_bytes))
    return m


def engine_checksum(b: np.ndarray) -> int:
    """The synthetic engine's checksum of a unit: sum of its little-endian u32 words w_j x ((j mod 251) + 1), mod 2^64
    (the formula tierstream_amd/engine/engine.hip computes on the device)."""
    w = np.frombuffer(np.ascontiguousarray(b).tobytes(), dtype="<u4").astype(np.uint64)
    mult = (np.arange(w.size, dtype=np.uint64) % np.uint64(251)) + np.uint64(1)
    with np.errstate(over="ignore"):
        return int(np.sum(w * mult, dtype=np.uint64))


def uniform_routes(layers, units, top_k, steps, seed, tokens=1):
    """[steps][layers][tokens * top_k] ids, each row top_k distinct uniform ids."""
    rng = np.random.default_rng(seed)
    out = np.full((steps, layers, tokens * top_k), -1, dtype=np.int32)
    for s in range(steps):
        for L in range(layers):
            out[s, L] = np.concatenate([rng.choice(units, size=top_k, replace=False) for _ in range(tokens)])
    return out
