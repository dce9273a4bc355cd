"""Descriptor and plan formats against the reference's own planner (oracle/_ref, compiled from its sources), on the
CPU: the same desc-v1 JSON and budget give the same canonical descriptor JSON, the same plan-v1 JSON (every unit's
tier, the rings, the spare blocks, the byte totals) or the same refusal status. The grid mixes MoE and blob layers,
ranked and prefix order, inclusive and exclusive tier modes, margins, dynamic and ring slots, spare units and engine
benefits (reference src/desc.cpp, src/plan.cpp:36-477)."""
import json

import numpy as np
import pytest

from oracle import ref
from tierstream_amd import SsError, ss

pytestmark = pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built (needs the reference sources)")

MiB = 1 << 20


def desc(rng, order, kinds):
    layers = []
    off = 0
    for L, kind in enumerate(kinds):
        n = 1 if kind == "blob" else int(rng.choice([4, 8, 16]))
        n_parts = 1 if kind == "blob" else int(rng.choice([1, 2, 3]))
        parts_b = [int(rng.choice([64, 96, 256, 1000])) * 4096 for _ in range(n_parts)]
        ub = sum(parts_b)
        stride = (ub + 4095) // 4096 * 4096
        parts, po = [], 0
        for p, pb in enumerate(parts_b):
            parts.append({"name": f"p{p}", "format": "U8", "source": 0, "offset": off + po, "stride": stride,
                          "bytes": pb})
            po += pb
        lay = {"index": L, "kind": kind, "n_units": n, "unit_bytes": ub, "parts": parts,
               "hash": [f"{int(h):016x}" for h in rng.integers(0, 2**63, size=n)]}
        if kind == "moe":
            lay["top_k"] = int(min(2, n))
        layers.append(lay)
        off += n * stride
    return json.dumps({"schema": "strix-stream/desc-v1", "model": "grid", "engine": "oracle", "unit_align": 256,
                       "order": order, "tiers": "pinned", "sources": [{"name": "w", "path": "/nonexistent/w.bin",
                                                                         "align": 4096}], "layers": layers})


def cases(n=150):
    rng = np.random.default_rng(2024)
    for i in range(n):
        kinds = list(rng.choice(["moe", "moe", "blob"], size=int(rng.integers(2, 7))))
        order = str(rng.choice(["ranked", "prefix"]))
        d = desc(rng, order, kinds)
        dj = json.loads(d)
        total = sum(l["n_units"] * ((l["unit_bytes"] + 255) // 256 * 256) for l in dj["layers"])
        host_total = sum(l["n_units"] * ((l["unit_bytes"] + 4095) // 4096 * 4096) for l in dj["layers"])
        host_frac = rng.uniform(0.3, 0.9) if rng.uniform() < 0.15 else rng.uniform(1.0, 1.4)  # some too small
        ring_slots = int(rng.choice([0, 3, 5]))
        strides = {(l["unit_bytes"] + 255) // 256 * 256 for l in dj["layers"]}
        widest = max(l["n_units"] for l in dj["layers"])
        rings = sum(strides) * (ring_slots or 2 * widest)  # the stream rings the planner reserves first
        kw = dict(device_bytes=int(rings + total * rng.uniform(0.0, 0.8)), host_pinned_bytes=int(host_total * host_frac),
                  tier_mode=int(rng.integers(0, 2)), dynamic_slots_per_layer=int(rng.choice([0, 0, 1, 2])),
                  ring_slots=ring_slots, host_spare_units=int(rng.choice([0, 0, 2, 6])))
        if rng.uniform() < 0.3:
            kw.update(margin_gib=float(rng.choice([0.0, 0.001])), margin_fraction=float(rng.choice([0.0, 0.02])))
        n_units = sum(l["n_units"] for l in dj["layers"])
        benefit = list(rng.uniform(0, 1, size=n_units)) if rng.uniform() < 0.4 else None
        yield pytest.param(d, kw, benefit, id=f"case{i}")


@pytest.mark.parametrize("d,kw,benefit", list(cases()))
def test_plan_matches_reference(d, kw, benefit):
    want_status = ref.plan_status(d, ss.budget(**kw), benefit)
    desc_ = ss.Desc(d)
    assert desc_.json() == ref.desc_roundtrip(d)
    if want_status != 0:
        with pytest.raises(SsError) as e:
            ss.Plan(desc_, ss.budget(**kw), benefit)
        assert e.value.status == want_status
        return
    got = ss.Plan(desc_, ss.budget(**kw), benefit)
    assert got.json() == ref.plan_json(d, ss.budget(**kw), benefit)


def _from_json(L, desc_text: str, budget, plan_text: bytes):
    """Status and canonical plan JSON of ss_plan_from_json over `plan_text` (None when refused)."""
    import ctypes as C
    vp = C.c_void_p
    L.ss_plan_from_json.restype = C.c_int
    L.ss_plan_from_json.argtypes = [vp, C.POINTER(ss.SsBudget), C.c_char_p, C.c_size_t, C.POINTER(vp)]
    d, p = vp(), vp()
    b = desc_text.encode()
    assert L.ss_desc_from_json(b, len(b), C.byref(d)) == 0
    try:
        st = L.ss_plan_from_json(d, C.byref(budget), plan_text, len(plan_text), C.byref(p))
        if st != 0:
            return st, None
        s, n = C.c_char_p(), C.c_size_t()
        assert L.ss_plan_to_json(p, C.byref(s), C.byref(n)) == 0
        out = C.string_at(s, n.value)
        L.ss_free(s)
        L.ss_plan_free(p)
        return 0, out
    finally:
        L.ss_desc_free(d)


def _tier_edits(tiers, rng):
    """The reference's plan tiers, and broken or re-lettered copies of them."""
    yield "same", tiers
    L = int(rng.integers(len(tiers)))
    yield "missing", None
    yield "short-list", tiers[:-1]
    if tiers[L]:
        yield "short-layer", tiers[:L] + [tiers[L][:-1]] + tiers[L + 1:]
        for letter in "RPDXBZr\x00":
            yield f"letter-{letter!r}", tiers[:L] + [letter + tiers[L][1:]] + tiers[L + 1:]
        yield "all-pinned", [("P" * len(t)) for t in tiers]
        yield "all-resident", [("R" * len(t)) for t in tiers]
        yield "all-backed", [("B" * len(t)) for t in tiers]
        yield "all-disk", [("D" * len(t)) for t in tiers]
    yield "number", tiers[:L] + [7] + tiers[L + 1:]


@pytest.mark.parametrize("d,kw,benefit", list(cases(40)))
def test_plan_from_json_matches_reference(d, kw, benefit):
    """ss_plan_from_json on the reference's own plan document and on edited copies of its tier letters (other tiers,
    a letter outside R P D X B, a NUL, wrong lengths, a missing or mistyped list): the same status and, when accepted,
    the same canonical plan (reference src/plan.cpp:460-477, src/capi.cpp:384-391)."""
    if ref.plan_status(d, ss.budget(**kw), benefit) != 0:
        pytest.skip("the reference makes no plan for this budget")
    want = ref.plan_json(d, ss.budget(**kw), benefit)
    rng = np.random.default_rng(len(d))
    for name, tiers in _tier_edits(want["tiers"], rng):
        doc = dict(want)
        if tiers is None:
            doc.pop("tiers")
        else:
            doc["tiers"] = tiers
        text = json.dumps(doc).encode()
        got_o = _from_json(ss._declare(), d, ss.budget(**kw), text)
        got_t = _from_json(ref.lib(), d, ss.budget(**kw), text)
        assert got_o == got_t, (name, got_o[0], got_t[0])
