"""The device-gated open's geometry and refusals on the CPU, against the reference's dg_layout (oracle/_ref): the same
descriptor, budget, plan and options through this library's dg_geometry (tsa_test_dg_geometry) and the reference's.
Either both refuse with the same status, or both lay out the same keys, gated layers, residents (R and their keys),
spare slots D, bank size B, pinned homes P, file homes F, spare blocks Q, clean-copy share I, staging buffers and reads
in flight, slot counts, guard slot, blocks, score weights and the landing settings (blocks, pieces running, TTL,
piece bytes).

Configurations are drawn per seed around valid ones: layers and units, one to five parts (now and then not a multiple
of 256, or five), the planner's tiers or explicit ones (with file homes), dynamic and explicit spare slots, ring slots
around 2 x dg_max_ids + 1, spare blocks, clean copies, the file tier's options, the policy and its weights, and a broken
option now and then (dg_bank_keep, dg_disk_queue_adapt and the landing options among them). Options the reference
accepts but this library does not serve (no-admit, prefetch revert, strict admission) must be refused with
SS_E_UNSUPPORTED."""
import ctypes as C

import numpy as np
import pytest

from oracle import fixtures, ref
from tierstream_amd import ss

KiB = 1024
u32 = C.c_uint32
FIELDS = ["keys", "G", "R", "D", "B", "P", "F", "Q", "I", "S", "disk_queue", "persistent_slots", "slots", "guard_slot",
          "blocks", "scored", "w_trans", "w_freq", "w_rec", "L", "landing_queued", "landing_ttl", "landing_chunk"]
UNSERVED = ["dg_no_admit", "dg_pf_revert_unused", "dg_pf_strict_admit"]


def _case(seed, tmp_path, landing=False):
    """landing: the file tier with explicit file homes and reads in flight, and the landing options drawn (mostly
    valid)."""
    rng = np.random.default_rng(seed)
    layers, units = int(rng.integers(1, 5)), int(rng.integers(2, 17))
    n_parts = int(rng.choice([1, 2, 3, 3, 4])) if rng.random() < 0.97 else 5
    parts = [int(rng.integers(1, 9)) * 4 * KiB for _ in range(n_parts)]
    if rng.random() < 0.05:
        parts[0] += 128  # not a multiple of 256
    m = fixtures.write_model(tmp_path, layers, units, parts, top_k=2, seed=seed % 997,
                             tiers="pinned|disk" if landing else str(rng.choice(["pinned", "pinned|disk"])))
    st = (m.unit_bytes + 255) // 256 * 256
    hs = (m.unit_bytes + 4095) // 4096 * 4096
    B = int(rng.choice([1, 2, 4, 8])) if rng.random() < 0.95 else int(rng.choice([0, 65]))
    total = layers * units
    n_res = int(rng.integers(0, total // 2 + 1))
    dyn = int(rng.integers(1, 3)) if rng.random() < 0.9 else 0
    ring = max(0, 2 * max(B, 1) + 1 + int(rng.integers(-1, 3)))
    spares = int(rng.integers(0, 8))
    S_opt = int(rng.choice([0, 0, 4, 2, 16])) if rng.random() < 0.95 else 300
    bkw = dict(device_bytes=n_res * st + ring * st + dyn * layers * st + st // 2,
               host_pinned_bytes=(total + spares + 2 * 300) * hs + (512 << 20), dynamic_slots_per_layer=dyn,
               ring_slots=ring, tier_mode=1 if rng.random() < 0.97 else 0, host_spare_units=spares)
    okw = dict(forward_mode=1, dg_max_ids=B, pin_planned=0 if rng.random() < 0.97 else 1)
    tiers = None
    disk = landing or rng.random() < 0.4
    if landing or rng.random() < 0.5:  # explicit tiers (with file homes when the file tier is on)
        t = rng.choice([0, 1, 2] if disk else [0, 1], size=total, p=[0.3, 0.5, 0.2] if disk else [0.4, 0.6])
        tiers = [int(v) for v in t]
        n_res = sum(1 for v in tiers if v == 0)
        bkw["device_bytes"] = n_res * st + ring * st + dyn * layers * st + st // 2
    if disk:
        okw.update(dg_disk_tier=1, dg_disk_staging=S_opt,
                   dg_disk_queue=int(rng.choice([0, 1, 3, 8, 16, 0xFFFFFFFF, 65])),
                   dg_disk_prefetch=int(rng.integers(0, 2)))
    elif rng.random() < 0.05:
        okw.update(dg_disk_staging=4)  # without the file tier: refused
    if rng.random() < 0.3:
        okw.update(dg_inclusive_blocks=int(rng.integers(0, spares + 2)))
    if rng.random() < 0.2:
        okw.update(dg_spare_slots=int(rng.integers(0, total)))
    if rng.random() < 0.3:
        okw.update(policy=int(rng.choice([1, 2])) if rng.random() < 0.9 else 3)
        if rng.random() < 0.5:
            a, b = sorted(int(x) for x in rng.integers(0, 1001, size=2))
            okw.update(dg_score_w_trans=a, dg_score_w_freq=b - a, dg_score_w_recency=1000 - b + int(rng.random() < 0.1))
    if rng.random() < 0.15:
        okw.update(dg_bank_keep=int(rng.choice([0, 1, 2, 3])))
    if rng.random() < 0.1:  # (valid with the file tier at the AUTO queue only)
        okw.update(dg_disk_queue_adapt=int(rng.choice([1, 1, 2])))
        if disk and rng.random() < 0.7:
            okw.update(dg_disk_queue=0xFFFFFFFF)
    if landing or rng.random() < 0.2:  # landings: mostly valid (the file tier with reads in flight), now and then not
        lb = int(rng.choice([1, 2, 8, 64, 600])) if rng.random() < 0.95 else 5000
        okw.update(dg_landing_blocks=lb if rng.random() < 0.9 else 0)
        if rng.random() < 0.5:
            okw.update(dg_landing_max_queued=int(rng.choice([0, 1, 4, 4, 65])))
        if rng.random() < 0.5:
            okw.update(dg_landing_ttl=int(rng.choice([0, 1, 7, 7, 1025])))
        if rng.random() < 0.4:
            okw.update(dg_landing_chunk=int(rng.choice([0, 4096, 1 << 20, 0xFFFFFFFF, 5000])))
        if disk and rng.random() < 0.8 and okw.get("dg_disk_queue") in (0, 1, 65):
            okw.update(dg_disk_queue=int(rng.choice([3, 8])))
        if landing and rng.random() < 0.85:  # (no other broken option, mostly)
            for k in ("dg_bank_keep", "dg_disk_queue_adapt", "dg_wb_defer", "dg_wait_timeout_ms", "policy",
                      "dg_disk_staging"):
                okw.pop(k, None)
        if landing and rng.random() < 0.15:  # a host budget that holds the plan but not the landing blocks
            bkw["host_pinned_bytes"] = (total + spares) * hs + (okw.get("dg_landing_blocks") or 0) * hs // 2
    if rng.random() < 0.02:
        okw.update(dg_wb_defer=2)
    if rng.random() < 0.02:
        okw.update(dg_wait_timeout_ms=0)
    unserved = None
    if not landing and rng.random() < 0.08:
        unserved = str(rng.choice(UNSERVED))
        okw[unserved] = 1
    return m, bkw, okw, tiers, unserved


def _ours(js, b, tiers, o):
    import tierstream_amd as tsa
    L = tsa.lib()
    L.tsa_test_dg_geometry.restype = C.c_int
    L.tsa_test_dg_geometry.argtypes = [C.c_char_p, C.c_size_t, C.POINTER(ss.SsBudget), C.POINTER(C.c_uint8),
                                       C.c_size_t, C.POINTER(ss.SsOptions), C.POINTER(u32), C.POINTER(u32), u32]
    out = (u32 * len(FIELDS))()
    res = (u32 * 4096)()
    t = (C.c_uint8 * len(tiers))(*tiers) if tiers is not None else None
    st = L.tsa_test_dg_geometry(js, len(js), C.byref(b), t, len(tiers) if tiers else 0, C.byref(o), out, res, 4096)
    return st, dict(zip(FIELDS, list(out))), list(res)


def _theirs(js, b, tiers, o):
    L = ref.lib()
    f = L.ref_dg_layout
    f.restype = C.c_int
    f.argtypes = [C.c_char_p, C.c_size_t, C.POINTER(ss.SsBudget), C.POINTER(C.c_uint8), C.c_size_t,
                  C.POINTER(ss.SsOptions), C.POINTER(u32), C.POINTER(u32), u32, C.c_char_p, C.c_size_t]
    out = (u32 * len(FIELDS))()
    res = (u32 * 4096)()
    err = C.create_string_buffer(512)
    t = (C.c_uint8 * len(tiers))(*tiers) if tiers is not None else None
    st = f(js, len(js), C.byref(b), t, len(tiers) if tiers else 0, C.byref(o), out, res, 4096, err, 512)
    return st, dict(zip(FIELDS, list(out))), list(res), err.value.decode()


def _plan_ok(m, bkw, tiers):
    d = ss.Desc(m.desc_json())
    try:
        ss.Plan(d, ss.budget(**bkw), tiers=tiers).close()
        return True
    except ss.SsError:
        return False
    finally:
        d.close()


@pytest.mark.parametrize("seed", range(300))
def test_geometry_matches_reference(seed, tmp_path):
    if not ref.available():
        pytest.skip("oracle/_ref is not built")
    m, bkw, okw, tiers, unserved = _case(seed, tmp_path)
    if not _plan_ok(m, bkw, tiers):
        pytest.skip("the planner refuses this budget (a plan test's matter)")
    js = m.desc_json().encode()
    st_o, got, res_o = _ours(js, ss.budget(**bkw), tiers, ss.options(**okw))
    st_t, want, res_t, why = _theirs(js, ss.budget(**bkw), tiers, ss.options(**okw))
    if unserved:
        assert st_o in (st_t, 8) and (st_t != 0 or st_o == 8), (seed, unserved, st_o, st_t, why)  # 8: UNSUPPORTED
        return
    assert st_o == st_t, (seed, st_o, st_t, why)
    if st_t == 0:
        assert got == want, seed
        assert res_o[:want["R"]] == res_t[:want["R"]], seed


def test_cases_cover_layouts_and_refusals(tmp_path):
    """The draws are not vacuous: many lay out (with file homes, clean copies, scoring), and each refusal status
    occurs."""
    if not ref.available():
        pytest.skip("oracle/_ref is not built")
    laid = file_homes = statuses = 0
    seen = set()
    for seed in range(300):
        d = tmp_path / str(seed)
        d.mkdir()
        m, bkw, okw, tiers, unserved = _case(seed, d)
        if unserved or not _plan_ok(m, bkw, tiers):
            continue
        js = m.desc_json().encode()
        st, got, _, _ = _theirs(js, ss.budget(**bkw), tiers, ss.options(**okw))
        seen.add(st)
        if st == 0:
            laid += 1
            file_homes += got["F"] > 0
    assert laid > 60 and file_homes > 5, (laid, file_homes)
    assert {0, 1, 6, 8} <= seen, seen  # laid out; INVALID; CAPACITY; UNSUPPORTED


@pytest.mark.parametrize("seed", range(200))
def test_landing_geometry_matches_reference(seed, tmp_path):
    """The landing options on file-tier opens (dg_landing_blocks, _max_queued, _ttl, _chunk): the same refusals
    (out-of-range values, options without blocks, blocks without reads in flight, a host budget that cannot also
    hold the landing blocks) and the same resolved settings as the reference's layout."""
    if not ref.available():
        pytest.skip("oracle/_ref is not built")
    m, bkw, okw, tiers, _ = _case(50000 + seed, tmp_path, landing=True)
    if not _plan_ok(m, bkw, tiers):
        pytest.skip("the planner refuses this budget (a plan test's matter)")
    js = m.desc_json().encode()
    st_o, got, res_o = _ours(js, ss.budget(**bkw), tiers, ss.options(**okw))
    st_t, want, res_t, why = _theirs(js, ss.budget(**bkw), tiers, ss.options(**okw))
    assert st_o == st_t, (seed, st_o, st_t, why, okw)
    if st_t == 0:
        assert got == want, (seed, got, want)


def test_landing_geometry_cases_lay_out_landings(tmp_path):
    if not ref.available():
        pytest.skip("oracle/_ref is not built")
    laid, refused = 0, set()
    for seed in range(200):
        (tmp_path / str(seed)).mkdir()
        m, bkw, okw, tiers, _ = _case(50000 + seed, tmp_path / str(seed), landing=True)
        if not _plan_ok(m, bkw, tiers):
            continue
        js = m.desc_json().encode()
        st, got, _ = _ours(js, ss.budget(**bkw), tiers, ss.options(**okw))
        laid += st == 0 and got["L"] > 0
        refused.add(st)
    assert laid >= 20 and {1, 6} <= refused, (laid, refused)
