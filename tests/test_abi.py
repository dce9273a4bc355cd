"""The drop-in boundary on the CPU (no GPU call):

- every struct of include/strix_stream/ss.h has the size and field offsets the reference's own header gives them
  (tests/golden/abi_layout.json, written by tests/golden/gen_abi_layout.py against the reference's ss.h);
- libtierstream_amd.so loads and exports every function that include/strix_stream/ss.h, include/tierstream/ts.h,
  include/tierstream_amd/tsa.h and include/tierstream_amd/tsa_test.h declare;
- include/tierstream/ts.h and tierstream_amd/csrc/ts_api.cpp are what tierstream_amd/gen_ts.py makes of ss.h;
- version and status calls that touch no device answer as the reference's do (ss_abi_version, refusals of a bad
  descriptor)."""
import ctypes as C
import json
import re
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "tests" / "golden"))

import gen_abi_layout  # noqa: E402

HEADERS = ["strix_stream/ss.h", "tierstream/ts.h", "tierstream_amd/tsa.h", "tierstream_amd/tsa_test.h"]


def declared(header: Path) -> list[str]:
    code = re.sub(r"/\*.*?\*/", " ", header.read_text(), flags=re.S)
    return re.findall(r"(?:SS_API|TS_API)\s+[^;(]*?\b(\w+)\s*\([^)]*\)\s*;", code)


def test_struct_layouts_match_the_reference_header():
    want = json.loads((ROOT / "tests" / "golden" / "abi_layout.json").read_text())
    layout = gen_abi_layout.structs(ROOT / "include" / "strix_stream" / "ss.h")
    assert set(layout) == set(want)
    got = gen_abi_layout.measure(ROOT / "include", layout)
    for s in want:
        assert got[s]["size"] == want[s]["size"], s
        assert got[s]["fields"] == want[s]["fields"], s


@pytest.mark.parametrize("header", HEADERS)
def test_library_exports_every_declared_function(header):
    import tierstream_amd
    lib = tierstream_amd.lib()
    names = declared(ROOT / "include" / header)
    assert names, header
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_reference_test_hooks_and_clean_evict_are_exported():
    """The host and device-gated test hooks the reference's own tests link by name (reference
    include/strix_stream/ss_test.h:14-28, src/capi.cpp:691-737, :898-921), and ss_dg_set_clean_evict (reference
    include/strix_stream/ss.h:1760) with its ts_ name."""
    import tierstream_amd
    lib = tierstream_amd.lib()
    names = ["ss_test_inject", "ss_test_check_exclusive", "ss_test_hold_readers", "ss_test_ra_quiesce",
             "ss_test_dg_check", "ss_test_dg_stop_service", "ss_dg_set_clean_evict", "ts_dg_set_clean_evict"]
    assert [n for n in names if not hasattr(lib, n)] == []
    test_h = set(declared(ROOT / "include" / "tierstream_amd" / "tsa_test.h"))
    assert {n for n in names[:6]} <= test_h
    assert "ss_dg_set_clean_evict" in set(declared(ROOT / "include" / "strix_stream" / "ss.h"))


def test_minimum_export_set_of_the_serve_path():
    """Every function of the reference header's serve-path sections (tests/golden/min_exports.json: descriptor, plan,
    defaults, context and forward, stats, device-gated calls) is declared in ss.h and exported, under its ss_ and its
    ts_ name."""
    import tierstream_amd
    lib = tierstream_amd.lib()
    want = json.loads((ROOT / "tests" / "golden" / "min_exports.json").read_text())["functions"]
    ours = set(declared(ROOT / "include" / "strix_stream" / "ss.h"))
    assert len(want) > 50
    assert [n for n in want if n not in ours] == []
    assert [n for n in want if not hasattr(lib, n) or not hasattr(lib, "ts_" + n[3:])] == []


def test_lookahead_select_matches_the_reference():
    """ss_lookahead_select against the reference's own (oracle/_ref): random score rows with ties (scores drawn from a
    few values), every top_k, max_out below and above the union, zero rows; and the argument refusals."""
    import numpy as np

    import tierstream_amd
    from oracle import ref
    if not ref.available():
        pytest.skip("oracle/_ref is not built")
    ours, theirs = tierstream_amd.lib(), ref.lib()
    for L in (ours, theirs):
        L.ss_lookahead_select.restype = C.c_int
        L.ss_lookahead_select.argtypes = [C.POINTER(C.c_float), C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int32),
                                          C.c_int, C.POINTER(C.c_int)]
    rng = np.random.default_rng(3)
    fp = C.POINTER(C.c_float)
    for case in range(400):
        n_exp = int(rng.integers(1, 80))
        rows = int(rng.integers(0, 9))
        k = int(rng.integers(1, n_exp + 1))
        levels = rng.choice([2, 5, 1000])
        s = (rng.integers(0, levels, size=(max(rows, 1), n_exp)) / levels).astype(np.float32)
        s = np.ascontiguousarray(s)
        max_out = int(rng.integers(0, n_exp + 3))
        got = []
        for L in (ours, theirs):
            out = np.full(n_exp + 3, -7, dtype=np.int32)
            n = C.c_int(-1)
            st = L.ss_lookahead_select(s.ctypes.data_as(fp), rows, n_exp, k, out.ctypes.data_as(C.POINTER(C.c_int32)),
                                       max_out, C.byref(n))
            got.append((st, n.value, out.tolist()))
        assert got[0] == got[1], (case, rows, n_exp, k, max_out)
    out = np.zeros(4, dtype=np.int32)
    n = C.c_int(0)
    s = np.zeros(8, dtype=np.float32)
    for args in [(2, 4, 0), (2, 4, 5), (-1, 4, 2), (2, 0, 1)]:  # top_k 0, top_k > n_experts, rows < 0, no experts
        for L in (ours, theirs):
            st = L.ss_lookahead_select(s.ctypes.data_as(fp), args[0], args[1], args[2],
                                       out.ctypes.data_as(C.POINTER(C.c_int32)), 4, C.byref(n))
            assert st == tierstream_amd.SS_E_INVALID, (args, st)


def test_ts_names_are_generated_from_ss_h():
    r = subprocess.run([sys.executable, "-m", "tierstream_amd.gen_ts", "--check"], cwd=ROOT, capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stdout + r.stderr


def test_host_only_calls():
    import tierstream_amd
    lib = tierstream_amd.lib()
    lib.ss_abi_version.restype = C.c_int
    lib.ts_abi_version.restype = C.c_int
    assert lib.ss_abi_version() == lib.ts_abi_version() > 0
    from tierstream_amd import ss
    from oracle import ref
    bad = '{"schema": "strix-stream/desc-v1", "layers": "no"}'
    with pytest.raises(tierstream_amd.SsError) as e:
        ss.Desc(bad)
    assert e.value.status == tierstream_amd.SS_E_DESC
    if ref.available():
        with pytest.raises(RuntimeError, match="reference status 2"):
            ref.desc_roundtrip(bad)
