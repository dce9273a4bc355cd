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
