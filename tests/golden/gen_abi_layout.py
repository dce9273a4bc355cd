"""Writes tests/golden/abi_layout.json: sizeof and offsetof of every field of every struct this library's
include/strix_stream/ss.h declares, as the REFERENCE's own header lays them out (the probe is compiled with gcc against
the reference's include/strix_stream/ss.h). tests/test_abi.py compiles the same probe against this library's header and
requires the same numbers: an engine built against either header passes the same bytes.

    python tests/golden/gen_abi_layout.py [/path/to/reference]     (default /root/reference)
"""
from __future__ import annotations

import json
import os
import re
import subprocess
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
OURS = ROOT / "include"


def structs(header: Path) -> dict[str, list[str]]:
    """typedef struct NAME { ... } NAME; -> field names, in order (arrays and comma lists expanded to names)."""
    code = re.sub(r"/\*.*?\*/", " ", header.read_text(), flags=re.S)
    code = re.sub(r"//[^\n]*", " ", code)
    out = {}
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*(\w+)\s*;", code, flags=re.S):
        name, body = m.group(3), m.group(2)
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            decl = re.sub(r"\[[^\]]*\]", "", decl)  # arrays: the name is what is left
            if "(" in decl:  # a function pointer member: (*name)(...)
                fields.append(re.search(r"\(\s*\*\s*(\w+)\s*\)", decl).group(1))
                continue
            head, *rest = decl.split(",")
            fields.append(re.search(r"(\w+)\s*$", head).group(1))
            fields.extend(r.strip().lstrip("*").strip() for r in rest)
        out[name] = fields
    return out


def probe_source(layout: dict[str, list[str]]) -> str:
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "strix_stream/ss.h"', "int main(void) {",
             '  printf("{");']
    first = True
    for s, fields in layout.items():
        sep = "" if first else ","
        first = False
        lines.append(f'  printf("{sep}\\"{s}\\": {{\\"size\\": %zu, \\"fields\\": {{", sizeof({s}));')
        for i, f in enumerate(fields):
            fs = "" if i == 0 else ","
            lines.append(f'  printf("{fs}\\"{f}\\": %zu", offsetof({s}, {f}));')
        lines.append('  printf("}}");')
    lines += ['  printf("}\\n");', "  return 0;", "}"]
    return "\n".join(lines)


def measure(include_dir: Path, layout) -> dict:
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "probe.c")
        exe = os.path.join(d, "probe")
        Path(src).write_text(probe_source(layout))
        subprocess.run(["gcc", "-std=c11", "-I", str(include_dir), src, "-o", exe], check=True)
        return json.loads(subprocess.run([exe], check=True, capture_output=True, text=True).stdout)


def main(argv):
    ref = Path(argv[0]) if argv else Path("/root/reference")
    layout = structs(OURS / "strix_stream" / "ss.h")
    got = measure(ref / "include", layout)
    (HERE / "abi_layout.json").write_text(json.dumps(got, indent=1, sort_keys=True) + "\n")
    print(f"{len(got)} structs written")


if __name__ == "__main__":
    main(sys.argv[1:])
