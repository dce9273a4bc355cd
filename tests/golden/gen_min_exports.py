"""Writes tests/golden/min_exports.json: the functions of the reference's include/strix_stream/ss.h that the serve
path's drop-in boundary must export at a minimum - the descriptor and plan calls (ss.h:78-175), defaults
(:451-452), the context and forward calls (:457-527), stats (:545-571, :894-897), the device-gated calls
(:671-701) and the device-gated stats (:1052). Run where the reference sources exist:

    python tests/golden/gen_min_exports.py [/root/reference]
"""
import json
import re
import sys
from pathlib import Path

RANGES = [(78, 175), (451, 527), (545, 571), (894, 897), (671, 701), (1052, 1052)]


def main(ref: Path) -> None:
    lines = (ref / "include" / "strix_stream" / "ss.h").read_text().splitlines()
    names = []
    for a, b in RANGES:
        for line in lines[a - 1:b]:
            m = re.search(r"SS_API\s[^(]*?\b(\w+)\s*\(", line)
            if m and m.group(1) not in names:
                names.append(m.group(1))
    out = Path(__file__).with_name("min_exports.json")
    out.write_text(json.dumps({"source": "include/strix_stream/ss.h", "ranges": RANGES, "functions": names},
                              indent=1) + "\n")
    print(f"{len(names)} functions -> {out}")


if __name__ == "__main__":
    main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
