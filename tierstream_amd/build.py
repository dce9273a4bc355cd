"""Build recipe of the native libraries (hipcc for gfx950, in-tree outputs).

libtierstream_amd.so  the product: the ss_* / ts_* / tsa_* C ABI, host runtime and HIP kernels (csrc/).
libtsa_engine.so      the synthetic engine the tests and the benchmark drive the library with (engine/): graph-captured
                      device-gated tokens, checksum kernels that read units through the tables. Not part of the product.
libtierstream.a       the product's objects as a static archive, under the reference's archive name, and an identical
libstrix_stream.a     copy under its older name (engines link either by name; they add -lamdhip64 -lstdc++ -lpthread).

Every call recompiles every source (objects under _build/, compiled in parallel).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
BUILD = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = ["-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wno-unused-function", f"-I{ROOT / 'include'}",
          f"-I{PKG / 'csrc'}", "-I/opt/rocm/include", "-D__HIP_PLATFORM_AMD__"]
# Device code: gfx950 only; packed FP32 instructions disabled (-packed-fp32-ops).
HIP_FLAGS = ["-x", "hip", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-fno-gpu-rdc"]
CXX_FLAGS = ["-x", "c++"]
LINK = ["-shared", "-fPIC", f"--offload-arch={ARCH}", "-Wl,-rpath,/opt/rocm/lib", "-L/opt/rocm/lib", "-lamdhip64",
        "-lpthread"]

ARCHIVES = ["libtierstream.a", "libstrix_stream.a"]
LIBS = {
    "libtierstream_amd.so": {"dir": PKG / "csrc", "extra_link": []},
    "libtsa_engine.so": {"dir": PKG / "engine", "extra_link": [f"-L{PKG}", "-ltierstream_amd",
                                                                 "-Wl,-rpath,$ORIGIN"]},
}


def _compile(src: Path, obj: Path) -> tuple[Path, int, str]:
    flags = HIP_FLAGS if src.suffix == ".hip" else CXX_FLAGS
    cmd = [HIPCC, *COMMON, *flags, "-c", str(src), "-o", str(obj)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    return src, p.returncode, (p.stdout + p.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> list[Path]:
    BUILD.mkdir(exist_ok=True)
    out = []
    jobs = jobs or min(8, os.cpu_count() or 4)
    for name, spec in LIBS.items():
        srcs = sorted(p for p in spec["dir"].glob("*") if p.suffix in (".cpp", ".hip"))
        if not srcs:
            continue
        objdir = BUILD / name.replace(".so", "")
        objdir.mkdir(exist_ok=True)
        objs = [objdir / (s.name + ".o") for s in srcs]
        errors = []
        with cf.ThreadPoolExecutor(jobs) as ex:
            for src, rc, log in ex.map(lambda a: _compile(*a), zip(srcs, objs)):
                if verbose and log.strip():
                    print(f"[{src.name}]\n{log}", file=sys.stderr)
                if rc != 0:
                    errors.append(f"{src.name}:\n{log}")
        if errors:
            raise RuntimeError("hipcc failed:\n" + "\n".join(errors))
        target = PKG / name
        tmp = PKG / (name + ".tmp")
        cmd = [HIPCC, *LINK, *[str(o) for o in objs], *spec["extra_link"], "-o", str(tmp)]
        p = subprocess.run(cmd, capture_output=True, text=True)
        if p.returncode != 0:
            raise RuntimeError(f"link of {name} failed:\n{p.stdout}{p.stderr}")
        os.replace(tmp, target)
        out.append(target)
        if name == "libtierstream_amd.so":  # the static archives of the same objects
            for a in ARCHIVES:
                tmp = PKG / (a + ".tmp")
                tmp.unlink(missing_ok=True)
                p = subprocess.run(["ar", "rcs", str(tmp), *[str(o) for o in objs]], capture_output=True, text=True)
                if p.returncode != 0:
                    raise RuntimeError(f"ar of {a} failed:\n{p.stdout}{p.stderr}")
                os.replace(tmp, PKG / a)
                out.append(PKG / a)
    return out


if __name__ == "__main__":
    for t in build(verbose="-v" in sys.argv):
        print(t)
