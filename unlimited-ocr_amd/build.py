"""Build libsrswa.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

Usage: ``python unlimited-ocr_amd/build.py [-j N] [-v]``.  Every ``csrc/*.hip``
file is compiled to an object in parallel and linked into
``srswa/libsrswa.so`` next to the Python package that loads it.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
OUT = os.path.join(HERE, "srswa", "libsrswa.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # no packed-fp32 instructions anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


# Files whose results must follow a fixed rounding order (each product and sum
# rounded on its own): hipcc fuses a*b + c into an FMA by default and its
# backend does so even under `#pragma clang fp contract(off)`.
NO_CONTRACT = {"rope2d.hip", "router.hip", "route_serve.hip"}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libsrswa.so)")


def _compile(src: str, obj: str, verbose: bool) -> str:
    extra = ["-ffp-contract=off"] if os.path.basename(src) in NO_CONTRACT else []
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    msg = "\n".join(line for line in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in line and line.strip())
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{msg}")
    return msg


def build(jobs: int | None = None, verbose: bool = False) -> str:
    """Compile all kernels and link ``srswa/libsrswa.so``; returns its path."""
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    if not srcs:
        raise RuntimeError("no HIP sources under csrc/")
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with tempfile.TemporaryDirectory(prefix="srswa_build_") as tmp:
        objs = [os.path.join(tmp, os.path.basename(s)[:-4] + ".o") for s in srcs]
        with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
            futs = [ex.submit(_compile, s, o, verbose) for s, o in zip(srcs, objs)]
            for f in futs:
                warn = f.result()
                if warn and verbose:
                    print(warn, flush=True)
        tmp_out = OUT + ".tmp"
        # --no-undefined: a kernel whose host stub was not emitted fails here, not at load time
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", tmp_out, *objs]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
        os.replace(tmp_out, OUT)
    return OUT


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("-j", "--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args(argv)
    path = build(args.jobs, args.verbose)
    print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
