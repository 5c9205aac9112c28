"""Build libssmoe.so (gfx950) in-tree with hipcc: one object per .hip source, then a shared link.

Usage: python -m slotstream_spark_amd.build  (or build() from Python). Always recompiles.
"""
import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libssmoe.so"
BUILD = PKG / "_build"
ARCH = os.environ.get("SSMOE_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    # Packed fp32 VALU forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = ("is not a recognized feature for this target", "kernel-resource-usage")
    lines = (r.stderr or "").splitlines()
    # Drop the resource remarks with their include-stack and source-snippet lines; keep every other diagnostic whole.
    kept, pending, drop = [], [], False
    for l in lines:
        if l.startswith("In file included from"):
            pending.append(l)
        elif re.match(r"^\s*\d*\s*\|", l):
            if not drop:
                kept.append(l)
        else:
            drop = any(n in l for n in noise)
            if not drop:
                kept += pending + [l]
            pending = []
    err = "\n".join(kept)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    # No kernel may use private scratch: a spill or a local array addressed at run time means a slow (and, for
    # selects of whole vectors, once miscompiled) path, so the build refuses it.
    name = None
    for line in lines:
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and int(m.group(1)) > 0:
            raise RuntimeError(f"{src.name}: kernel {name} uses {m.group(1)} bytes of private scratch per lane")
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    with ThreadPoolExecutor(max_workers=min(len(srcs), 8)) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} ({OUT.stat().st_size} bytes)")
    return OUT


if __name__ == "__main__":
    build()
