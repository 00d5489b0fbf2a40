"""Build librewy_hip.so (every HIP source under rewy_amd/csrc) for gfx950.

Compiles in-tree with hipcc, one object per source (in parallel), then links
the shared library next to this file so it travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import json
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "librewy_hip.so"
MANIFEST = HERE / "librewy_hip.manifest.json"
BUILD = HERE / "_build"
ARCH = "gfx950"
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed fp32 ops off: some of their forms have given wrong results on this pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(HERE.parent / "include"),
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build rewy_amd)")


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    extra = os.environ.get("REWY_HIPCC_FLAGS", "").split()   # e.g. -DREWY_CHUNK_PIPE=2
    cmd = [hipcc(), *FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr[-4000:]}")
    return obj


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, OUT)
    from rewy_amd.runtime import source_fingerprint
    MANIFEST.write_text(json.dumps({"arch": ARCH, "sources": source_fingerprint()}, indent=1))
    if verbose:
        print(f"built {OUT} from {[s.name for s in sources]}", file=sys.stderr)
    return OUT


if __name__ == "__main__":
    sys.path.insert(0, str(HERE.parent))
    build(verbose=True)
