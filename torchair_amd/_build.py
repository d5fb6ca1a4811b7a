"""In-tree build of libtai_kernels.so (hipcc, gfx950 only).

Every ``csrc/*.hip`` file is compiled to an object under ``_build/`` and the objects are
linked into ``torchair_amd/libtai_kernels.so``, which travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures
import hashlib
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libtai_kernels.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # packed fp32 VALU ops are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]
# Files whose float arithmetic must follow the CPU oracle's operation order exactly.
NO_CONTRACT = {"quant.hip", "moe_routing.hip", "norm_cache.hip", "gemm_i8.hip"}


INCLUDE = PKG.parent / "include"


def source_id() -> str:
    """Hash of every source and flag the library is built from. It is compiled into the library
    (``tai_build_id``) and compared at load time, so a library built from other sources is refused."""
    h = hashlib.sha256()
    files = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.h")) + sorted(INCLUDE.glob("*.h"))
    for f in files:
        h.update(f.name.encode())
        h.update(f.read_bytes())
    h.update(" ".join(COMMON_FLAGS + sorted(NO_CONTRACT)).encode())
    return h.hexdigest()[:20]


def _compile(src: Path, build_id: str) -> Path:
    obj = BUILD / (src.stem + ".o")
    flags = list(COMMON_FLAGS)
    if src.name == "runtime.hip":
        flags.append(f'-DTAI_BUILD_ID="{build_id}"')
    if src.name in NO_CONTRACT:
        flags.append("-ffp-contract=off")
    cmd = [HIPCC, *flags, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(jobs, 1)) as ex:
        bid = source_id()
        objs = list(ex.map(lambda src: _compile(src, bid), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
