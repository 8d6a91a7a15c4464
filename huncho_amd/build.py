"""Builds libhuncho_rocm.so (gfx950) in-tree: huncho_amd/_build/libhuncho_rocm.so.

Every HIP and host source under huncho_amd/csrc is compiled with hipcc for gfx950 only,
then linked against the HIP runtime and hipBLASLt. Run as `python -m huncho_amd.build`.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "_build"
LIB = OUT / "libhuncho_rocm.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

COMMON = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-result",
    # packed fp32 ops stay off in every kernel (host pass warns it does not know the feature)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    p = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    if not Path(p).exists():
        raise RuntimeError("hipcc not found: a ROCm toolchain is required to build libhuncho_rocm")
    return p


# per-source flags: the standalone delta-rule recurrence runs 5-6 % faster with the
# max-memory-clause machine scheduler (the fused layer kernel, in gdn16.hip, does not)
EXTRA = {"gdn16_standalone.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"]}


def _compile(src: Path) -> Path:
    obj = OUT / (src.name + ".o")
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    cmd = [hipcc(), *COMMON, *EXTRA.get(src.name, []), *lang, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    OUT.mkdir(parents=True, exist_ok=True)
    sources = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
           f"-L{ROCM / 'lib'}", "-lhipblaslt", f"-Wl,-rpath,{ROCM / 'lib'}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
