"""Builds the gfx950 library libllm_engine_amd.so in-tree with hipcc.

    python llm-engine_amd/build.py          # compile every source, link
    python llm-engine_amd/build.py --jobs 8

Each .hip/.cpp under csrc/ is compiled to an object in _build/ (parallel),
then linked into llm-engine_amd/lib/libllm_engine_amd.so. Everything is
compiled for gfx950 only, with packed-FP32 instruction selection disabled.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = ROOT / "_build"
LIB = PKG / "lib" / "libllm_engine_amd.so"
BRIDGE_SRC = PKG / "bridge" / "le_cuda_kernels.cpp"
BRIDGE_LIB = PKG / "lib" / "libllm_engine_amd_bridge.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(CSRC), "-I", str(ROOT / "include"),
    "-Wall", "-Wno-unused-function",
]


def sources() -> list[Path]:
    return sorted(list(CSRC.rglob("*.hip")) + list(CSRC.rglob("*.cpp")))


def _compile(src: Path, defines=(), build_dir: Path = BUILD) -> Path:
    rel = src.relative_to(CSRC)
    obj = build_dir / ("_".join(rel.parts[:-1] + (src.stem,)) + src.suffix.replace(".", "_") + ".o")
    cmd = [HIPCC, *COMMON, *[f"-D{d}" for d in defines], "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr[-6000:]}")
    return obj


def build(jobs: int | None = None, verbose: bool = False, out: Path = LIB, defines=()) -> Path:
    """Compiles every source and links `out` (the in-tree library by default;
    `defines` builds a variant with extra -D flags into a separate object dir)."""
    build_dir = BUILD if not defines else BUILD / ("v_" + "_".join(d.replace("=", "") for d in defines))
    build_dir.mkdir(parents=True, exist_ok=True)
    out.parent.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(8, os.cpu_count() or 4)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, defines, build_dir), srcs))
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "--offload-arch=gfx950", "-fPIC", "-o", str(tmp), *map(str, objs),
           "-L/opt/rocm/lib", "-lrocblas", "-Wl,-rpath,/opt/rocm/lib", "-Wl,--no-undefined"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    shutil.move(str(tmp), str(out))
    if out == LIB:
        build_bridge()
    if verbose:
        print(f"built {out} from {len(srcs)} sources, and {BRIDGE_LIB.name}")
    return out


def build_bridge() -> Path:
    """libllm_engine_amd_bridge.so: the reference's launcher signatures
    (include/le_cuda_kernels.h) over the C ABI; host code only."""
    tmp = BRIDGE_LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-O2", "-std=c++17", "-fPIC", "-shared", "-I", str(ROOT / "include"), str(BRIDGE_SRC),
           "-L", str(LIB.parent), "-lllm_engine_amd", "-Wl,-rpath,$ORIGIN", "-Wl,--no-undefined",
           "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"bridge build failed:\n{r.stderr[-6000:]}")
    shutil.move(str(tmp), str(BRIDGE_LIB))
    return BRIDGE_LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--out", type=Path, default=LIB)
    ap.add_argument("-D", dest="defines", action="append", default=[])
    a = ap.parse_args()
    build(a.jobs, verbose=True, out=a.out, defines=a.defines)
    sys.exit(0)
