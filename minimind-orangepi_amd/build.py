#!/usr/bin/env python3
"""Build libmmr.so (HIP kernels + C++ runtime + C ABI) and the CLI tools for gfx950.

    python minimind-orangepi_amd/build.py            # incremental
    python minimind-orangepi_amd/build.py --force    # rebuild everything

Outputs (git-ignored, shipped with the tree to the GPU box):
    minimind-orangepi_amd/lib/libmmr.so
    minimind-orangepi_amd/bin/bench_decode, bin/minimind_generate, bin/check_prefill_consistency
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "lib"
BIN = PKG / "bin"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = ["-std=c++17", "-O3", "-fPIC", "-Wall", "-Wno-unused-result", f"-I{ROOT / 'include'}"]
# Packed FP32 (v_pk_*_f32) is disabled for all device code.
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

SOURCES = sorted(CSRC.glob("kernels/*.hip")) + sorted(CSRC.glob("runtime/*.cpp")) + [CSRC / "capi.cpp",
                                                                                      CSRC / "host_ops.cpp"]
TOOLS = {name: CSRC / "tools" / f"{name}.cpp"
         for name in ("bench_decode", "minimind_generate", "check_prefill_consistency")}


def _headers() -> list[Path]:
    return sorted(CSRC.rglob("*.h")) + sorted((ROOT / "include").glob("*.h"))


def _stale(out: Path, deps: list[Path]) -> bool:
    if not out.exists():
        return True
    t = out.stat().st_mtime
    return any(d.stat().st_mtime > t for d in deps)


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature flag; drop that noise.
    noise = ("packed-fp32-ops", "is not a recognized feature")
    err = "\n".join(l for l in proc.stderr.splitlines() if l.strip() and not any(n in l for n in noise))
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if err:
        print(err, file=sys.stderr)


def _compile(src: Path) -> Path:
    rel = src.relative_to(CSRC)
    obj = OBJ / (str(rel).replace("/", "__") + ".o")
    cmd = [HIPCC, *COMMON, *DEVICE, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [HIPCC, *COMMON, *DEVICE, "-x", "hip", "-c", str(src), "-o", str(obj)]
    _run(cmd)
    return obj


def build(force: bool = False, jobs: int | None = None, verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    BIN.mkdir(exist_ok=True)
    headers = _headers()
    todo = []
    objs = []
    for src in SOURCES:
        obj = OBJ / (str(src.relative_to(CSRC)).replace("/", "__") + ".o")
        objs.append(obj)
        if force or _stale(obj, [src, *headers]):
            todo.append(src)
    jobs = jobs or min(8, os.cpu_count() or 4)
    if todo:
        if verbose:
            print(f"[build] compiling {len(todo)} source(s) for {ARCH} with {jobs} jobs", flush=True)
        with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
            for obj in ex.map(_compile, todo):
                if verbose:
                    print(f"[build]   {obj.name}", flush=True)
    lib = LIB / "libmmr.so"
    if force or todo or _stale(lib, objs):
        tmp = lib.with_suffix(".so.tmp")
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
        os.replace(tmp, lib)
        if verbose:
            print(f"[build] linked {lib}", flush=True)
    for name, src in TOOLS.items():
        exe = BIN / name
        if src.exists() and (force or _stale(exe, [src, lib, *headers])):
            _run([HIPCC, *COMMON, "-x", "hip", str(src), "-o", str(exe), f"-L{LIB}", "-lmmr",
                  "-Wl,-rpath,$ORIGIN/../lib", f"--offload-arch={ARCH}"])
            if verbose:
                print(f"[build] linked {exe}", flush=True)
    return lib


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    args = ap.parse_args()
    build(force=args.force, jobs=args.jobs)
    return 0


if __name__ == "__main__":
    sys.exit(main())
