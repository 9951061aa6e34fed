"""Compile the HIP sources of this package into libprismkv_hip.so (gfx950).

`compile_hip` mirrors the reference's `compile_ppu` contract
(src/prismkv/native8b.py:16-31): the output directory must not exist yet; the
call writes build.log and build.json (command, seconds, return code, source
sha256) there and returns the library path.  `build_inplace` produces the
in-tree library the package loads by default.
"""
from __future__ import annotations

import hashlib
import json
import os
import shutil
import subprocess
import tempfile
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
INCLUDE = PACKAGE.parent / "include"
SOURCES = ["route.hip", "union.hip", "attend.hip", "decode.hip", "update.hip"]
LIBRARY_NAME = "libprismkv_hip.so"
ARCH = "gfx950"

# Packed-fp32 VALU forms are disabled for every HIP translation unit.
HIP_FLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-Wno-unused-command-line-argument"]
# Per-source flags.  The fused decode is scheduled for instruction-level
# parallelism: its latency-bound phases (selection chains, polls, the
# attention's load rounds) ran faster in every measured configuration
# (MI355X, alternating graph-timed chains: 64K 24.93 -> 24.79 us per layer,
# 64K with a 2048-row tail 25.96 -> 25.57, 131K 34.66 -> 33.77, the capped
# 262K step 39.74 -> 39.07, prismkv_attend 14.62 -> 14.57).  The index
# update and build kernels keep the default scheduler: with max-ilp the 64K
# build took 7.08 ms instead of 6.25 and a 1024-token update 178 us instead
# of 157 (the encode's MFMA loop).
SOURCE_FLAGS = {"decode.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]}


def _hipcc(rocm_root) -> str:
    cand = Path(rocm_root) / "bin" / "hipcc"
    return str(cand) if cand.exists() else (shutil.which("hipcc") or "hipcc")


def _sources(source_root: Path):
    return [source_root / s for s in SOURCES if (source_root / s).exists()]


def _compile(hipcc, sources, output: Path, include_dirs, log, defines=()):
    """Compile each source to an object in parallel, then link the shared library."""
    with tempfile.TemporaryDirectory(prefix="prismkv_build_") as tmp:
        objects, commands = [], []
        for src in sources:
            obj = Path(tmp) / (src.stem + ".o")
            cmd = [hipcc, *HIP_FLAGS, *SOURCE_FLAGS.get(src.name, []), *[f"-D{d}" for d in defines],
                   *[f"-I{d}" for d in include_dirs], "-c", str(src), "-o", str(obj)]
            objects.append(obj)
            commands.append(cmd)
        with ThreadPoolExecutor(max_workers=min(len(commands), os.cpu_count() or 4)) as pool:
            results = list(pool.map(lambda c: subprocess.run(c, capture_output=True, text=True), commands))
        for cmd, res in zip(commands, results):
            log.append(" ".join(cmd) + "\n" + res.stdout + res.stderr)
        rc = next((r.returncode for r in results if r.returncode), 0)
        if rc == 0:
            tmp_out = output.with_name(output.name + ".tmp")
            link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp_out)]
            commands.append(link)
            res = subprocess.run(link, capture_output=True, text=True)
            log.append(" ".join(link) + "\n" + res.stdout + res.stderr)
            rc = res.returncode
            if rc == 0:
                os.replace(tmp_out, output)
        return rc, commands


def compile_hip(source_root=CSRC, output_dir=None, rocm_root="/opt/rocm", defines=()):
    """Build libprismkv_hip.so into a NEW directory; returns the library path.
    `defines` are NAME=VALUE preprocessor definitions (e.g.
    PRISMKV_VALU_ATTENTION=1, the decode's VALU-attention A/B build)."""
    source_root = Path(source_root)
    if output_dir is None:
        raise ValueError("output_dir is required")
    output_dir = Path(output_dir)
    output_dir.mkdir(parents=True, exist_ok=False)
    sources = _sources(source_root)
    log: list[str] = []
    start = time.perf_counter()
    rc, commands = _compile(_hipcc(rocm_root), sources, output_dir / LIBRARY_NAME,
                            [source_root, INCLUDE], log, defines)
    (output_dir / "build.log").write_text("\n".join(log), encoding="utf8")
    (output_dir / "build.json").write_text(json.dumps(dict(
        command=commands, seconds=time.perf_counter() - start, returncode=rc,
        sources={p.name: hashlib.sha256(p.read_bytes()).hexdigest() for p in sources}), indent=2), encoding="utf8")
    if rc:
        raise subprocess.CalledProcessError(rc, commands[-1])
    return output_dir / LIBRARY_NAME


def build_inplace(rocm_root="/opt/rocm") -> Path:
    """(Re)build the in-tree library next to this file; always compiles."""
    out = PACKAGE / LIBRARY_NAME
    log: list[str] = []
    rc, commands = _compile(_hipcc(rocm_root), _sources(CSRC), out, [CSRC, INCLUDE], log)
    if rc:
        raise RuntimeError("HIP build failed:\n" + "\n".join(log))
    return out


if __name__ == "__main__":
    import argparse
    ap = argparse.ArgumentParser(description="build libprismkv_hip.so (in-tree by default)")
    ap.add_argument("--output-dir", help="build into this new directory instead of in-tree")
    ap.add_argument("--define", action="append", default=[], help="NAME=VALUE preprocessor definition")
    args = ap.parse_args()
    if args.output_dir:
        print(compile_hip(CSRC, args.output_dir, defines=args.define))
    else:
        print(build_inplace())
