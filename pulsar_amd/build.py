"""Builds libpulsar_moe.so (the HIP kernels + C ABI) in-tree for gfx950.

    python -m pulsar_amd.build [--changed]

Each .hip translation unit compiles in parallel to an object under
pulsar_amd/_build/, then the objects link into pulsar_amd/libpulsar_moe.so.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libpulsar_moe.so"
SOURCES = ["q8k.hip", "matvec.hip", "mmq.hip", "moe.hip", "router.hip", "route.hip", "fused.hip", "selftest.hip"]
ARCH = os.environ.get("PULSAR_OFFLOAD_ARCH", "gfx950")

# -ffp-contract=off: the compiler fuses no a*b+c on its own, so fp32
#   epilogues round in source order, as the reference CPU lane does. The
#   grouped matrix-core stages are the one exception, by choice: their
#   per-super-block epilogues call __builtin_fmaf (one rounding instead of
#   two), and their tests hold them to an explicit error bound instead of
#   bit equality.
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 emitted by the compiler.
# -mcode-object-version=5: loadable by the HIP runtime torch bundles.
HIPFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libpulsar_moe.so)")


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIPFLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    noise = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n" + "\n".join(noise))
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")


def _stale(src: Path, obj: Path) -> bool:
    """True when obj is missing or older than its source or any header it
    may include (the package's and include/'s)."""
    if not obj.exists():
        return True
    deps = [src, *CSRC.glob("*.h"), *(PKG.parent / "include").glob("*.h")]
    return obj.stat().st_mtime < max(d.stat().st_mtime for d in deps)


def build_library(jobs: int | None = None, changed_only: bool = False) -> Path:
    """Compiles the HIP sources (all of them, or with changed_only only those
    whose object is older than the source or a header) and links
    libpulsar_moe.so; returns its path."""
    BUILD.mkdir(exist_ok=True)
    objs = [BUILD / (Path(s).stem + ".o") for s in SOURCES]
    todo = [(CSRC / s, o) for s, o in zip(SOURCES, objs) if not changed_only or _stale(CSRC / s, o)]
    with ThreadPoolExecutor(max_workers=jobs or min(8, len(SOURCES))) as ex:
        list(ex.map(lambda so: _compile(*so), todo))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link of libpulsar_moe.so failed:\n" + res.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build_library(changed_only="--changed" in sys.argv))
