"""Ahead-of-time build of libreelcache_hip.so for gfx950 (hipcc, no JIT).

``python -m reelcache_amd.csrc.build`` (or :func:`build`) compiles every ``*.hip``
source of this directory in parallel into ``reelcache_amd/_build/`` and links
``reelcache_amd/libreelcache_hip.so``.  The library travels with the tree; the
package loads it and never compiles at import time.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PACKAGE = HERE.parent
ROOT = PACKAGE.parent
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libreelcache_hip.so"
ARCH = "gfx950"

# Packed FP32 VALU instructions are disabled (they have produced silent errors on this
# hardware pool); FP contraction is off so dequantization and RoPE keep separate roundings.
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build the HIP library")
    return found


def sources() -> list[Path]:
    return sorted(HERE.glob("*.hip"))


def _compile(hipcc: str, source: Path, verbose: bool) -> Path:
    target = BUILD / (source.stem + ".o")
    command = [hipcc, *FLAGS, "-c", str(source), "-o", str(target)]
    if verbose:
        print(" ".join(command), flush=True)
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stderr[-6000:]}")
    return target


def _dependencies(source: Path) -> set[Path]:
    """The source and every header it includes with quotes, transitively."""
    seen: set[Path] = set()
    pending = [source]
    while pending:
        path = pending.pop()
        if path in seen or not path.exists():
            continue
        seen.add(path)
        for line in path.read_text().splitlines():
            line = line.strip()
            if line.startswith("#include \""):
                pending.append((path.parent / line.split('"')[1]).resolve())
    return seen


def _stale(source: Path) -> bool:
    target = BUILD / (source.stem + ".o")
    if not target.exists():
        return True
    built = target.stat().st_mtime
    return any(path.stat().st_mtime > built for path in _dependencies(source))


def build(*, jobs: int | None = None, verbose: bool = False, incremental: bool = False) -> Path:
    """Compile all sources (with ``incremental``, only those whose object is older than the
    source or a header it includes) and link the shared library; returns its path."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    files = sources()
    if incremental:
        files = [source for source in files if _stale(source)]
    workers = max(1, min(len(files), jobs or min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(lambda source: _compile(hipcc, source, verbose), files))
    objects = [BUILD / (source.stem + ".o") for source in sources()]
    temporary = LIBRARY.with_suffix(".so.tmp")
    command = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(temporary)]
    if verbose:
        print(" ".join(command), flush=True)
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"linking {LIBRARY.name} failed:\n{result.stderr[-6000:]}")
    os.replace(temporary, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv, incremental="--incremental" in sys.argv)
    print(path)
