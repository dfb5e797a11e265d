"""Build recipe for the summa_amd HIP library (gfx950 only).

Compiles every ``csrc/*.hip`` translation unit with hipcc for ``gfx950`` and
links them into ``summa_amd/libsumma_amd.so`` (in-tree, so the built library
travels with the source tree to the GPU host), and archives the same objects
as ``summa_amd/libsumma_amd.a``: the static library a Rust ``build.rs`` links
(each object carries its own gfx950 code object and registers it at load, so
the archive links with the host linker plus ``-lamdhip64 -lstdc++``). Run
``python -m summa_amd.build``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libsumma_amd.so"
ARCHIVE = PKG / "libsumma_amd.a"
ARCH = "gfx950"

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # Keep the compiler from forming packed-fp32 VALU ops.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{PKG.parent / 'include'}",
]


# AddressSanitizer on the host side only (the argument checks, plans and
# HQUANT parsing that run on the CPU); device code is built as usual.
ASAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer",
              "-Xarch_host", "-g"]


def _compile(src: Path, obj_dir: Path = OBJ, extra=()) -> Path:
    obj = obj_dir / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    tmp_a = ARCHIVE.with_suffix(".a.tmp")
    if tmp_a.exists():
        tmp_a.unlink()
    proc = subprocess.run([shutil.which("ar") or "ar", "rcs", str(tmp_a), *map(str, objs)],
                          capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"ar failed:\n{proc.stderr}")
    os.replace(tmp_a, ARCHIVE)
    if verbose:
        print(f"built {LIB} and {ARCHIVE.name} from {len(sources)} sources", flush=True)
    return LIB


def build_asan(verbose: bool = True) -> Path:
    """The library with AddressSanitizer on its host code, in summa_amd/_asan/
    (for the CPU test suite: SUMMA_AMD_LIB=summa_amd/_asan/libsumma_amd.so
    with clang's ASan runtime preloaded)."""
    out_dir = PKG / "_asan"
    out_dir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda src: _compile(src, out_dir, ASAN_FLAGS), sources))
    lib = out_dir / "libsumma_amd.so"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-fsanitize=address",
           *map(str, objs), "-o", str(lib)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    if verbose:
        print(f"built {lib} (host AddressSanitizer)", flush=True)
    return lib


if __name__ == "__main__":
    if "--asan" in sys.argv[1:]:
        build_asan()
    else:
        build()
    sys.exit(0)
