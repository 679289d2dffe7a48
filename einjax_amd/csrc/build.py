"""Builds libejhip.so (the C-ABI HIP library) in-tree for gfx950.

Usage: python -m einjax_amd.csrc.build   (or einjax_amd.csrc.build.build())
       python -m einjax_amd.csrc.build --sanitize   (ASan/UBSan on the host code, for
                                                     the host-side tests)

Each ``*.hip`` file under this directory is compiled with hipcc to an
object in ``_build/`` and linked into ``einjax_amd/libejhip.so``.  Packed
fp32 VALU forms are disabled for all device code.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
BUILD_DIR = HERE / "_build"
LIB_PATH = PKG / "libejhip.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build libejhip.so")


def sources() -> list[Path]:
    return sorted(HERE.glob("*.hip"))


def _compile(hipcc: str, src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    """Compiles every HIP source and links libejhip.so; returns its path."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    try:  # every symbol must resolve (a kernel whose host stub was not emitted would not)
        import ctypes

        ctypes.CDLL(str(tmp), mode=os.RTLD_NOW)
    except OSError as e:
        raise RuntimeError(f"built library does not load: {e}") from e
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources")
    return LIB_PATH


# Sanitized build: AddressSanitizer and UndefinedBehaviorSanitizer on the
# host code only (the device code is built as usual and is never launched
# from it), into a separate library.  It serves the host-side tests
# (argument validation, workspace sizing, error paths: tests/test_abi.py);
# loading it needs the shared ASan runtime first in the process
# (san_runtime(), preloaded by the test that runs it).
SAN_DIR = HERE / "_build_san"
SAN_LIB_PATH = SAN_DIR / "libejhip_san.so"
SAN_FLAGS = [
    f"--offload-arch={ARCH}", "-O1", "-g", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
    "-shared-libasan", "-Wno-unused-result",
]


def san_runtime() -> Path:
    """The shared AddressSanitizer runtime of the HIP compiler."""
    res = subprocess.run([_hipcc(), "-print-file-name=libclang_rt.asan-x86_64.so"],
                         capture_output=True, text=True)
    p = Path(res.stdout.strip())
    if res.returncode != 0 or not p.is_absolute() or not p.exists():
        raise RuntimeError("the HIP compiler's shared ASan runtime was not found")
    return p


def build_sanitized(verbose: bool = True) -> Path:
    """Builds the sanitized library (when a source or header is newer than
    it); returns its path."""
    hipcc = _hipcc()
    SAN_DIR.mkdir(exist_ok=True)
    deps = [*sources(), *HERE.glob("*.h"), PKG.parent / "include" / "einjax_hip.h",
            Path(__file__)]
    if SAN_LIB_PATH.exists() and all(d.stat().st_mtime <= SAN_LIB_PATH.stat().st_mtime
                                     for d in deps if d.exists()):
        return SAN_LIB_PATH

    def comp(src: Path) -> Path:
        obj = SAN_DIR / (src.stem + ".o")
        res = subprocess.run([hipcc, *SAN_FLAGS, "-c", str(src), "-o", str(obj)],
                             capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"sanitized hipcc failed on {src.name}:\n{res.stderr}")
        return obj

    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(len(srcs), 8)) as ex:
        objs = list(ex.map(comp, srcs))
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-shared-libasan",
           "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-o", str(SAN_LIB_PATH), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"sanitized link failed:\n{res.stderr}")
    if verbose:
        print(f"built {SAN_LIB_PATH} (ASan + UBSan on the host code)")
    return SAN_LIB_PATH


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "--sanitize":
        build_sanitized()
    else:
        build()
