"""Build libwfbitnet.so (the HIP kernels + C ABI) in-tree for gfx950 with hipcc.

Run as ``python wrinklefree-monorepo_amd/_build.py`` or through ``__graft_entry__.build()``.
Objects go to ``wrinklefree-monorepo_amd/_build/``; the library lands next to this file so it
travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
OBJ_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libwfbitnet.so"
ARCH = os.environ.get("WFB_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    # packed fp32 VALU ops are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libwfbitnet")
    return exe


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip for the target arch and link libwfbitnet.so; returns its path."""
    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")

    def compile_one(src: Path) -> Path:
        obj = OBJ_DIR / (src.stem + ".o")
        cmd = [hipcc, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)
        return obj

    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")), 16)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(compile_one, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


ASAN_DIR = OBJ_DIR / "asan"
ASAN_DRIVER_SRC = PKG_DIR.parent / "tests" / "asan" / "abi_driver.cpp"


# Sources with host code only (no kernels): the entry points' validation and dispatch, the native engine.
HOST_ONLY_SOURCES = ("api.hip", "engine.hip")


def build_asan(verbose: bool = False) -> Path:
    """Host-code AddressSanitizer build for the CPU tests of the C ABI: the host-only sources (argument
    validation, dispatch, the engine's loader and state) compiled with ASan, linked with the kernel objects
    of the product build (run build() first) into _build/asan/libwfbitnet_asan.so, and the driver
    tests/asan/abi_driver.cpp linked against it.  Returns the driver's path."""
    hipcc = _hipcc()
    ASAN_DIR.mkdir(parents=True, exist_ok=True)
    host = ["--offload-host-only", "-O1", "-g", "-fPIC", "-std=c++17", "-Wno-unused-command-line-argument"]
    san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]
    objs = []
    for src in sorted(CSRC.glob("*.hip")):
        if src.name in HOST_ONLY_SOURCES:
            obj = ASAN_DIR / (src.stem + ".o")
            cmd = [hipcc, *host, *san, "-c", str(src), "-o", str(obj)]
            if verbose:
                print(" ".join(cmd), flush=True)
            _run(cmd)
        else:
            obj = OBJ_DIR / (src.stem + ".o")
            if not obj.exists():
                raise RuntimeError(f"{obj} missing: build() the library first")
        objs.append(obj)
    lib = ASAN_DIR / "libwfbitnet_asan.so"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *san, *map(str, objs), "-o", str(lib)])
    driver = ASAN_DIR / "abi_driver"
    dobj = ASAN_DIR / "abi_driver.o"
    _run([hipcc, *host, *san, f"-I{PKG_DIR.parent / 'include'}", "-c", str(ASAN_DRIVER_SRC), "-o", str(dobj)])
    _run([hipcc, "--offload-host-only", *san, str(dobj), f"-L{ASAN_DIR}", "-lwfbitnet_asan",
          f"-Wl,-rpath,{ASAN_DIR}", "-o", str(driver)])
    return driver


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
    if "--asan" in sys.argv:
        print(build_asan(verbose="-v" in sys.argv))
