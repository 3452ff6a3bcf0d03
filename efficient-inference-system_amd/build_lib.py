"""Build libpaged_hip.so (the C-ABI paged-attention library) for gfx950 with hipcc.

Every `csrc/*.hip` file is compiled to an object under `_build/` and linked into
`libpaged_hip.so` next to this file; `csrc/host/paged_host.cpp` becomes the CPython module
`src/cache/_paged_host` (native host bookkeeping of graph steps). The library links against the HIP runtime that torch bundles
(rpath to torch/lib), so a process that imports torch and then loads the library maps a single
HIP runtime. Usage: `python build_lib.py [--verbose]`.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libpaged_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Keep the compiler from forming packed fp32 instructions (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs instead of AGPRs: with AGPR accumulators the prefill
    # kernels copied their 64 output accumulators between the two register files every KV step
    # (around the lazy-rescale branch) and needed 244-296 registers; in VGPR form no copies and
    # 146-212 registers (large prefill: bf16 417 -> 371 us, fp32 2018 -> 1908 us; others equal).
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _torch_lib_dir() -> Path | None:
    try:
        import torch  # noqa: F401  (only to locate the bundled HIP runtime)
    except ImportError:
        return None
    d = Path(torch.__file__).resolve().parent / "lib"
    return d if (d / "libamdhip64.so").exists() else None


def _filter(out: str) -> str:
    # The host pass reports the gfx-only target feature as unknown; that line is noise.
    return "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l)


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    msg = _filter(proc.stdout)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{msg}")
    if msg.strip() and verbose:
        print(msg, flush=True)


HOST_SRC = CSRC / "host" / "paged_host.cpp"
HOST_DIR = PKG_DIR / "src" / "cache"


def build_host(verbose: bool = False) -> Path:
    """Compile the native host bookkeeping module (CPython extension, plain g++ against this
    interpreter's headers) to src/cache/_paged_host<EXT_SUFFIX>; returns its path."""
    import sysconfig

    out = HOST_DIR / ("_paged_host" + sysconfig.get_config_var("EXT_SUFFIX"))
    cxx = os.environ.get("CXX") or shutil.which("g++") or "g++"
    _run([cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Wextra",
          f"-I{sysconfig.get_paths()['include']}", str(HOST_SRC), "-o", str(out) + ".tmp"], verbose)
    os.replace(str(out) + ".tmp", out)
    return out


def build(verbose: bool = False) -> Path:
    """Compile all sources and link the library (and the host module); returns the library path."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no sources under {CSRC}")
    incs = [f"-I{INCLUDE}", f"-I{CSRC}"]

    def compile_one(src: Path) -> Path:
        obj = BUILD_DIR / (src.stem + ".o")
        _run([hipcc, *HIPCC_FLAGS, *incs, "-c", str(src), "-o", str(obj)], verbose)
        return obj

    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(compile_one, sources))

    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(LIB_PATH) + ".tmp"]
    tlib = _torch_lib_dir()
    if tlib is not None:
        link += [f"-L{tlib}", f"-Wl,-rpath,{tlib}"]
    _run(link, verbose)
    os.replace(str(LIB_PATH) + ".tmp", LIB_PATH)
    build_host(verbose)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="--verbose" in sys.argv)
    print(path)
