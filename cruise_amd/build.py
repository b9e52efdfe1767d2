"""Build libresident_epoch.so for gfx950 with hipcc (in-tree, no JIT cache).

``python -m cruise_amd.build`` compiles ``cruise_amd/csrc/*.hip`` into
``cruise_amd/lib/libresident_epoch.so``.  The library links the HIP runtime
only: every kernel, the batched-prefill GEMMs included, is hand-written, and
PyTorch is never linked into it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
LIBDIR = PACKAGE / "lib"
LIBRARY = LIBDIR / "libresident_epoch.so"
SERVER = LIBDIR / "resident_epoch_server"
SERVER_SOURCE = "re_server.cpp"
INCLUDE = PACKAGE.parent / "include"
SOURCES = ("re_step.hip", "re_attn.hip", "re_ctrl.hip", "re_prefill.hip", "re_mfma.hip", "re_engine.hip")
LINK_LIBS: tuple[str, ...] = ()

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # Packed FP32 instructions are kept out of the device code.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found: the resident epoch library needs ROCm's hipcc")
    return found


def build(verbose: bool = False, defines: tuple[str, ...] = (), output: Path | None = None) -> Path:
    """Compile the library.  ``defines`` are extra ``-D`` macros (tuning
    variants such as ``NORMED_MIN_WAVES=3``); ``output`` another .so path."""
    library = Path(output) if output is not None else LIBRARY
    library.parent.mkdir(parents=True, exist_ok=True)
    build_dir = PACKAGE / "_build" / (library.stem if output is not None else "default")
    build_dir.mkdir(parents=True, exist_ok=True)
    objects = []

    def compile_one(src: str) -> Path:
        obj = build_dir / (Path(src).stem + ".o")
        cmd = [hipcc(), *HIPCC_FLAGS, *(f"-D{d}" for d in defines), f"-I{INCLUDE}", "-c", str(CSRC / src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr[-6000:]}")
        if verbose and res.stderr.strip():
            noise = "is not a recognized feature for this target"
            lines = [ln for ln in res.stderr.splitlines() if noise not in ln]
            if lines:
                print("\n".join(lines), file=sys.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        objects = list(pool.map(compile_one, SOURCES))
    tmp = library.with_suffix(".so.tmp")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objects), *LINK_LIBS, "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, library)
    if output is None:
        build_server(library, SERVER)
    return library


def build_server(library: Path = LIBRARY, output: Path = SERVER) -> Path:
    """Compile the sidecar server (host C++ only) against ``library``; it
    finds the library next to itself at run time (rpath $ORIGIN)."""
    compiler = shutil.which("g++") or "g++"
    tmp = output.with_name(output.name + ".tmp")
    cmd = [
        compiler, "-O2", "-std=c++17", "-Wall", "-Wextra", f"-I{INCLUDE}", str(CSRC / SERVER_SOURCE),
        f"-L{library.parent}", f"-l:{library.name}", "-Wl,-rpath,$ORIGIN", "-Wl,-rpath-link,/opt/rocm/lib",
        "-o", str(tmp),
    ]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"server build failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, output)
    return output


if __name__ == "__main__":
    print(build(verbose=True))
