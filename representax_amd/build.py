"""Build librepresentax_amd.so for gfx950 with hipcc (in-tree, no JIT cache).

``python -m representax_amd.build`` compiles every HIP source under
``representax_amd/csrc`` in parallel and links them into
``representax_amd/_lib/librepresentax_amd.so``, then builds the CPython
fast-call binding of the small-M forward entry points (``csrc/pyfast.c``)
next to it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
OUT_DIR = PACKAGE / "_lib"
LIB_NAME = "librepresentax_amd.so"
FAST_NAME = "_rpxfast" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so")
ARCH = os.environ.get("RPX_OFFLOAD_ARCH", "gfx950")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 VALU forms stay disabled on this target
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build")
    return exe


def _compile(src: Path, obj: Path) -> tuple[Path, str]:
    cmd = [hipcc(), *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    log = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{log}")
    return obj, log


def build(verbose: bool = False) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = [(src, obj_dir / (src.stem + ".o")) for src in sources]
    workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        results = list(pool.map(lambda j: _compile(*j), jobs))
    if verbose:
        for obj, log in results:
            if log.strip():
                print(f"[{obj.name}]\n{log}")
    lib = OUT_DIR / LIB_NAME
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp)]
    cmd += [str(o) for o, _ in results]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, lib)
    build_fast()
    return lib


def build_fast() -> Path:
    """The CPython binding: plain C, linked against the library in the same
    directory (rpath $ORIGIN) so both bindings share one loaded instance."""

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no C compiler for the CPython binding")
    out = OUT_DIR / FAST_NAME
    tmp = OUT_DIR / (FAST_NAME + ".tmp")
    cmd = [cc, "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-Werror",
           f"-I{sysconfig.get_paths()['include']}", str(CSRC / "pyfast.c"),
           f"-L{OUT_DIR}", "-lrepresentax_amd", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"building the CPython binding failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
