"""Build libeverserve_mi355x.so for gfx950 with hipcc, in tree, and stamp it.

The library is plain C ABI over the HIP runtime: no torch headers, no pybind. It is built where
there is no GPU (hipcc cross-compiles for the architectures it is told) and loaded by
:mod:`everserve_amd.kernels`, which refuses a build whose stamp does not match the sources beside
it. This mirrors the reference's ``python -m everserve.kernels --into DIR``
(core/everserve/kernels.py:93-107), with ``PYTORCH_ROCM_ARCH`` in place of
``TORCH_CUDA_ARCH_LIST``.

Run as ``python -m everserve_amd.build``.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
INCLUDE = ROOT / "include"
LIBRARY = "libeverserve_mi355x.so"
STAMP = "stamp.json"
SOURCES = ("rows.hip", "order.hip", "reduce.hip", "slot.hip", "host_rows.hip", "store.hip",
           "runtime.hip")
HEADERS = ("common.hpp", "host_copy.hpp", "workers.hpp")
PUBLIC_HEADERS = ("everserve_mi355x.h",)
DEFAULT_ARCHS = "gfx950"
# Flags for one source only. The local reduce's counting atomics run in one lane and their
# answers are read late; the atomic optimizer would rewrite each into a wave-wide form that reads
# its answer at once (to hand it to every lane), which waits out the atomic in front of the
# payload loads.
SOURCE_FLAGS = {"reduce.hip": ("-mllvm", "-amdgpu-atomic-optimizer-strategy=None")}

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # no packed fp32 instructions anywhere: some of their forms have miscomputed on these boxes
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    """The hipcc to build with: $HIPCC, else ROCm's."""
    return os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def source_files() -> list[Path]:
    """Every file whose bytes the library is built from, in a fixed order."""
    return (
        [CSRC / s for s in SOURCES]
        + [CSRC / h for h in HEADERS]
        + [INCLUDE / h for h in PUBLIC_HEADERS]
    )


def sources_digest() -> str:
    """sha256 over the names and bytes of every source file, and the flags they are built with."""
    digest = hashlib.sha256()
    for f in source_files():
        digest.update(f.name.encode())
        digest.update(f.read_bytes())
    digest.update(json.dumps([HIPCC_FLAGS, SOURCE_FLAGS], sort_keys=True).encode())
    return digest.hexdigest()


def archs_from_env() -> str:
    return os.environ.get("PYTORCH_ROCM_ARCH", "") or DEFAULT_ARCHS


def stamp(archs: str | None = None) -> dict[str, str]:
    """What a build is made from: the sources by content and the GPU architectures."""
    return {"sources": sources_digest(), "archs": archs or archs_from_env()}


def build(out_dir: Path = PACKAGE, archs: str | None = None, verbose: bool = False,
          defines: tuple[str, ...] = ()) -> Path:
    """Compile every source for ``archs`` (``;``-separated, default gfx950) into ``out_dir``.

    Always compiles: the build is the check that the sources build. ``defines`` (``NAME=VALUE``)
    override the kernels' tuning macros, for building variants side by side. Raises
    ``subprocess.CalledProcessError`` when hipcc fails.
    """
    archs = archs or archs_from_env()
    arch_flags = [f"--offload-arch={a.strip()}" for a in archs.replace(" ", ";").split(";") if a]
    out_dir.mkdir(parents=True, exist_ok=True)
    obj_dir = out_dir / "_build"
    obj_dir.mkdir(exist_ok=True)
    cc = hipcc()
    includes = [f"-I{INCLUDE}", f"-I{CSRC}"]

    def compile_one(src: str) -> Path:
        obj = obj_dir / (Path(src).stem + ".o")
        cmd = [cc, *HIPCC_FLAGS, *SOURCE_FLAGS.get(src, ()), *arch_flags, *includes,
               *[f"-D{d}" for d in defines], "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        return obj

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), 4)) as pool:
        try:
            objs = list(pool.map(compile_one, SOURCES))
        except subprocess.CalledProcessError as e:
            sys.stderr.write(e.stdout or "")
            raise
    lib = out_dir / LIBRARY
    tmp = out_dir / (LIBRARY + ".tmp")
    cmd = [cc, *arch_flags, "-shared", "-fPIC", *[str(o) for o in objs], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, lib)
    (out_dir / STAMP).write_text(json.dumps(stamp(archs), indent=2) + "\n")
    return lib


def main(argv: list[str] | None = None) -> None:
    ap = argparse.ArgumentParser(prog="everserve_amd.build", description=__doc__)
    ap.add_argument("--into", type=Path, default=PACKAGE, help="output directory")
    ap.add_argument("--archs", default=None, help="GPU architectures (default $PYTORCH_ROCM_ARCH or gfx950)")
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args(argv)
    print(build(a.into, a.archs, a.verbose))


if __name__ == "__main__":
    main()
