"""Build the gfx950 shared library ``mintext_amd/_lib/libmintext_moe.so`` with hipcc.

Each ``csrc/*.hip`` file is compiled to an object in parallel and the objects are linked
into one shared library exporting the C-ABI of ``include/mintext_moe.h``.  The library is
built in-tree so that it travels with the source tree to the GPU host.

    python -m mintext_amd.build            # build (always recompiles)
    python -m mintext_amd.build --report   # also print per-kernel register/LDS usage
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB_NAME = "libmintext_moe.so"
ARCH = os.environ.get("MTX_OFFLOAD_ARCH", "gfx950")

# Packed-FP32 VALU instructions are disabled on purpose for every device compile.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the MI355X library needs ROCm's hipcc")
    return path


def _compile(src: Path, obj: Path, report: bool) -> str:
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    if report:
        cmd.insert(1, "-Rpass-analysis=kernel-resource-usage")
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr[-6000:]}")
    lines = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
    return "\n".join(lines)


def build(report: bool = False, verbose: bool = True) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    objs = [OUT_DIR / (s.stem + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        logs = list(ex.map(lambda so: _compile(so[0], so[1], report), zip(srcs, objs)))
    if report and verbose:
        for s, log in zip(srcs, logs):
            print(f"==== {s.name}\n{log}")
    lib = OUT_DIR / LIB_NAME
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, lib)
    for o in objs:
        o.unlink(missing_ok=True)
    if verbose:
        print(f"built {lib}")
    return lib


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--report", action="store_true")
    a = ap.parse_args(argv)
    build(report=a.report)
    return 0


if __name__ == "__main__":
    sys.exit(main())
