"""Builds libvkhip.so (the gfx950 device backend) in-tree with hipcc.

The library is compiled here, on a machine with no GPU (hipcc cross-compiles
for gfx950), and the resulting .so travels with the source tree.

Flags:
  --offload-arch=gfx950          CDNA4 only; no other targets, no host fallback.
  -ffp-contract=off              no FMA contraction in hand-written arithmetic:
                                 products and sums round where the CPU oracle's do.
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                 keep the compiler from forming packed-fp32 ops.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libvkhip.so"
OBJDIR = ROOT / "_build" / "vkhip"

SOURCES = ["runtime.hip", "allocator.hip", "observe.hip", "program.hip", "gemm.hip", "movement.hip",
           "reduce.hip", "elementwise.hip", "conv_small.hip"]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the gfx950 backend cannot be built")
    return exe


def compile_flags() -> list[str]:
    return [
        "--offload-arch=gfx950",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-result",
        f"-I{ROOT / 'include'}",
        f"-I{CSRC}",
    ]


# Per-source additions: the small-window convolution kernels keep their MFMA
# accumulators in VGPRs, which their epilogues read with plain VALU
# instructions (from AGPRs each value would first be copied out).
FILE_FLAGS = {"conv_small.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: Path, obj: Path, verbose: bool) -> tuple[Path, str]:
    cmd = [hipcc(), *compile_flags(), *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = res.stdout + res.stderr
    # hipcc's host pass does not know the packed-fp32 feature and says so; that
    # line is expected and harmless.
    out = "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, file=sys.stderr)
    return obj, out


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    OBJDIR.mkdir(parents=True, exist_ok=True)
    LIBDIR.mkdir(parents=True, exist_ok=True)
    srcs = [CSRC / s for s in SOURCES]
    objs = [OBJDIR / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], verbose), zip(srcs, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
