"""Build the HIP C-ABI library libmlxnufft_amd.so for gfx950.

    python -m mlx_nufft_amd.build            # or: python mlx_nufft_amd/build.py

Every csrc/*.hip file is compiled with hipcc to an object under _build/ (in
parallel), then linked into the package directory against rocFFT. The .so
is loaded with ctypes after `import torch`, so it binds to the HIP runtime
and rocFFT that torch already loaded (same SONAMEs as /opt/rocm).
"""

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libmlxnufft_amd.so"
ARCH = os.environ.get("MN_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

CFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed fp32 VALU ops are disabled (the compiler would otherwise form them)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]


def _run(cmd):
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n"
                           f"{p.stdout}\n{p.stderr}")
    return p


# Per-source additions. The z-gather reads its MFMA results with VALU code
# right away: in the VGPR form of the MFMAs they need no copy out of the
# accumulation registers (one v_accvgpr_read per result element otherwise).
# The max-ILP scheduler interleaves its tile reductions with the next tile's
# MFMAs more tightly: 1 % faster at 2e7 points on 512^3 (three runs,
# bit-identical). It also speeds the 2D y-window MFMA sweep with 8 vectors
# per wave by 1-3 % (1e7 points, 2048^2, within 1 % for one vector); it made
# the z-sweep spread 1.3 % slower, left the sort unchanged and moved the
# type-1 FFT by -0.3 to +0.7 %, so those keep the default scheduler.
EXTRA_FLAGS = {
    "mn_zgather.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form",
                       "-mllvm", "-amdgpu-sched-strategy=max-ilp"],
    "mn_ymfma.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
}


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = BUILD / (src.stem + ".o")
    _run([HIPCC, *CFLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)])
    return obj


def build(jobs: int | None = None, verbose: bool = True) -> pathlib.Path:
    """Compile every csrc/*.hip and link the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs),
          "-L/opt/rocm/lib", "-lrocfft", "-Wl,-rpath,/opt/rocm/lib", "-o", str(tmp)])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} ({LIB.stat().st_size / 1e6:.1f} MB) from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
