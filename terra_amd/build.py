"""Builds ``terra_amd/libterra_swin.so`` from ``terra_amd/csrc`` with hipcc for gfx950.

    python -m terra_amd.build

The library is written in-tree (it travels with the source tree to the GPU
host; nothing is JIT-compiled at run time).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
SOURCES = ("abi.hip", "window_copy.hip", "window_attention.hip", "window_attention_bwd.hip", "swin_block.hip",
           "swin_mlp.hip", "linear.hip", "mlp_backward.hip")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Packed-fp32 VALU ops are kept out of the device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in arch VGPRs (no AGPR round trip): keeps the attention
    # kernel at <= 128 VGPRs, i.e. 4 waves per SIMD.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wall",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libterra_swin.so)")


def _run(cmd, verbose: bool) -> str:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{out}")
    return out


# Host-side AddressSanitizer (the C-ABI validation code; device code is built
# as usual): each flag applies to the host compilation only.
ASAN_HOST_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]
ASAN_LIB_PATH = os.path.join(HERE, "libterra_swin_asan.so")


def build_library(verbose: bool = False, jobs: int = 0, asan_host: bool = False) -> str:
    """Compile every HIP source (one hipcc process per source, in parallel)
    and link them into the shared library; returns its path.  ``asan_host``
    builds ``libterra_swin_asan.so`` instead, its host code under
    AddressSanitizer (load it with the sanitizer runtime preloaded and
    TERRA_SWIN_LIB naming it)."""
    from concurrent.futures import ThreadPoolExecutor

    from ._lib import LIB_PATH as default_path  # noqa: WPS433 (path only; does not open the library)

    LIB_PATH = ASAN_LIB_PATH if asan_host else default_path
    extra = ASAN_HOST_FLAGS if asan_host else []
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1, 8)
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"] + extra
    with tempfile.TemporaryDirectory(prefix="_build.", dir=HERE) as tmpdir:
        objs = [os.path.join(tmpdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
        cmds = [[hipcc(), *compile_flags, "-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(SOURCES, objs)]
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            outs = list(pool.map(lambda c: _run(c, verbose), cmds))
        fd, tmp = tempfile.mkstemp(prefix="libterra_swin.", suffix=".so.tmp", dir=HERE)
        os.close(fd)
        try:
            outs.append(_run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *extra, *objs, "-o", tmp],
                             verbose))
        except RuntimeError:
            os.unlink(tmp)
            raise
    if verbose:
        for out in outs:
            if out.strip():
                print(out, flush=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def asan_runtime() -> str:
    """Path of the clang AddressSanitizer runtime that hipcc links against."""
    out = subprocess.run([hipcc(), "-print-file-name=libclang_rt.asan-x86_64.so"], stdout=subprocess.PIPE,
                         stderr=subprocess.DEVNULL, text=True).stdout.strip()
    if out and os.path.isabs(out) and os.path.exists(out):
        return out
    import glob

    for cand in sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so")):
        return cand
    raise RuntimeError("clang AddressSanitizer runtime not found")


if __name__ == "__main__":
    path = build_library(verbose=True, asan_host="--asan-host" in sys.argv)
    print(path)
    sys.exit(0)
