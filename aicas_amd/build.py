"""Build recipe for libaicas_decode.so (gfx950). Run as ``python -m aicas_amd.build``.

hipcc cross-compiles for gfx950 without a GPU. Flags:
  -mcode-object-version=5   loadable by both the system ROCm 7.2 runtime and torch's bundled 7.0 runtime;
  -Xclang -target-feature -Xclang -packed-fp32-ops
                            keep the compiler from forming packed fp32 VALU ops (v_pk_*_f32) out of
                            ordinary float code; the host pass warns that it does not know the feature.
"""

from __future__ import annotations

import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
SOURCES = [
    os.path.join(CSRC, "aicas_decode.hip"),
    os.path.join(CSRC, "decode_bf16_bf16.hip"),
    os.path.join(CSRC, "decode_fp16_fp16.hip"),
    os.path.join(CSRC, "decode_bf16_fp8.hip"),
    os.path.join(CSRC, "decode_fp16_fp8.hip"),
]
INCLUDE = os.path.join(os.path.dirname(PKG_DIR), "include")
OUTPUT = os.path.join(PKG_DIR, "libaicas_decode.so")
# bandwidth calibration kernels for bench.py --config calib (a library of their own, outside the decode ABI)
CALIB_SOURCES = [os.path.join(CSRC, "calib.hip")]
CALIB_OUTPUT = os.path.join(PKG_DIR, "libaicas_calib.so")
OBJ_DIR = os.path.join(PKG_DIR, "_build")
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    return path if os.path.exists(path) else "hipcc"


COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def compile_command(source: str, obj: str, include: str = INCLUDE) -> list[str]:
    return [hipcc(), *COMMON_FLAGS, "-I", include, "-c", "-o", obj, source]


def link_command(objs: list[str], output: str) -> list[str]:
    return [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", output, *objs]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("[aicas build]", " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(verbose: bool = True, sources: list[str] | None = None, output: str = OUTPUT,
          include: str = INCLUDE, obj_dir: str = OBJ_DIR, calib: bool = True) -> str:
    """Compile every translation unit in parallel and link the library in-tree (always recompiles); with calib
    (the default build), also the calibration library libaicas_calib.so."""
    from concurrent.futures import ThreadPoolExecutor

    sources = sources or SOURCES
    libs = [(list(sources), output)] + ([(CALIB_SOURCES, CALIB_OUTPUT)] if calib else [])
    os.makedirs(obj_dir, exist_ok=True)
    obj = lambda src: os.path.join(obj_dir, os.path.splitext(os.path.basename(src))[0] + ".o")  # noqa: E731
    units = [src for srcs, _ in libs for src in srcs]
    jobs = max(1, min(len(units), os.cpu_count() or 1, 8))
    with ThreadPoolExecutor(jobs) as pool:
        list(pool.map(lambda src: _run(compile_command(src, obj(src), include), verbose), units))
    for srcs, out in libs:
        tmp = out + ".tmp"
        _run(link_command([obj(src) for src in srcs], tmp), verbose)
        os.replace(tmp, out)
    return output


if __name__ == "__main__":
    print(build())
