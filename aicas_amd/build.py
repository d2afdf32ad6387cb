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
SOURCES = [os.path.join(CSRC, "aicas_decode.hip")]
HEADERS = [
    os.path.join(CSRC, "common.hpp"),
    os.path.join(CSRC, "kv_append.hpp"),
    os.path.join(CSRC, "decode_attn.hpp"),
    os.path.join(os.path.dirname(PKG_DIR), "include", "aicas_decode.h"),
]
OUTPUT = os.path.join(PKG_DIR, "libaicas_decode.so")
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    return path if os.path.exists(path) else "hipcc"


def command(output: str = OUTPUT) -> list[str]:
    return [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-mcode-object-version=5",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-o", output,
        *SOURCES,
    ]


def build(verbose: bool = True) -> str:
    """Compile the library in-tree (always recompiles) and return its path."""
    tmp = OUTPUT + ".tmp"
    cmd = command(tmp)
    if verbose:
        print("[aicas build]", " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build())
