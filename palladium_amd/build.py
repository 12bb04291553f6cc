"""Build the native pieces in-tree: `libpalladium_hip.so` (the C-ABI
launcher, include/palladium_hip.h). Run `python -m palladium_amd.build`.

Every hipcc line carries `-Xclang -target-feature -Xclang -packed-fp32-ops`
so no packed-FP32 VALU forms reach a code object.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
LIB = PKG / "libpalladium_hip.so"
NO_PACKED = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def build_launcher(verbose: bool = False) -> Path:
    src = PKG / "csrc" / "palladium_hip.cpp"
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [
        HIPCC, "--offload-arch=gfx950", *NO_PACKED, "-O2", "-fPIC", "-shared", "-std=c++17",
        f"-I{ROOT / 'include'}", str(src), "-o", str(tmp), "-lhiprtc",
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


def build_ffi(verbose: bool = False) -> Path:
    """The jax.ffi handler (csrc/xla_ffi_handler.cc) over the C ABI; needs
    jax for the XLA FFI headers."""
    import jax

    out = PKG / "libpalladium_hip_ffi.so"
    cmd = [
        HIPCC, "--offload-arch=gfx950", *NO_PACKED, "-O2", "-fPIC", "-shared", "-std=c++17",
        f"-I{ROOT / 'include'}", f"-I{jax.ffi.include_dir()}", str(PKG / "csrc" / "xla_ffi_handler.cc"),
        str(PKG / "csrc" / "palladium_hip.cpp"), "-o", str(out), "-lhiprtc",
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return out


def build_all(verbose: bool = False, ffi: bool = False) -> list[Path]:
    out = [build_launcher(verbose)]
    if ffi:
        out.append(build_ffi(verbose))
    return out


if __name__ == "__main__":
    for p in build_all(verbose="-v" in sys.argv, ffi="--ffi" in sys.argv):
        print(p)
