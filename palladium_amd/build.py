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


def build_all(verbose: bool = False) -> list[Path]:
    return [build_launcher(verbose)]


if __name__ == "__main__":
    for p in build_all(verbose="-v" in sys.argv):
        print(p)
