"""Build ``libt2i_hip.so`` (gfx950) in-tree with hipcc.

``python -m torch2iron_amd.build`` compiles every ``csrc/*.hip`` into one shared
library next to this file.  The library exports the C ABI of
``include/t2i_hip.h`` and is loaded with ctypes by ``torch2iron_amd._lib``.

``python -m torch2iron_amd.build --tuning PATH`` writes a second library to PATH
with ``T2I_TUNING`` defined: its plan functions then honour the environment
overrides ``T2I_PLAN`` and ``T2I_RT`` (decode linear tile plan and row-tile
height), ``T2I_GEMM_MIN_M`` (smallest M routed to the prompt GEMM) and
``T2I_ATTN_ROWS`` (decode attention rows per chunk), for sweeps of the launch
shapes.  Swap it in place of ``libt2i_hip.so`` to use it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_PATH = PKG_DIR / "libt2i_hip.so"
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False, out: Path | None = None, tuning: bool = False) -> Path:
    """Compile all HIP sources into ``out`` (default ``LIB_PATH``) and return its path."""
    out = Path(out) if out is not None else LIB_PATH
    tmp = out.with_suffix(".so.tmp")
    cmd = [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-shared",
        "-fPIC",
        # packed fp32 VALU forms are kept out of the device code
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # leading scalar kernel arguments arrive in SGPRs at wave launch (no
        # kernarg load before the first address can be formed)
        "-mllvm", "-amdgpu-kernarg-preload-count=16",
        # MFMA accumulators in VGPRs rather than AGPRs: the prompt GEMM's per-group
        # scale step then reads them without a v_accvgpr_read each (qkv GEMM at
        # 8192 rows 132 -> 127 us, down 99 -> 94 us)
        "-mllvm", "-amdgpu-mfma-vgpr-form",
        *(["-DT2I_TUNING"] if tuning else []),
        f"-I{INCLUDE}",
        f"-I{CSRC}",
        *[str(s) for s in sources()],
        "-o", str(tmp),
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    if len(sys.argv) == 3 and sys.argv[1] == "--tuning":
        print(build(verbose=True, out=Path(sys.argv[2]).resolve(), tuning=True))
    elif len(sys.argv) == 1:
        print(build(verbose=True))
    else:
        sys.exit("usage: python -m torch2iron_amd.build [--tuning PATH]")
