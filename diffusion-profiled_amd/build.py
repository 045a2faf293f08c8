"""Build the gfx950 HIP library ``lib/libdpa_fp8.so`` from ``csrc/*.hip``.

The library has a plain C ABI (``include/dpa_fp8.h``); nothing here links against torch.
Sources compile in parallel (one ``hipcc -c`` per file) and link with ``hipcc -shared``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC_DIR = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_DIR = PKG_DIR / "lib"
LIB_PATH = LIB_DIR / "libdpa_fp8.so"

OFFLOAD_ARCH = "gfx950"

# -ffp-contract=off keeps every fp32 rounding step of the reference recipe explicit; the
# packed-fp32 target feature is switched off for all device code.
HIPCC_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = shutil.which("hipcc") or os.path.join(rocm, "bin", "hipcc")
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the FP8 HIP library cannot be built")
    return path


def sources() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.hip"))


def build_library(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip for gfx950 and link lib/libdpa_fp8.so. Always rebuilds."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    cc = hipcc()
    procs = []
    objs = []
    for src in sources():
        obj = BUILD_DIR / (src.stem + ".o")
        objs.append(obj)
        cmd = [cc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    errors = []
    for src, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        # the host pass warns that it does not know the packed-fp32 feature: harmless
        lines = [ln for ln in text.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
        if p.returncode != 0:
            errors.append(f"{src.name}:\n" + "\n".join(lines))
        elif verbose and lines:
            print("\n".join(lines), flush=True)
    if errors:
        raise RuntimeError("hipcc failed:\n" + "\n\n".join(errors))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if r.returncode != 0:
        raise RuntimeError("hipcc link failed:\n" + r.stdout.decode(errors="replace"))
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
