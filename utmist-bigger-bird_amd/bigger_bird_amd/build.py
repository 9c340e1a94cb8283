"""Build libbb_attn.so (gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python -m bigger_bird_amd.build            # from utmist-bigger-bird_amd/
    python utmist-bigger-bird_amd/bigger_bird_amd/build.py

The library lands next to this file, so it travels with the source tree (and to a GPU box) without installation.
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / "csrc"
INCLUDE = PKG.parent.parent / "include"
LIB = PKG / "libbb_attn.so"
ARCH = os.environ.get("BB_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # packed fp32 VALU ops stay off (the device compiler would otherwise form v_pk_* from scalar float code)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]
SOURCES = ["bb_flash.hip", "bb_flash_pipe.hip", "bb_routes.hip", "bb_int8.hip", "bb_decode.hip", "bb_probe.hip",
           "bb_capi.cpp"]


def _compile(src: Path, obj: Path) -> None:
    cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        noise = "is not a recognized feature for this target"
        err = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")


def build(verbose: bool = True) -> Path:
    """Compile every HIP source for the target arch and link the shared library. Always rebuilds."""
    objdir = PKG.parent / "_build"
    objdir.mkdir(exist_ok=True)
    objs = [objdir / (Path(s).stem + ".o") for s in SOURCES]
    jobs = min(len(SOURCES), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda so: _compile(CSRC / so[0], so[1]), zip(SOURCES, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", flush=True)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
