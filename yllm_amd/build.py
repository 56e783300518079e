"""Build the gfx950 attention library in-tree: yllm_amd/libyllm_hip.so.

Every source under yllm_amd/csrc is compiled with hipcc for gfx950 and
linked into one shared library with a plain C ABI (include/yllm_hip.h).
Packed-fp32 instruction selection is switched off for device code
(-Xclang -target-feature -Xclang -packed-fp32-ops).

    python -m yllm_amd.build          # or yllm_amd.build.build()
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_build"
LIB = PKG / "libyllm_hip.so"
ARCH = os.environ.get("YLLM_HIP_ARCH", "gfx950")

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(hipcc: str, src: Path) -> Path:
    obj = OUT_DIR / (src.stem + ".o")
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    cmd = [hipcc, *COMMON_FLAGS, *lang, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the packed-fp32 feature; that warning is expected
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l and "(ignoring feature)" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(verbose: bool = True) -> Path:
    hipcc = _hipcc()
    OUT_DIR.mkdir(exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    rocm_lib = Path(hipcc).resolve().parent.parent / "lib"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
           f"-L{rocm_lib}", f"-Wl,-rpath,{rocm_lib}"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    # A kernel whose body the host pass could not instantiate leaves its
    # launch stub undefined without any compiler error; the library would
    # then fail to load.  Refuse it here.
    nm = subprocess.run(["nm", "-D", "--undefined-only", str(tmp)], capture_output=True, text=True)
    stubs = [l.split()[-1] for l in nm.stdout.splitlines() if "__device_stub__" in l]
    if stubs:
        tmp.unlink()
        raise RuntimeError("kernel launch stubs missing from the host objects: " + ", ".join(stubs))
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources for {ARCH}")
    return LIB


if __name__ == "__main__":
    build()
