"""Ahead-of-time build of librumik_hip.so (all HIP kernels + the C ABI of include/rumik_hip.h) for gfx950.

    python rumik-fast_amd/build.py          # -> rumik-fast_amd/lib/librumik_hip.so

Each .hip file is compiled separately (in parallel) and the objects are linked into one shared library. There is
no JIT anywhere: the Python wrappers load the prebuilt library with ctypes.
"""
import os
import shutil
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "librumik_hip.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-mcode-object-version=5", "-Wall", "-Wno-unused-function",
    # export only what include/rumik_hip.h declares (it pushes default visibility around its declarations)
    "-fvisibility=hidden",
    # packed fp32 ops (v_pk_*_f32) stay off: only scalar fp32 VALU ops are emitted
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


# per-source additions: the prefill attention keeps its MFMA accumulators in VGPRs (its online-softmax rescale
# multiplies them between MFMAs; in AGPRs every multiply costs a copy out and back)
EXTRA = {"prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def sources():
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, obj: Path):
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src.name, []), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the packed-fp32 feature and says so; that warning is expected
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    return err.strip()


def build(verbose: bool = True, jobs: int | None = None) -> Path:
    t0 = time.time()
    obj_dir = PKG / "_build"
    obj_dir.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    srcs = sources()
    objs = [obj_dir / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(jobs) as ex:
        warns = list(ex.map(_compile, srcs, objs))
    for s, w in zip(srcs, warns):
        if w and verbose:
            print(f"[build] {s.name}:\n{w}", file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[build] {LIB.relative_to(ROOT)} ({len(srcs)} sources) in {time.time() - t0:.1f}s", flush=True)
    return LIB


if __name__ == "__main__":
    build()
