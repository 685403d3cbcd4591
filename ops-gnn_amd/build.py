"""Build libogn_hip.so (the gfx950 kernels + C ABI) in-tree.

    python ops-gnn_amd/build.py [-j N]

Every ``csrc/*.hip`` file is compiled separately with hipcc for gfx950 and the
objects are linked into ``ops_gnn/libogn_hip.so`` next to the Python package
that loads it.  ``csrc/pybind.cpp`` (host C++) becomes the torch extension
``ops_gnn/_pybind.so`` over that library.  Packed-fp32 instruction selection is disabled for all device
code (``-packed-fp32-ops``).
"""

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT_DIR = HERE / "ops_gnn"
LIB_NAME = "libogn_hip.so"
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build ops-gnn)")


COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # let `#pragma unroll` fully unroll the engine's consume loop (its body
    # holds the row-finishing code) so that staged loads stay in registers
    "-mllvm", "-pragma-unroll-threshold=200000",
]


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    # The host pass does not know the packed-fp32 feature; drop that warning.
    noise = [l for l in proc.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip()]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")


def _stale(src: Path, obj: Path, headers) -> bool:
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    return src.stat().st_mtime > t or any(h.stat().st_mtime > t for h in headers)


def build(jobs: int = 8, verbose: bool = True, incremental: bool = False) -> Path:
    """Compile every source (or, with incremental, those whose object is older
    than the source or any header) and link the library."""
    # the engine instance files take minutes each: start them first
    sources = sorted(CSRC.glob("*.hip"), key=lambda f: (not f.name.startswith("engine_"), f.name))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    obj_dir = HERE / "_build"
    obj_dir.mkdir(exist_ok=True)
    objs = [obj_dir / (s.stem + ".o") for s in sources]
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        headers = list(CSRC.glob("*.h")) + [HERE.parent / "include" / "ogn.h"]
        futures = [pool.submit(_compile, s, o) for s, o in zip(sources, objs)
                   if not incremental or _stale(s, o, headers)]
        for f in futures:
            f.result()
    target = OUT_DIR / LIB_NAME
    tmp = target.with_suffix(".so.tmp")
    # the SONAME lets the extension's dependency on libogn_hip.so resolve to a
    # copy already loaded from $OGN_LIB, so both routes share one library
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,-soname,{LIB_NAME}", *map(str, objs),
           "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, target)
    if verbose:
        print(f"built {target} from {len(sources)} sources")
    return target


EXT_NAME = "_pybind"


def build_extension(verbose: bool = True) -> Path:
    """Compile csrc/pybind.cpp (host C++, no device code) into the torch
    extension ops_gnn/_pybind.so, linked against libogn_hip.so (found next to
    it through an $ORIGIN rpath) and torch's libraries."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    target = OUT_DIR / (EXT_NAME + ".so")
    tmp = target.with_suffix(".so.tmp")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-shared", "-fPIC", "-w",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           *[f"-I{p}" for p in cpp_extension.include_paths(device_type="cuda")],
           f"-I{sysconfig.get_paths()['include']}", "-I/opt/rocm/include",
           str(CSRC / "pybind.cpp"), "-o", str(tmp),
           f"-L{OUT_DIR}", "-logn_hip", "-Wl,-rpath,$ORIGIN",
           f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
           f"-Wl,-rpath,{torch_lib}"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"extension build failed:\n{proc.stderr}")
    os.replace(tmp, target)
    if verbose:
        print(f"built {target}")
    return target


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", "--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--incremental", action="store_true", help="recompile only out-of-date objects")
    ap.add_argument("--extension-only", action="store_true", help="rebuild only the torch extension")
    args = ap.parse_args()
    if not args.extension_only:
        build(args.jobs, incremental=args.incremental)
    build_extension()
