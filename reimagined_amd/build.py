"""Compiles the nsosx HIP library for gfx950 in-tree: reimagined_amd/libnsosx.so.

    python -m reimagined_amd.build

Every .hip file under csrc/ becomes one object (compiled in parallel), then
one shared library.  Flags:
  -ffp-contract=off                      no implicit fma: every fusion the
                                         reference's arithmetic performs is
                                         written out in the source
  -fhip-fp32-correctly-rounded-divide-sqrt  IEEE division and square root
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed-fp32 VALU ops
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libnsosx.so")
BUILD_DIR = os.path.join(HERE, "_build")

ARCH = os.environ.get("NSOSX_OFFLOAD_ARCH", "gfx950")
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the nsosx library needs ROCm's hipcc")


def _compile(src: str) -> str:
    obj = _obj(src)
    cmd = [hipcc(), *CFLAGS, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def _obj(src: str) -> str:
    return os.path.join(BUILD_DIR, os.path.basename(src).replace(".hip", ".o"))


def build(verbose: bool = False, incremental: bool = False) -> str:
    """Compiles every csrc/*.hip and links the library.  incremental: keep an object
    newer than its source and than every csrc/*.hpp (a header change rebuilds all)."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    hdr_time = max((os.path.getmtime(os.path.join(CSRC, f)) for f in os.listdir(CSRC)
                    if f.endswith(".hpp")), default=0.0)

    def stale(src: str) -> bool:
        obj = _obj(src)
        return (not incremental or not os.path.exists(obj) or
                os.path.getmtime(obj) < max(os.path.getmtime(src), hdr_time))

    todo = [s for s in srcs if stale(s)]
    # longest units first, so the slowest compile starts at once
    todo.sort(key=os.path.getsize, reverse=True)
    with cf.ThreadPoolExecutor(max_workers=max(1, min(8, len(todo)))) as ex:
        list(ex.map(_compile, todo))
    objs = [_obj(s) for s in srcs]
    tmp = OUT + ".tmp"
    # --no-undefined: a kernel whose host launch stub was not emitted fails here, at build
    # time, instead of when the library is loaded
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", tmp,
           *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


CONSUMER_SRC = os.path.join(os.path.dirname(HERE), "tests", "abi_consumer.cpp")
CONSUMER_OUT = os.path.join(HERE, "host", "abi_consumer")


def consumer_cmd(out: str = CONSUMER_OUT) -> list:
    """g++ line of the C++ consumer of the C ABI (tests/abi_consumer.cpp through
    reimagined_amd/host/nsosx.hpp): warnings are errors, linked to libnsosx.so."""
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    inc = os.path.join(os.path.dirname(HERE), "include")
    return ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
            f"-I{inc}", f"-I{os.path.join(HERE, 'host')}", f"-I{rocm}/include", CONSUMER_SRC,
            "-o", out, f"-L{HERE}", "-lnsosx", f"-Wl,-rpath,{HERE}", f"-L{rocm}/lib",
            "-lamdhip64", f"-Wl,-rpath,{rocm}/lib"]


def build_consumer(verbose: bool = False) -> str:
    proc = subprocess.run(consumer_cmd(), capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"C++ consumer build failed:\n{proc.stderr}")
    if verbose:
        print(f"built {CONSUMER_OUT}")
    return CONSUMER_OUT


if __name__ == "__main__":
    build(verbose=True, incremental="--incremental" in sys.argv)
    build_consumer(verbose=True)
