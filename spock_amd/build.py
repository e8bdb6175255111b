"""Builds the gfx950 HIP library and the C++ host layer in-tree.

* spock_amd/libspock_hip.so: every .hip file under spock_amd/csrc, compiled
  with hipcc for gfx950 only, with -ffp-contract=off (the bit-exact kernels
  spell out every fma) and packed fp32 instructions disabled; its C ABI is
  include/spock_hip.h.
* spock_amd/libspock_hip_host.so: the C++ host classes under csrc/host
  (run_deltanet_chunk_rule, DeltaNetSession), plain C++17 built with g++
  against the HIP runtime and libspock_hip.so.
* spock_amd/bin/: the command-line drivers under csrc/apps.
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
OBJ = PKG / "_obj"
LIB = PKG / "libspock_hip.so"
HOST_LIB = PKG / "libspock_hip_host.so"
BIN = PKG / "bin"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
CXX = os.environ.get("CXX_HOST", shutil.which("g++") or "g++")
HOST_FLAGS = ["-std=c++17", "-O2", "-fPIC", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
              "-I", str(ROCM / "include"), "-I", str(ROOT / "include")]
HOST_LINK = ["-L", str(ROCM / "lib"), "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}"]
# csrc/apps/<name>.cpp -> bin/<name with - for _>

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-I", str(ROOT / "include"),
]


def _compile(src: Path) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr[-6000:]}")
    noise = [ln for ln in r.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")
    return obj


def build(verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


def _run(cmd: list[str], what: str) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{r.stderr[-6000:]}")
    if r.stderr.strip():
        sys.stderr.write(r.stderr)


def _host_compile(src: Path) -> Path:
    obj = OBJ / ("host_" + src.stem + ".o")
    _run([CXX, *HOST_FLAGS, "-c", str(src), "-o", str(obj)], f"g++ {src.name}")
    return obj


def build_host(verbose: bool = False) -> list[Path]:
    """C++ host layer (needs libspock_hip.so built first)."""
    OBJ.mkdir(exist_ok=True)
    BIN.mkdir(exist_ok=True)
    host_srcs = sorted((CSRC / "host").glob("*.cpp"))
    app_srcs = sorted((CSRC / "apps").glob("*.cpp"))
    with ThreadPoolExecutor(max_workers=8) as ex:
        host_objs = list(ex.map(_host_compile, host_srcs))
        app_objs = list(ex.map(_host_compile, app_srcs))
    tmp = HOST_LIB.with_suffix(".so.tmp")
    _run([CXX, "-shared", "-fPIC", *map(str, host_objs), "-o", str(tmp), "-L", str(PKG), "-lspock_hip",
          "-Wl,-rpath,$ORIGIN", *HOST_LINK], "host library link")
    os.replace(tmp, HOST_LIB)
    outs = [HOST_LIB]
    for src, obj in zip(app_srcs, app_objs):
        exe = BIN / src.stem.replace("_", "-")
        tmp = exe.with_suffix(".tmp")
        _run([CXX, str(obj), "-o", str(tmp), "-L", str(PKG), "-lspock_hip_host", "-lspock_hip",
              "-Wl,-rpath,$ORIGIN/..", *HOST_LINK], f"link {exe.name}")
        os.replace(tmp, exe)
        outs.append(exe)
    if verbose:
        print(f"built {HOST_LIB.name} and {len(app_srcs)} drivers in {BIN}")
    return outs


def build_oracle(verbose: bool = False) -> None:
    """Test infrastructure: the CPU oracle and, when the reference checkout is
    present, oracle/_ref (see oracle/Makefile)."""
    r = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}\n{r.stderr}")
    if verbose and r.stdout.strip():
        print(r.stdout.strip())


if __name__ == "__main__":
    build(verbose=True)
    build_host(verbose=True)
    build_oracle(verbose=True)
