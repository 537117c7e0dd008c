"""Build recipe for the MI355X attention libraries (gfx950 only).

Produces, in-tree:
  runtherder_amd/lib/libruntherder_attn.so      C ABI + HIP kernels (the product)
  runtherder_amd/lib/libruntherder_attn_cpp.so  C++20 AttentionBackend / KVCache
                                                layer over the C ABI
Run as ``python -m runtherder_amd.build`` or through __graft_entry__.build().
"""
from __future__ import annotations

import concurrent.futures as _cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
HOST = PKG / "host"
LIB_DIR = PKG / "lib"
OBJ_DIR = PKG / "lib" / "obj"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++20",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]

KERNEL_SOURCES = [
    "kv_quant.hip",
    "flash_decode.hip",
    "flash_prefill.hip",
    "attention_naive.hip",
    "rope.hip",
    "rmsnorm.hip",
    "capi.cpp",
]
HOST_SOURCES = ["attention_backends.cpp"]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (res.stdout + res.stderr).splitlines()
        if "packed-fp32-ops" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def _compile(src: Path, obj: Path, verbose: bool) -> Path:
    cmd = [HIPCC, *DEVICE_FLAGS, "-x", "hip", "-c", str(src), "-o", str(obj)]
    _run(cmd, verbose)
    return obj


def build(verbose: bool = False, jobs: int = 8) -> dict[str, Path]:
    """Compile every HIP/C++ source for gfx950 and link the two libraries."""
    if not Path(HIPCC).exists() and shutil.which(HIPCC) is None:
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    work = [(CSRC / s, OBJ_DIR / (Path(s).stem + ".o")) for s in KERNEL_SOURCES]
    work += [(HOST / s, OBJ_DIR / ("host_" + Path(s).stem + ".o")) for s in HOST_SOURCES]
    with _cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = [ex.submit(_compile, s, o, verbose) for s, o in work]
        for f in futs:
            f.result()
    core = LIB_DIR / "libruntherder_attn.so"
    kernel_objs = [str(o) for _, o in work[: len(KERNEL_SOURCES)]]
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(core), *kernel_objs],
         verbose)
    cpp = LIB_DIR / "libruntherder_attn_cpp.so"
    host_objs = [str(o) for _, o in work[len(KERNEL_SOURCES):]]
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(cpp), *host_objs,
          f"-L{LIB_DIR}", "-lruntherder_attn", "-Wl,-rpath,$ORIGIN"], verbose)
    return {"core": core, "cpp": cpp}


def build_oracle(verbose: bool = False) -> Path:
    """Compile the CPU oracle (test infrastructure) with its Makefile."""
    _run(["make", "-s", "-C", str(ROOT / "oracle")], verbose)
    return ROOT / "oracle" / "librth_oracle.so"


def build_cpp_tests(verbose: bool = False) -> Path:
    """Compile the C++ drop-in test driver against the C++ layer."""
    out_dir = ROOT / "tests" / "cpp" / "bin"
    out_dir.mkdir(parents=True, exist_ok=True)
    exe = out_dir / "test_backend"
    _run([HIPCC, *DEVICE_FLAGS, "-x", "hip", str(ROOT / "tests" / "cpp" / "test_backend.cpp"),
          f"-I{ROOT / 'oracle'}", "-o", str(exe), f"-L{LIB_DIR}", "-lruntherder_attn_cpp",
          "-lruntherder_attn", f"-L{ROOT / 'oracle'}", "-lrth_oracle",
          f"-Wl,-rpath,{LIB_DIR}", f"-Wl,-rpath,{ROOT / 'oracle'}",
          "-Wl,-rpath,$ORIGIN/../../../runtherder_amd/lib",
          "-Wl,-rpath,$ORIGIN/../../../oracle"], verbose)
    return exe


if __name__ == "__main__":
    v = "-v" in sys.argv
    libs = build(verbose=v)
    print({k: str(p) for k, p in libs.items()})
