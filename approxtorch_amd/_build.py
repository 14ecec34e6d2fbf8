"""Builds libatx.so (the HIP kernels + C ABI) in-tree for gfx950.

Every translation unit under csrc/ is compiled by hipcc in parallel and
linked into approxtorch_amd/libatx.so; the measurement probes under diag/
go into a separate approxtorch_amd/libatx_diag.so that only bench.py
--probe-lds loads.  The built libraries travel with the source tree; nothing
is installed elsewhere.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
DIAG = os.path.join(PKG_DIR, "diag")
LIB_PATH = os.path.join(PKG_DIR, "libatx.so")
DIAG_LIB_PATH = os.path.join(PKG_DIR, "libatx_diag.so")
OBJ_DIR = os.path.join(PKG_DIR, "_build")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: every a*b+c in the fake-quant / EMA code stays two
# rounded operations, matching the separate torch ops they restate.
# -packed-fp32-ops: packed fp32 VALU forms are disabled on this platform.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _sources(folder):
    out = []
    for name in sorted(os.listdir(folder)):
        if name.endswith((".hip", ".cpp")):
            out.append(os.path.join(folder, name))
    return out


def _compile(src):
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC] + COMMON_FLAGS + ["-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC, "-O2", "-std=c++17", "-fPIC", "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def _link(objs, path):
    tmp = path + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, path)


def build_library(verbose=False):
    """Compile every source, link libatx.so and libatx_diag.so; returns the
    product library's path."""
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs, diag = _sources(CSRC), _sources(DIAG)
    workers = min(len(srcs) + len(diag), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(_compile, srcs + diag))
    _link(objs[:len(srcs)], LIB_PATH)
    _link(objs[len(srcs):], DIAG_LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources and {DIAG_LIB_PATH}",
              file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build_library(verbose=True)
