"""Build the HIP kernels into the in-tree shared library ``lib/libmoe_fp8.so``.

Compiles every ``csrc/*.hip`` for gfx950 with hipcc (one process per file, in
parallel) and links them into one shared object that exports the C ABI
declared in ``include/moe_fp8.h``. Run as ``python -m vllm_neuron_amd._build``.
"""
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
PROJ_DIR = os.path.dirname(PKG_DIR)
CSRC_DIR = os.path.join(PROJ_DIR, "csrc")
REPO_DIR = os.path.dirname(PROJ_DIR)
INCLUDE_DIR = os.path.join(REPO_DIR, "include")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libmoe_fp8.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed fp32 VALU forms are disabled for all device code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
CFLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall",
          "-Wno-unused-command-line-argument", "-I", INCLUDE_DIR, "-I", CSRC_DIR] + DEVICE_FLAGS


def sources():
    return sorted(os.path.join(CSRC_DIR, f) for f in os.listdir(CSRC_DIR) if f.endswith(".hip"))


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    return r.returncode, out


def build(verbose=False):
    """Compile and link; returns the library path. Raises RuntimeError on failure."""
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sources()
    with tempfile.TemporaryDirectory(prefix="moe_fp8_build_") as tmp:
        objs = [os.path.join(tmp, os.path.basename(s)[:-4] + ".o") for s in srcs]
        cmds = [[HIPCC] + CFLAGS + ["-c", s, "-o", o] for s, o in zip(srcs, objs)]
        with ThreadPoolExecutor(max_workers=min(8, len(cmds))) as ex:
            results = list(ex.map(_run, cmds))
        for cmd, (rc, out) in zip(cmds, results):
            if verbose and out.strip():
                print(out)
            if rc != 0:
                raise RuntimeError(f"hipcc failed for {cmd[-3]}:\n{out}")
        tmp_lib = LIB_PATH + ".tmp"
        rc, out = _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", tmp_lib] + objs)
        if rc != 0:
            raise RuntimeError(f"link failed:\n{out}")
        os.replace(tmp_lib, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
