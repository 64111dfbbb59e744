"""Builds the native libraries of metalfish_amd in-tree.

* ``libmfhip.so``  -- gfx950 kernels + the C ABI of include/mfhip.h (hipcc),
  with the host-only network-file reader (g++, zlib).
* ``libmfhost.so`` -- seeded nets and chess positions, include/mfh_synth.h (g++).
* ``libmfadapter.so`` / ``hip_network_test`` -- the C++ ``HipNetwork``
  adapter (NN::Network over the C ABI) and its self-test driver.

All HIP code is compiled for gfx950 only, with packed-fp32 instructions
disabled.  The build always recompiles (it is the "does it build" check).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")

HIP_SOURCES = ["hip/gemm.hip", "hip/panel_gemm.hip", "hip/skinny_gemm.hip", "hip/attention.hip", "hip/rowops.hip",
               "hip/policy.hip",
               "hip/mfh_api.cpp", "host/policy_tables.cpp"]
# Host-only parts of libmfhip.so (no device code), compiled with g++.
HIP_HOST_SOURCES = ["host/weights_file.cpp"]
HOST_SOURCES = ["host/chess.cpp", "host/policy_tables.cpp", "host/synth_api.cpp"]

HIPCC_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-Wall", "-Wno-unused-function"]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd, cwd=None):
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                          text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops" not in l)  # host-pass notice, harmless
    if proc.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    return out


def build_hip(jobs=8):
    """Compile each HIP/C++ translation unit to an object, then link."""
    hipcc = _hipcc()
    objdir = os.path.join(PKG, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = []
    procs = []
    for src in HIP_SOURCES:
        obj = os.path.join(objdir, src.replace("/", "_") + ".o")
        objs.append(obj)
        cmd = [hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
        if src.endswith(".cpp"):
            cmd = [hipcc, *HIPCC_FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                            stderr=subprocess.STDOUT, text=True)))
        if len(procs) >= jobs:
            _wait(procs)
            procs = []
    for src in HIP_HOST_SOURCES:
        obj = os.path.join(objdir, src.replace("/", "_") + ".o")
        objs.append(obj)
        cmd = ["g++", "-std=c++17", "-O2", "-fPIC", "-Wall", "-Wextra", "-c",
               os.path.join(CSRC, src), "-o", obj]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                            stderr=subprocess.STDOUT, text=True)))
    _wait(procs)
    out = os.path.join(PKG, "libmfhip.so")
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-lz", "-o",
          out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def _wait(procs):
    for cmd, p in procs:
        text, _ = p.communicate()
        if p.returncode != 0:
            text = "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l)
            raise RuntimeError(f"build failed: {' '.join(cmd)}\n{text}")


def build_host():
    out = os.path.join(PKG, "libmfhost.so")
    srcs = [os.path.join(CSRC, s) for s in HOST_SOURCES]
    _run(["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-fopenmp", "-Wall", "-Wextra",
          *srcs, "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_adapter():
    """C++ NN::Network adapter over the C ABI, plus its self-test driver."""
    src = os.path.join(CSRC, "host", "hip_network.cpp")
    if not os.path.exists(src):
        return None
    inc = ["-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(CSRC, "host")]
    out = os.path.join(PKG, "libmfadapter.so")
    _run(["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", *inc, src,
          "-L" + PKG, "-lmfhip", "-Wl,-rpath,$ORIGIN", "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    test_src = os.path.join(ROOT, "tests", "native", "hip_network_test.cpp")
    if os.path.exists(test_src):
        exe = os.path.join(PKG, "hip_network_test")
        _run(["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", *inc, test_src,
              "-L" + PKG, "-lmfadapter", "-lmfhip", "-lmfhost",
              "-Wl,-rpath,$ORIGIN", "-o", exe + ".tmp"])
        os.replace(exe + ".tmp", exe)
    return out


def build_oracle():
    """The CPU oracle (test infrastructure) and, when the reference tree is
    present, the reference-table dumper in oracle/_ref."""
    _run(["make", "-C", os.path.join(ROOT, "oracle"), "-B", "all"])


def build_all():
    build_host()
    build_hip()
    build_adapter()
    build_oracle()


if __name__ == "__main__":
    build_all()
    print("built", file=sys.stderr)
