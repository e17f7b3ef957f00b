"""Builds the native libraries in-tree.

  lib/libxvram.so          the product: C++20 host runtime + gfx950 HIP kernel,
                           exporting exactly ``xvram_get_api@@XVRAM_0.1`` (the
                           extension table is one more version of it);
  lib/build_info.json      compiler, HIP and source versions of that build;
  lib/libxvram_synth.so    seeded synthetic operands for the benchmark;
  lib/libxvram_hostsim.so  the same host runtime over a host-memory device
                           simulation, for CPU-only tests (never used on the
                           product path).

Run ``python -m xvram_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import json
import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "lib")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

HOST_SOURCES = ["api.cpp", "errors.cpp", "session.cpp", "runtime.cpp", "gemm.cpp", "policy.cpp"]
HIP_SOURCES = ["sgemm_mfma.hip", "sgemm_wide.hip", "sgemm_direct.hip"]
COMMON_FLAGS = ["-std=c++20", "-O2", "-fPIC", "-fvisibility=hidden", "-DXVRAM_BUILDING_LIBRARY",
                f"-I{INCLUDE}", f"-I{CSRC}", "-Wall", "-Wextra", "-Wno-unused-parameter"]
# Packed-FP32 instructions are disabled for every HIP compile.
HIP_FLAGS = ["-std=c++20", "-O3", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature",
             "-Xclang", "-packed-fp32-ops", f"-I{CSRC}", f"-I{INCLUDE}"]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + proc.stdout)
        raise RuntimeError(f"build step failed: {cmd[0]} {cmd[-1]}")
    return proc.stdout


def _compile_host(src, obj, extra):
    _run(["g++", *COMMON_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def _first_line(cmd):
    try:
        out = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                             timeout=60).stdout
        return out.strip().splitlines()[0] if out.strip() else "unknown"
    except (OSError, subprocess.SubprocessError):
        return "unknown"


def build_info() -> dict:
    """Versions recorded next to the libraries (read by reports)."""
    hip_version = 0
    try:
        text = open(os.path.join(ROCM, "include", "hip", "hip_version.h")).read()
        parts = {k: int(v) for k, v in re.findall(r"#define HIP_VERSION_(MAJOR|MINOR|PATCH) (\d+)", text)}
        hip_version = parts["MAJOR"] * 10000000 + parts["MINOR"] * 100000 + parts["PATCH"]
    except (OSError, KeyError):
        pass
    commit = _first_line(["git", "-C", ROOT, "rev-parse", "HEAD"])
    if not re.fullmatch(r"[0-9a-f]{40}", commit):
        commit = "unknown"
    return {"version": "0.1.0", "git_commit": commit, "build_type": "Release",
            "compiler": f"{_first_line([HIPCC, '--version'])}; {_first_line(['g++', '--version'])}",
            "hip_version": hip_version, "offload_arch": ARCH}


def build(hostsim: bool = True, product: bool = True, verbose: bool = True) -> None:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    jobs = []
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as pool:
        if product:
            hip_flags = [f"-I{ROCM}/include", "-D__HIP_PLATFORM_AMD__"]
            for src in HOST_SOURCES + ["device_hip.cpp"]:
                jobs.append(pool.submit(_compile_host, src,
                                        os.path.join(OBJ, "hip_" + src.replace(".cpp", ".o")),
                                        hip_flags))
            for src in HIP_SOURCES:
                jobs.append(pool.submit(_run, [HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src),
                                               "-o", os.path.join(OBJ, src.replace(".hip", ".o"))]))
        if hostsim:
            for src in HOST_SOURCES + ["device_hostsim.cpp"]:
                jobs.append(pool.submit(_compile_host, src,
                                        os.path.join(OBJ, "sim_" + src.replace(".cpp", ".o")),
                                        ["-DXVRAM_HOSTSIM"]))
        for j in jobs:
            j.result()
    if product:
        objs = [os.path.join(OBJ, "hip_" + s.replace(".cpp", ".o"))
                for s in HOST_SOURCES + ["device_hip.cpp"]] + [
                    os.path.join(OBJ, s.replace(".hip", ".o")) for s in HIP_SOURCES]
        out = os.path.join(LIB, "libxvram.so")
        _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", out + ".tmp", *objs,
              f"-Wl,--version-script={os.path.join(CSRC, 'exports.map')}", "-Wl,--no-undefined",
              "-Wl,-soname,libxvram.so",
              f"-L{ROCM}/lib", "-lamdhip64", "-lpthread"])
        os.replace(out + ".tmp", out)
        with open(os.path.join(LIB, "build_info.json"), "w") as f:
            json.dump(build_info(), f, indent=1)
        if verbose:
            print(f"built {out}")
    synth = os.path.join(LIB, "libxvram_synth.so")
    _run(["gcc", "-std=c11", "-O3", "-fopenmp", "-fPIC", "-shared", "-o", synth + ".tmp",
          os.path.join(CSRC, "synth.c"), "-lm"])
    os.replace(synth + ".tmp", synth)
    if hostsim:
        objs = [os.path.join(OBJ, "sim_" + s.replace(".cpp", ".o"))
                for s in HOST_SOURCES + ["device_hostsim.cpp"]]
        out = os.path.join(LIB, "libxvram_hostsim.so")
        _run(["g++", "-shared", "-o", out + ".tmp", *objs,
              f"-Wl,--version-script={os.path.join(CSRC, 'exports_hostsim.map')}",
              "-Wl,--no-undefined", "-lpthread"])
        os.replace(out + ".tmp", out)
        if verbose:
            print(f"built {out}")


if __name__ == "__main__":
    build()
