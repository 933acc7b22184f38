"""Build recipe for the gfx950 HIP library and the host runtime.

* ``arcllm_amd/libarcllm_hip.so``: every source under ``arcllm_amd/csrc``
  compiled with hipcc for gfx950 (the kernels and their C ABI).
* ``arcllm_amd/libarcllm_runtime.so``: the C++17 host layer under
  ``arcllm_amd/host`` (GGUF reader, ``arcllm::v1::runtime::generate``),
  compiled with g++ against the C ABI only.
* ``arcllm_amd/arcllm_runtime``: the command-line front end.
* ``arcllm_amd/arcllm_q4_paths``: the Q4_K ffn_down route / EXEC148
  acquisition path exerciser and timer.

``python -m arcllm_amd.build`` or ``__graft_entry__.build()`` runs it; it
always recompiles.  Libraries and the CLI find each other through
``$ORIGIN`` run paths, so the tree can move as a whole.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libarcllm_hip.so")
HOST = os.path.join(PKG, "host")
RUNTIME_LIB = os.path.join(PKG, "libarcllm_runtime.so")
CLI = os.path.join(PKG, "arcllm_runtime")
Q4_PATHS = os.path.join(PKG, "arcllm_q4_paths")
HOST_SOURCES = ["gguf.cpp", "qwen2_binding.cpp", "runtime.cpp", "inspect.cpp", "registry_v2.cpp", "policy_v4.cpp", "binding_v4.cpp",
                "q4_down_backend.cpp", "registrations/arcllm_v1_q4k_down_reference_registration_v2.cpp"]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra"]
ARCH = "gfx950"

# -packed-fp32-ops: keep v_pk_{add,mul,fma}_f32 out of the generated code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", f"--offload-arch={ARCH}"]

SOURCES = ["arc_runtime.cpp", "arc_synth.cpp", "arc_kernels.hip", "arc_probe.hip", "arc_decode.hip", "arc_prefill.hip",
           "arc_exec148.hip"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *COMMON, *DEVICE_FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (proc.stdout + proc.stderr).splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{out}")
    if out.strip():
        print(out, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("link failed:\n" + proc.stdout + proc.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_host(verbose)
    return LIB


def _run(cmd: list[str], what: str) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"{what} failed:\n" + proc.stdout + proc.stderr)
    if (proc.stdout + proc.stderr).strip():
        print(proc.stdout + proc.stderr, file=sys.stderr)


def build_host(verbose: bool = True) -> None:
    """g++ build of the host runtime library and CLI over libarcllm_hip.so."""
    cxx = shutil.which(os.environ.get("CXX", "g++")) or "g++"
    srcs = [os.path.join(HOST, s) for s in HOST_SOURCES]
    rpath = "-Wl,-rpath,$ORIGIN"
    tmp = RUNTIME_LIB + ".tmp"
    _run([cxx, *HOST_FLAGS, "-shared", "-o", tmp, *srcs, f"-L{PKG}", "-l:libarcllm_hip.so", rpath], "host library")
    os.replace(tmp, RUNTIME_LIB)
    tmp = CLI + ".tmp"
    _run([cxx, *HOST_FLAGS, "-o", tmp, os.path.join(HOST, "cli.cpp"), f"-L{PKG}", "-l:libarcllm_runtime.so",
          "-l:libarcllm_hip.so", rpath], "CLI")
    os.replace(tmp, CLI)
    tmp = Q4_PATHS + ".tmp"
    _run([cxx, *HOST_FLAGS, "-o", tmp, os.path.join(HOST, "q4_paths.cpp"), f"-L{PKG}", "-l:libarcllm_runtime.so",
          "-l:libarcllm_hip.so", rpath], "Q4 path tool")
    os.replace(tmp, Q4_PATHS)
    if verbose:
        print(f"built {RUNTIME_LIB}, {CLI} and {Q4_PATHS}")


if __name__ == "__main__":
    if sys.argv[1:] == ["host"]:
        build_host()
    else:
        build()
