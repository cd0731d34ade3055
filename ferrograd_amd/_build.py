"""Ahead-of-time build of the gfx950 backend library.

Compiles every source under ``ferrograd_amd/csrc`` with hipcc for gfx950 and
links ``ferrograd_amd/libferrograd_hip.so`` in-tree, so the library travels
with the source tree.  ``python -m ferrograd_amd._build`` runs it.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_obj")
LIB = os.path.join(HERE, "libferrograd_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = [
    "fg_runtime.cpp",
    "k_elementwise.hip",
    "k_optim.hip",
    "k_softmax.hip",
    "k_gemm.hip",
    "k_gemm_nn.hip",
    "k_gemm_nt.hip",
    "k_gemm_tn.hip",
    "k_gemm_nt_pro.hip",
    "k_gemm_tn_pro.hip",
    "k_gemm_skinny.hip",
    "k_gemm_pair.hip",
    "k_gemm16.hip",
    "k_gemm16_bf16.hip",
    "k_gemm16_f16.hip",
    "k_eltwise_prog.hip",
    "k_noalloc.hip",
    "fg_graph.cpp",
    "fg_bpat.cpp",
    "fg_telemetry.cpp",
    "fg_elt_jit.cpp",
]

# Device headers that kernels compiled at run time include (fg_elt_jit.cpp):
# their text goes into the library, written into the build folder as
# fg_jit_headers.inc before the compile.
JIT_HEADERS = ["fg_half.h", "fg_act.h", "fg_elt_ops.h"]

# Packed-fp32 VALU instructions are disabled for all device code: some of
# their forms have produced silent wrong results on the target machines.
COMMON = [
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
]
DEVICE = [
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-source flags.  The optimiser kernels must round every fp32 operation
# where it is written (bit-exact with the CPU restatement): no contraction
# of a*b+c into fma -- HIP's __fmul_rn is a plain, contractable multiply.
EXTRA = {
    "k_optim.hip": ["-ffp-contract=off"],
}


def _compile(src: str, obj_dir: str = OBJ, defines=()) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMMON, *DEVICE, *EXTRA.get(src, []), *[f"-D{d}" for d in defines],
           f"-I{obj_dir}"]
    if src.endswith(".hip"):
        cmd += ["-x", "hip"]
    cmd += ["-c", path, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    if res.stderr.strip():
        # Keep warnings visible (the packed-fp32 feature warning of the host
        # pass is expected and filtered).
        lines = [l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l]
        if any(l.strip() for l in lines):
            sys.stderr.write("\n".join(lines) + "\n")
    return obj


def write_jit_headers(obj_dir: str) -> str:
    """fg_jit_headers.inc: {name, text} of each JIT_HEADERS file, as raw
    string literals."""
    out = ["struct FgJitHeader { const char *name; const char *text; };",
           "static const FgJitHeader kJitHeaders[] = {"]
    for name in JIT_HEADERS:
        text = open(os.path.join(CSRC, name)).read()
        if ")FGJITH\"" in text:
            raise RuntimeError(f"{name} holds the raw-string delimiter")
        out.append(f'    {{"{name}", R"FGJITH({text})FGJITH"}},')
    out.append("};")
    path = os.path.join(obj_dir, "fg_jit_headers.inc")
    tmp = path + ".tmp"
    with open(tmp, "w") as f:
        f.write("\n".join(out) + "\n")
    os.replace(tmp, path)
    return path


def build(verbose: bool = True, lib: str = LIB, obj_dir: str = OBJ, defines=()) -> str:
    """Compile all sources and link the shared library; returns its path.
    `defines` (e.g. ["FG_GEMM_BK=32"]) builds a tuning variant into `lib`."""
    os.makedirs(obj_dir, exist_ok=True)
    write_jit_headers(obj_dir)
    jobs = min(len(SOURCES), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda s: _compile(s, obj_dir, defines), SOURCES))
    tmp = lib + ".tmp"
    # -z defs: an undefined symbol (e.g. a kernel launch stub that a
    # compilation pass failed to emit) fails the link, not the first load.
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", "-Wl,-z,defs", "-o", tmp, *objs,
           "-L/opt/rocm/lib", "-lhiprtc", "-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    return lib


ROOF_SRC = os.path.join(CSRC, "probe", "k_hbm_roof.hip")
ROOF_LIB = os.path.join(HERE, "libfg_hbm_roof.so")


def build_roof(verbose: bool = True) -> str:
    """The measurement kernels of bench.py's HBM-roof mode (their own
    library; the product never loads it)."""
    tmp = ROOF_LIB + ".tmp"
    cmd = [HIPCC, *COMMON, *DEVICE, "-shared", "-x", "hip", ROOF_SRC, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {ROOF_SRC}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, ROOF_LIB)
    if verbose:
        print(f"built {ROOF_LIB}")
    return ROOF_LIB


if __name__ == "__main__":
    build()
    build_roof()
