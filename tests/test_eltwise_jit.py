"""Compiled elementwise kernels (ferrograd_amd/csrc/fg_elt_jit.h), on the CPU:
hipRTC compiles generated kernel sources for gfx950 without a GPU, with
each compiler the library may get (below).

tests/cpp/elt_jit_check.cpp generates the source of random programs over
every op, element type (fp32 / fp16 / bf16 loads, stores and rounds),
addressing mode (whole tensor, row broadcast, scalar), alignment and quad
count, with a destination that is also a source, and compiles each as the
library does.  The code objects are then read back with llvm-objdump:

* none holds a packed-fp32 VALU instruction (the library builds all device
  code without them);
* the program a*b + c compiles to a separate multiply and add, as the
  interpreter evaluates it (two ops, two roundings), while the same source
  with the op barriers removed compiles to fused multiply-adds -- so the
  check fails if the barrier stops separating ops, and shows that hipRTC
  would otherwise contract across them.

* each unary op compiles to the same arithmetic (opcodes and literal
  constants of its vector instructions) with hipcc -- the interpreter's
  compiler -- and with every compiler behind hipRTC that the library may
  get: ROCm's, and in a PyTorch process the older hipRTC and comgr that
  PyTorch ships and has loaded, which the library's libhiprtc.so.7
  dependency then resolves to.  The ops are written so that no device
  math-library routine enters them: that compiler's build of logf ends
  with an add where hipcc's ends with an fma, a one-ulp difference in a
  third of the results (checked against this test: it fails with logf).

Bit-equality of compiled and interpreted results is checked on the GPU
(tests/test_eltwise_jit_gpu.py)."""
import glob
import importlib.util
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "ferrograd_amd", "csrc")
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"
UNARY = ["relu", "gelu", "elu", "tanh", "exp", "log", "abs", "relu_d", "gelu_d", "elu_d", "sign"]


def _rtc_envs():
    """The compilers behind hipRTC that the library may get: ROCm's, and in
    a PyTorch process the hipRTC and comgr (the compiler itself) that
    PyTorch's HIP runtime has already loaded -- preloaded here to the same
    effect (their sonames match the library's dependencies)."""
    envs = {"rocm": {}}
    spec = importlib.util.find_spec("torch")  # located, not imported
    if spec and spec.origin:
        lib = os.path.join(os.path.dirname(spec.origin), "lib")
        libs = [os.path.join(lib, n) for n in ("libamd_comgr.so", "libhiprtc.so")]
        if all(os.path.exists(x) for x in libs):
            envs["torch"] = {"LD_PRELOAD": ":".join(libs)}
    return envs


def _checker(d):
    exe = str(d / "elt_jit_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", "-I", CSRC,
                    "-I", "/opt/rocm/include", "-D__HIP_PLATFORM_AMD__",
                    os.path.join(ROOT, "tests", "cpp", "elt_jit_check.cpp"), "-o", exe,
                    "-L/opt/rocm/lib", "-lhiprtc", "-Wl,-rpath,/opt/rocm/lib"], check=True)
    return exe


@pytest.fixture(scope="module", params=list(_rtc_envs()))
def objects(tmp_path_factory, request):
    d = tmp_path_factory.mktemp("jit")
    exe = _checker(d)
    r = subprocess.run([exe, CSRC, str(d), "40", "7"], capture_output=True, text=True,
                       timeout=600, env={**os.environ, **_rtc_envs()[request.param]})
    assert r.returncode == 0 and r.stdout.startswith("OK"), r.stdout[-4000:] + r.stderr
    return d


def disasm(path):
    r = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", str(path)], capture_output=True,
                       text=True, check=True)
    return re.findall(r"^\s+(v_[a-z0-9_]+)", r.stdout, re.M)


def test_generated_programs_compile_without_packed_fp32(objects):
    cos = sorted(glob.glob(str(objects / "k*.co")))
    assert len(cos) == 40
    for co in cos:
        ops = disasm(co)
        assert ops, co
        bad = [o for o in ops if re.match(r"v_pk_(add|mul|fma)_f32", o)]
        assert not bad, (co, bad)


def test_op_barrier_keeps_multiply_and_add_apart(objects):
    kept = disasm(objects / "fma_bar.co")
    fused = disasm(objects / "fma_nobar.co")
    fma = re.compile(r"v_(fma|fmac|fmamk|fmaak|mad|mac)_f32")
    assert not [o for o in kept if fma.match(o)], kept
    assert sum(o.startswith("v_mul_f32") for o in kept) == 16   # 4 quads x 4 elements
    assert sum(o.startswith("v_add_f32") for o in kept) == 16
    assert sum(bool(fma.match(o)) for o in fused) == 16, fused


def _arith(lines):
    """Sorted opcodes and literal constants of a kernel's vector instructions."""
    out = []
    for l in lines:
        m = re.match(r"\s+(v_[a-z0-9_]+)(.*)", l)
        if m:
            out.append(m.group(1))
            out += re.findall(r"0x[0-9a-f]+", m.group(2).split("//")[0].split(";")[0])
    return sorted(out)


@pytest.mark.parametrize("rtc", list(_rtc_envs()))
def test_ops_compile_alike_under_hipcc_and_hiprtc(tmp_path, rtc):
    exe = _checker(tmp_path)
    r = subprocess.run([exe, "ops", CSRC, str(tmp_path)], capture_output=True, text=True,
                       timeout=600, env={**os.environ, **_rtc_envs()[rtc]})
    assert r.returncode == 0 and r.stdout.startswith("OK"), r.stdout[-3000:] + r.stderr
    for op in UNARY:
        src = tmp_path / f"k_{op}.hip"
        src.write_text('#include <hip/hip_runtime.h>\n#include "fg_elt_ops.h"\n'
                       'extern "C" __global__ void k(const float *a, float *o) '
                       f'{{ o[threadIdx.x] = fg::elt_{op}(a[threadIdx.x]); }}\n')
        asm = tmp_path / f"k_{op}.s"
        subprocess.run(["/opt/rocm/bin/hipcc", "-O3", "--offload-arch=gfx950", "-Xclang",
                        "-target-feature", "-Xclang", "-packed-fp32-ops", "-I", CSRC,
                        "--cuda-device-only", "-S", str(src), "-o", str(asm)], check=True,
                       capture_output=True)
        aot = _arith(asm.read_text().splitlines())
        jit = _arith(subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950",
                                     str(tmp_path / f"op_{op}.co")], capture_output=True,
                                    text=True, check=True).stdout.splitlines())
        assert aot and aot == jit, (rtc, op)
