"""Register allocation of elementwise programs (fg::elt_allocate in
ferrograd_amd/csrc/fg_eltwise.h), on the CPU.

The launch code rewrites every program before it runs: whole-tensor loads
that are safe to hoist become registers filled before the program runs, and
registers are reassigned by liveness, so short programs fit a 4- or
8-register file and run over 4 or 2 quads per thread.  tests/cpp/
elt_alloc_check.cpp builds random programs (in-place writes, repeated loads,
row / scalar loads, a destination that is also a source, a misaligned
source), runs each before and after allocation with a scalar interpreter of
the kernel's semantics, and requires the same bits in every destination,
no register at or above the reported count, and (without prefetch) exactly
as many registers as values live at once.  Each of those checks fails when
the allocator frees a register one instruction early, ignores the
destination overlap, or binds a hoisted load to a fresh value instead of
its source's register."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("elt") / "elt_alloc_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror",
                    "-I", os.path.join(ROOT, "ferrograd_amd", "csrc"),
                    os.path.join(ROOT, "tests", "cpp", "elt_alloc_check.cpp"), "-o", exe],
                   check=True)
    return exe


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_allocation_preserves_every_destination(checker, seed):
    r = subprocess.run([checker, "3000", str(seed)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.startswith("OK"), r.stdout + r.stderr
    # The generator must exercise both the prefetch and the small files.
    words = r.stdout.split()
    assert int(words[3]) > 1000 and int(words[7]) > 300, r.stdout
