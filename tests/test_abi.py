"""CPU checks of the C-ABI library: it loads, exports exactly what
include/ferrograd_hip.h declares, and its host-only code paths (argument
validation, the synthetic-data generator) behave.  No GPU work is issued."""
import ctypes
import os
import re

import numpy as np
import pytest

import ferrograd_amd as fa
from ferrograd_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(fg_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = header_functions()
    assert declared, "no declarations parsed"
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # The Python binding covers exactly the declared surface.
    assert declared == set(_lib.SIGNATURES), (
        declared ^ set(_lib.SIGNATURES))


@pytest.mark.parametrize("lang,compiler", [("c", "gcc"), ("c++", "g++")])
def test_headers_compile_standalone(lang, compiler, tmp_path):
    """Every public header is valid C and C++ on its own (a library built
    before a header edit would hide a broken declaration from the symbol
    check above)."""
    import shutil
    import subprocess
    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} not installed")
    for fn in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not fn.endswith(".h"):
            continue
        r = subprocess.run([compiler, "-fsyntax-only", "-Wall", "-Werror", "-x", lang,
                            os.path.join(ROOT, "include", fn)],
                           capture_output=True, text=True, cwd=tmp_path)
        assert r.returncode == 0, f"{fn} ({lang}):\n{r.stderr}"


def test_version_and_error_message():
    lib = _lib.load()
    assert lib.fg_version() >= 100
    rc = lib.fg_sync(None)
    assert rc == 1  # FG_ERR_INVALID_ARGUMENT
    assert b"ctx is NULL" in lib.fg_last_error_msg()
    with pytest.raises(fa.FgError) as e:
        _lib.call("fg_upload", None, None, None, 4, 0)
    assert e.value.code == 1


def test_host_rng_is_deterministic_and_keyed():
    a = fa.rng_normal(4, 7, (1000,))
    b = fa.rng_normal(4, 7, (1000,))
    c = fa.rng_normal(4, 8, (1000,))
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    # Counter-based: a prefix of a longer fill is the shorter fill.
    assert np.array_equal(fa.rng_normal(4, 7, (300000,))[:1000], a)


def test_host_rng_distributions():
    u = fa.rng_uniform(0, 1, (1 << 20,))
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 2e-3 and abs(u.var() - 1 / 12) < 2e-3
    n = fa.rng_normal(1, 2, (1 << 20,), 0.0, 2.0).astype(np.float64)
    assert abs(n.mean()) < 1e-2 and abs(n.std() - 2.0) < 1e-2
    k = fa.rng_int(2, 3, (1 << 20,), 1000)
    assert k.min() == 0 and k.max() == 999
    counts = np.bincount(k, minlength=1000)
    assert counts.min() > 800 and counts.max() < 1300
    # Uniform lo/hi mapping (Kaiming-uniform bounds).
    w = fa.rng_uniform(0, 5, (4096,), -0.5, 0.5)
    assert w.min() >= -0.5 and w.max() < 0.5


@pytest.mark.parametrize("fn", ["fg_matmul_bwd_f32", "fg_matmul_bwd_x16"])
def test_matmul_bwd_rejects_null_context(fn):
    """A matmul node's gradient entry points check their context before
    anything else: INVALID_ARGUMENT and a message, no device touched."""
    args = [None, 64, 32, 16, None, 16, None, 32, None, 32, 0, None, 0, None, 16, None, 32,
            None, 0]
    if fn.endswith("x16"):
        args.insert(1, 2)  # dtype bf16
    with pytest.raises(fa.FgError) as e:
        _lib.call(fn, *args)
    assert e.value.code == 1 and "ctx is NULL" in str(e.value)


def test_context_without_gpu_reports_no_device():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(fa.FgError) as e:
        fa.Context(0)
    assert e.value.code in (8, 4)


def test_rust_ffi_crate_declares_every_function():
    """crates/ferrograd-hip-sys (unbuilt here: no Rust toolchain) declares
    each function of include/ferrograd_hip.h with the same parameter names in
    the same order, and nothing else."""
    hdr = open(os.path.join(ROOT, "include", "ferrograd_hip.h")).read()
    hdr = re.sub(r"/\*.*?\*/", "", hdr, flags=re.S)
    c_decl = {}
    for m in re.finditer(r"\b(fg_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", hdr):
        args = [a.strip() for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        c_decl[m.group(1)] = [re.findall(r"[A-Za-z_][A-Za-z_0-9]*$", a)[0] for a in args]
    rs = open(os.path.join(ROOT, "crates", "ferrograd-hip-sys", "src", "lib.rs")).read()
    r_decl = {}
    for m in re.finditer(r"pub fn (fg_[a-z0-9_]+)\(([^)]*)\)", rs, re.S):
        args = [a.strip() for a in m.group(2).split(",") if a.strip()]
        r_decl[m.group(1)] = [a.split(":")[0].strip() for a in args]
    assert set(c_decl) == set(r_decl), set(c_decl) ^ set(r_decl)
    for name, params in c_decl.items():
        assert r_decl[name] == params, name
