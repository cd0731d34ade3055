"""CPU restatement of ferrograd's fused-training-path math (ctypes wrapper).

TEST INFRASTRUCTURE ONLY.  This package is the parity checker and the timed
CPU baseline.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg import it; the product (``ferrograd_amd``) never does.

The C sources (``fg_oracle.c``) cite the reference file:line each function
restates.  ``build()`` compiles ``libfg_oracle.so`` in place with the
committed Makefile.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfg_oracle.so")

NN, NT, TN = 0, 1, 2
F32, F16, BF16 = 0, 1, 2
ACT_NONE, ACT_RELU, ACT_GELU = 0, 1, 2

_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")


def build() -> str:
    """Compile the oracle library with its Makefile (gcc + OpenMP)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    c_int, c_float, c_double, c_i64 = ctypes.c_int, ctypes.c_float, ctypes.c_double, ctypes.c_int64
    vp = ctypes.c_void_p
    lib.fgo_gemm.argtypes = [c_int, c_int, c_int, c_int, vp, c_int, vp, c_int, vp, c_int]
    lib.fgo_gemm.restype = None
    lib.fgo_bias_act.argtypes = [c_int, c_int, vp, c_int, vp, c_int, vp, vp]
    lib.fgo_bias_act.restype = None
    lib.fgo_act.argtypes = [c_int, c_float]
    lib.fgo_act.restype = c_float
    lib.fgo_act_grad.argtypes = [c_int, c_float]
    lib.fgo_act_grad.restype = c_float
    lib.fgo_act_bwd.argtypes = [c_int, c_i64, vp, vp, vp]
    lib.fgo_act_bwd.restype = None
    lib.fgo_bias_grad.argtypes = [c_int, c_int, vp, c_int, vp]
    lib.fgo_bias_grad.restype = None
    lib.fgo_softmax_ce.argtypes = [c_int, c_int, vp, c_int, vp, c_float, vp, vp, c_int, vp]
    lib.fgo_softmax_ce.restype = c_double
    lib.fgo_softmax.argtypes = [c_int, c_int, vp, vp]
    lib.fgo_softmax.restype = None
    lib.fgo_softmax_bwd.argtypes = [c_int, c_int, vp, vp, vp]
    lib.fgo_softmax_bwd.restype = None
    lib.fgo_sgd.argtypes = [c_i64, vp, vp, c_float, c_int]
    lib.fgo_sgd.restype = None
    lib.fgo_adam_scalars.argtypes = [c_double, c_double, c_double, c_int,
                                     ctypes.POINTER(c_float), ctypes.POINTER(c_float)]
    lib.fgo_adam_scalars.restype = None
    lib.fgo_adam.argtypes = [c_i64, vp, vp, vp, vp, c_float, c_float, c_float, c_float, c_float]
    lib.fgo_adam.restype = None
    lib.fgo_f32_to_f16.argtypes = [c_float]
    lib.fgo_f32_to_f16.restype = ctypes.c_uint16
    lib.fgo_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.fgo_f16_to_f32.restype = c_float
    lib.fgo_f32_to_bf16.argtypes = [c_float]
    lib.fgo_f32_to_bf16.restype = ctypes.c_uint16
    lib.fgo_bf16_to_f32.argtypes = [ctypes.c_uint16]
    lib.fgo_bf16_to_f32.restype = c_float
    lib.fgo_to_f32.argtypes = [c_int, c_i64, vp, vp]
    lib.fgo_to_f32.restype = None
    lib.fgo_from_f32.argtypes = [c_int, c_i64, vp, vp]
    lib.fgo_from_f32.restype = None
    lib.fgo_gemm_x16.argtypes = [c_int, c_int, c_int, c_int, c_int, vp, c_int, vp, c_int, vp,
                                 c_int, vp, c_int, vp, c_int, c_int]
    lib.fgo_gemm_x16.restype = None
    lib.fgo_gemm_bwd_x16.argtypes = [c_int, c_int, c_int, c_int, c_int, vp, c_int, vp, c_int,
                                     c_int, vp, c_int, vp, c_int, c_int]
    lib.fgo_gemm_bwd_x16.restype = None
    lib.fgo_num_threads.argtypes = []
    lib.fgo_num_threads.restype = c_int
    lib.fgo_set_num_threads.argtypes = [c_int]
    lib.fgo_set_num_threads.restype = None
    _lib = lib
    return lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def num_threads() -> int:
    return _load().fgo_num_threads()


def set_num_threads(n: int) -> None:
    _load().fgo_set_num_threads(int(n))


def gemm(layout: int, A, B) -> np.ndarray:
    """C = op(A).op(B) with layout NN (A[M,K], B[K,N]), NT (B given [N,K]) or
    TN (A given [K,M])."""
    A, B = _c32(A), _c32(B)
    if layout == NN:
        M, K = A.shape
        N = B.shape[1]
        assert B.shape[0] == K
    elif layout == NT:
        M, K = A.shape
        N = B.shape[0]
        assert B.shape[1] == K
    elif layout == TN:
        K, M = A.shape
        N = B.shape[1]
        assert B.shape[0] == K
    else:
        raise ValueError(layout)
    C = np.empty((M, N), dtype=np.float32)
    _load().fgo_gemm(layout, M, N, K, _p(A), A.shape[1], _p(B), B.shape[1], _p(C), N)
    return C


def bias_act(C, bias, act: int):
    """Returns (Z, H) with Z = C + bias (row broadcast), H = act(Z)."""
    C = _c32(C)
    M, N = C.shape
    b = None if bias is None else _c32(bias)
    Z = np.empty_like(C)
    H = np.empty_like(C)
    _load().fgo_bias_act(M, N, _p(C), N, _p(b), act, _p(Z), _p(H))
    return Z, H


def act(act_kind: int, z) -> np.ndarray:
    z = _c32(z)
    Z, H = bias_act(z.reshape(1, -1), None, act_kind)
    return H.reshape(z.shape)


def act_grad_scalar(act_kind: int, z: float) -> float:
    return float(_load().fgo_act_grad(act_kind, float(z)))


def act_bwd(act_kind: int, dH, Z) -> np.ndarray:
    dH, Z = _c32(dH), _c32(Z)
    out = np.empty_like(dH)
    _load().fgo_act_bwd(act_kind, dH.size, _p(dH), _p(Z), _p(out))
    return out


def bias_grad(dZ) -> np.ndarray:
    dZ = _c32(dZ)
    M, N = dZ.shape
    out = np.empty(N, dtype=np.float32)
    _load().fgo_bias_grad(M, N, _p(dZ), N, _p(out))
    return out


def softmax_ce(x, labels, grad_scale: float = 1.0, want_grad: bool = True):
    """Returns (row_loss, dlogits or None, argmax, mean_loss)."""
    x = _c32(x)
    R, C = x.shape
    labels = np.ascontiguousarray(labels, dtype=np.uint32)
    row_loss = np.empty(R, dtype=np.float32)
    argmax = np.empty(R, dtype=np.uint32)
    d = np.empty_like(x) if want_grad else None
    mean = _load().fgo_softmax_ce(R, C, _p(x), C, _p(labels), float(grad_scale), _p(row_loss),
                                  _p(d), C, _p(argmax))
    return row_loss, d, argmax, mean


def softmax(x) -> np.ndarray:
    x = _c32(x)
    R, C = x.shape
    y = np.empty_like(x)
    _load().fgo_softmax(R, C, _p(x), _p(y))
    return y


def softmax_bwd(y, dy) -> np.ndarray:
    y, dy = _c32(y), _c32(dy)
    R, C = y.shape
    dx = np.empty_like(y)
    _load().fgo_softmax_bwd(R, C, _p(y), _p(dy), _p(dx))
    return dx


def sgd_(w: np.ndarray, g: np.ndarray, lr: float, zero_grad: bool = True) -> None:
    """In-place SGD on float32 C-contiguous arrays."""
    assert w.dtype == np.float32 and g.dtype == np.float32
    assert w.flags.c_contiguous and g.flags.c_contiguous and w.size == g.size
    _load().fgo_sgd(w.size, _p(w), _p(g), float(lr), int(zero_grad))


def adam_scalars(lr: float, b1: float, b2: float, step: int):
    s = ctypes.c_float()
    r = ctypes.c_float()
    _load().fgo_adam_scalars(float(lr), float(b1), float(b2), int(step), ctypes.byref(s),
                             ctypes.byref(r))
    return s.value, r.value


def adam_(p, g, m, v, b1, b2, eps, step_size, inv_sqrt_bc2) -> None:
    """In-place Adam update of float32 C-contiguous arrays."""
    for a in (p, g, m, v):
        assert a.dtype == np.float32 and a.flags.c_contiguous and a.size == p.size
    _load().fgo_adam(p.size, _p(p), _p(g), _p(m), _p(v), float(b1), float(b2), float(eps),
                     float(step_size), float(inv_sqrt_bc2))


# ------------------------------------------------------ 16-bit storage types
def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


def to_f32(dtype: int, bits) -> np.ndarray:
    """Widen 16-bit words (F16 or BF16) to float32."""
    bits = _u16(bits)
    out = np.empty(bits.shape, dtype=np.float32)
    _load().fgo_to_f32(dtype, bits.size, _p(bits), _p(out))
    return out


def from_f32(dtype: int, x) -> np.ndarray:
    """Round float32 values to 16-bit words (F16 or BF16), nearest even."""
    x = _c32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    _load().fgo_from_f32(dtype, x.size, _p(x), _p(out))
    return out


def _x16_dims(layout, A, B):
    if layout == NN:
        (M, K), N = A.shape, B.shape[1]
    elif layout == NT:
        (M, K), N = A.shape, B.shape[0]
    else:
        (K, M), N = A.shape, B.shape[1]
    return M, N, K


def gemm_x16(dtype: int, layout: int, A, B, bias=None, act: int = ACT_NONE, C=None,
             want_z: bool = False):
    """16-bit GEMM (16-bit word arrays in and out): returns C, or (C, Z).
    With C given, accumulates into a copy of it (act must be NONE)."""
    A, B = _u16(A), _u16(B)
    M, N, K = _x16_dims(layout, A, B)
    acc = C is not None
    out = _u16(C).copy() if acc else np.zeros((M, N), dtype=np.uint16)
    Z = np.zeros((M, N), dtype=np.uint16) if want_z else None
    b = None if bias is None else _u16(bias)
    _load().fgo_gemm_x16(dtype, layout, M, N, K, _p(A), A.shape[1], _p(B), B.shape[1], _p(b),
                         act, _p(out), N, _p(Z), N, int(acc))
    return (out, Z) if want_z else out


def gemm_bwd_x16(dtype: int, layout: int, A, B, act: int = ACT_NONE, Zs=None, C=None):
    """C (=|+=) round(round(op(A).op(B)) * act'(Zs)) on 16-bit words."""
    A, B = _u16(A), _u16(B)
    M, N, K = _x16_dims(layout, A, B)
    acc = C is not None
    out = _u16(C).copy() if acc else np.zeros((M, N), dtype=np.uint16)
    zs = None if Zs is None else _u16(Zs)
    _load().fgo_gemm_bwd_x16(dtype, layout, M, N, K, _p(A), A.shape[1], _p(B), B.shape[1], act,
                             _p(zs), N, _p(out), N, int(acc))
    return out
