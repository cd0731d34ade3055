"""ferrograd_amd -- MI355X (gfx950) backend for ferrograd's fused training path.

The product is the C-ABI library ``libferrograd_hip.so`` (declared in
``include/ferrograd_hip.h``): hand-written HIP kernels for gfx950 and the C++
host runtime around them.  This package is the thin Python face of that ABI:

* ``Context`` / direct-kernel helpers below take device pointers (``int``) or
  any object with ``data_ptr()`` (e.g. a torch tensor used purely as device
  memory);
* ``graph`` mirrors ferrograd's Graph / GpuContext API (build, lower,
  schedule, dispatch_forward / loss / backward / optim) on top of the
  library's planner.

Nothing here computes on the CPU: every call goes to the library, and the
import fails loudly when the library has not been built.
"""
from __future__ import annotations

import ctypes
import weakref
from typing import Optional, Sequence

import numpy as np

from . import _lib
from ._lib import FgError, call, load

NN, NT, TN = 0, 1, 2
ACT_NONE, ACT_RELU, ACT_GELU = 0, 1, 2
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
ELTWISE_INTERPRET, ELTWISE_COMPILE_LARGE, ELTWISE_COMPILE_ALL = 0, 1, 2

__all__ = [
    "NN", "NT", "TN", "ACT_NONE", "ACT_RELU", "ACT_GELU", "FgError", "Context",
    "MultiTensor", "load", "rng_uniform", "rng_normal", "rng_int", "torch_context",
    "eltwise_mode", "eltwise_stats",
]


def _ptr(x) -> Optional[int]:
    """Device address of x: None, an int address, or an object with data_ptr()."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return int(x.data_ptr())


class Context:
    """An fg_ctx bound to ``device`` and a HIP stream.

    ``stream`` is a raw hipStream_t address (e.g. ``torch.cuda.current_stream()
    .cuda_stream``) or None for a private stream."""

    def __init__(self, device: int = 0, stream: Optional[int] = None):
        h = ctypes.c_void_p()
        call("fg_ctx_create", device, stream, ctypes.byref(h))
        self.handle = h
        arch = ctypes.create_string_buffer(64)
        flags = ctypes.c_uint32()
        cus = ctypes.c_int()
        call("fg_ctx_target", h, arch, 64, ctypes.byref(flags), ctypes.byref(cus))
        self.arch = arch.value.decode()
        self.flags = flags.value
        self.cu_count = cus.value
        # Plans and tensor lists made on this context (they keep a pointer to
        # it): closed before it, whatever order the garbage collector picks.
        self._dependents = weakref.WeakSet()

    def adopt(self, obj) -> None:
        """Close `obj` (anything with close()) before this context closes."""
        self._dependents.add(obj)

    @property
    def stream(self) -> int:
        s = ctypes.c_void_p()
        call("fg_ctx_stream", self.handle, ctypes.byref(s))
        return int(s.value or 0)

    def sync(self) -> None:
        call("fg_sync", self.handle)

    def is_ready(self) -> bool:
        r = ctypes.c_int()
        call("fg_is_ready", self.handle, ctypes.byref(r))
        return bool(r.value)

    def reserve_workspace(self, nbytes: int) -> None:
        call("fg_ctx_reserve_workspace", self.handle, nbytes)

    def close(self) -> None:
        if self.handle:
            for d in list(getattr(self, "_dependents", ())):
                d.close()
            call("fg_ctx_destroy", self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------ direct kernels
    def gemm(self, layout: int, M: int, N: int, K: int, A, lda: int, B, ldb: int, C, ldc: int,
             bias=None, act: int = ACT_NONE, Z=None, ldz: int = 0,
             accumulate: bool = False) -> None:
        call("fg_gemm_f32", self.handle, layout, M, N, K, _ptr(A), lda, _ptr(B), ldb, _ptr(bias),
             act, _ptr(C), ldc, _ptr(Z), ldz, int(accumulate))

    def gemm_bwd(self, layout: int, M: int, N: int, K: int, A, lda: int, B, ldb: int, C,
                 ldc: int, act: int = ACT_NONE, Zs=None, ldzs: int = 0,
                 accumulate: bool = False) -> None:
        call("fg_gemm_bwd_f32", self.handle, layout, M, N, K, _ptr(A), lda, _ptr(B), ldb, act,
             _ptr(Zs), ldzs, _ptr(C), ldc, int(accumulate))

    def gemm_dw(self, M: int, N: int, K: int, A, lda: int, B, ldb: int, C, ldc: int,
                accumulate: bool = False, colsum=None, colsum_accumulate: bool = False) -> None:
        """C (=|+=) A^T.B and colsum (=|+=) column sums of B in one launch."""
        call("fg_gemm_dw_f32", self.handle, M, N, K, _ptr(A), lda, _ptr(B), ldb, _ptr(C), ldc,
             int(accumulate), _ptr(colsum), int(colsum_accumulate))

    def linear_bwd(self, act: int, M: int, N: int, K: int, X, ldx: int, W, ldw: int, Zs,
                   ldzs: int, dC, lddc: int, dX=None, lddx: int = 0, dW=None, lddw: int = 0,
                   dbias=None, accumulate: bool = False, dZ=None, lddz: int = 0) -> None:
        """Backward of C = act(X.W + bias): dZ = dC * act'(Zs), dX = dZ.W^T,
        dW = X^T.dZ, dbias = colsum(dZ) (any output may be None).  With a dZ
        buffer, dZ is materialised by one pass; without, act' is applied to
        the dC tiles as the GEMMs load them."""
        call("fg_linear_bwd_f32", self.handle, act, M, N, K, _ptr(X), ldx, _ptr(W), ldw,
             _ptr(Zs), ldzs, _ptr(dC), lddc, _ptr(dX), lddx or K, _ptr(dW), lddw or N,
             _ptr(dbias), int(accumulate), _ptr(dZ), lddz or N)

    def matmul_bwd(self, M: int, N: int, K: int, X, ldx: int, W, ldw: int, dZ, lddz: int, dX,
                   lddx: int, dW, lddw: int, dbias=None, act: int = ACT_NONE, Zs=None,
                   ldzs: int = 0, accumulate: bool = False) -> None:
        """A matmul node's gradients from dZ: dW = X^T.dZ (+ dbias = colsum(dZ))
        and dX = (dZ.W^T) * act'(Zs), in one launch when their kernels pair."""
        call("fg_matmul_bwd_f32", self.handle, M, N, K, _ptr(X), ldx, _ptr(W), ldw, _ptr(dZ),
             lddz, act, _ptr(Zs), ldzs, _ptr(dX), lddx, _ptr(dW), lddw, _ptr(dbias),
             int(accumulate))

    def matmul_bwd_x16(self, dtype: int, M: int, N: int, K: int, X, ldx: int, W, ldw: int, dZ,
                       lddz: int, dX, lddx: int, dW, lddw: int, dbias=None, act: int = ACT_NONE,
                       Zs=None, ldzs: int = 0, accumulate: bool = False) -> None:
        """matmul_bwd with 16-bit tensors (dtype DTYPE_F16 / DTYPE_BF16)."""
        call("fg_matmul_bwd_x16", self.handle, dtype, M, N, K, _ptr(X), ldx, _ptr(W), ldw,
             _ptr(dZ), lddz, act, _ptr(Zs), ldzs, _ptr(dX), lddx, _ptr(dW), lddw, _ptr(dbias),
             int(accumulate))

    def gemm_dw_x16(self, dtype: int, M: int, N: int, K: int, A, lda: int, B, ldb: int, C,
                    ldc: int, accumulate: bool = False, colsum=None,
                    colsum_accumulate: bool = False) -> None:
        """16-bit C (=|+=) A^T.B and colsum (=|+=) column sums of B in one launch."""
        call("fg_gemm_dw_x16", self.handle, dtype, M, N, K, _ptr(A), lda, _ptr(B), ldb, _ptr(C),
             ldc, int(accumulate), _ptr(colsum), int(colsum_accumulate))

    def gemm_x16(self, dtype: int, layout: int, M: int, N: int, K: int, A, lda: int, B,
                 ldb: int, C, ldc: int, bias=None, act: int = ACT_NONE, Z=None, ldz: int = 0,
                 accumulate: bool = False) -> None:
        """16-bit GEMM (dtype DTYPE_F16 / DTYPE_BF16 for every operand)."""
        call("fg_gemm_x16", self.handle, dtype, layout, M, N, K, _ptr(A), lda, _ptr(B), ldb,
             _ptr(bias), act, _ptr(C), ldc, _ptr(Z), ldz, int(accumulate))

    def gemm_bwd_x16(self, dtype: int, layout: int, M: int, N: int, K: int, A, lda: int, B,
                     ldb: int, C, ldc: int, act: int = ACT_NONE, Zs=None, ldzs: int = 0,
                     accumulate: bool = False) -> None:
        call("fg_gemm_bwd_x16", self.handle, dtype, layout, M, N, K, _ptr(A), lda, _ptr(B),
             ldb, act, _ptr(Zs), ldzs, _ptr(C), ldc, int(accumulate))

    def bias_grad(self, M: int, N: int, dZ, ld: int, dbias, accumulate: bool = False,
                  dtype: int = DTYPE_F32) -> None:
        call("fg_bias_grad", self.handle, dtype, M, N, _ptr(dZ), ld, _ptr(dbias),
             int(accumulate))

    def act_bwd(self, act: int, n: int, dH, Z, dZ) -> None:
        call("fg_act_bwd_f32", self.handle, act, n, _ptr(dH), _ptr(Z), _ptr(dZ))

    def softmax_ce(self, logits, ldx: int, labels, R: int, C: int, grad_scale: float = 1.0,
                   row_loss=None, mean_loss=None, dlogits=None, ldd: int = 0,
                   argmax=None, dtype: int = DTYPE_F32) -> None:
        call("fg_softmax_ce", self.handle, dtype, _ptr(logits), ldx, _ptr(labels), R, C,
             grad_scale, _ptr(row_loss), _ptr(mean_loss), _ptr(dlogits), ldd or C, _ptr(argmax))

    def softmax(self, x, R: int, C: int, y, dtype: int = DTYPE_F32) -> None:
        call("fg_softmax", self.handle, dtype, _ptr(x), R, C, _ptr(y))

    def softmax_bwd(self, y, dy, R: int, C: int, dx, accumulate: bool = False,
                    dtype: int = DTYPE_F32) -> None:
        call("fg_softmax_bwd", self.handle, dtype, _ptr(y), _ptr(dy), R, C, _ptr(dx),
             int(accumulate))

    def fill_u32(self, dst, value: int, count: int) -> None:
        call("fg_fill_u32", self.handle, _ptr(dst), value, count)

    def rng_uniform(self, seed, tensor_id, lo, hi, dst, n) -> None:
        call("fg_rng_uniform_dev", self.handle, seed, tensor_id, lo, hi, _ptr(dst), n)

    def rng_normal(self, seed, tensor_id, mean, std, dst, n) -> None:
        call("fg_rng_normal_dev", self.handle, seed, tensor_id, mean, std, _ptr(dst), n)

    def rng_int(self, seed, tensor_id, bound, dst, n) -> None:
        call("fg_rng_int_dev", self.handle, seed, tensor_id, bound, _ptr(dst), n)


def torch_context(device: int = 0):
    """A Context sharing a fresh default-priority torch stream, made current.

    torch's default stream has the handle 0, which fg_ctx_create reads as
    "create a private stream"; binding an explicit stream instead keeps
    torch ops (allocation, copies, events) and library launches in one
    ordered queue.  Returns (context, torch stream)."""
    import torch

    torch.cuda.init()
    s = torch.cuda.Stream(device)
    torch.cuda.set_stream(s)
    return Context(device, s.cuda_stream), s


class MultiTensor:
    """A device-resident tensor list for the one-launch SGD / Adam updates."""

    def __init__(self, ctx: Context, params: Sequence, grads: Sequence,
                 m: Optional[Sequence] = None, v: Optional[Sequence] = None,
                 sizes: Optional[Sequence[int]] = None, dtypes: Optional[Sequence[int]] = None):
        """dtypes: element type per tensor (DTYPE_*) of params / grads; m and
        v are always fp32."""
        n = len(params)
        if sizes is None:
            sizes = [int(p.numel()) for p in params]
        arr = ctypes.c_void_p * n
        P = arr(*[_ptr(p) for p in params])
        G = arr(*[_ptr(g) for g in grads])
        Mv = arr(*[_ptr(x) for x in m]) if m is not None else None
        Vv = arr(*[_ptr(x) for x in v]) if v is not None else None
        S = (ctypes.c_uint64 * n)(*sizes)
        h = ctypes.c_void_p()
        D = (ctypes.c_int * n)(*dtypes) if dtypes is not None else None
        call("fg_mt_create_x", ctx.handle, n, D, P, G, Mv, Vv, S, ctypes.byref(h))
        self.ctx = ctx
        self.handle = h
        ctx.adopt(self)

    def sgd(self, lr: float, zero_grad: bool = True) -> None:
        call("fg_sgd_step", self.ctx.handle, self.handle, lr, int(zero_grad))

    def adam(self, lr: float, b1: float, b2: float, eps: float, step: int,
             zero_grad: bool = False) -> None:
        call("fg_adam_step", self.ctx.handle, self.handle, lr, b1, b2, eps, step, int(zero_grad))

    def adam_scalars(self, b1: float, b2: float, eps: float, step_size: float,
                     inv_sqrt_bc2: float, zero_grad: bool = False) -> None:
        call("fg_adam_step_scalars", self.ctx.handle, self.handle, b1, b2, eps, step_size,
             inv_sqrt_bc2, int(zero_grad))

    def close(self) -> None:
        if self.handle:
            call("fg_mt_destroy", self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------------ synthetic data
def rng_uniform(seed: int, tensor_id: int, shape, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    call("fg_rng_uniform_host", seed, tensor_id, lo, hi, out.ctypes.data, out.size)
    return out


def rng_normal(seed: int, tensor_id: int, shape, mean: float = 0.0,
               std: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    call("fg_rng_normal_host", seed, tensor_id, mean, std, out.ctypes.data, out.size)
    return out


def rng_int(seed: int, tensor_id: int, shape, bound: int) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint32)
    call("fg_rng_int_host", seed, tensor_id, bound, out.ctypes.data, out.size)
    return out


# ------------------------------------------------ compiled elementwise kernels
def eltwise_mode(mode: int) -> int:
    """Sets how plans run elementwise programs (ELTWISE_INTERPRET,
    ELTWISE_COMPILE_LARGE -- the default -- or ELTWISE_COMPILE_ALL), process-wide;
    returns the previous mode."""
    prev = ctypes.c_int32(0)
    call("fg_eltwise_set_mode", mode, ctypes.byref(prev))
    return prev.value


def eltwise_stats() -> dict:
    """Process-wide counts: kernels compiled, launches of compiled kernels,
    launches of the interpreter."""
    c, j, i = ctypes.c_uint64(0), ctypes.c_uint64(0), ctypes.c_uint64(0)
    call("fg_eltwise_stats", ctypes.byref(c), ctypes.byref(j), ctypes.byref(i))
    return {"compiled": c.value, "compiled_launches": j.value, "interpreted_launches": i.value}
