"""bpat tensor files: the mirror of ``fused_gpu::io``
(crates/fused_gpu/src/io/mod.rs:20-196) over the C ABI.

``save_tensors(path, ctx, tensors, header)`` and ``load_tensors(path, ctx)``
keep the reference's names and argument meaning; ``BpatFile`` exposes the
parsed file (shapes, host values, upload into existing device memory) and
``save_checkpoint`` / ``load_checkpoint`` store a plan's inputs and
optimiser state.
"""
from __future__ import annotations

import ctypes
import os
from typing import List, Sequence

import numpy as np

from ._lib import FgError, call


class BpatHeader:
    """BpatHeader (io/mod.rs:20-54), in declaration order."""
    BpatV0 = 0
    BpatV1 = 1
    BpatV1M = 2
    BpatV2f16 = 3
    BpatV2bf16 = 4
    BpatV2f32 = 5


_HOST_DTYPE = {0: np.float32, 1: np.float16, 2: np.uint16}
# Element type (FG_DTYPE_*) a loaded tensor gets on the device per header:
# fp64 files load as fp32 (the device kernels have no fp64 path).
_LOAD_DTYPE = {0: 0, 1: 0, 2: 0, 3: 1, 4: 2, 5: 0}


class _BpatTensor(ctypes.Structure):
    _fields_ = [("d_ptr", ctypes.c_void_p), ("dtype", ctypes.c_int), ("rank", ctypes.c_int),
                ("shape", ctypes.c_uint32 * 8)]


def _dtype_code(t) -> int:
    dt = getattr(t, "dtype", np.float32)
    try:  # torch dtypes
        import torch

        if isinstance(dt, torch.dtype):
            codes = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
            if dt not in codes:
                raise FgError(1, f"bpat: unsupported tensor element type {dt}")
            return codes[dt]
    except ImportError:
        pass
    dt = np.dtype(dt)
    if dt == np.float16:
        return 1
    if dt == np.uint16:  # bfloat16 words
        return 2
    if dt == np.float32:
        return 0
    raise FgError(1, f"bpat: unsupported tensor element type {dt}")


def _describe(tensors, shapes=None) -> ctypes.Array:
    arr = (_BpatTensor * len(tensors))()
    for i, t in enumerate(tensors):
        shape = tuple(shapes[i]) if shapes is not None else tuple(t.shape)
        if len(shape) > 8:
            raise FgError(1, f"bpat: tensor {i} has rank {len(shape)} (at most 8)")
        ptr = t.data_ptr() if hasattr(t, "data_ptr") else t.ptr
        arr[i].d_ptr = ptr
        arr[i].dtype = _dtype_code(t)
        arr[i].rank = len(shape)
        for d, n in enumerate(shape):
            arr[i].shape[d] = int(n)
    return arr


def save_tensors(path, ctx, tensors: Sequence, header: int = BpatHeader.BpatV2f32,
                 shapes=None) -> None:
    """save_tensors (io/mod.rs:95-123): device tensors (graph.Tensor or
    torch tensors on the device) to a bpat file, converted to the header's
    element type.  Parent directories are created."""
    parent = os.path.dirname(os.fspath(path))
    if parent:
        os.makedirs(parent, exist_ok=True)
    arr = _describe(tensors, shapes)
    handle = getattr(ctx, "ctx", ctx).handle
    call("fg_bpat_save", handle, os.fsencode(path), int(header), len(tensors), arr)


def save_arrays(path, arrays: Sequence[np.ndarray], header: int = BpatHeader.BpatV2f32) -> None:
    """Host arrays (float32, float16, or uint16 bfloat16 words) to a bpat
    file, without a device."""
    arrs = [np.ascontiguousarray(a) for a in arrays]

    class _H:
        def __init__(self, a):
            self.ptr, self.shape, self.dtype = a.ctypes.data, a.shape, a.dtype

    call("fg_bpat_save_host", os.fsencode(path), int(header), len(arrs),
         _describe([_H(a) for a in arrs]))


class BpatFile:
    """A parsed bpat file held in host memory (CRCs of V1 / V1M checked)."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        call("fg_bpat_open", os.fsencode(path), ctypes.byref(h))
        self.handle = h
        hdr, cnt = ctypes.c_int(), ctypes.c_int()
        call("fg_bpat_info", h, ctypes.byref(hdr), ctypes.byref(cnt))
        self.header, self.count = hdr.value, cnt.value

    def shape(self, i: int) -> tuple:
        rank = ctypes.c_int()
        dims = (ctypes.c_uint32 * 8)()
        call("fg_bpat_tensor_info", self.handle, i, ctypes.byref(rank), dims, None)
        return tuple(int(dims[d]) for d in range(rank.value))

    def read_f32(self, i: int) -> np.ndarray:
        out = np.empty(self.shape(i), dtype=np.float32)
        call("fg_bpat_read_f32", self.handle, i, out.ctypes.data)
        return out

    def upload(self, ctx, i: int, dst, dtype: int = 0) -> None:
        """Copy tensor i into device memory dst as element type dtype."""
        ptr = dst.data_ptr() if hasattr(dst, "data_ptr") else int(dst)
        call("fg_bpat_upload", getattr(ctx, "ctx", ctx).handle, self.handle, i, ptr, int(dtype))

    def close(self) -> None:
        if self.handle:
            call("fg_bpat_close", self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass


def load_tensors(path, ctx) -> List:
    """load_tensors (io/mod.rs:125-160): one new device tensor per file
    tensor (graph.Tensor owned by ctx, a graph.GpuContext); fp64 files load
    as fp32, 16-bit files keep their type."""
    from .graph import Tensor, call_ptr

    out = []
    with BpatFile(path) as f:
        dt = _LOAD_DTYPE[f.header]
        for i in range(f.count):
            shape = f.shape(i)
            n = int(np.prod(shape)) if shape else 1
            host = np.zeros(n, dtype=_HOST_DTYPE[dt])
            h = ctypes.c_void_p()
            call("fg_buf_alloc_init", ctx.ctx.handle, host.ctypes.data, host.nbytes,
                 ctypes.byref(h))
            ptr = call_ptr(h)
            t = Tensor(ptr, host.nbytes, shape, _HOST_DTYPE[dt], owner=ctx, buf=h)
            f.upload(ctx, i, ptr, dt)
            out.append(t)
    return out


def save_checkpoint(schedule, path, header: int = BpatHeader.BpatV2f32) -> None:
    """Every input of the schedule's plan, then (Adam) m, v and the step
    count, to a bpat file."""
    parent = os.path.dirname(os.fspath(path))
    if parent:
        os.makedirs(parent, exist_ok=True)
    call("fg_plan_save", schedule.plan.handle, os.fsencode(path), int(header))


def load_checkpoint(schedule, path) -> None:
    """Restore what save_checkpoint wrote into the plan's bound inputs and
    optimiser state (tensor count and sizes are checked)."""
    call("fg_plan_load", schedule.plan.handle, os.fsencode(path))
