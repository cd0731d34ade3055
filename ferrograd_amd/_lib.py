"""ctypes binding of the C ABI in include/ferrograd_hip.h.

The library is built in-tree (``libferrograd_hip.so`` next to this file) by
``ferrograd_amd._build``.  Loading fails loudly when it is missing: there is
no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libferrograd_hip.so")

vp = ctypes.c_void_p
i32 = ctypes.c_int
u32 = ctypes.c_uint32
u64 = ctypes.c_uint64
f32 = ctypes.c_float
sz = ctypes.c_size_t
cp = ctypes.c_char_p
pvp = ctypes.POINTER(ctypes.c_void_p)

# name -> (restype, argtypes); one entry per declaration of the header.
SIGNATURES = {
    "fg_last_error_msg": (cp, []),
    "fg_version": (i32, []),
    "fg_ctx_create": (i32, [i32, vp, pvp]),
    "fg_ctx_destroy": (i32, [vp]),
    "fg_ctx_target": (i32, [vp, cp, sz, ctypes.POINTER(u32), ctypes.POINTER(i32)]),
    "fg_ctx_stream": (i32, [vp, pvp]),
    "fg_ctx_reserve_workspace": (i32, [vp, u64]),
    "fg_sync": (i32, [vp]),
    "fg_is_ready": (i32, [vp, ctypes.POINTER(i32)]),
    "fg_buf_alloc": (i32, [vp, u64, pvp]),
    "fg_buf_alloc_zeroed": (i32, [vp, u64, pvp]),
    "fg_buf_alloc_init": (i32, [vp, vp, u64, pvp]),
    "fg_buf_free": (i32, [vp]),
    "fg_buf_size_bytes": (u64, [vp]),
    "fg_buf_device_ptr": (vp, [vp]),
    "fg_upload": (i32, [vp, vp, vp, u64, u64]),
    "fg_download": (i32, [vp, vp, vp, u64, u64]),
    "fg_copy": (i32, [vp, vp, vp]),
    "fg_fill_u32": (i32, [vp, vp, u32, u64]),
    "fg_gemm_f32": (i32, [vp, i32, i32, i32, i32, vp, i32, vp, i32, vp, i32, vp, i32, vp, i32,
                          i32]),
    "fg_gemm_bwd_f32": (i32, [vp, i32, i32, i32, i32, vp, i32, vp, i32, i32, vp, i32, vp, i32,
                              i32]),
    "fg_bias_grad_f32": (i32, [vp, i32, i32, vp, i32, vp, i32]),
    "fg_gemm_dw_f32": (i32, [vp, i32, i32, i32, vp, i32, vp, i32, vp, i32, i32, vp, i32]),
    "fg_linear_bwd_f32": (i32, [vp, i32, i32, i32, i32, vp, i32, vp, i32, vp, i32, vp, i32, vp,
                                i32, vp, i32, vp, i32, vp, i32]),
    "fg_matmul_bwd_f32": (i32, [vp, i32, i32, i32, vp, i32, vp, i32, vp, i32, i32, vp, i32, vp,
                                i32, vp, i32, vp, i32]),
    "fg_matmul_bwd_x16": (i32, [vp, i32, i32, i32, i32, vp, i32, vp, i32, vp, i32, i32, vp, i32,
                                vp, i32, vp, i32, vp, i32]),
    "fg_gemm_dw_x16": (i32, [vp, i32, i32, i32, i32, vp, i32, vp, i32, vp, i32, i32, vp, i32]),
    "fg_bias_grad": (i32, [vp, i32, i32, i32, vp, i32, vp, i32]),
    "fg_bias_grad_noalloc": (i32, [vp, i32, i32, i32, vp, i32, vp, i32]),
    "fg_softmax_ce": (i32, [vp, i32, vp, i32, vp, i32, i32, f32, vp, vp, vp, i32, vp]),
    "fg_softmax": (i32, [vp, i32, vp, i32, i32, vp]),
    "fg_softmax_bwd": (i32, [vp, i32, vp, vp, i32, i32, vp, i32]),
    "fg_mt_create_x": (i32, [vp, i32, vp, vp, vp, vp, vp, vp, vp]),
    "fg_graph_input_x": (i32, [vp, vp, i32, i32, vp]),
    "fg_graph_constant": (i32, [vp, i32, f32, vp]),
    "fg_plan_tensor_dtype": (i32, [vp, i32, i32, vp]),
    "fg_monitor_start": (i32, [vp, i32, vp]),
    "fg_monitor_stop": (i32, [vp, vp]),
    "fg_monitor_sample": (i32, [vp, i32, vp, vp, vp]),
    "fg_monitor_destroy": (i32, [vp]),
    "fg_plan_save": (i32, [vp, ctypes.c_char_p, i32]),
    "fg_plan_load": (i32, [vp, ctypes.c_char_p]),
    "fg_bpat_save": (i32, [vp, ctypes.c_char_p, i32, i32, vp]),
    "fg_bpat_save_host": (i32, [ctypes.c_char_p, i32, i32, vp]),
    "fg_bpat_open": (i32, [ctypes.c_char_p, vp]),
    "fg_bpat_close": (i32, [vp]),
    "fg_bpat_info": (i32, [vp, vp, vp]),
    "fg_bpat_tensor_info": (i32, [vp, i32, vp, vp, vp]),
    "fg_bpat_read_f32": (i32, [vp, i32, vp]),
    "fg_bpat_upload": (i32, [vp, vp, i32, vp, i32]),
    "fg_gemm_x16": (i32, [vp, i32, i32, i32, i32, i32, vp, i32, vp, i32, vp, i32, vp, i32, vp,
                          i32, i32]),
    "fg_gemm_bwd_x16": (i32, [vp, i32, i32, i32, i32, i32, vp, i32, vp, i32, i32, vp, i32, vp,
                              i32, i32]),
    "fg_act_bwd_f32": (i32, [vp, i32, u64, vp, vp, vp]),
    "fg_softmax_ce_f32": (i32, [vp, vp, i32, vp, i32, i32, f32, vp, vp, vp, i32, vp]),
    "fg_softmax_f32": (i32, [vp, vp, i32, i32, vp]),
    "fg_softmax_bwd_f32": (i32, [vp, vp, vp, i32, i32, vp, i32]),
    "fg_mt_create": (i32, [vp, i32, vp, vp, vp, vp, vp, pvp]),
    "fg_mt_destroy": (i32, [vp]),
    "fg_sgd_step": (i32, [vp, vp, f32, i32]),
    "fg_adam_step": (i32, [vp, vp, f32, f32, f32, f32, i32, i32]),
    "fg_adam_step_scalars": (i32, [vp, vp, f32, f32, f32, f32, f32, i32]),
    "fg_memcpy_h2d": (i32, [vp, vp, vp, u64]),
    "fg_memcpy_d2h": (i32, [vp, vp, vp, u64]),
    "fg_eltwise_set_mode": (i32, [i32, ctypes.POINTER(i32)]),
    "fg_eltwise_stats": (i32, [ctypes.POINTER(u64), ctypes.POINTER(u64), ctypes.POINTER(u64)]),
    "fg_graph_create": (i32, [i32, i32, pvp]),
    "fg_graph_destroy": (i32, [vp]),
    "fg_graph_new_field": (i32, [vp, ctypes.POINTER(u32)]),
    "fg_graph_input": (i32, [vp, vp, i32, ctypes.POINTER(u32)]),
    "fg_graph_constant_f32": (i32, [vp, f32, ctypes.POINTER(u32)]),
    "fg_graph_op": (i32, [vp, i32, vp, i32, ctypes.POINTER(u32)]),
    "fg_graph_set_input_flags": (i32, [vp, u32, u32]),
    "fg_graph_num_nodes": (i32, [vp, ctypes.POINTER(u32)]),
    "fg_graph_validate": (i32, [vp, vp, i32]),
    "fg_plan_create": (i32, [vp, vp, vp, i32, pvp]),
    "fg_plan_destroy": (i32, [vp]),
    "fg_plan_count": (i32, [vp, i32, ctypes.POINTER(i32)]),
    "fg_plan_tensor": (i32, [vp, i32, i32, pvp, ctypes.POINTER(u64), ctypes.POINTER(u32)]),
    "fg_plan_bind_input": (i32, [vp, i32, vp, u64]),
    "fg_plan_bind_target": (i32, [vp, vp, u64]),
    "fg_plan_set_lr": (i32, [vp, f32]),
    "fg_plan_set_adam": (i32, [vp, f32, f32, f32]),
    "fg_plan_forward": (i32, [vp]),
    "fg_plan_loss": (i32, [vp]),
    "fg_plan_backward": (i32, [vp]),
    "fg_plan_optim": (i32, [vp]),
    "fg_plan_single_optim": (i32, [vp, i32]),
    "fg_plan_capture_step": (i32, [vp]),
    "fg_plan_launch_step": (i32, [vp]),
    "fg_plan_describe": (i32, [vp, cp, sz, ctypes.POINTER(sz)]),
    "fg_rng_uniform_host": (i32, [u64, u64, f32, f32, vp, u64]),
    "fg_rng_normal_host": (i32, [u64, u64, f32, f32, vp, u64]),
    "fg_rng_int_host": (i32, [u64, u64, u32, vp, u64]),
    "fg_rng_uniform_dev": (i32, [vp, u64, u64, f32, f32, vp, u64]),
    "fg_rng_normal_dev": (i32, [vp, u64, u64, f32, f32, vp, u64]),
    "fg_rng_int_dev": (i32, [vp, u64, u64, u32, vp, u64]),
}

STATUS_NAMES = {
    0: "OK", 1: "INVALID_ARGUMENT", 2: "OUT_OF_MEMORY", 3: "UNSUPPORTED", 4: "DEVICE",
    5: "SHAPE", 6: "GRAPH", 7: "INTERNAL", 8: "NO_DEVICE", 9: "OUT_OF_BOUNDS",
    10: "SERIALIZATION", 11: "FILE_NOT_FOUND",
}


class FgError(RuntimeError):
    """A non-zero fg_status; ``code`` is the status, the message is the
    library's fg_last_error_msg()."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{STATUS_NAMES.get(code, code)}] {msg}")
        self.code = code


_lib = None


def load():
    """Load the in-tree library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m ferrograd_amd._build` "
            "(there is no fallback implementation)")
    # PyTorch-ROCm ships its own libamdhip64 with the same SONAME.  Loading
    # torch first lets the dynamic linker resolve this library's HIP
    # dependency to that already-loaded copy, so the process has a single HIP
    # runtime (streams and allocations are then shared with torch).
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != 0:
        msg = load().fg_last_error_msg()
        raise FgError(rc, msg.decode() if msg else "")


def call(name: str, *args):
    """Call ``name`` and raise FgError on a non-zero status."""
    check(getattr(load(), name)(*args))
