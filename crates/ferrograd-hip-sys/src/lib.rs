//! Raw FFI declarations of `libferrograd_hip.so`, the MI355X (gfx950) backend
//! for ferrograd's fused training path.  One declaration per function of
//! `include/ferrograd_hip.h`, in the same order and with the same parameter
//! names; the header's comments document each call and the reference
//! interface it replaces (ferrograd's `fused_gpu::dispatch::GpuBackend`,
//! crates/fused_gpu/src/dispatch/mod.rs:161-261, and its graph and IO types).
//!
//! Every function returns an `fg_status` (0 = success, otherwise a code that
//! maps one to one onto `fused_gpu::errors::ErrorKind`, see [`FgStatus`]); the
//! message of the last failure on the calling thread is `fg_last_error_msg()`.
#![no_std]
#![allow(non_camel_case_types, non_snake_case)]

use core::ffi::{c_char, c_int, c_void};

/// Opaque handles.
#[repr(C)]
pub struct fg_ctx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct fg_buf {
    _p: [u8; 0],
}
#[repr(C)]
pub struct fg_mt {
    _p: [u8; 0],
}
#[repr(C)]
pub struct fg_monitor {
    _p: [u8; 0],
}
#[repr(C)]
pub struct fg_bpat {
    _p: [u8; 0],
}
#[repr(C)]
pub struct fg_graph {
    _p: [u8; 0],
}
#[repr(C)]
pub struct fg_plan {
    _p: [u8; 0],
}

/// One device tensor to save (`fg_bpat_tensor`).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct fg_bpat_tensor {
    pub d_ptr: *const c_void,
    pub dtype: c_int,
    pub rank: c_int,
    pub shape: [u32; 8],
}

/// `fg_status`: 0 = success; the others are `fused_gpu::errors::ErrorKind`s
/// (crates/fused_gpu/src/errors.rs:102-140).
#[repr(i32)]
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum FgStatus {
    Ok = 0,
    InvalidArgument = 1,
    OutOfMemory = 2,
    Unsupported = 3,
    Device = 4,
    Shape = 5,
    Graph = 6,
    Internal = 7,
    NoDevice = 8,
    OutOfBounds = 9,
    Serialization = 10,
    FileNotFound = 11,
}

impl FgStatus {
    /// The status of a returned code (unknown codes read as `Internal`).
    pub fn from_code(code: c_int) -> FgStatus {
        match code {
            0 => FgStatus::Ok,
            1 => FgStatus::InvalidArgument,
            2 => FgStatus::OutOfMemory,
            3 => FgStatus::Unsupported,
            4 => FgStatus::Device,
            5 => FgStatus::Shape,
            6 => FgStatus::Graph,
            8 => FgStatus::NoDevice,
            9 => FgStatus::OutOfBounds,
            10 => FgStatus::Serialization,
            11 => FgStatus::FileNotFound,
            _ => FgStatus::Internal,
        }
    }
}

pub const FG_TARGET_LIN_ACC: u32 = 0x1;

// fg_layout
pub const FG_NN: c_int = 0;
pub const FG_NT: c_int = 1;
pub const FG_TN: c_int = 2;
// fg_act
pub const FG_ACT_NONE: c_int = 0;
pub const FG_ACT_RELU: c_int = 1;
pub const FG_ACT_GELU: c_int = 2;
// fg_dtype (SimpleDType F32 / F16 / BF16)
pub const FG_DTYPE_F32: c_int = 0;
pub const FG_DTYPE_F16: c_int = 1;
pub const FG_DTYPE_BF16: c_int = 2;
// fg_bpat_header (BpatHeader declaration order)
pub const FG_BPAT_V0: c_int = 0;
pub const FG_BPAT_V1: c_int = 1;
pub const FG_BPAT_V1M: c_int = 2;
pub const FG_BPAT_V2_F16: c_int = 3;
pub const FG_BPAT_V2_BF16: c_int = 4;
pub const FG_BPAT_V2_F32: c_int = 5;
// elementwise program modes (fg_eltwise_set_mode)
pub const FG_ELTWISE_INTERPRET: c_int = 0;
pub const FG_ELTWISE_COMPILE_LARGE: c_int = 1;
pub const FG_ELTWISE_COMPILE_ALL: c_int = 2;
// fg_loss (ferrograd-nn LossType constants)
pub const FG_LOSS_MSE: c_int = 0;
pub const FG_LOSS_BCE: c_int = 1;
pub const FG_LOSS_CE: c_int = 2;
// fg_optim
pub const FG_OPTIM_SGD: c_int = 0;
pub const FG_OPTIM_ADAM: c_int = 1;
// fg_op (ferrograd-nn builders)
pub const FG_OP_INPUT: c_int = 0;
pub const FG_OP_CONST: c_int = 1;
pub const FG_OP_ADD: c_int = 2;
pub const FG_OP_SUB: c_int = 3;
pub const FG_OP_MUL: c_int = 4;
pub const FG_OP_DIV: c_int = 5;
pub const FG_OP_MATMUL: c_int = 6;
pub const FG_OP_RELU: c_int = 7;
pub const FG_OP_GELU: c_int = 8;
pub const FG_OP_ELU: c_int = 9;
pub const FG_OP_TANH: c_int = 10;
pub const FG_OP_EXP: c_int = 11;
pub const FG_OP_LOG: c_int = 12;
pub const FG_OP_ABS: c_int = 13;
pub const FG_OP_NEG: c_int = 14;
pub const FG_OP_SOFTMAX: c_int = 15;
pub const FG_OP_BIAS_ADD: c_int = 16;
// input flags
pub const FG_INPUT_NO_GRAD: u32 = 0x1;
pub const FG_INPUT_FROZEN: u32 = 0x2;
// fg_role (AllocTensors fields)
pub const FG_ROLE_FORWARD_OUT: c_int = 0;
pub const FG_ROLE_SEED: c_int = 1;
pub const FG_ROLE_LOSS: c_int = 2;
pub const FG_ROLE_FORWARD_SAVED: c_int = 3;
pub const FG_ROLE_GRAD: c_int = 4;
pub const FG_ROLE_INPUT: c_int = 5;
pub const FG_ROLE_STATE: c_int = 6;
pub const FG_ROLE_MEAN_LOSS: c_int = 7;
pub const FG_ROLE_TARGET: c_int = 8;

#[link(name = "ferrograd_hip")]
extern "C" {
    pub fn fg_last_error_msg() -> *const c_char;
    pub fn fg_version() -> c_int;
    pub fn fg_ctx_create(device: c_int, stream: *mut c_void, out: *mut *mut fg_ctx) -> c_int;
    pub fn fg_ctx_destroy(ctx: *mut fg_ctx) -> c_int;
    pub fn fg_ctx_target(
        ctx: *mut fg_ctx,
        arch: *mut c_char,
        arch_len: usize,
        flags: *mut u32,
        cu_count: *mut c_int,
    ) -> c_int;
    pub fn fg_ctx_stream(ctx: *mut fg_ctx, stream: *mut *mut c_void) -> c_int;
    pub fn fg_ctx_reserve_workspace(ctx: *mut fg_ctx, bytes: u64) -> c_int;
    pub fn fg_sync(ctx: *mut fg_ctx) -> c_int;
    pub fn fg_is_ready(ctx: *mut fg_ctx, ready: *mut c_int) -> c_int;
    pub fn fg_buf_alloc(ctx: *mut fg_ctx, bytes: u64, out: *mut *mut fg_buf) -> c_int;
    pub fn fg_buf_alloc_zeroed(ctx: *mut fg_ctx, bytes: u64, out: *mut *mut fg_buf) -> c_int;
    pub fn fg_buf_alloc_init(
        ctx: *mut fg_ctx,
        src: *const c_void,
        bytes: u64,
        out: *mut *mut fg_buf,
    ) -> c_int;
    pub fn fg_buf_free(buf: *mut fg_buf) -> c_int;
    pub fn fg_buf_size_bytes(buf: *const fg_buf) -> u64;
    pub fn fg_buf_device_ptr(buf: *const fg_buf) -> *mut c_void;
    pub fn fg_upload(
        ctx: *mut fg_ctx,
        dst: *mut fg_buf,
        src: *const c_void,
        bytes: u64,
        dst_off: u64,
    ) -> c_int;
    pub fn fg_download(
        ctx: *mut fg_ctx,
        src: *const fg_buf,
        dst: *mut c_void,
        bytes: u64,
        src_off: u64,
    ) -> c_int;
    pub fn fg_copy(ctx: *mut fg_ctx, src: *const fg_buf, dst: *mut fg_buf) -> c_int;
    pub fn fg_fill_u32(ctx: *mut fg_ctx, d_dst: *mut c_void, value: u32, count: u64) -> c_int;
    pub fn fg_gemm_f32(
        ctx: *mut fg_ctx,
        layout: c_int,
        M: c_int,
        N: c_int,
        K: c_int,
        d_A: *const f32,
        lda: c_int,
        d_B: *const f32,
        ldb: c_int,
        d_bias: *const f32,
        act: c_int,
        d_C: *mut f32,
        ldc: c_int,
        d_Z: *mut f32,
        ldz: c_int,
        accumulate: c_int,
    ) -> c_int;
    pub fn fg_gemm_bwd_f32(
        ctx: *mut fg_ctx,
        layout: c_int,
        M: c_int,
        N: c_int,
        K: c_int,
        d_A: *const f32,
        lda: c_int,
        d_B: *const f32,
        ldb: c_int,
        act: c_int,
        d_Zs: *const f32,
        ldzs: c_int,
        d_C: *mut f32,
        ldc: c_int,
        accumulate: c_int,
    ) -> c_int;
    pub fn fg_matmul_bwd_f32(
        ctx: *mut fg_ctx,
        M: c_int,
        N: c_int,
        K: c_int,
        d_X: *const f32,
        ldx: c_int,
        d_W: *const f32,
        ldw: c_int,
        d_dZ: *const f32,
        lddz: c_int,
        act: c_int,
        d_Zs: *const f32,
        ldzs: c_int,
        d_dX: *mut f32,
        lddx: c_int,
        d_dW: *mut f32,
        lddw: c_int,
        d_dbias: *mut f32,
        accumulate: c_int,
    ) -> c_int;
    pub fn fg_matmul_bwd_x16(
        ctx: *mut fg_ctx,
        dtype: c_int,
        M: c_int,
        N: c_int,
        K: c_int,
        d_X: *const c_void,
        ldx: c_int,
        d_W: *const c_void,
        ldw: c_int,
        d_dZ: *const c_void,
        lddz: c_int,
        act: c_int,
        d_Zs: *const c_void,
        ldzs: c_int,
        d_dX: *mut c_void,
        lddx: c_int,
        d_dW: *mut c_void,
        lddw: c_int,
        d_dbias: *mut c_void,
        accumulate: c_int,
    ) -> c_int;
    pub fn fg_linear_bwd_f32(
        ctx: *mut fg_ctx,
        act: c_int,
        M: c_int,
        N: c_int,
        K: c_int,
        d_X: *const f32,
        ldx: c_int,
        d_W: *const f32,
        ldw: c_int,
        d_Zs: *const f32,
        ldzs: c_int,
        d_dC: *const f32,
        lddc: c_int,
        d_dX: *mut f32,
        lddx: c_int,
        d_dW: *mut f32,
        lddw: c_int,
        d_dbias: *mut f32,
        accumulate: c_int,
        d_dZ: *mut f32,
        lddz: c_int,
    ) -> c_int;
    pub fn fg_gemm_x16(
        ctx: *mut fg_ctx,
        dtype: c_int,
        layout: c_int,
        M: c_int,
        N: c_int,
        K: c_int,
        d_A: *const c_void,
        lda: c_int,
        d_B: *const c_void,
        ldb: c_int,
        d_bias: *const c_void,
        act: c_int,
        d_C: *mut c_void,
        ldc: c_int,
        d_Z: *mut c_void,
        ldz: c_int,
        accumulate: c_int,
    ) -> c_int;
    pub fn fg_gemm_bwd_x16(
        ctx: *mut fg_ctx,
        dtype: c_int,
        layout: c_int,
        M: c_int,
        N: c_int,
        K: c_int,
        d_A: *const c_void,
        lda: c_int,
        d_B: *const c_void,
        ldb: c_int,
        act: c_int,
        d_Zs: *const c_void,
        ldzs: c_int,
        d_C: *mut c_void,
        ldc: c_int,
        accumulate: c_int,
    ) -> c_int;
    pub fn fg_gemm_dw_f32(
        ctx: *mut fg_ctx,
        M: c_int,
        N: c_int,
        K: c_int,
        d_A: *const f32,
        lda: c_int,
        d_B: *const f32,
        ldb: c_int,
        d_C: *mut f32,
        ldc: c_int,
        accumulate: c_int,
        d_colsum: *mut f32,
        colsum_accumulate: c_int,
    ) -> c_int;
    pub fn fg_gemm_dw_x16(
        ctx: *mut fg_ctx,
        dtype: c_int,
        M: c_int,
        N: c_int,
        K: c_int,
        d_A: *const c_void,
        lda: c_int,
        d_B: *const c_void,
        ldb: c_int,
        d_C: *mut c_void,
        ldc: c_int,
        accumulate: c_int,
        d_colsum: *mut c_void,
        colsum_accumulate: c_int,
    ) -> c_int;
    pub fn fg_bias_grad_f32(
        ctx: *mut fg_ctx,
        M: c_int,
        N: c_int,
        d_dZ: *const f32,
        ld: c_int,
        d_dbias: *mut f32,
        accumulate: c_int,
    ) -> c_int;
    pub fn fg_bias_grad(
        ctx: *mut fg_ctx,
        dtype: c_int,
        M: c_int,
        N: c_int,
        d_dZ: *const c_void,
        ld: c_int,
        d_dbias: *mut c_void,
        accumulate: c_int,
    ) -> c_int;
    pub fn fg_bias_grad_noalloc(
        ctx: *mut fg_ctx,
        dtype: c_int,
        M: c_int,
        N: c_int,
        d_dZ: *const c_void,
        ld: c_int,
        d_dbias: *mut c_void,
        accumulate: c_int,
    ) -> c_int;
    pub fn fg_act_bwd_f32(
        ctx: *mut fg_ctx,
        act: c_int,
        n: u64,
        d_dH: *const f32,
        d_Z: *const f32,
        d_dZ: *mut f32,
    ) -> c_int;
    pub fn fg_softmax_ce_f32(
        ctx: *mut fg_ctx,
        d_logits: *const f32,
        ldx: c_int,
        d_labels: *const u32,
        R: c_int,
        C: c_int,
        grad_scale: f32,
        d_row_loss: *mut f32,
        d_mean_loss: *mut f32,
        d_dlogits: *mut f32,
        ldd: c_int,
        d_argmax: *mut u32,
    ) -> c_int;
    pub fn fg_softmax_ce(
        ctx: *mut fg_ctx,
        dtype: c_int,
        d_logits: *const c_void,
        ldx: c_int,
        d_labels: *const u32,
        R: c_int,
        C: c_int,
        grad_scale: f32,
        d_row_loss: *mut f32,
        d_mean_loss: *mut f32,
        d_dlogits: *mut c_void,
        ldd: c_int,
        d_argmax: *mut u32,
    ) -> c_int;
    pub fn fg_softmax_f32(
        ctx: *mut fg_ctx,
        d_x: *const f32,
        R: c_int,
        C: c_int,
        d_y: *mut f32,
    ) -> c_int;
    pub fn fg_softmax_bwd_f32(
        ctx: *mut fg_ctx,
        d_y: *const f32,
        d_dy: *const f32,
        R: c_int,
        C: c_int,
        d_dx: *mut f32,
        accumulate: c_int,
    ) -> c_int;
    pub fn fg_softmax(
        ctx: *mut fg_ctx,
        dtype: c_int,
        d_x: *const c_void,
        R: c_int,
        C: c_int,
        d_y: *mut c_void,
    ) -> c_int;
    pub fn fg_softmax_bwd(
        ctx: *mut fg_ctx,
        dtype: c_int,
        d_y: *const c_void,
        d_dy: *const c_void,
        R: c_int,
        C: c_int,
        d_dx: *mut c_void,
        accumulate: c_int,
    ) -> c_int;
    pub fn fg_mt_create(
        ctx: *mut fg_ctx,
        n: c_int,
        d_params: *const *mut f32,
        d_grads: *const *mut f32,
        d_m: *const *mut f32,
        d_v: *const *mut f32,
        sizes: *const u64,
        out: *mut *mut fg_mt,
    ) -> c_int;
    pub fn fg_mt_create_x(
        ctx: *mut fg_ctx,
        n: c_int,
        dtypes: *const c_int,
        d_params: *const *mut c_void,
        d_grads: *const *mut c_void,
        d_m: *const *mut f32,
        d_v: *const *mut f32,
        sizes: *const u64,
        out: *mut *mut fg_mt,
    ) -> c_int;
    pub fn fg_mt_destroy(mt: *mut fg_mt) -> c_int;
    pub fn fg_sgd_step(ctx: *mut fg_ctx, mt: *mut fg_mt, lr: f32, zero_grad: c_int) -> c_int;
    pub fn fg_adam_step(
        ctx: *mut fg_ctx,
        mt: *mut fg_mt,
        lr: f32,
        b1: f32,
        b2: f32,
        eps: f32,
        step: c_int,
        zero_grad: c_int,
    ) -> c_int;
    pub fn fg_adam_step_scalars(
        ctx: *mut fg_ctx,
        mt: *mut fg_mt,
        b1: f32,
        b2: f32,
        eps: f32,
        step_size: f32,
        inv_sqrt_bc2: f32,
        zero_grad: c_int,
    ) -> c_int;
    pub fn fg_memcpy_h2d(
        ctx: *mut fg_ctx,
        d_dst: *mut c_void,
        src: *const c_void,
        bytes: u64,
    ) -> c_int;
    pub fn fg_memcpy_d2h(
        ctx: *mut fg_ctx,
        dst: *mut c_void,
        d_src: *const c_void,
        bytes: u64,
    ) -> c_int;
    pub fn fg_monitor_start(
        ctx: *mut fg_ctx,
        interval_us: c_int,
        out: *mut *mut fg_monitor,
    ) -> c_int;
    pub fn fg_monitor_stop(m: *mut fg_monitor, n_samples: *mut c_int) -> c_int;
    pub fn fg_monitor_sample(
        m: *const fg_monitor,
        index: c_int,
        t_s: *mut f64,
        used: *mut u64,
        budget: *mut u64,
    ) -> c_int;
    pub fn fg_monitor_destroy(m: *mut fg_monitor) -> c_int;
    pub fn fg_bpat_save(
        ctx: *mut fg_ctx,
        path: *const c_char,
        header: c_int,
        n: c_int,
        tensors: *const fg_bpat_tensor,
    ) -> c_int;
    pub fn fg_bpat_save_host(
        path: *const c_char,
        header: c_int,
        n: c_int,
        tensors: *const fg_bpat_tensor,
    ) -> c_int;
    pub fn fg_bpat_open(path: *const c_char, out: *mut *mut fg_bpat) -> c_int;
    pub fn fg_bpat_close(f: *mut fg_bpat) -> c_int;
    pub fn fg_bpat_info(f: *const fg_bpat, header: *mut c_int, count: *mut c_int) -> c_int;
    pub fn fg_bpat_tensor_info(
        f: *const fg_bpat,
        index: c_int,
        rank: *mut c_int,
        shape: *mut u32,
        numel: *mut u64,
    ) -> c_int;
    pub fn fg_bpat_read_f32(f: *const fg_bpat, index: c_int, dst: *mut f32) -> c_int;
    pub fn fg_bpat_upload(
        ctx: *mut fg_ctx,
        f: *const fg_bpat,
        index: c_int,
        d_dst: *mut c_void,
        dtype: c_int,
    ) -> c_int;
    pub fn fg_eltwise_set_mode(mode: c_int, previous: *mut c_int) -> c_int;
    pub fn fg_eltwise_stats(
        kernels_compiled: *mut u64,
        compiled_launches: *mut u64,
        interpreted_launches: *mut u64,
    ) -> c_int;
    pub fn fg_graph_create(loss: c_int, optim: c_int, out: *mut *mut fg_graph) -> c_int;
    pub fn fg_graph_destroy(g: *mut fg_graph) -> c_int;
    pub fn fg_graph_new_field(g: *mut fg_graph, field: *mut u32) -> c_int;
    pub fn fg_graph_input(
        g: *mut fg_graph,
        fields: *const u32,
        rank: c_int,
        node: *mut u32,
    ) -> c_int;
    pub fn fg_graph_input_x(
        g: *mut fg_graph,
        fields: *const u32,
        rank: c_int,
        dtype: c_int,
        node: *mut u32,
    ) -> c_int;
    pub fn fg_graph_constant_f32(g: *mut fg_graph, value: f32, node: *mut u32) -> c_int;
    pub fn fg_graph_constant(g: *mut fg_graph, dtype: c_int, value: f32, node: *mut u32) -> c_int;
    pub fn fg_graph_op(
        g: *mut fg_graph,
        op: c_int,
        inputs: *const u32,
        n_inputs: c_int,
        node: *mut u32,
    ) -> c_int;
    pub fn fg_graph_set_input_flags(g: *mut fg_graph, node: u32, flags: u32) -> c_int;
    pub fn fg_graph_num_nodes(g: *const fg_graph, n: *mut u32) -> c_int;
    pub fn fg_graph_validate(g: *const fg_graph, meta: *const u32, n_meta: c_int) -> c_int;
    pub fn fg_plan_create(
        ctx: *mut fg_ctx,
        g: *const fg_graph,
        meta: *const u32,
        n_meta: c_int,
        out: *mut *mut fg_plan,
    ) -> c_int;
    pub fn fg_plan_destroy(p: *mut fg_plan) -> c_int;
    pub fn fg_plan_count(p: *const fg_plan, role: c_int, count: *mut c_int) -> c_int;
    pub fn fg_plan_tensor(
        p: *const fg_plan,
        role: c_int,
        index: c_int,
        d_ptr: *mut *mut c_void,
        bytes: *mut u64,
        node: *mut u32,
    ) -> c_int;
    pub fn fg_plan_tensor_dtype(
        p: *const fg_plan,
        role: c_int,
        index: c_int,
        dtype: *mut c_int,
    ) -> c_int;
    pub fn fg_plan_bind_input(
        p: *mut fg_plan,
        index: c_int,
        d_ptr: *mut c_void,
        bytes: u64,
    ) -> c_int;
    pub fn fg_plan_bind_target(p: *mut fg_plan, d_ptr: *const c_void, bytes: u64) -> c_int;
    pub fn fg_plan_set_lr(p: *mut fg_plan, lr: f32) -> c_int;
    pub fn fg_plan_set_adam(p: *mut fg_plan, b1: f32, b2: f32, eps: f32) -> c_int;
    pub fn fg_plan_forward(p: *mut fg_plan) -> c_int;
    pub fn fg_plan_loss(p: *mut fg_plan) -> c_int;
    pub fn fg_plan_backward(p: *mut fg_plan) -> c_int;
    pub fn fg_plan_optim(p: *mut fg_plan) -> c_int;
    pub fn fg_plan_single_optim(p: *mut fg_plan, input_index: c_int) -> c_int;
    pub fn fg_plan_capture_step(p: *mut fg_plan) -> c_int;
    pub fn fg_plan_launch_step(p: *mut fg_plan) -> c_int;
    pub fn fg_plan_save(p: *mut fg_plan, path: *const c_char, header: c_int) -> c_int;
    pub fn fg_plan_load(p: *mut fg_plan, path: *const c_char) -> c_int;
    pub fn fg_plan_describe(
        p: *const fg_plan,
        buf: *mut c_char,
        len: usize,
        needed: *mut usize,
    ) -> c_int;
    pub fn fg_rng_uniform_host(
        seed: u64,
        tensor_id: u64,
        lo: f32,
        hi: f32,
        dst: *mut f32,
        n: u64,
    ) -> c_int;
    pub fn fg_rng_normal_host(
        seed: u64,
        tensor_id: u64,
        mean: f32,
        std: f32,
        dst: *mut f32,
        n: u64,
    ) -> c_int;
    pub fn fg_rng_int_host(seed: u64, tensor_id: u64, bound: u32, dst: *mut u32, n: u64) -> c_int;
    pub fn fg_rng_uniform_dev(
        ctx: *mut fg_ctx,
        seed: u64,
        tensor_id: u64,
        lo: f32,
        hi: f32,
        d_dst: *mut f32,
        n: u64,
    ) -> c_int;
    pub fn fg_rng_normal_dev(
        ctx: *mut fg_ctx,
        seed: u64,
        tensor_id: u64,
        mean: f32,
        std: f32,
        d_dst: *mut f32,
        n: u64,
    ) -> c_int;
    pub fn fg_rng_int_dev(
        ctx: *mut fg_ctx,
        seed: u64,
        tensor_id: u64,
        bound: u32,
        d_dst: *mut u32,
        n: u64,
    ) -> c_int;
}
