//! Safe Rust face of `libferrograd_hip.so`, the MI355X (gfx950) backend for
//! ferrograd's fused training path, and the pieces a ferrograd maintainer
//! adds for a `Dynamic::Hip` backend.
//!
//! Not built in this repository's image (it has no Rust toolchain); the C
//! ABI it wraps is `include/ferrograd_hip.h`, whose functions the
//! `ferrograd-hip-sys` crate declares one for one.
//!
//! # Where it plugs in
//!
//! ferrograd selects a backend through `ferrograd::backend::Dynamic`
//! (crates/ferrograd/src/backend.rs:316-325).  The reference backends
//! implement `fused_gpu::dispatch::GpuBackend` (crates/fused_gpu/src/dispatch/
//! mod.rs:161-261), whose `compile` consumes generated kernel IR; this backend
//! plans the graph instead and launches ahead-of-time kernels, so its seam is
//! one level up, in `GpuContext`:
//!
//! ```text
//! pub enum Dynamic {
//!     None(NopGpuContext),
//!     #[cfg(feature = "wgsl")] Wgsl(wgsl::GpuContext),
//!     #[cfg(feature = "rocm")] Rocm(rocm::GpuContext),
//!     #[cfg(feature = "hip")]  Hip(ferrograd_hip::Context),     // new arm
//! }
//! ```
//!
//! and `GpuContext<Dynamic>`'s methods route the `Hip` arm as follows:
//!
//! | `GpuContext` (backend.rs)            | here                                   |
//! |--------------------------------------|----------------------------------------|
//! | `new()` / `detect_target()`          | [`Context::new`] / [`Context::target`] |
//! | `alloc_tensors(graph, saved, meta)`  | [`mirror_graph`] + [`Plan::create`]    |
//! | `compile(ir)`                        | nothing (kernels are ahead of time)    |
//! | `init_tensor_*`, `upload`, `download`| [`Context::alloc_init`], [`Context::upload`], [`Context::download`] |
//! | `schedule(kernels, meta, ins, ..)`   | [`Plan::bind_input`] per input, [`Plan::set_lr`] |
//! | `dispatch_forward / _loss / _backward / _optim / _single_optim` | [`Plan::forward`] ... [`Plan::single_optim`] |
//! | `save_tensors` / `load_tensors`      | `fg_bpat_save` / `fg_bpat_open` + `fg_bpat_upload` |
//! | `sync()`                             | [`Context::sync`]                      |
#![allow(clippy::missing_safety_doc)]

use core::ffi::{c_char, c_int, c_void};
use core::marker::PhantomData;
use std::ffi::{CStr, CString};

use ferrograd_hip_sys as sys;

/// The `fused_gpu::errors::ErrorKind`s this backend raises
/// (crates/fused_gpu/src/errors.rs:102-140), one per `fg_status`.
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum ErrorKind {
    InvalidArgument,
    OutOfMemory,
    UnsupportedFeature,
    DeviceError,
    ShapeMismatch,
    ComputeGraphError,
    InternalError,
    NoDevice,
    OutOfBounds,
    SerializationError,
    FileNotFound,
}

/// A failed call: its kind and the library's message for it.
#[derive(Clone, Debug)]
pub struct Error {
    pub kind: ErrorKind,
    pub msg: String,
}

impl core::fmt::Display for Error {
    fn fmt(&self, f: &mut core::fmt::Formatter<'_>) -> core::fmt::Result {
        write!(f, "{:?}: {}", self.kind, self.msg)
    }
}

impl std::error::Error for Error {}

fn last_message() -> String {
    // SAFETY: the library returns a NUL-terminated thread-local string.
    unsafe {
        let p = sys::fg_last_error_msg();
        if p.is_null() {
            String::new()
        } else {
            CStr::from_ptr(p).to_string_lossy().into_owned()
        }
    }
}

/// Maps a returned `fg_status` to `Ok(())` or the matching [`Error`].
pub fn check(code: c_int) -> Result<(), Error> {
    use sys::FgStatus as S;
    let kind = match S::from_code(code) {
        S::Ok => return Ok(()),
        S::InvalidArgument => ErrorKind::InvalidArgument,
        S::OutOfMemory => ErrorKind::OutOfMemory,
        S::Unsupported => ErrorKind::UnsupportedFeature,
        S::Device => ErrorKind::DeviceError,
        S::Shape => ErrorKind::ShapeMismatch,
        S::Graph => ErrorKind::ComputeGraphError,
        S::Internal => ErrorKind::InternalError,
        S::NoDevice => ErrorKind::NoDevice,
        S::OutOfBounds => ErrorKind::OutOfBounds,
        S::Serialization => ErrorKind::SerializationError,
        S::FileNotFound => ErrorKind::FileNotFound,
    };
    Err(Error { kind, msg: last_message() })
}

fn unsupported(msg: String) -> Error {
    Error { kind: ErrorKind::UnsupportedFeature, msg }
}

// ------------------------------------------------------------------ context
/// One device and one stream (`rocm::GpuContext`, rocm/mod.rs:57-79).
pub struct Context {
    raw: *mut sys::fg_ctx,
}

impl Context {
    /// Opens `device` with a private default-priority stream.
    pub fn new(device: i32) -> Result<Self, Error> {
        let mut raw = core::ptr::null_mut();
        check(unsafe { sys::fg_ctx_create(device, core::ptr::null_mut(), &mut raw) })?;
        Ok(Context { raw })
    }

    /// (architecture name, `FG_TARGET_*` flags, CU count).
    pub fn target(&self) -> Result<(String, u32, i32), Error> {
        let mut arch = [0 as c_char; 64];
        let (mut flags, mut cus) = (0u32, 0 as c_int);
        check(unsafe { sys::fg_ctx_target(self.raw, arch.as_mut_ptr(), arch.len(), &mut flags, &mut cus) })?;
        let name = unsafe { CStr::from_ptr(arch.as_ptr()) }.to_string_lossy().into_owned();
        Ok((name, flags, cus))
    }

    pub fn sync(&self) -> Result<(), Error> {
        check(unsafe { sys::fg_sync(self.raw) })
    }

    pub fn raw(&self) -> *mut sys::fg_ctx {
        self.raw
    }

    pub fn alloc(&self, bytes: u64) -> Result<Buffer, Error> {
        let mut raw = core::ptr::null_mut();
        check(unsafe { sys::fg_buf_alloc(self.raw, bytes, &mut raw) })?;
        Ok(Buffer { raw })
    }

    pub fn alloc_zeroed(&self, bytes: u64) -> Result<Buffer, Error> {
        let mut raw = core::ptr::null_mut();
        check(unsafe { sys::fg_buf_alloc_zeroed(self.raw, bytes, &mut raw) })?;
        Ok(Buffer { raw })
    }

    pub fn alloc_init(&self, data: &[u8]) -> Result<Buffer, Error> {
        let mut raw = core::ptr::null_mut();
        check(unsafe {
            sys::fg_buf_alloc_init(self.raw, data.as_ptr() as *const c_void, data.len() as u64, &mut raw)
        })?;
        Ok(Buffer { raw })
    }

    pub fn upload(&self, dst: &Buffer, data: &[u8], dst_off: u64) -> Result<(), Error> {
        check(unsafe {
            sys::fg_upload(self.raw, dst.raw, data.as_ptr() as *const c_void, data.len() as u64, dst_off)
        })
    }

    pub fn download(&self, src: &Buffer, out: &mut [u8], src_off: u64) -> Result<(), Error> {
        check(unsafe {
            sys::fg_download(self.raw, src.raw, out.as_mut_ptr() as *mut c_void, out.len() as u64, src_off)
        })
    }

    /// Copies between host memory and a device address (plan tensors).
    pub unsafe fn memcpy_h2d(&self, d_dst: *mut c_void, data: &[u8]) -> Result<(), Error> {
        check(sys::fg_memcpy_h2d(self.raw, d_dst, data.as_ptr() as *const c_void, data.len() as u64))
    }

    pub unsafe fn memcpy_d2h(&self, out: &mut [u8], d_src: *const c_void) -> Result<(), Error> {
        check(sys::fg_memcpy_d2h(self.raw, out.as_mut_ptr() as *mut c_void, d_src, out.len() as u64))
    }
}

impl Drop for Context {
    fn drop(&mut self) {
        unsafe { sys::fg_ctx_destroy(self.raw) };
    }
}

/// A device allocation (`rocm_rt::hip::memory::Buffer`).
pub struct Buffer {
    raw: *mut sys::fg_buf,
}

impl Buffer {
    pub fn device_ptr(&self) -> *mut c_void {
        unsafe { sys::fg_buf_device_ptr(self.raw) }
    }

    pub fn size_bytes(&self) -> u64 {
        unsafe { sys::fg_buf_size_bytes(self.raw) }
    }
}

impl Drop for Buffer {
    fn drop(&mut self) {
        unsafe { sys::fg_buf_free(self.raw) };
    }
}

// -------------------------------------------------------------------- graph
/// The C mirror of a `fused_gpu::Graph` (dispatch/backend/mod.rs:499-1316):
/// node ids are creation order, the last node is the forward output.
pub struct Graph {
    raw: *mut sys::fg_graph,
}

impl Graph {
    /// `loss`: `FG_LOSS_*`; `optim`: `FG_OPTIM_*`.
    pub fn new(loss: c_int, optim: c_int) -> Result<Self, Error> {
        let mut raw = core::ptr::null_mut();
        check(unsafe { sys::fg_graph_create(loss, optim, &mut raw) })?;
        Ok(Graph { raw })
    }

    /// A new metadata field (`Metadata::new_field`); index 0 is the learning rate.
    pub fn new_field(&mut self) -> Result<u32, Error> {
        let mut f = 0u32;
        check(unsafe { sys::fg_graph_new_field(self.raw, &mut f) })?;
        Ok(f)
    }

    /// An input whose dims are metadata fields, of element type `dtype`.
    pub fn input(&mut self, fields: &[u32], dtype: c_int) -> Result<u32, Error> {
        let mut id = 0u32;
        check(unsafe { sys::fg_graph_input_x(self.raw, fields.as_ptr(), fields.len() as c_int, dtype, &mut id) })?;
        Ok(id)
    }

    pub fn constant(&mut self, dtype: c_int, value: f32) -> Result<u32, Error> {
        let mut id = 0u32;
        check(unsafe { sys::fg_graph_constant(self.raw, dtype, value, &mut id) })?;
        Ok(id)
    }

    /// An operation node (`FG_OP_*`) on existing nodes.
    pub fn op(&mut self, kind: c_int, inputs: &[u32]) -> Result<u32, Error> {
        let mut id = 0u32;
        check(unsafe { sys::fg_graph_op(self.raw, kind, inputs.as_ptr(), inputs.len() as c_int, &mut id) })?;
        Ok(id)
    }

    pub fn set_input_flags(&mut self, node: u32, flags: u32) -> Result<(), Error> {
        check(unsafe { sys::fg_graph_set_input_flags(self.raw, node, flags) })
    }

    /// `Graph::validate` against a meta binding `[lr_bits, dim1, ...]`.
    pub fn validate(&self, meta: &[u32]) -> Result<(), Error> {
        check(unsafe { sys::fg_graph_validate(self.raw, meta.as_ptr(), meta.len() as c_int) })
    }

    pub fn raw(&self) -> *const sys::fg_graph {
        self.raw
    }
}

impl Drop for Graph {
    fn drop(&mut self) {
        unsafe { sys::fg_graph_destroy(self.raw) };
    }
}

/// The operation kind of a ferrograd-nn node from its `display` output: each
/// builder prints a fixed form (op/binary.rs:218,431,626,864,
/// op/matmul/mod.rs:288, op/softmax.rs:751, op/unary.rs:252,311,418,474,
/// 717,758,828,863).  A `GraphOp::Custom` of any other form is not an
/// operation this backend lowers: `UnsupportedFeature`, naming the text.
/// (ferrograd-nn's `log` prints "log2(" but computes the natural log.)
pub fn op_kind_from_display(display: &str) -> Result<c_int, Error> {
    const PREFIX: [(&str, c_int); 9] = [
        ("softmax(", sys::FG_OP_SOFTMAX),
        ("bias_add(", sys::FG_OP_BIAS_ADD),
        ("log2(", sys::FG_OP_LOG),
        ("tanh(", sys::FG_OP_TANH),
        ("GELU(", sys::FG_OP_GELU),
        ("ReLU(", sys::FG_OP_RELU),
        ("ELU(", sys::FG_OP_ELU),
        ("e^", sys::FG_OP_EXP),
        ("|", sys::FG_OP_ABS),
    ];
    for (p, k) in PREFIX {
        if display.starts_with(p) {
            return Ok(k);
        }
    }
    const INFIX: [(&str, c_int); 5] = [
        (" @ ", sys::FG_OP_MATMUL),
        (" + ", sys::FG_OP_ADD),
        (" - ", sys::FG_OP_SUB),
        (" * ", sys::FG_OP_MUL),
        (" / ", sys::FG_OP_DIV),
    ];
    for (p, k) in INFIX {
        if display.contains(p) {
            return Ok(k);
        }
    }
    if display.starts_with('-') {
        return Ok(sys::FG_OP_NEG);
    }
    Err(unsupported(format!(
        "GraphOp::Custom node `{display}` is not a ferrograd-nn operation this backend lowers"
    )))
}

/// What [`mirror_graph`] needs of a ferrograd graph's nodes, in creation
/// order: an Input (its metadata fields and element type), a scalar
/// constant, or a custom operation (its display text and input ids).
pub enum NodeView<'a> {
    Input { fields: &'a [u32], dtype: c_int, trainable: bool },
    Constant { dtype: c_int, value: f32 },
    Op { display: String, inputs: &'a [u32] },
}

/// Builds the C mirror of a ferrograd graph (`loss`, `optim` as in
/// [`Graph::new`], `n_fields` metadata fields after the learning rate).
/// Non-trainable inputs are marked `FG_INPUT_FROZEN`: their gradient is
/// computed, as ferrograd computes one for every Input, but never applied.
pub fn mirror_graph<'a>(
    loss: c_int,
    optim: c_int,
    n_fields: usize,
    nodes: impl IntoIterator<Item = NodeView<'a>>,
) -> Result<Graph, Error> {
    let mut g = Graph::new(loss, optim)?;
    for _ in 0..n_fields {
        g.new_field()?;
    }
    for node in nodes {
        match node {
            NodeView::Input { fields, dtype, trainable } => {
                let id = g.input(fields, dtype)?;
                if !trainable {
                    g.set_input_flags(id, sys::FG_INPUT_FROZEN)?;
                }
            }
            NodeView::Constant { dtype, value } => {
                g.constant(dtype, value)?;
            }
            NodeView::Op { display, inputs } => {
                let kind = op_kind_from_display(&display)?;
                g.op(kind, inputs)?;
            }
        }
    }
    Ok(g)
}

// --------------------------------------------------------------------- plan
/// A lowered, allocated graph (Graph::lower + compile + alloc_tensors +
/// schedule, kernel/mod.rs:107-152 and dispatch/mod.rs:509-764); borrows its
/// context.
pub struct Plan<'c> {
    raw: *mut sys::fg_plan,
    _ctx: PhantomData<&'c Context>,
}

impl<'c> Plan<'c> {
    pub fn create(ctx: &'c Context, graph: &Graph, meta: &[u32]) -> Result<Self, Error> {
        let mut raw = core::ptr::null_mut();
        check(unsafe { sys::fg_plan_create(ctx.raw, graph.raw, meta.as_ptr(), meta.len() as c_int, &mut raw) })?;
        Ok(Plan { raw, _ctx: PhantomData })
    }

    /// Tensors of a role (`FG_ROLE_*`, the fields of `AllocTensors`).
    pub fn count(&self, role: c_int) -> Result<usize, Error> {
        let mut n = 0 as c_int;
        check(unsafe { sys::fg_plan_count(self.raw, role, &mut n) })?;
        Ok(n as usize)
    }

    /// (device address, bytes, node id) of a role's index-th tensor.
    pub fn tensor(&self, role: c_int, index: usize) -> Result<(*mut c_void, u64, u32), Error> {
        let (mut p, mut bytes, mut node) = (core::ptr::null_mut(), 0u64, 0u32);
        check(unsafe { sys::fg_plan_tensor(self.raw, role, index as c_int, &mut p, &mut bytes, &mut node) })?;
        Ok((p, bytes, node))
    }

    pub unsafe fn bind_input(&mut self, index: usize, d_ptr: *mut c_void, bytes: u64) -> Result<(), Error> {
        check(sys::fg_plan_bind_input(self.raw, index as c_int, d_ptr, bytes))
    }

    pub unsafe fn bind_target(&mut self, d_ptr: *const c_void, bytes: u64) -> Result<(), Error> {
        check(sys::fg_plan_bind_target(self.raw, d_ptr, bytes))
    }

    /// Meta field 0 (kernel/optim.rs:119-131).
    pub fn set_lr(&mut self, lr: f32) -> Result<(), Error> {
        check(unsafe { sys::fg_plan_set_lr(self.raw, lr) })
    }

    pub fn set_adam(&mut self, b1: f32, b2: f32, eps: f32) -> Result<(), Error> {
        check(unsafe { sys::fg_plan_set_adam(self.raw, b1, b2, eps) })
    }

    pub fn forward(&mut self) -> Result<(), Error> {
        check(unsafe { sys::fg_plan_forward(self.raw) })
    }

    pub fn loss(&mut self) -> Result<(), Error> {
        check(unsafe { sys::fg_plan_loss(self.raw) })
    }

    pub fn backward(&mut self) -> Result<(), Error> {
        check(unsafe { sys::fg_plan_backward(self.raw) })
    }

    pub fn optim(&mut self) -> Result<(), Error> {
        check(unsafe { sys::fg_plan_optim(self.raw) })
    }

    pub fn single_optim(&mut self, input_index: usize) -> Result<(), Error> {
        check(unsafe { sys::fg_plan_single_optim(self.raw, input_index as c_int) })
    }

    /// Forward, loss, backward and optimiser as one captured hipGraph.
    pub fn capture_step(&mut self) -> Result<(), Error> {
        check(unsafe { sys::fg_plan_capture_step(self.raw) })
    }

    pub fn launch_step(&mut self) -> Result<(), Error> {
        check(unsafe { sys::fg_plan_launch_step(self.raw) })
    }

    /// Checkpoint (inputs and optimiser state) to a bpat file of `header`.
    pub fn save(&mut self, path: &str, header: c_int) -> Result<(), Error> {
        let c = CString::new(path).map_err(|_| Error { kind: ErrorKind::InvalidArgument, msg: "path contains NUL".into() })?;
        check(unsafe { sys::fg_plan_save(self.raw, c.as_ptr(), header) })
    }

    pub fn load(&mut self, path: &str) -> Result<(), Error> {
        let c = CString::new(path).map_err(|_| Error { kind: ErrorKind::InvalidArgument, msg: "path contains NUL".into() })?;
        check(unsafe { sys::fg_plan_load(self.raw, c.as_ptr()) })
    }

    /// The planned launch list, as text.
    pub fn describe(&self) -> Result<String, Error> {
        let mut need = 0usize;
        check(unsafe { sys::fg_plan_describe(self.raw, core::ptr::null_mut(), 0, &mut need) })?;
        let mut buf = vec![0 as c_char; need.max(1)];
        check(unsafe { sys::fg_plan_describe(self.raw, buf.as_mut_ptr(), buf.len(), core::ptr::null_mut()) })?;
        Ok(unsafe { CStr::from_ptr(buf.as_ptr()) }.to_string_lossy().into_owned())
    }
}

impl Drop for Plan<'_> {
    fn drop(&mut self) {
        unsafe { sys::fg_plan_destroy(self.raw) };
    }
}
