"""Mirror of ferrograd's graph / context API over the gfx950 planner.

The names, argument order and meaning follow the reference so that its
tests read the same here:

  reference (Rust)                                  here (Python)
  ------------------------------------------------  -------------------------
  Metadata::new() / new_field() / validate_meta     Metadata
  Graph::new(LOSS, Optim::sgd().lower)              Graph(LOSS, Optim.sgd().lower)
  graph.define_ops().input/matmul/add/...           graph.define_ops().input/...
  graph.compute_saved_nodes() / validate / lower    same
  GpuContext::new()                                 GpuContext.new()
  ctx.alloc_meta / alloc_tensors / compile          same
  ctx.init_tensor_f32 / new_onehot_init             same
  ctx.upload / download / sync                      same
  ctx.schedule(kernels, meta, in_tensors, saved,    same
               state)
  ctx.dispatch_forward / dispatch_loss /            same
      dispatch_backward / dispatch_optim /
      dispatch_single_optim

(crates/ferrograd/src/graph.rs:15-159, crates/ferrograd/src/backend.rs:54-314,
crates/fused_gpu/src/dispatch/mod.rs:340-833, crates/ferrograd/tests/*.rs.)

Differences, all deliberate:
  * dims need not be multiples of 16 (the reference asserts they are,
    backend/mod.rs:617-619);
  * `bias_add` (and broadcast in add / sub) exist;
  * `Optim.adam()` exists; `SimpleDType` covers F32, F16 and BF16 (F64 and
    the integer types have no op on this path);
  * after `dispatch_loss` with CROSS_ENTROPY on a final softmax the next
    `dispatch_backward` starts from dlogits = p - onehot (the reference
    pushes that gradient through the softmax Jacobian a second time);
  * `alloc_tensors` lowers and allocates in one step (the plan owns one
    device arena); `compile` is a no-op (kernels are ahead-of-time).
"""
from __future__ import annotations

import ctypes
import struct
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

from . import Context
from ._lib import FgError, call

# fg_op
OP_INPUT, OP_CONST, OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_MATMUL = 0, 1, 2, 3, 4, 5, 6
OP_RELU, OP_GELU, OP_ELU, OP_TANH, OP_EXP, OP_LOG, OP_ABS, OP_NEG = 7, 8, 9, 10, 11, 12, 13, 14
OP_SOFTMAX, OP_BIAS_ADD = 15, 16
# fg_role
ROLE_FORWARD_OUT, ROLE_SEED, ROLE_LOSS, ROLE_FORWARD_SAVED, ROLE_GRAD = 0, 1, 2, 3, 4
ROLE_INPUT, ROLE_STATE, ROLE_MEAN_LOSS, ROLE_TARGET = 5, 6, 7, 8
INPUT_NO_GRAD, INPUT_FROZEN = 1, 2


# ------------------------------------------------------------- constants
@dataclass(frozen=True)
class LossType:
    name: str
    code: int


MEAN_SQUARED_ERROR = LossType("MEAN_SQUARED_ERROR", 0)
BINARY_CROSS_ENTROPY = LossType("BINARY_CROSS_ENTROPY", 1)
CROSS_ENTROPY = LossType("CROSS_ENTROPY", 2)


class SimpleDType:
    """Element types of tensors (backend/mod.rs:335-427).  F16 tensors are
    numpy float16 on the host; BF16 tensors are raw 16-bit words (numpy has
    no bfloat16; see bf16_from_f32 / bf16_to_f32)."""
    F32 = "f32"
    F16 = "f16"
    BF16 = "bf16"


DTYPE_CODE = {SimpleDType.F32: 0, SimpleDType.F16: 1, SimpleDType.BF16: 2}
_CODE_NP = {0: np.float32, 1: np.float16, 2: np.uint16}


def bf16_from_f32(x) -> np.ndarray:
    """Round float32 values to bfloat16 words (nearest, ties to even; NaN
    stays NaN)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + np.uint32(0x7FFF) + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_to_f32(bits) -> np.ndarray:
    """Widen bfloat16 words to float32 (exact)."""
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


@dataclass(frozen=True)
class OptimType:
    name: str
    code: int


class Optim:
    """Optim{state, lower} (crates/ferrograd/src/optim.rs:4-15)."""

    def __init__(self, lower: OptimType, state: tuple):
        self.lower = lower
        self.state = state

    @staticmethod
    def sgd() -> "Optim":
        return Optim(OptimType("SGD", 0), ())

    @staticmethod
    def adam() -> "Optim":
        return Optim(OptimType("ADAM", 1), ("m", "v"))


def f32_bits(x: float) -> int:
    """The u32 bit pattern of an f32 (meta field 0 holds the lr this way)."""
    return struct.unpack("<I", struct.pack("<f", x))[0]


# ------------------------------------------------------------- metadata
@dataclass(frozen=True)
class Field:
    index: int


class Metadata:
    """Metadata::new / new_field / validate_meta (backend/mod.rs:576-620).
    Field 0 holds the learning rate; dims are fields 1, 2, ..."""

    def __init__(self):
        self.fields = 0

    @staticmethod
    def new() -> "Metadata":
        return Metadata()

    def new_field(self) -> Field:
        self.fields += 1
        return Field(self.fields)

    def validate_meta(self, binding: Sequence[int]) -> bool:
        return len(binding) == self.fields + 1 and all(int(d) > 0 for d in binding[1:])


# ----------------------------------------------------------------- graph
@dataclass
class _Node:
    op: int
    inputs: List[int] = field(default_factory=list)
    fields: List[int] = field(default_factory=list)
    value: float = 0.0
    flags: int = 0
    dtype: int = 0  # DTYPE_CODE of an input / constant


class _DefineOps:
    """graph.define_ops(): the builder view (crates/ferrograd/src/graph.rs:106-159)."""

    def __init__(self, graph: "Graph"):
        self.g = graph

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False

    def _push(self, node: _Node) -> int:
        for i in node.inputs:
            if not 0 <= i < len(self.g.nodes):
                raise FgError(6, f"input node {i} does not exist")
        self.g.nodes.append(node)
        return len(self.g.nodes) - 1

    def input(self, shape: Sequence[Field], dtype: str = SimpleDType.F32,
              trainable: bool = True, requires_grad: bool = True) -> int:
        if dtype not in DTYPE_CODE:
            raise FgError(3, f"element type {dtype!r} is not supported on this path")
        flags = (0 if requires_grad else INPUT_NO_GRAD) | (0 if trainable else INPUT_FROZEN)
        return self._push(_Node(OP_INPUT, fields=[f.index for f in shape], flags=flags,
                                dtype=DTYPE_CODE[dtype]))

    def constant_f32(self, value: float) -> int:
        return self._push(_Node(OP_CONST, value=float(value)))

    def constant_f16(self, value: float) -> int:
        return self._push(_Node(OP_CONST, value=float(value), dtype=1))

    def constant_bf16(self, value: float) -> int:
        return self._push(_Node(OP_CONST, value=float(value), dtype=2))

    def _op(self, op: int, *xs: int) -> int:
        return self._push(_Node(op, inputs=list(xs)))

    def add(self, a, b): return self._op(OP_ADD, a, b)
    def sub(self, a, b): return self._op(OP_SUB, a, b)
    def mul(self, a, b): return self._op(OP_MUL, a, b)
    def div(self, a, b): return self._op(OP_DIV, a, b)
    def matmul(self, a, b): return self._op(OP_MATMUL, a, b)
    def bias_add(self, x, b): return self._op(OP_BIAS_ADD, x, b)
    def relu(self, x): return self._op(OP_RELU, x)
    def gelu(self, x): return self._op(OP_GELU, x)
    def elu(self, x): return self._op(OP_ELU, x)
    def tanh(self, x): return self._op(OP_TANH, x)
    def exp(self, x): return self._op(OP_EXP, x)
    def log(self, x): return self._op(OP_LOG, x)
    def abs(self, x): return self._op(OP_ABS, x)
    def neg(self, x): return self._op(OP_NEG, x)
    def softmax(self, x): return self._op(OP_SOFTMAX, x)


class Graph:
    """Graph::new(loss, optim_lower) (crates/ferrograd/src/graph.rs:34)."""

    def __init__(self, loss: LossType, optim: OptimType):
        self.loss = loss
        self.optim = optim
        self.nodes: List[_Node] = []

    def define_ops(self) -> _DefineOps:
        return _DefineOps(self)

    def compute_saved_nodes(self) -> List[int]:
        """SaveIndicator flags per node (1 = defined in forward, 2 = defined
        in backward), by the rules of matmul/mod.rs:191-202,
        softmax.rs:699-718, unary.rs:15-21 and binary.rs:66-72."""
        n = len(self.nodes)
        save = [0] * n
        users = [[] for _ in range(n)]
        for i, nd in enumerate(self.nodes):
            for x in nd.inputs:
                users[x].append(i)
        nonleaf = [bool(nd.inputs) for nd in self.nodes]
        for i, nd in enumerate(self.nodes):
            if nd.op == OP_INPUT:
                save[i] |= 2
            elif nd.op == OP_MATMUL:
                save[i] |= 3
                for x in nd.inputs:
                    if nonleaf[x]:
                        save[x] |= 1
            elif nd.op == OP_SOFTMAX:
                save[i] |= 3
                for x in nd.inputs:
                    if self.nodes[x].op in (OP_MATMUL, OP_GELU, OP_SOFTMAX):
                        save[x] |= 3
                for u in users[i]:
                    save[u] |= 2
            elif nd.op in (OP_MUL, OP_DIV):
                for x in nd.inputs:
                    if nonleaf[x]:
                        save[x] |= 1
            elif OP_RELU <= nd.op <= OP_NEG and nonleaf[nd.inputs[0]]:
                save[nd.inputs[0]] |= 1
        return save

    def _c_graph(self, nfields: int):
        h = ctypes.c_void_p()
        call("fg_graph_create", self.loss.code, self.optim.code, ctypes.byref(h))
        try:
            f = ctypes.c_uint32()
            for _ in range(nfields):
                call("fg_graph_new_field", h, ctypes.byref(f))
            out = ctypes.c_uint32()
            for nd in self.nodes:
                if nd.op == OP_INPUT:
                    arr = (ctypes.c_uint32 * len(nd.fields))(*nd.fields)
                    call("fg_graph_input_x", h, arr, len(nd.fields), nd.dtype, ctypes.byref(out))
                    if nd.flags:
                        call("fg_graph_set_input_flags", h, out.value, nd.flags)
                elif nd.op == OP_CONST:
                    call("fg_graph_constant", h, nd.dtype, nd.value, ctypes.byref(out))
                else:
                    arr = (ctypes.c_uint32 * len(nd.inputs))(*nd.inputs)
                    call("fg_graph_op", h, nd.op, arr, len(nd.inputs), ctypes.byref(out))
        except Exception:
            call("fg_graph_destroy", h)
            raise
        return h

    def _nfields(self) -> int:
        return max([max(nd.fields) for nd in self.nodes if nd.fields] + [0])

    def validate(self, meta: Metadata, binding: Optional[Sequence[int]] = None) -> None:
        """Graph::validate.  Structural checks always; shape checks when a
        meta binding is given (or default dims of 16 otherwise)."""
        nf = max(meta.fields, self._nfields())
        b = list(binding) if binding is not None else [0] + [16] * nf
        h = self._c_graph(nf)
        try:
            arr = (ctypes.c_uint32 * len(b))(*b)
            call("fg_graph_validate", h, arr, len(b))
        finally:
            call("fg_graph_destroy", h)

    def lower(self, meta: Metadata, options=None, saved=None) -> "LoweredGraph":
        return LoweredGraph(self, meta)

    def describe(self, binding: Sequence[int]) -> str:
        """The fused launch list the planner builds for a meta binding (no
        device needed)."""
        nf = max(len(binding) - 1, self._nfields())
        h = self._c_graph(nf)
        p = ctypes.c_void_p()
        try:
            arr = (ctypes.c_uint32 * len(binding))(*binding)
            call("fg_plan_create", None, h, arr, len(binding), ctypes.byref(p))
            need = ctypes.c_size_t()
            call("fg_plan_describe", p, None, 0, ctypes.byref(need))
            buf = ctypes.create_string_buffer(need.value)
            call("fg_plan_describe", p, buf, need.value, None)
            return buf.value.decode()
        finally:
            if p:
                call("fg_plan_destroy", p)
            call("fg_graph_destroy", h)


@dataclass
class LoweredGraph:
    graph: Graph
    meta: Metadata


# ----------------------------------------------------------------- tensors
class Tensor:
    """A device tensor: either context-allocated (init_tensor_*) or a view
    of a plan-owned buffer."""

    def __init__(self, ptr: int, nbytes: int, shape, dtype=np.float32, owner=None, buf=None):
        self.ptr = int(ptr)
        self.nbytes = int(nbytes)
        self.shape = tuple(shape)
        self.dtype = np.dtype(dtype)
        self._owner = owner
        self._buf = buf

    def data_ptr(self) -> int:
        return self.ptr

    def len(self) -> int:
        return self.nbytes // self.dtype.itemsize

    def __len__(self) -> int:
        return self.len()

    def free(self) -> None:
        if self._buf is not None:
            call("fg_buf_free", self._buf)
            self._buf = None


@dataclass
class AllocTensors:
    """AllocTensors (dispatch/mod.rs:835-845)."""
    forward_saved: List[Tensor]
    grad_tensors: List[Tensor]
    forward_out: Tensor
    seed: Tensor
    loss_t: Tensor
    state: List[Tensor]
    mean_loss: Optional[Tensor]
    plan: "Plan"


class Plan:
    """Owns an fg_plan (lowered graph + device arena)."""

    def __init__(self, ctx: "GpuContext", graph: Graph, binding: Sequence[int]):
        self.ctx = ctx
        nf = max(len(binding) - 1, graph._nfields())
        h = graph._c_graph(nf)
        p = ctypes.c_void_p()
        try:
            arr = (ctypes.c_uint32 * len(binding))(*binding)
            call("fg_plan_create", ctx.ctx.handle, h, arr, len(binding), ctypes.byref(p))
        finally:
            call("fg_graph_destroy", h)
        self.handle = p
        ctx.ctx.adopt(self)

    def count(self, role: int) -> int:
        c = ctypes.c_int()
        call("fg_plan_count", self.handle, role, ctypes.byref(c))
        return c.value

    def tensor(self, role: int, index: int = 0, dtype=None) -> Tensor:
        """A role's index-th tensor; its host dtype follows the plan's element
        type (float32, float16, or uint16 words for bfloat16) unless given
        (labels are u32: pass np.uint32)."""
        ptr = ctypes.c_void_p()
        nb = ctypes.c_uint64()
        node = ctypes.c_uint32()
        call("fg_plan_tensor", self.handle, role, index, ctypes.byref(ptr), ctypes.byref(nb),
             ctypes.byref(node))
        if dtype is None:
            code = ctypes.c_int()
            call("fg_plan_tensor_dtype", self.handle, role, index, ctypes.byref(code))
            dtype = _CODE_NP[code.value]
        t = Tensor(ptr.value or 0, nb.value, (nb.value // np.dtype(dtype).itemsize,), dtype,
                   owner=self)
        t.node = node.value
        return t

    def describe(self) -> str:
        need = ctypes.c_size_t()
        call("fg_plan_describe", self.handle, None, 0, ctypes.byref(need))
        buf = ctypes.create_string_buffer(need.value)
        call("fg_plan_describe", self.handle, buf, need.value, None)
        return buf.value.decode()

    def close(self) -> None:
        if self.handle:
            call("fg_plan_destroy", self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass


class Schedule:
    def __init__(self, plan: Plan, in_tensors: Sequence[Tensor]):
        self.plan = plan
        self.in_tensors = list(in_tensors)


# ----------------------------------------------------------------- context
class GpuContext:
    """GpuContext (crates/ferrograd/src/backend.rs:54-314)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx

    @staticmethod
    def new(device: int = 0) -> "GpuContext":
        """Bind device 0 on a fresh torch stream when torch is present (so
        torch tensors and this context share one queue), else a private
        stream.  Raises FgError when there is no gfx950 device."""
        try:
            import torch  # noqa: F401
            from . import torch_context

            if torch.cuda.is_available():
                ctx, _ = torch_context(device)
                return GpuContext(ctx)
        except ImportError:
            pass
        return GpuContext(Context(device))

    def detect_target(self):
        return {"arch": self.ctx.arch, "lin_acc": bool(self.ctx.flags & 1)}

    def alloc_meta(self, binding: Sequence[int]) -> List[int]:
        return [int(x) for x in binding]

    def alloc_tensors(self, graph: Graph, saved, meta_binding: Sequence[int],
                      state=None) -> AllocTensors:
        plan = Plan(self, graph, meta_binding)
        fs = [plan.tensor(ROLE_FORWARD_SAVED, i) for i in range(plan.count(ROLE_FORWARD_SAVED))]
        gr = [plan.tensor(ROLE_GRAD, i) for i in range(plan.count(ROLE_GRAD))]
        st = [plan.tensor(ROLE_STATE, i) for i in range(plan.count(ROLE_STATE))]
        mean = plan.tensor(ROLE_MEAN_LOSS) if plan.count(ROLE_MEAN_LOSS) else None
        return AllocTensors(fs, gr, plan.tensor(ROLE_FORWARD_OUT), plan.tensor(ROLE_SEED),
                            plan.tensor(ROLE_LOSS), st, mean, plan)

    def compile(self, ir: LoweredGraph, options=None) -> LoweredGraph:
        return ir  # kernels are compiled ahead of time for gfx950

    def _alloc(self, data: np.ndarray, shape) -> Tensor:
        data = np.ascontiguousarray(data)
        h = ctypes.c_void_p()
        call("fg_buf_alloc_init", self.ctx.handle, data.ctypes.data, data.nbytes, ctypes.byref(h))
        ptr = call_ptr(h)
        return Tensor(ptr, data.nbytes, shape, data.dtype, owner=self, buf=h)

    def init_tensor_f32(self, shape: Sequence[int], data) -> Tensor:
        a = np.asarray(data, dtype=np.float32).reshape(-1)
        if a.size != int(np.prod(shape)):
            raise FgError(5, f"init_tensor_f32: {a.size} values for shape {tuple(shape)}")
        return self._alloc(a, shape)

    def init_tensor_f16(self, shape: Sequence[int], data) -> Tensor:
        """GpuContext::init_tensor_f16 (dispatch/mod.rs:614-628)."""
        a = np.asarray(data, dtype=np.float16).reshape(-1)
        if a.size != int(np.prod(shape)):
            raise FgError(5, f"init_tensor_f16: {a.size} values for shape {tuple(shape)}")
        return self._alloc(a, shape)

    def init_tensor_bf16(self, shape: Sequence[int], data) -> Tensor:
        """GpuContext::init_tensor_bf16 (dispatch/mod.rs:630-645): float
        values are rounded to bfloat16; uint16 arrays are taken as words."""
        a = np.asarray(data)
        a = (a.astype(np.uint16) if a.dtype == np.uint16 else bf16_from_f32(a)).reshape(-1)
        if a.size != int(np.prod(shape)):
            raise FgError(5, f"init_tensor_bf16: {a.size} values for shape {tuple(shape)}")
        return self._alloc(a, shape)

    def new_onehot_init(self, labels: Sequence[int]) -> Tensor:
        """u32 class labels, one per row (dispatch/mod.rs:647-662)."""
        a = np.asarray(labels, dtype=np.uint32).reshape(-1)
        return self._alloc(a, (a.size,))

    def upload(self, t: Tensor, data, offset: int = 0) -> None:
        """Copy host data into t (converted to t's element type; float data
        for a bfloat16 tensor is rounded to it)."""
        d = np.asarray(data)
        if t.dtype == np.uint16 and d.dtype != np.uint16:
            d = bf16_from_f32(d)
        a = np.ascontiguousarray(np.asarray(d, dtype=t.dtype).reshape(-1))
        off = int(offset) * t.dtype.itemsize
        if off + a.nbytes > t.nbytes:
            raise FgError(9, f"upload: {a.nbytes} bytes at {off} exceed {t.nbytes}")
        call("fg_memcpy_h2d", self.ctx.handle, t.ptr + off, a.ctypes.data, a.nbytes)

    def download(self, t: Tensor, dst: Optional[np.ndarray] = None, offset: int = 0) -> np.ndarray:
        off = int(offset) * t.dtype.itemsize
        if dst is None:
            dst = np.empty((t.nbytes - off) // t.dtype.itemsize, dtype=t.dtype)
        n = min(dst.nbytes, t.nbytes - off)
        call("fg_memcpy_d2h", self.ctx.handle, dst.ctypes.data, t.ptr + off, n)
        return dst

    def schedule(self, kernels: LoweredGraph, meta, in_tensors: Sequence[Tensor],
                 saved_tensors: AllocTensors, state=None, *_extra) -> Schedule:
        plan = saved_tensors.plan
        n = plan.count(ROLE_INPUT)
        if len(in_tensors) != n:
            raise FgError(1, f"schedule: {len(in_tensors)} in_tensors for {n} inputs")
        for i, t in enumerate(in_tensors):
            call("fg_plan_bind_input", plan.handle, i, t.data_ptr(), tensor_nbytes(t))
        lr_bits = int(meta[0]) if meta else f32_bits(1e-3)
        call("fg_plan_set_lr", plan.handle, struct.unpack("<f", struct.pack("<I", lr_bits))[0])
        return Schedule(plan, in_tensors)

    def dispatch_forward(self, s: Schedule) -> None:
        call("fg_plan_forward", s.plan.handle)

    def dispatch_loss(self, s: Schedule, target: Tensor) -> None:
        call("fg_plan_bind_target", s.plan.handle, target.data_ptr(), tensor_nbytes(target))
        call("fg_plan_loss", s.plan.handle)

    def dispatch_backward(self, s: Schedule) -> None:
        call("fg_plan_backward", s.plan.handle)

    def dispatch_optim(self, s: Schedule) -> None:
        call("fg_plan_optim", s.plan.handle)

    def dispatch_single_optim(self, s: Schedule, weight: Tensor, grad: int = 0,
                              tensors: Optional[AllocTensors] = None) -> None:
        idx = [t.data_ptr() for t in s.in_tensors].index(weight.data_ptr())
        call("fg_plan_single_optim", s.plan.handle, idx)

    def sync(self) -> None:
        self.ctx.sync()

    # ---------------------------------------------------- extensions
    def capture_step(self, s: Schedule, target: Tensor) -> None:
        """Capture forward + loss + backward + optim into one hipGraph."""
        call("fg_plan_bind_target", s.plan.handle, target.data_ptr(), tensor_nbytes(target))
        call("fg_plan_capture_step", s.plan.handle)

    def launch_step(self, s: Schedule) -> None:
        """Replay the captured training step."""
        call("fg_plan_launch_step", s.plan.handle)


def call_ptr(buf_handle) -> int:
    from ._lib import load

    return int(load().fg_buf_device_ptr(buf_handle) or 0)


def tensor_nbytes(t) -> int:
    if isinstance(t, Tensor):
        return t.nbytes
    return int(t.numel() * t.element_size())
