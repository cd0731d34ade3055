"""CPU tests of the graph planner: validation errors and the fused launch
lists it builds (dry plans -- lowering only, no device)."""
import re

import pytest

from ferrograd_amd import FgError
from ferrograd_amd.graph import (BINARY_CROSS_ENTROPY, CROSS_ENTROPY, MEAN_SQUARED_ERROR, Graph,
                                 Metadata, Optim, SimpleDType, f32_bits)


def section(desc, name):
    m = re.search(rf"^{re.escape(name)}: (\d+) launches\n((?:  .*\n)*)", desc, re.M)
    assert m, desc
    return int(m.group(1)), [l.strip() for l in m.group(2).splitlines() if l.strip()]


def mlp_graph(dims, act="gelu", optim=None, loss=CROSS_ENTROPY):
    meta = Metadata.new()
    B = meta.new_field()
    d = [meta.new_field() for _ in dims]
    g = Graph(loss, (optim or Optim.adam()).lower)
    with g.define_ops() as ops:
        x = ops.input([B, d[0]], SimpleDType.F32, trainable=False)
        h = x
        for l in range(len(dims) - 1):
            W = ops.input([d[l], d[l + 1]])
            b = ops.input([d[l + 1]])
            z = ops.bias_add(ops.matmul(h, W), b)
            h = getattr(ops, act)(z) if l < len(dims) - 2 else z
        ops.softmax(h)
    return g, meta


def test_mlp_lowers_to_fused_gemm_launches():
    dims = [1024, 4096, 4096, 1000]
    g, meta = mlp_graph(dims)
    desc = g.describe([f32_bits(1e-3), 2048] + dims)
    n, fwd = section(desc, "forward")
    assert n == 4  # 3 GEMMs (bias + act fused) + the softmax for forward_out
    assert fwd[0].startswith("forward gemm NN 2048x4096x1024 +bias +gelu")
    assert fwd[1].startswith("forward gemm NN 2048x4096x4096 +bias +gelu")
    assert fwd[2].startswith("forward gemm NN 2048x1000x4096 +bias ->")
    assert fwd[3].startswith("forward softmax 2048x1000")
    n, loss = section(desc, "loss")
    assert n == 1 and loss[0].startswith("loss softmax+ce 2048x1000")
    n, bwd = section(desc, "backward(ce-fused)")
    kinds = [l.split(" ")[1] + " " + l.split(" ")[2] for l in bwd]
    # per layer: dW (TN) with the bias gradient fused, dX (NT, with the lower
    # layer's gelu' fused); no separate bias-gradient launch
    assert kinds.count("gemm TN") == 3 and not any("bias_grad" in k for k in kinds)
    assert sum("+dbias" in l for l in bwd) == 3
    assert sum("gelu'" in l for l in bwd) == 2
    assert sum(l.startswith("backward gemm NT") for l in bwd) == 3  # incl. dX of the data
    assert "eltwise" not in "\n".join(bwd)  # no standalone activation backward
    assert "adam over 6 inputs" in desc      # X is frozen: grads but no update
    # A captured step leaves the final softmax to the loss launch (which
    # writes forward_out too): forward 3; the loss is the row kernel + mean.
    assert "kernels per step: 13 (forward 3, loss 2, backward 6, optim 2)" in desc


def test_reference_graph_mul_add_is_one_elementwise_launch():
    meta = Metadata.new()
    m, n = meta.new_field(), meta.new_field()
    g = Graph(MEAN_SQUARED_ERROR, Optim.sgd().lower)
    with g.define_ops() as ops:
        a = ops.input([m, n], SimpleDType.F32)
        b = ops.input([m, n], SimpleDType.F32)
        c = ops.input([m, n], SimpleDType.F32)
        ops.add(c, ops.mul(a, b))
    desc = g.describe([f32_bits(1e-3), 32, 32])
    n_f, fwd = section(desc, "forward")
    assert n_f == 1 and "mul#3,add#4" in fwd[0]
    assert g.compute_saved_nodes() == [2, 2, 2, 0, 0]


def test_reference_graph_matmul_chain3_saved_nodes():
    meta = Metadata.new()
    m, n, k, h = (meta.new_field() for _ in range(4))
    g = Graph(MEAN_SQUARED_ERROR, Optim.sgd().lower)
    with g.define_ops() as ops:
        a = ops.input([m, k], SimpleDType.F32)
        b = ops.input([k, n], SimpleDType.F32)
        c = ops.input([h, m], SimpleDType.F32)
        d = ops.input([n, h], SimpleDType.F32)
        e = ops.input([h, h], SimpleDType.F32)
        x = ops.matmul(a, b)
        y = ops.matmul(c, x)
        z = ops.matmul(y, d)
        ops.add(z, e)
    saved = g.compute_saved_nodes()
    assert [i for i, s in enumerate(saved) if s & 1] == [5, 6, 7]  # X, Y, Z
    desc = g.describe([f32_bits(1e-3), 32, 64, 128, 256])
    n_f, fwd = section(desc, "forward")
    assert n_f == 4  # three GEMMs and the elementwise add
    n_b, bwd = section(desc, "backward(seed)")
    assert sum(l.startswith("backward gemm") for l in bwd) == 6


def test_validation_errors():
    meta = Metadata.new()
    m, n, k = meta.new_field(), meta.new_field(), meta.new_field()
    g = Graph(MEAN_SQUARED_ERROR, Optim.sgd().lower)
    with g.define_ops() as ops:
        a = ops.input([m, k])
        b = ops.input([n, k])
        ops.matmul(a, b)
    with pytest.raises(FgError) as e:
        g.validate(meta, [f32_bits(1e-3), 32, 64, 16])
    assert e.value.code == 5 and "inner dims" in str(e.value)
    g.validate(meta, [f32_bits(1e-3), 32, 16, 16])  # k == n: fine
    with pytest.raises(FgError) as e:                 # missing metadata field
        g.validate(meta, [f32_bits(1e-3), 32, 16])
    assert e.value.code == 6
    g2 = Graph(MEAN_SQUARED_ERROR, Optim.sgd().lower)
    with g2.define_ops() as ops:
        with pytest.raises(FgError):
            ops.add(0, 1)  # nodes that do not exist
    # arbitrary dims (the reference requires multiples of 16)
    assert meta.validate_meta([f32_bits(1e-3), 10, 1000, 3])


def test_losses_lower():
    for loss in (MEAN_SQUARED_ERROR, BINARY_CROSS_ENTROPY, CROSS_ENTROPY):
        meta = Metadata.new()
        m, n = meta.new_field(), meta.new_field()
        g = Graph(loss, Optim.sgd().lower)
        with g.define_ops() as ops:
            a = ops.input([m, n])
            ops.tanh(a)
        desc = g.describe([f32_bits(1e-3), 8, 10])
        n_l, lines = section(desc, "loss")
        assert n_l == 1 and "eltwise" in lines[0]


def test_unknown_operation_kind_is_unsupported():
    """An operation code outside fg_op -- a GraphOp::Custom the Rust mirror
    could not map to a ferrograd-nn builder -- is refused with
    FG_ERR_UNSUPPORTED (ErrorKind::UnsupportedFeature) and a message that
    names it; leaves passed to fg_graph_op are invalid arguments."""
    import ctypes

    from ferrograd_amd._lib import call
    g = ctypes.c_void_p()
    call("fg_graph_create", 0, 0, ctypes.byref(g))
    try:
        f = ctypes.c_uint32()
        call("fg_graph_new_field", g, ctypes.byref(f))
        fields = (ctypes.c_uint32 * 2)(f.value, f.value)
        x = ctypes.c_uint32()
        call("fg_graph_input", g, fields, 2, ctypes.byref(x))
        ins = (ctypes.c_uint32 * 1)(x.value)
        node = ctypes.c_uint32()
        with pytest.raises(FgError) as e:
            call("fg_graph_op", g, 99, ins, 1, ctypes.byref(node))
        assert e.value.code == 3 and "operation kind 99" in str(e.value)
        with pytest.raises(FgError) as e:
            call("fg_graph_op", g, 0, ins, 1, ctypes.byref(node))  # FG_OP_INPUT
        assert e.value.code == 1
        call("fg_graph_op", g, 7, ins, 1, ctypes.byref(node))  # relu: fine
    finally:
        call("fg_graph_destroy", g)


def test_c1_step_dispatches():
    """BASELINE c1 (batch 64, 784 -> 256 -> ReLU -> 10, CE, SGD), planned
    without a device (so no GEMM splits K): a captured step is 2 forward
    GEMMs (the final softmax is left to the loss launch), 1 loss launch (one
    workgroup, the mean included), 4 backward GEMMs (dbias fused into the dW
    GEMMs) and 1 SGD update."""
    g, meta = mlp_graph([784, 256, 10], act="relu", optim=Optim.sgd())
    desc = g.describe([f32_bits(0.01), 64, 784, 256, 10])
    assert "kernels per step: 8 (forward 2, loss 1, backward 4, optim 1)" in desc, desc
