"""GPU tests of the graph path with 16-bit tensors (SimpleDType F16 / BF16).

The first test re-hosts the reference's own 16-bit test
(crates/ferrograd/tests/nonf32.rs:11-99) with its exact expectations; the
second runs a two-layer MLP step (bias + ReLU, softmax-CE, SGD) in each
16-bit type against the oracle's 16-bit operations composed the same way,
small and at a size whose GEMMs split K; the third checks a 16-bit step whose
plan pairs a 4096-wide layer's gradient GEMMs in one launch against the
same step from single calls, bit for bit.
"""
import math

import numpy as np
import pytest

import oracle as O
from conftest import normwise_rel

pytestmark = pytest.mark.gpu

f32 = np.float32


def api():
    from ferrograd_amd import graph as G
    return G


@pytest.fixture(scope="module")
def ctx(gpu_ctx):
    from ferrograd_amd.graph import GpuContext
    return GpuContext(gpu_ctx)


@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_mul_add_16bit(ctx, kind):
    """nonf32.rs:11-99 (mul_add_f16): c + a*b over 32x32 inputs of 3, 2, 1;
    seed 1; out 7, grads 2, 3, 1 exactly (run for bf16 as well)."""
    G = api()
    graph, meta = G.Graph(G.MEAN_SQUARED_ERROR, G.Optim.sgd().lower), G.Metadata.new()
    m, n = meta.new_field(), meta.new_field()
    with graph.define_ops() as ops:
        a = ops.input([m, n], kind)
        b = ops.input([m, n], kind)
        c = ops.input([m, n], kind)
        x = ops.mul(a, b)
        ops.add(c, x)
    saved = graph.compute_saved_nodes()
    graph.validate(meta)
    mb = [G.f32_bits(1e-3), 32, 32]
    st = ctx.alloc_tensors(graph, saved, mb, G.Optim.sgd().state)
    init = ctx.init_tensor_f16 if kind == "f16" else ctx.init_tensor_bf16
    ins = [init([32, 32], [3.0] * 1024), init([32, 32], [2.0] * 1024),
           init([32, 32], [1.0] * 1024)]
    ctx.upload(st.seed, [1.0] * 1024, 0)
    sch = ctx.schedule(ctx.compile(graph.lower(meta, None, saved)), mb, ins, st)
    ctx.dispatch_forward(sch)
    ctx.dispatch_backward(sch)
    ctx.sync()

    def vals(t):
        d = ctx.download(t)
        return d.astype(f32) if kind == "f16" else G.bf16_to_f32(d)

    assert st.forward_out.nbytes == 1024 * 2
    assert np.all(vals(st.forward_out) == 7.0)
    assert np.all(vals(st.grad_tensors[0]) == 2.0)
    assert np.all(vals(st.grad_tensors[1]) == 3.0)
    assert np.all(vals(st.grad_tensors[2]) == 1.0)


@pytest.mark.parametrize("size", ["small", "split"])
@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_mlp_step_16bit_matches_oracle(ctx, kind, size):
    """batch 64, 96 -> 128 -> ReLU -> 40 (small), or batch 2048, 1024 ->
    1024 -> ReLU -> 1000 (split: the two forward GEMMs and the first layer's
    data gradient split K into the plan's workspace), softmax-CE, SGD lr
    0.01, all tensors of one 16-bit type.  The oracle composes its 16-bit
    GEMMs (fp32 sums, each node value rounded), softmax-CE on the widened
    logits with dlogits rounded, column sums rounded; the GPU must agree
    within two units in the last place of the type (normwise)."""
    import ferrograd_amd as fa
    G = api()
    dt = O.F16 if kind == "f16" else O.BF16
    eps = 2.0 ** -10 if kind == "f16" else 2.0 ** -7
    dims, B = ([96, 128, 40], 64) if size == "small" else ([1024, 1024, 1000], 2048)
    graph, meta = G.Graph(G.CROSS_ENTROPY, G.Optim.sgd().lower), G.Metadata.new()
    fb = meta.new_field()
    fd = [meta.new_field() for _ in dims]
    with graph.define_ops() as ops:
        h = ops.input([fb, fd[0]], kind, trainable=False)
        for l in range(2):
            W = ops.input([fd[l], fd[l + 1]], kind)
            b = ops.input([fd[l + 1]], kind)
            z = ops.bias_add(ops.matmul(h, W), b)
            h = ops.relu(z) if l == 0 else z
        ops.softmax(h)
    mb = [G.f32_bits(0.01), B] + dims
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    X16 = O.from_f32(dt, fa.rng_uniform(0, 0, (B, dims[0])))
    y = fa.rng_int(0, 1, (B,), dims[-1])
    W16 = [O.from_f32(dt, fa.rng_uniform(0, 10 + l, (dims[l], dims[l + 1]),
                                         -math.sqrt(6 / dims[l]), math.sqrt(6 / dims[l])))
           for l in range(2)]
    b16 = [O.from_f32(dt, 0.05 * fa.rng_normal(0, 20 + l, (dims[l + 1],))) for l in range(2)]

    def dev(bits):
        if kind == "f16":
            return ctx.init_tensor_f16(bits.shape, bits.view(np.float16))
        return ctx.init_tensor_bf16(bits.shape, bits)

    ins = [dev(X16)]
    for W, b in zip(W16, b16):
        ins += [dev(W), dev(b)]
    tgt = ctx.new_onehot_init(y)
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    desc = st.plan.describe()
    assert ("[K split: slices + summing kernel]" in desc) == (size == "split"), desc
    ctx.dispatch_forward(sch)
    ctx.dispatch_loss(sch, tgt)
    ctx.dispatch_backward(sch)
    ctx.sync()

    # Oracle, in the same node order.
    H1, Z1 = O.gemm_x16(dt, O.NN, X16, W16[0], bias=b16[0], act=O.ACT_RELU, want_z=True)
    Z2 = O.gemm_x16(dt, O.NN, H1, W16[1], bias=b16[1])
    rl, d2, _, mean = O.softmax_ce(O.to_f32(dt, Z2), y)
    dZ2 = O.from_f32(dt, d2)
    db2 = O.from_f32(dt, O.to_f32(dt, dZ2).astype(np.float64).sum(0).astype(f32))
    dW2 = O.gemm_x16(dt, O.TN, H1, dZ2)
    dZ1 = O.gemm_bwd_x16(dt, O.NT, dZ2, W16[1], act=O.ACT_RELU, Zs=Z1)
    db1 = O.from_f32(dt, O.to_f32(dt, dZ1).astype(np.float64).sum(0).astype(f32))
    dW1 = O.gemm_x16(dt, O.TN, X16, dZ1)
    dX = O.gemm_bwd_x16(dt, O.NT, dZ1, W16[0])

    def gpu(t):
        d = ctx.download(t)
        return d.astype(f32) if kind == "f16" else G.bf16_to_f32(d)

    assert abs(float(ctx.download(st.mean_loss)[0]) - mean) < 4 * eps * max(1.0, abs(mean))
    grads = {t.node: gpu(t) for t in st.grad_tensors}
    in_nodes = [i for i, nd in enumerate(graph.nodes) if nd.op == 0]
    for node, ref in zip(in_nodes, [dX, dW1, db1, dW2, db2]):
        r = O.to_f32(dt, ref)
        assert normwise_rel(grads[node].reshape(r.shape), r) <= 2 * eps, node
    # SGD on the device's own gradients: w = round(w - g*lr), bit for bit.
    ctx.dispatch_optim(sch)
    ctx.sync()
    for k, (t, w0) in enumerate(zip(ins[1:], [W16[0], b16[0], W16[1], b16[1]])):
        w = O.to_f32(dt, w0).reshape(-1).copy()
        g = grads[in_nodes[k + 1]].reshape(-1).astype(f32).copy()
        O.sgd_(w, g, f32(0.01), True)
        got = ctx.download(t)
        got = got.view(np.uint16) if kind == "f16" else got
        assert np.array_equal(got.reshape(-1), O.from_f32(dt, w)), k


@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_step_with_pair_and_split_matches_single_calls(ctx, kind):
    """16-bit MLP (batch 2048, 256 -> 4096 -> 4096 -> 16, GELU, CE): the plan
    runs the 4096-wide layer's dW and dX as one launch (gemm16_pair_big) and
    splits the first layer's dW with its column sums into its workspace; the
    same step from single calls, on a context whose workspace takes the same
    K splits, gives every gradient bit for bit."""
    torch = pytest.importorskip("torch")
    import ferrograd_amd as fa
    G = api()
    dt, bf = (O.F16, fa.DTYPE_F16) if kind == "f16" else (O.BF16, fa.DTYPE_BF16)
    dims, B = [256, 4096, 4096, 16], 2048
    graph, meta = G.Graph(G.CROSS_ENTROPY, G.Optim.sgd().lower), G.Metadata.new()
    fb = meta.new_field()
    fd = [meta.new_field() for _ in dims]
    with graph.define_ops() as ops:
        h = ops.input([fb, fd[0]], kind, trainable=False)
        for l in range(3):
            W = ops.input([fd[l], fd[l + 1]], kind)
            b = ops.input([fd[l + 1]], kind)
            z = ops.bias_add(ops.matmul(h, W), b)
            h = ops.gelu(z) if l < 2 else z
        ops.softmax(h)
    mb = [G.f32_bits(0.01), B] + dims
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    X16 = O.from_f32(dt, fa.rng_uniform(0, 0, (B, dims[0])))
    y = fa.rng_int(0, 1, (B,), dims[-1])
    Ws = [O.from_f32(dt, fa.rng_uniform(0, 10 + l, (dims[l], dims[l + 1]),
                                        -math.sqrt(6 / dims[l]), math.sqrt(6 / dims[l])))
          for l in range(3)]
    bs = [O.from_f32(dt, 0.05 * fa.rng_normal(0, 20 + l, (dims[l + 1],))) for l in range(3)]
    def dev(bits):
        if kind == "f16":
            return ctx.init_tensor_f16(bits.shape, bits.view(np.float16))
        return ctx.init_tensor_bf16(bits.shape, bits)

    ins = [dev(X16)]
    for W, b in zip(Ws, bs):
        ins += [dev(W), dev(b)]
    tgt = ctx.new_onehot_init(y)
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    ctx.dispatch_forward(sch)
    ctx.dispatch_loss(sch, tgt)
    ctx.dispatch_backward(sch)
    ctx.sync()
    grads = {t.node: np.asarray(ctx.download(t)).view(np.uint16).reshape(-1)
             for t in st.grad_tensors}
    in_nodes = [i for i, nd in enumerate(graph.nodes) if nd.op == 0]
    own = fa.Context(0, ctx.ctx.stream)
    try:
        own.reserve_workspace(64 << 20)
        x, w1, b1, w2, b2, w3, b3 = ins

        def buf(*shape):
            return torch.zeros(shape, dtype=torch.int16, device="cuda")
        d0, d1, d2, d3 = dims
        Z1, H1, Z2, H2, L = buf(B, d1), buf(B, d1), buf(B, d2), buf(B, d2), buf(B, d3)
        own.gemm_x16(bf, fa.NN, B, d1, d0, x, d0, w1, d1, H1, d1, bias=b1, act=fa.ACT_GELU,
                     Z=Z1, ldz=d1)
        own.gemm_x16(bf, fa.NN, B, d2, d1, H1, d1, w2, d2, H2, d2, bias=b2, act=fa.ACT_GELU,
                     Z=Z2, ldz=d2)
        own.gemm_x16(bf, fa.NN, B, d3, d2, H2, d2, w3, d3, L, d3, bias=b3)
        dl = buf(B, d3)
        own.softmax_ce(L, d3, tgt, B, d3, 1.0, dlogits=dl, ldd=d3, dtype=bf)
        dW3, db3, dZ2 = buf(d2, d3), buf(d3), buf(B, d2)
        own.gemm_dw_x16(bf, d2, d3, B, H2, d2, dl, d3, dW3, d3, colsum=db3)
        own.gemm_bwd_x16(bf, fa.NT, B, d2, d3, dl, d3, w3, d3, dZ2, d2, act=fa.ACT_GELU,
                         Zs=Z2, ldzs=d2)
        dW2, db2, dZ1 = buf(d1, d2), buf(d2), buf(B, d1)
        own.gemm_dw_x16(bf, d1, d2, B, H1, d1, dZ2, d2, dW2, d2, colsum=db2)
        own.gemm_bwd_x16(bf, fa.NT, B, d1, d2, dZ2, d2, w2, d2, dZ1, d1, act=fa.ACT_GELU,
                         Zs=Z1, ldzs=d1)
        dW1, db1, dX = buf(d0, d1), buf(d1), buf(B, d0)
        own.gemm_dw_x16(bf, d0, d1, B, x, d0, dZ1, d1, dW1, d1, colsum=db1)
        own.gemm_bwd_x16(bf, fa.NT, B, d0, d1, dZ1, d1, w1, d1, dX, d0)
        own.sync()
        ref = [dX, dW1, db1, dW2, db2, dW3, db3]
        for node, r in zip(in_nodes, ref):
            assert np.array_equal(grads[node], r.cpu().numpy().view(np.uint16).reshape(-1)), node
    finally:
        own.close()
