"""GPU tests of the graph path (planner + executor) through the ferrograd
API mirror.

The first block re-hosts the reference's own integration tests
(crates/ferrograd/tests/std_wgsl.rs, tests/optim.rs) with their exact
closed-form expectations; the rest compare whole training steps with the CPU
oracle (BASELINE configs c1 and a reduced c5), the three losses and every
elementwise op's backward with float64 numpy, and check that a captured
hipGraph step replays like the eager step.
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


def new_graph(loss, optim=None):
    G = api()
    return G.Graph(loss, (optim or G.Optim.sgd()).lower), G.Metadata.new()


# ------------------------------------------------ reference tests, re-hosted
def test_mul_add_forward_backward(ctx):
    """std_wgsl.rs:10-94."""
    G = api()
    graph, meta = new_graph(G.MEAN_SQUARED_ERROR)
    m, n = meta.new_field(), meta.new_field()
    with graph.define_ops() as ops:
        a = ops.input([m, n], G.SimpleDType.F32)
        b = ops.input([m, n], G.SimpleDType.F32)
        c = ops.input([m, n], G.SimpleDType.F32)
        x = ops.mul(a, b)
        ops.add(c, x)
    saved = graph.compute_saved_nodes()
    graph.validate(meta)
    mb = [G.f32_bits(1e-3), 32, 32]
    assert meta.validate_meta(mb)
    mb = ctx.alloc_meta(mb)
    st = ctx.alloc_tensors(graph, saved, mb, G.Optim.sgd().state)
    kernels = ctx.compile(graph.lower(meta, None, saved))
    ins = [ctx.init_tensor_f32([32, 32], [3.0] * 1024), ctx.init_tensor_f32([32, 32], [2.0] * 1024),
           ctx.init_tensor_f32([32, 32], [1.0] * 1024)]
    ctx.upload(st.seed, [1.0] * 1024, 0)
    sch = ctx.schedule(kernels, mb, ins, st, [], G.Optim.sgd().state)
    ctx.dispatch_forward(sch)
    ctx.dispatch_backward(sch)
    ctx.sync()
    assert np.all(ctx.download(st.forward_out) == 7.0)
    assert np.all(ctx.download(st.grad_tensors[0]) == 2.0)
    assert np.all(ctx.download(st.grad_tensors[1]) == 3.0)
    assert np.all(ctx.download(st.grad_tensors[2]) == 1.0)


def test_matmul_sub_softmax_forward_backward(ctx):
    """std_wgsl.rs:97-187: softmax(c - a@b), seed 1 -> every grad 0."""
    G = api()
    graph, meta = new_graph(G.CROSS_ENTROPY)
    m, n, k = meta.new_field(), meta.new_field(), meta.new_field()
    with graph.define_ops() as ops:
        a = ops.input([m, k])
        b = ops.input([k, n])
        c = ops.input([m, n])
        ops.softmax(ops.sub(c, ops.matmul(a, b)))
    mb = [G.f32_bits(1e-3), 16, 64, 32]
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    ins = [ctx.init_tensor_f32([16, 32], [3.0] * 512), ctx.init_tensor_f32([32, 64], [2.0] * 2048),
           ctx.init_tensor_f32([16, 64], [1.0] * 1024)]
    ctx.upload(st.seed, [1.0] * 1024, 0)
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    ctx.dispatch_forward(sch)
    ctx.dispatch_backward(sch)
    ctx.sync()
    assert np.all(ctx.download(st.forward_out) == f32(1 / 64))
    assert np.all(ctx.download(st.grad_tensors[0])[:512] == 0.0)
    assert np.all(ctx.download(st.grad_tensors[1]) == 0.0)
    assert np.all(ctx.download(st.grad_tensors[2])[:1024] == 0.0)


def test_div_const_softmax_forward_backward(ctx):
    """std_wgsl.rs:190-265: softmax(2/x) + 2 -> 2 + 1/32, grad 0."""
    G = api()
    graph, meta = new_graph(G.CROSS_ENTROPY)
    m, n = meta.new_field(), meta.new_field()
    with graph.define_ops() as ops:
        x = ops.input([m, n])
        two = ops.constant_f32(2.0)
        ops.add(ops.softmax(ops.div(two, x)), two)
    mb = [G.f32_bits(1e-3), 16, 32]
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    ins = [ctx.init_tensor_f32([16, 32], [3.0] * 512)]
    ctx.upload(st.seed, [1.0] * 512, 0)
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    ctx.dispatch_forward(sch)
    ctx.dispatch_backward(sch)
    ctx.sync()
    assert np.all(ctx.download(st.forward_out) == f32(2.0 + 1.0 / 32.0))
    assert np.all(ctx.download(st.grad_tensors[0]) == 0.0)


def test_matmul_add_forward_backward(ctx):
    """std_wgsl.rs:268-373: a@b + c -> 97; dA 128, dB 96, dC 1."""
    G = api()
    M, N, K = 32, 64, 16
    graph, meta = new_graph(G.MEAN_SQUARED_ERROR)
    m, n, k = meta.new_field(), meta.new_field(), meta.new_field()
    with graph.define_ops() as ops:
        a = ops.input([m, k])
        b = ops.input([k, n])
        c = ops.input([m, n])
        ops.add(ops.matmul(a, b), c)
    mb = [G.f32_bits(1e-3), M, N, K]
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    ins = [ctx.init_tensor_f32([M, K], [3.0] * (M * K)), ctx.init_tensor_f32([K, N], [2.0] * (K * N)),
           ctx.init_tensor_f32([M, N], [1.0] * (M * N))]
    ctx.upload(st.seed, [1.0] * (M * N), 0)
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    ctx.dispatch_forward(sch)
    ctx.dispatch_backward(sch)
    ctx.sync()
    assert np.all(ctx.download(st.forward_out) == 97.0)
    assert np.all(ctx.download(st.grad_tensors[0]) == 128.0)
    assert np.all(ctx.download(st.grad_tensors[1]) == 96.0)
    assert np.all(ctx.download(st.grad_tensors[2]) == 1.0)


def test_matmul_chain3_forward_backward(ctx):
    """std_wgsl.rs:376-520."""
    G = api()
    M, N, K, H = 32, 64, 128, 256
    A_VAL, B_VAL, C_VAL, D_VAL, E_VAL = 3.0, 2.0, 1.0, 0.5, 1.0
    X_VAL = A_VAL * B_VAL * K
    Y_VAL = C_VAL * X_VAL * M
    Z_VAL = Y_VAL * D_VAL * N
    Y_GRAD = D_VAL * H
    X_GRAD = Y_GRAD * C_VAL * H
    D_GRAD = Y_VAL * H
    C_GRAD = Y_GRAD * X_VAL * N
    B_GRAD = A_VAL * X_GRAD * M
    A_GRAD = X_GRAD * B_VAL * N
    graph, meta = new_graph(G.MEAN_SQUARED_ERROR)
    m, n, k, h = (meta.new_field() for _ in range(4))
    with graph.define_ops() as ops:
        a = ops.input([m, k])
        b = ops.input([k, n])
        c = ops.input([h, m])
        d = ops.input([n, h])
        e = ops.input([h, h])
        x = ops.matmul(a, b)
        y = ops.matmul(c, x)
        z = ops.matmul(y, d)
        ops.add(z, e)
    mb = [G.f32_bits(1e-3), M, N, K, H]
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    ins = [ctx.init_tensor_f32([M, K], [A_VAL] * (M * K)),
           ctx.init_tensor_f32([K, N], [B_VAL] * (K * N)),
           ctx.init_tensor_f32([H, M], [C_VAL] * (H * M)),
           ctx.init_tensor_f32([N, H], [D_VAL] * (N * H)),
           ctx.init_tensor_f32([H, H], [E_VAL] * (H * H))]
    ctx.upload(st.seed, [1.0] * (H * H), 0)
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    ctx.dispatch_forward(sch)
    ctx.dispatch_backward(sch)
    ctx.sync()
    fs = st.forward_saved
    assert np.all(ctx.download(fs[0]) == X_VAL)
    assert np.all(ctx.download(fs[1]) == Y_VAL)
    assert np.all(ctx.download(fs[2]) == Z_VAL)
    assert np.all(ctx.download(st.forward_out) == Z_VAL + E_VAL)
    gt = st.grad_tensors
    assert np.all(ctx.download(gt[0]) == A_GRAD)
    assert np.all(ctx.download(gt[1]) == B_GRAD)
    assert np.all(ctx.download(gt[2]) == C_GRAD)
    assert np.all(ctx.download(gt[3]) == D_GRAD)
    assert np.all(ctx.download(gt[4]) == 1.0)


def test_matmul_sub_forward_backward(ctx):
    """std_wgsl.rs:523-653."""
    G = api()
    M, N, K = 32, 64, 128
    graph, meta = new_graph(G.MEAN_SQUARED_ERROR)
    m, n, k = meta.new_field(), meta.new_field(), meta.new_field()
    with graph.define_ops() as ops:
        a = ops.input([m, k])
        b = ops.input([k, n])
        c = ops.input([m, k])
        d = ops.input([k, n])
        ops.sub(ops.matmul(a, b), ops.matmul(c, d))
    mb = [G.f32_bits(1e-3), M, N, K]
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    ins = [ctx.init_tensor_f32([M, K], [3.0] * (M * K)), ctx.init_tensor_f32([K, N], [2.0] * (K * N)),
           ctx.init_tensor_f32([M, K], [1.0] * (M * K)), ctx.init_tensor_f32([K, N], [0.5] * (K * N))]
    ctx.upload(st.seed, [1.0] * (M * N), 0)
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    ctx.dispatch_forward(sch)
    ctx.dispatch_backward(sch)
    ctx.sync()
    assert np.all(ctx.download(st.forward_saved[0]) == 768.0)
    assert np.all(ctx.download(st.forward_saved[1]) == 64.0)
    assert np.all(ctx.download(st.forward_out) == 704.0)
    gt = st.grad_tensors
    assert np.all(ctx.download(gt[0]) == 128.0)
    assert np.all(ctx.download(gt[1]) == 96.0)
    assert np.all(ctx.download(gt[2]) == -32.0)
    assert np.all(ctx.download(gt[3]) == -32.0)


def _mul_add_optim(ctx, separate):
    G = api()
    graph, meta = new_graph(G.MEAN_SQUARED_ERROR)
    m, n = meta.new_field(), meta.new_field()
    with graph.define_ops() as ops:
        a = ops.input([m, n])
        b = ops.input([m, n])
        c = ops.input([m, n])
        ops.add(c, ops.mul(a, b))
    mb = [G.f32_bits(1e-3), 32, 32]
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    ins = [ctx.init_tensor_f32([32, 32], [3.0] * 1024), ctx.init_tensor_f32([32, 32], [2.0] * 1024),
           ctx.init_tensor_f32([32, 32], [1.0] * 1024)]
    ctx.upload(st.seed, [1.0] * 1024, 0)
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    ctx.dispatch_forward(sch)
    ctx.dispatch_backward(sch)
    if separate:
        for i, t in enumerate(ins):
            ctx.dispatch_single_optim(sch, t, i, st)
    else:
        ctx.dispatch_optim(sch)
    ctx.sync()
    assert np.all(ctx.download(st.forward_out) == 7.0)
    for gt in st.grad_tensors[:3]:
        assert np.all(ctx.download(gt) == 0.0)
    assert np.all(ctx.download(ins[0]) == f32(3.0) - f32(2e-3))
    assert np.all(ctx.download(ins[1]) == f32(2.0) - f32(3e-3))
    assert np.all(ctx.download(ins[2]) == f32(1.0) - f32(1e-3))


def test_mul_add_optim(ctx):
    """tests/optim.rs:10-104."""
    _mul_add_optim(ctx, False)


def test_mul_add_separate_optim(ctx):
    """tests/optim.rs:107-207."""
    _mul_add_optim(ctx, True)


# --------------------------------------------------------- MLP steps
def build_mlp(ctx, dims, batch, act, optim, trainable_x=False):
    G = api()
    graph, meta = new_graph(G.CROSS_ENTROPY, optim)
    B = meta.new_field()
    d = [meta.new_field() for _ in dims]
    with graph.define_ops() as ops:
        x = ops.input([B, d[0]], trainable=trainable_x)
        h = x
        for l in range(len(dims) - 1):
            W = ops.input([d[l], d[l + 1]])
            b = ops.input([d[l + 1]])
            z = ops.bias_add(ops.matmul(h, W), b)
            h = getattr(ops, act)(z) if l < len(dims) - 2 else z
        ops.softmax(h)
    mb = [G.f32_bits(1e-3), batch] + list(dims)
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    return graph, meta, mb, st


def oracle_mlp_step(X, Ws, bs, y, act):
    L = len(Ws)
    Zs, Hs = [], []
    inp = X
    for l in range(L):
        a = O.ACT_NONE if l == L - 1 else act
        Z, H = O.bias_act(O.gemm(O.NN, inp, Ws[l]), bs[l], a)
        Zs.append(Z)
        Hs.append(H)
        inp = H
    rl, dZ, _, mean = O.softmax_ce(Zs[-1], y)
    dW, db = [None] * L, [None] * L
    for l in range(L - 1, -1, -1):
        prev = Hs[l - 1] if l > 0 else X
        dW[l] = O.gemm(O.TN, prev, dZ)
        db[l] = O.bias_grad(dZ)
        up = O.gemm(O.NT, dZ, Ws[l])
        dZ = O.act_bwd(act, up, Zs[l - 1]) if l > 0 else up
    return mean, rl, dW, db, dZ, O.softmax(Zs[-1])


def test_c1_two_layer_mlp_sgd_step(ctx):
    """BASELINE config c1: batch 64, 784 -> 256 -> ReLU -> 10, CE, SGD lr 0.01;
    Kaiming-uniform weights and zero biases from seed 0, inputs U[0,1),
    labels U{0..9}.  Loss and every parameter gradient vs the oracle, then
    the SGD update bit for bit."""
    import ferrograd_amd as fa
    G = api()
    dims, B = [784, 256, 10], 64
    graph, meta, mb, st = build_mlp(ctx, dims, B, "relu", G.Optim.sgd())
    X = fa.rng_uniform(0, 0, (B, 784))
    y = fa.rng_int(0, 1, (B,), 10)
    Ws = [fa.rng_uniform(0, 10 + l, (dims[l], dims[l + 1]), -math.sqrt(6 / dims[l]),
                         math.sqrt(6 / dims[l])) for l in range(2)]
    bs = [np.zeros(d, f32) for d in dims[1:]]
    ins = [ctx.init_tensor_f32(X.shape, X)]
    for W, b in zip(Ws, bs):
        ins += [ctx.init_tensor_f32(W.shape, W), ctx.init_tensor_f32(b.shape, b)]
    tgt = ctx.new_onehot_init(y)
    sch = ctx.schedule(graph.lower(meta), [G.f32_bits(0.01)] + mb[1:], ins, st)
    ctx.dispatch_forward(sch)
    ctx.dispatch_loss(sch, tgt)
    ctx.dispatch_backward(sch)
    ctx.sync()
    mean, rl, dW, db, dX, probs = oracle_mlp_step(X, Ws, bs, y, O.ACT_RELU)
    assert abs(float(ctx.download(st.mean_loss)[0]) - mean) < 1e-5 * max(1, abs(mean))
    assert normwise_rel(ctx.download(st.loss_t), rl) < 1e-5
    assert normwise_rel(ctx.download(st.forward_out).reshape(B, 10), probs) < 1e-5
    tol = 1e-5 * math.sqrt(784)
    grads = {t.node: ctx.download(t) for t in st.grad_tensors}
    in_nodes = [i for i, nd in enumerate(graph.nodes) if nd.op == 0]
    exp = [dX] + [v for pair in zip(dW, db) for v in pair]
    for node, ref in zip(in_nodes, exp):
        assert normwise_rel(grads[node].reshape(ref.shape), ref) < tol, node
    # SGD: w - fl(g*lr), bit for bit against the oracle on the GPU's grads.
    ctx.dispatch_optim(sch)
    ctx.sync()
    host_params = [Ws[0], bs[0], Ws[1], bs[1]]
    for k, t in enumerate(ins[1:]):
        w = host_params[k].copy().reshape(-1)
        g = grads[in_nodes[k + 1]].copy()
        O.sgd_(w, g, f32(0.01), True)
        assert np.array_equal(ctx.download(t), w)
    assert np.array_equal(ctx.download(ins[0]), X.reshape(-1))  # data input is frozen


def test_mlp_gelu_adam_steps_match_oracle(ctx):
    """A reduced c5 (GELU hidden layers, CE, Adam) for 3 steps: loss,
    gradients and parameters against the oracle run on the same inputs."""
    import ferrograd_amd as fa
    G = api()
    dims, B = [96, 128, 128, 40], 64
    graph, meta, mb, st = build_mlp(ctx, dims, B, "gelu", G.Optim.adam())
    X = fa.rng_normal(4, 0, (B, dims[0]))
    y = fa.rng_int(4, 1, (B,), dims[-1])
    Ws = [fa.rng_uniform(4, 10 + l, (dims[l], dims[l + 1]), -math.sqrt(6 / dims[l]),
                         math.sqrt(6 / dims[l])) for l in range(3)]
    bs = [np.zeros(d, f32) for d in dims[1:]]
    ins = [ctx.init_tensor_f32(X.shape, X)]
    for W, b in zip(Ws, bs):
        ins += [ctx.init_tensor_f32(W.shape, W), ctx.init_tensor_f32(b.shape, b)]
    tgt = ctx.new_onehot_init(y)
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    P = [w.copy() for pair in zip(Ws, bs) for w in pair]
    Mh = [np.zeros_like(p) for p in P]
    Vh = [np.zeros_like(p) for p in P]
    in_nodes = [i for i, nd in enumerate(graph.nodes) if nd.op == 0]
    for step in range(1, 4):
        ctx.dispatch_forward(sch)
        ctx.dispatch_loss(sch, tgt)
        ctx.dispatch_backward(sch)
        ctx.sync()
        grads = {t.node: ctx.download(t) for t in st.grad_tensors}
        mean, rl, dW, db, dX, probs = oracle_mlp_step(X, P[0::2], P[1::2], y, O.ACT_GELU)
        assert abs(float(ctx.download(st.mean_loss)[0]) - mean) < 1e-5 * max(1, abs(mean))
        exp = [v for pair in zip(dW, db) for v in pair]
        for node, ref in zip(in_nodes[1:], exp):
            assert normwise_rel(grads[node].reshape(ref.shape), ref) < 1e-5 * math.sqrt(128)
        ctx.dispatch_optim(sch)
        ctx.sync()
        # Oracle Adam on the GPU's own gradients: any difference is the
        # update, not the gradient.
        s, r = O.adam_scalars(f32(1e-3), f32(0.9), f32(0.999), step)
        for k in range(len(P)):
            g = grads[in_nodes[k + 1]].reshape(P[k].shape).copy()
            O.adam_(P[k], g, Mh[k], Vh[k], f32(0.9), f32(0.999), f32(1e-8), s, r)
            got = ctx.download(ins[k + 1]).reshape(P[k].shape)
            assert normwise_rel(got, P[k]) < 1e-5, (step, k)
            P[k] = got.copy()  # continue from the device state


def test_captured_step_replays_like_eager(ctx):
    """fg_plan_capture_step: 4 graph replays, each followed by eager work and
    a sync, match 4 eager steps of an identical plan."""
    import ferrograd_amd as fa
    from ferrograd_amd._lib import call
    G = api()
    dims, B = [64, 96, 10], 32
    runs = []
    for captured in (False, True):
        graph, meta, mb, st = build_mlp(ctx, dims, B, "gelu", G.Optim.adam())
        X = fa.rng_normal(7, 0, (B, dims[0]))
        y = fa.rng_int(7, 1, (B,), dims[-1])
        ins = [ctx.init_tensor_f32(X.shape, X)]
        for l in range(2):
            W = fa.rng_uniform(7, 10 + l, (dims[l], dims[l + 1]), -0.3, 0.3)
            ins += [ctx.init_tensor_f32(W.shape, W), ctx.init_tensor_f32((dims[l + 1],),
                                                                         np.zeros(dims[l + 1]))]
        tgt = ctx.new_onehot_init(y)
        sch = ctx.schedule(graph.lower(meta), mb, ins, st)
        hist = []
        if captured:
            call("fg_plan_bind_target", sch.plan.handle, tgt.data_ptr(), tgt.nbytes)
            call("fg_plan_capture_step", sch.plan.handle)
        for _ in range(4):
            if captured:
                call("fg_plan_launch_step", sch.plan.handle)
                ctx.download(st.forward_out)  # eager work between replays
            else:
                ctx.dispatch_forward(sch)
                ctx.dispatch_loss(sch, tgt)
                ctx.dispatch_backward(sch)
                ctx.dispatch_optim(sch)
            ctx.sync()
            hist.append([ctx.download(t).copy() for t in ins[1:]] +
                        [ctx.download(st.mean_loss).copy()])
        runs.append(hist)
    for a, b in zip(*runs):
        for x, y2 in zip(a, b):
            assert np.array_equal(x, y2)


def test_paired_gradient_gemms_match_separate_calls(ctx):
    """Each layer's dW (+ dbias) and dX GEMMs share one launch when both take
    small kernels (the c1 shapes).  An eager c1 step through the planner
    against the same step built from single calls on a context with the
    plan's workspace size (so the same kernels and K splits): forward
    fg_gemm_f32, loss fg_softmax_ce, then fg_gemm_dw_f32 and fg_gemm_bwd_f32
    one at a time.  Every gradient equal bit for bit."""
    import ferrograd_amd as fa
    G = api()
    torch = pytest.importorskip("torch")
    own = fa.Context(0, ctx.ctx.stream)
    try:
        own.reserve_workspace(1 << 20)
        dims, B = [784, 256, 10], 64
        graph, meta, mb, st = build_mlp(ctx, dims, B, "relu", G.Optim.sgd())
        desc = st.plan.describe()
        # Both backward variants (seed, CE-fused) pair both layers.
        assert desc.count("[with the next]") == 4, desc
        # The first layer's K slices are summed by the second layer's kernel.
        assert "[K split: slices, summed by the next launch]" in desc, desc
        assert "kernels per step: 4 (forward 2, loss 0, backward 1, optim 1)" in desc, desc
        X = fa.rng_uniform(0, 0, (B, 784))
        y = fa.rng_int(0, 1, (B,), 10)
        Ws = [fa.rng_uniform(0, 10 + l, (dims[l], dims[l + 1]), -math.sqrt(6 / dims[l]),
                             math.sqrt(6 / dims[l])) for l in range(2)]
        bs = [(0.01 * np.arange(d) - 0.02).astype(f32) for d in dims[1:]]
        ins = [ctx.init_tensor_f32(X.shape, X)]
        for W, b in zip(Ws, bs):
            ins += [ctx.init_tensor_f32(W.shape, W), ctx.init_tensor_f32(b.shape, b)]
        tgt = ctx.new_onehot_init(y)
        sch = ctx.schedule(graph.lower(meta), [G.f32_bits(0.01)] + mb[1:], ins, st)
        ctx.dispatch_forward(sch)
        ctx.dispatch_loss(sch, tgt)
        ctx.dispatch_backward(sch)
        ctx.sync()
        grads = {t.node: ctx.download(t) for t in st.grad_tensors}
        in_nodes = [i for i, nd in enumerate(graph.nodes) if nd.op == 0]
        x, w1, b1, w2, b2 = ins

        def buf(*shape):
            return torch.empty(shape, device="cuda")
        Z1, H1, L = buf(B, 256), buf(B, 256), buf(B, 10)
        own.gemm(fa.NN, B, 256, 784, x, 784, w1, 256, H1, 256, bias=b1, act=fa.ACT_RELU, Z=Z1,
                 ldz=256)
        own.gemm(fa.NN, B, 10, 256, H1, 256, w2, 10, L, 10, bias=b2)
        dl = buf(B, 10)
        own.softmax_ce(L, 10, tgt, B, 10, 1.0, dlogits=dl, ldd=10)
        dW2, db2, dZ1 = buf(256, 10), buf(10), buf(B, 256)
        own.gemm_dw(256, 10, B, H1, 256, dl, 10, dW2, 10, colsum=db2)
        own.gemm_bwd(fa.NT, B, 256, 10, dl, 10, w2, 10, dZ1, 256, act=fa.ACT_RELU, Zs=Z1,
                     ldzs=256)
        dW1, db1, dX = buf(784, 256), buf(256), buf(B, 784)
        own.gemm_dw(784, 256, B, x, 784, dZ1, 256, dW1, 256, colsum=db1)
        own.gemm_bwd(fa.NT, B, 784, 256, dZ1, 256, w1, 256, dX, 784)
        own.sync()
        ref = [dX, dW1, db1, dW2, db2]
        for node, r in zip(in_nodes, ref):
            assert np.array_equal(grads[node], r.cpu().numpy().reshape(-1)), node
    finally:
        if "st" in locals():
            st.plan.close()
        own.close()


@pytest.mark.parametrize("d0", [256, 1024], ids=["in256", "in1024-mid-pair"])
def test_big_pair_matches_separate_calls(ctx, d0):
    """A 4096-wide hidden layer's dW (256x256 tiles) and dX (256x128 tiles)
    share one 512-thread launch, the dW tiles' output writes draining while
    dX tiles compute; with 1024 inputs the first layer's dW and dX (both on
    128x64 tiles) share another.  A 3-layer MLP (batch 2048, d0 -> 4096 ->
    4096 -> 16, GELU, CE) through the planner, against the same step from
    single calls on a context with the plan's workspace size (so the same
    kernels and K splits).  Every gradient equal bit for bit."""
    import ferrograd_amd as fa
    G = api()
    torch = pytest.importorskip("torch")
    dims, B = [d0, 4096, 4096, 16], 2048
    graph, meta, mb, st = build_mlp(ctx, dims, B, "gelu", G.Optim.sgd())
    own = fa.Context(0, ctx.ctx.stream)
    try:
        desc = st.plan.describe()
        # one launch per layer in the backward (each layer's pair)
        assert "kernels per step: 11 (forward 4, loss 2, backward 4, optim 1)" in desc, desc
        own.reserve_workspace(1 << 20)
        X = fa.rng_uniform(0, 0, (B, dims[0]))
        y = fa.rng_int(0, 1, (B,), dims[-1])
        ins = [ctx.init_tensor_f32(X.shape, X)]
        for l in range(3):
            W = fa.rng_uniform(0, 10 + l, (dims[l], dims[l + 1]), -math.sqrt(6 / dims[l]),
                               math.sqrt(6 / dims[l]))
            b = (0.01 * np.arange(dims[l + 1]) / dims[l + 1] - 0.005).astype(f32)
            ins += [ctx.init_tensor_f32(W.shape, W), ctx.init_tensor_f32(b.shape, b)]
        tgt = ctx.new_onehot_init(y)
        sch = ctx.schedule(graph.lower(meta), [G.f32_bits(0.01)] + mb[1:], ins, st)
        ctx.dispatch_forward(sch)
        ctx.dispatch_loss(sch, tgt)
        ctx.dispatch_backward(sch)
        ctx.sync()
        grads = {t.node: ctx.download(t) for t in st.grad_tensors}
        in_nodes = [i for i, nd in enumerate(graph.nodes) if nd.op == 0]
        x, w1, b1, w2, b2, w3, b3 = ins

        def buf(*shape):
            return torch.empty(shape, device="cuda")
        d0, d1, d2, d3 = dims
        Z1, H1, Z2, H2, L = buf(B, d1), buf(B, d1), buf(B, d2), buf(B, d2), buf(B, d3)
        own.gemm(fa.NN, B, d1, d0, x, d0, w1, d1, H1, d1, bias=b1, act=fa.ACT_GELU, Z=Z1, ldz=d1)
        own.gemm(fa.NN, B, d2, d1, H1, d1, w2, d2, H2, d2, bias=b2, act=fa.ACT_GELU, Z=Z2, ldz=d2)
        own.gemm(fa.NN, B, d3, d2, H2, d2, w3, d3, L, d3, bias=b3)
        dl = buf(B, d3)
        own.softmax_ce(L, d3, tgt, B, d3, 1.0, dlogits=dl, ldd=d3)
        dW3, db3, dZ2 = buf(d2, d3), buf(d3), buf(B, d2)
        own.gemm_dw(d2, d3, B, H2, d2, dl, d3, dW3, d3, colsum=db3)
        own.gemm_bwd(fa.NT, B, d2, d3, dl, d3, w3, d3, dZ2, d2, act=fa.ACT_GELU, Zs=Z2, ldzs=d2)
        dW2, db2, dZ1 = buf(d1, d2), buf(d2), buf(B, d1)
        own.gemm_dw(d1, d2, B, H1, d1, dZ2, d2, dW2, d2, colsum=db2)
        own.gemm_bwd(fa.NT, B, d1, d2, dZ2, d2, w2, d2, dZ1, d1, act=fa.ACT_GELU, Zs=Z1, ldzs=d1)
        dW1, db1, dX = buf(d0, d1), buf(d1), buf(B, d0)
        own.gemm_dw(d0, d1, B, x, d0, dZ1, d1, dW1, d1, colsum=db1)
        own.gemm_bwd(fa.NT, B, d0, d1, dZ1, d1, w1, d1, dX, d0)
        own.sync()
        ref = [dX, dW1, db1, dW2, db2, dW3, db3]
        for node, r in zip(in_nodes, ref):
            assert np.array_equal(grads[node], r.cpu().numpy().reshape(-1)), node
    finally:
        st.plan.close()
        own.close()


@pytest.mark.parametrize("k1,chained", [(768, True), (1000, False)],
                         ids=["K768-chained", "K1000-13-slices"])
def test_forward_chain_matches_separate_calls(ctx, k1, chained):
    """A split-K first layer whose output feeds a skinny second layer: the
    second layer's kernel sums the first's 12 K slices (slice order, bias,
    GELU, Z and H written) instead of a summing kernel.  100 rows (a partial
    last 16-row workgroup), 128 hidden, 12 classes.  With K = 1000 the first
    layer takes 13 slices, more than the summing prologue loads, and the
    plan falls back to the summing kernel.  An eager step through the plan
    against single calls on a context with the plan's workspace size: the
    loss and every gradient equal bit for bit."""
    import ferrograd_amd as fa
    G = api()
    torch = pytest.importorskip("torch")
    own = fa.Context(0, ctx.ctx.stream)
    try:
        own.reserve_workspace(1 << 20)
        dims, B = [k1, 128, 12], 100
        graph, meta, mb, st = build_mlp(ctx, dims, B, "gelu", G.Optim.sgd())
        desc = st.plan.describe()
        summed = "[K split: slices, summed by the next launch]" in desc
        assert summed == chained, desc
        assert ("summing kernel" in desc.split("loss:")[0]) != chained, desc
        X = fa.rng_uniform(0, 0, (B, k1))
        y = fa.rng_int(0, 1, (B,), 12)
        Ws = [fa.rng_uniform(0, 10 + l, (dims[l], dims[l + 1]), -math.sqrt(6 / dims[l]),
                             math.sqrt(6 / dims[l])) for l in range(2)]
        bs = [(0.01 * np.arange(d) - 0.3).astype(f32) for d in dims[1:]]
        ins = [ctx.init_tensor_f32(X.shape, X)]
        for W, b in zip(Ws, bs):
            ins += [ctx.init_tensor_f32(W.shape, W), ctx.init_tensor_f32(b.shape, b)]
        tgt = ctx.new_onehot_init(y)
        sch = ctx.schedule(graph.lower(meta), [G.f32_bits(0.01)] + mb[1:], ins, st)
        ctx.dispatch_forward(sch)
        ctx.dispatch_loss(sch, tgt)
        ctx.dispatch_backward(sch)
        ctx.sync()
        grads = {t.node: ctx.download(t) for t in st.grad_tensors}
        in_nodes = [i for i, nd in enumerate(graph.nodes) if nd.op == 0]
        x, w1, b1, w2, b2 = ins

        def buf(*shape):
            return torch.empty(shape, device="cuda")
        Z1, H1, L = buf(B, 128), buf(B, 128), buf(B, 12)
        own.gemm(fa.NN, B, 128, k1, x, k1, w1, 128, H1, 128, bias=b1, act=fa.ACT_GELU, Z=Z1,
                 ldz=128)
        own.gemm(fa.NN, B, 12, 128, H1, 128, w2, 12, L, 12, bias=b2)
        dl = buf(B, 12)
        own.softmax_ce(L, 12, tgt, B, 12, 1.0, dlogits=dl, ldd=12)
        dW2, db2, dZ1 = buf(128, 12), buf(12), buf(B, 128)
        own.gemm_dw(128, 12, B, H1, 128, dl, 12, dW2, 12, colsum=db2)
        own.gemm_bwd(fa.NT, B, 128, 12, dl, 12, w2, 12, dZ1, 128, act=fa.ACT_GELU, Zs=Z1,
                     ldzs=128)
        dW1, db1, dX = buf(k1, 128), buf(128), buf(B, k1)
        own.gemm_dw(k1, 128, B, x, k1, dZ1, 128, dW1, 128, colsum=db1)
        own.gemm_bwd(fa.NT, B, k1, 128, dZ1, 128, w1, 128, dX, k1)
        own.sync()
        ref = [dX, dW1, db1, dW2, db2]
        for node, r in zip(in_nodes, ref):
            assert np.array_equal(grads[node], r.cpu().numpy().reshape(-1)), node
    finally:
        if "st" in locals():
            st.plan.close()
        own.close()


@pytest.mark.parametrize("classes,dtype", [(10, "f32"), (1000, "f32"), (1001, "f32"),
                                           (1000, "bf16"), (37, "bf16")],
                         ids=["C10-small", "C1000-rows", "C1001-stream", "C1000-bf16",
                              "C37-bf16-small"])
def test_captured_step_softmax_output_matches_eager(ctx, classes, dtype):
    """A captured step leaves the final softmax to the fused CE launch, which
    writes forward_out itself (one-workgroup kernel for small heads, the
    register row kernels, the streaming kernel for unaligned rows, 16-bit
    rows).  Three captured steps against three eager steps of an identical
    plan: forward_out, the loss and every parameter bit for bit."""
    import ferrograd_amd as fa
    from ferrograd_amd._lib import call
    G = api()
    dims, B = [48, 64, classes], 32
    runs = []
    for captured in (False, True):
        graph, meta = new_graph(G.CROSS_ENTROPY, G.Optim.adam())
        fb = meta.new_field()
        fd = [meta.new_field() for _ in dims]
        with graph.define_ops() as ops:
            h = ops.input([fb, fd[0]], dtype, trainable=False)
            for l in range(2):
                W = ops.input([fd[l], fd[l + 1]], dtype)
                b = ops.input([fd[l + 1]], dtype)
                z = ops.bias_add(ops.matmul(h, W), b)
                h = ops.gelu(z) if l == 0 else z
            ops.softmax(h)
        mb = [G.f32_bits(1e-3), B] + dims
        st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
        init = ctx.init_tensor_f32 if dtype == "f32" else ctx.init_tensor_bf16
        X = fa.rng_normal(5, 0, (B, dims[0]))
        ins = [init(X.shape, X)]
        for l in range(2):
            W = fa.rng_uniform(5, 10 + l, (dims[l], dims[l + 1]), -0.3, 0.3)
            ins += [init(W.shape, W), init((dims[l + 1],), np.zeros(dims[l + 1], f32))]
        tgt = ctx.new_onehot_init(fa.rng_int(5, 1, (B,), classes))
        sch = ctx.schedule(graph.lower(meta), mb, ins, st)
        if captured:
            call("fg_plan_bind_target", sch.plan.handle, tgt.data_ptr(), tgt.nbytes)
            call("fg_plan_capture_step", sch.plan.handle)
        hist = []
        for _ in range(3):
            if captured:
                call("fg_plan_launch_step", sch.plan.handle)
            else:
                ctx.dispatch_forward(sch)
                ctx.dispatch_loss(sch, tgt)
                ctx.dispatch_backward(sch)
                ctx.dispatch_optim(sch)
            ctx.sync()
            hist.append([ctx.download(st.forward_out).copy(), ctx.download(st.mean_loss).copy()]
                        + [ctx.download(t).copy() for t in ins[1:]])
        runs.append(hist)
        st.plan.close()
    for a, b in zip(*runs):
        for x, y2 in zip(a, b):
            assert np.array_equal(x, y2)
    # The probabilities are a softmax: rows sum to 1 (fp32) / about 1 (bf16).
    p = runs[1][-1][0]
    p = p.astype(np.float32) if dtype == "f32" else G.bf16_to_f32(p)
    assert np.allclose(p.reshape(B, classes).sum(axis=1), 1.0, atol=1e-5 if dtype == "f32" else 2e-2)


def test_captured_step_survives_workspace_growth(ctx):
    """A captured c1 step (two of its GEMMs split K into the plan's workspace)
    replays bit for bit like eager steps of an identical plan after the
    context's workspace grows and a larger plan is created on the same
    context: each plan's workspace is its own, and a context workspace that
    grows is retired, not freed."""
    import ferrograd_amd as fa
    from ferrograd_amd._lib import call
    G = api()
    # A context of its own on the same stream: growing its workspace must not
    # change what later tests' direct GEMM calls on the shared context do.
    own = fa.Context(0, ctx.ctx.stream)
    gctx = G.GpuContext(own)
    dims, B = [784, 256, 10], 64
    runs, plans, extra = [], [], []
    try:
        for captured in (False, True):
            graph, meta, mb, st = build_mlp(gctx, dims, B, "relu", G.Optim.sgd())
            X = fa.rng_uniform(0, 0, (B, 784))
            y = fa.rng_int(0, 1, (B,), 10)
            ins = [gctx.init_tensor_f32(X.shape, X)]
            for l in range(2):
                W = fa.rng_uniform(0, 10 + l, (dims[l], dims[l + 1]), -math.sqrt(6 / dims[l]),
                                   math.sqrt(6 / dims[l]))
                ins += [gctx.init_tensor_f32(W.shape, W),
                        gctx.init_tensor_f32((dims[l + 1],), np.zeros(dims[l + 1]))]
            tgt = gctx.new_onehot_init(y)
            sch = gctx.schedule(graph.lower(meta), [G.f32_bits(0.01)] + mb[1:], ins, st)
            plans.append((sch, st, ins, tgt))
        desc = plans[1][1].plan.describe()
        # The first layer's forward and the data-input dX split K in the
        # plan's own workspace: the forward's slices are summed by the skinny
        # 64x10x256 second layer, dX's by blocks of the SGD launch (a
        # captured step); each layer's dW and dX share a launch; a captured
        # step leaves the softmax to the loss launch.
        fwd = desc.split("forward:")[1].split("loss:")[0]
        assert fwd.count("[K split: slices, summed by the next launch]") == 1, desc
        assert "the backward's last summing launch shares the SGD launch" in desc, desc
        assert "the head GEMM finishes the loss" in desc, desc
        assert "it also computes the head's data gradient" in desc, desc
        assert "kernels per step: 4 (forward 2, loss 0, backward 1, optim 1)" in desc, desc
        sch, st, ins, tgt = plans[1]
        call("fg_plan_bind_target", sch.plan.handle, tgt.data_ptr(), tgt.nbytes)
        call("fg_plan_capture_step", sch.plan.handle)
        # Grow the context's own workspace and create a larger plan on it.
        own.reserve_workspace(64 << 20)
        extra.append(build_mlp(gctx, [512, 2048, 1000], 256, "gelu", G.Optim.adam())[3])
        for captured, (sch, st, ins, tgt) in zip((False, True), plans):
            hist = []
            for _ in range(3):
                if captured:
                    call("fg_plan_launch_step", sch.plan.handle)
                    gctx.download(st.forward_out)  # eager work between replays
                else:
                    gctx.dispatch_forward(sch)
                    gctx.dispatch_loss(sch, tgt)
                    gctx.dispatch_backward(sch)
                    gctx.dispatch_optim(sch)
                gctx.sync()
                # Parameters, the mean loss, the probabilities and every
                # gradient: in the captured step the head GEMM finishes the
                # loss (dlogits, probabilities), the SGD launch its mean and
                # the data input's gradient.
                hist.append([gctx.download(t).copy() for t in ins[1:]] +
                            [gctx.download(st.mean_loss).copy(),
                             gctx.download(st.forward_out).copy()] +
                            [gctx.download(t).copy() for t in st.grad_tensors])
            runs.append(hist)
        for a, b in zip(*runs):
            for x, y2 in zip(a, b):
                assert np.array_equal(x, y2)
    finally:
        own.sync()
        for st in extra:
            st.plan.close()
        for _, st, _, _ in plans:
            st.plan.close()
        own.close()


# Shapes for the fused paths of captured SGD steps beyond c1's own: heads of
# at most 16 classes on hidden widths of at most 256 (the skinny head GEMM
# that finishes the loss and computes the head's data gradient, and the
# triple launch that follows), first layers long enough in K to split
# (the chained forward and the summing pass held for the SGD launch), odd
# batches, widths off multiples of 16.
FUSED_SGD_SHAPES = [([300, 128, 16], 32, "relu"), ([1000, 256, 3], 100, "gelu"),
                    ([640, 200, 7], 48, "relu"), ([784, 256, 10], 128, "gelu"),
                    ([96, 64, 12], 17, "relu")]


@pytest.mark.parametrize("dims,B,act", FUSED_SGD_SHAPES,
                         ids=["-".join(map(str, d)) + f"-b{b}" for d, b, _ in FUSED_SGD_SHAPES])
def test_captured_sgd_fused_paths_at_other_shapes(ctx, dims, B, act):
    """Captured SGD steps of two-layer MLPs at shapes other than c1's: three
    replays of the captured step against three eager steps of an identical
    plan, bit for bit (parameters, mean loss, probabilities, every gradient),
    and the first step against the oracle (loss within 1e-5, gradients
    within 1e-5 sqrt(K))."""
    import ferrograd_amd as fa
    from ferrograd_amd._lib import call
    G = api()
    print(f"fused SGD paths: dims {dims} batch {B} {act}", flush=True)
    runs, plans = [], []
    X = fa.rng_uniform(5, 0, (B, dims[0]))
    y = fa.rng_int(5, 1, (B,), dims[-1])
    Ws = [fa.rng_uniform(5, 10 + l, (dims[l], dims[l + 1]), -math.sqrt(6 / dims[l]),
                         math.sqrt(6 / dims[l])) for l in range(2)]
    bs = [fa.rng_uniform(5, 20 + l, (dims[l + 1],), -0.1, 0.1) for l in range(2)]
    graphs = []
    try:
        for captured in (False, True):
            graph, meta, mb, st = build_mlp(ctx, dims, B, act, G.Optim.sgd())
            ins = [ctx.init_tensor_f32(X.shape, X)]
            for W, b in zip(Ws, bs):
                ins += [ctx.init_tensor_f32(W.shape, W), ctx.init_tensor_f32(b.shape, b)]
            tgt = ctx.new_onehot_init(y)
            sch = ctx.schedule(graph.lower(meta), [G.f32_bits(0.01)] + mb[1:], ins, st)
            plans.append((sch, st, ins, tgt))
            graphs.append(graph)
        desc = plans[1][1].plan.describe()
        fused = [k for k in ("the head GEMM finishes the loss", "the head's data gradient",
                             "shares the SGD launch", "summed by the next launch")
                 if k in desc]
        print("  fused paths taken: " + (", ".join(fused) or "none"), flush=True)
        sch, st, ins, tgt = plans[1]
        call("fg_plan_bind_target", sch.plan.handle, tgt.data_ptr(), tgt.nbytes)
        call("fg_plan_capture_step", sch.plan.handle)
        first = None  # the eager plan's first-step gradients, before SGD zeroes them
        for captured, (sch, st, ins, tgt) in zip((False, True), plans):
            hist = []
            for step in range(3):
                if captured:
                    call("fg_plan_launch_step", sch.plan.handle)
                else:
                    ctx.dispatch_forward(sch)
                    ctx.dispatch_loss(sch, tgt)
                    ctx.dispatch_backward(sch)
                    if step == 0:
                        ctx.sync()
                        first = {t.node: ctx.download(t).copy() for t in st.grad_tensors}
                    ctx.dispatch_optim(sch)
                ctx.sync()
                hist.append([ctx.download(t).copy() for t in ins[1:]] +
                            [ctx.download(st.mean_loss).copy(),
                             ctx.download(st.forward_out).copy()] +
                            [ctx.download(t).copy() for t in st.grad_tensors])
            runs.append(hist)
        for step, (a, b) in enumerate(zip(*runs)):
            for k, (x, y2) in enumerate(zip(a, b)):
                assert np.array_equal(x, y2), (step, k)
        # The first step against the oracle: loss, probabilities, and every
        # gradient (dX of the data input included).
        mean, _, dW, db, dX, probs = oracle_mlp_step(X, Ws, bs, y.astype(np.uint32),
                                                     O.ACT_RELU if act == "relu" else O.ACT_GELU)
        assert abs(float(runs[0][0][4][0]) - mean) < 1e-5 * max(1.0, abs(mean))
        assert normwise_rel(runs[0][0][5].reshape(probs.shape), probs) < 1e-5
        in_nodes = [i for i, nd in enumerate(graphs[0].nodes) if nd.op == 0]
        exp = [dX] + [v for pair in zip(dW, db) for v in pair]
        tol = 1e-5 * math.sqrt(max(dims[0], dims[1], B))
        for node, ref in zip(in_nodes, exp):
            assert normwise_rel(first[node].reshape(ref.shape), ref) < tol, node
    finally:
        for _, st, _, _ in plans:
            st.plan.close()


@pytest.mark.parametrize("act", ["relu", "gelu"])
@pytest.mark.parametrize("seeded", [True, False], ids=["seed", "mse"])
def test_linear_root_activation_backward(ctx, act, seeded):
    """A graph that ends in act(bias_add(matmul(X, W), b)): the planner's
    root-activation path (dZ = dH * act'(Z) as an elementwise program that
    also fills the matmul's gradient tensor, then dW with the fused dbias and
    dX).  dH is an uploaded seed, or the MSE loss's gradient written by
    dispatch_loss (taken back from the seed buffer).  Forward output and
    every gradient, the matmul node's included, against the oracle."""
    import ferrograd_amd as fa
    G = api()
    M, K, N = 96, 200, 136
    graph, meta = new_graph(G.MEAN_SQUARED_ERROR)
    m, k, n = meta.new_field(), meta.new_field(), meta.new_field()
    with graph.define_ops() as ops:
        x = ops.input([m, k])
        w = ops.input([k, n])
        b = ops.input([n])
        mm = ops.matmul(x, w)
        getattr(ops, act)(ops.bias_add(mm, b))
    mb = [G.f32_bits(1e-3), M, K, N]
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    X = fa.rng_normal(9, 0, (M, K))
    Wv = fa.rng_uniform(9, 1, (K, N), -math.sqrt(6 / K), math.sqrt(6 / K))
    bv = fa.rng_normal(9, 2, (N,), 0.0, 0.1)
    ins = [ctx.init_tensor_f32(X.shape, X), ctx.init_tensor_f32(Wv.shape, Wv),
           ctx.init_tensor_f32(bv.shape, bv)]
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    a = O.ACT_RELU if act == "relu" else O.ACT_GELU
    Zr, Hr = O.bias_act(O.gemm(O.NN, X, Wv), bv, a)
    ctx.dispatch_forward(sch)
    if seeded:
        dH = fa.rng_normal(9, 3, (M, N))
        ctx.upload(st.seed, dH)
    else:
        tgt = ctx.init_tensor_f32((M, N), fa.rng_normal(9, 4, (M, N)))
        ctx.dispatch_loss(sch, tgt)
    ctx.dispatch_backward(sch)
    ctx.sync()
    assert normwise_rel(ctx.download(st.forward_out).reshape(M, N), Hr) < 1e-5 * math.sqrt(K)
    if not seeded:
        dH = ctx.download(st.seed).reshape(M, N)
    dZ = O.act_bwd(a, dH, Zr)
    grads = {t.node: ctx.download(t) for t in st.grad_tensors}
    exp = {x: O.gemm(O.NT, dZ, Wv), w: O.gemm(O.TN, X, dZ), b: O.bias_grad(dZ), mm: dZ}
    for node, ref in exp.items():
        tol = 1e-5 * math.sqrt(max(N, M))
        assert normwise_rel(grads[node].reshape(ref.shape), ref) < tol, node
    st.plan.close()


# --------------------------------------------------- losses and elementwise
@pytest.mark.parametrize("loss", ["MEAN_SQUARED_ERROR", "BINARY_CROSS_ENTROPY", "CROSS_ENTROPY"])
def test_losses_on_tanh_output(ctx, loss):
    """MSE / BCE / CE (no softmax) on pred = 0.5 + 0.4 tanh(x): loss_t and
    backward against float64 numpy (basic_loss.rs:3-133; BCE's 1-pred is
    taken from pred)."""
    G = api()
    R, C = 12, 10
    graph, meta = new_graph(getattr(G, loss))
    r, c = meta.new_field(), meta.new_field()
    with graph.define_ops() as ops:
        x = ops.input([r, c])
        half, scale = ops.constant_f32(0.5), ops.constant_f32(0.4)
        ops.add(ops.mul(ops.tanh(x), scale), half)
    mb = [G.f32_bits(1e-3), R, C]
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    rng = np.random.default_rng(5)
    X = rng.standard_normal((R, C)).astype(f32)
    ins = [ctx.init_tensor_f32([R, C], X)]
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    p = 0.5 + 0.4 * np.tanh(X.astype(np.float64))
    if loss == "CROSS_ENTROPY":
        lab = rng.integers(0, C, R)
        tgt = ctx.new_onehot_init(lab)
        oh = np.eye(C)[lab]
        exp_loss = np.where(oh > 0, -np.log(p), 0.0)
        seed = p - oh
    else:
        T = rng.uniform(0, 1, (R, C)).astype(f32)
        tgt = ctx.init_tensor_f32([R, C], T)
        t = T.astype(np.float64)
        if loss == "MEAN_SQUARED_ERROR":
            exp_loss, seed = (p - t) ** 2, 2 * (p - t)
        else:
            exp_loss = -(t * np.log(p) + (1 - t) * np.log(1 - p))
            seed = p - t
    ctx.dispatch_forward(sch)
    ctx.dispatch_loss(sch, tgt)
    ctx.dispatch_backward(sch)
    ctx.sync()
    assert normwise_rel(ctx.download(st.forward_out).reshape(R, C), p) < 1e-6
    assert normwise_rel(ctx.download(st.loss_t).reshape(R, C), exp_loss) < 1e-5
    assert normwise_rel(ctx.download(st.seed).reshape(R, C), seed) < 1e-5
    gx = seed * 0.4 * (1 - np.tanh(X.astype(np.float64)) ** 2)
    assert normwise_rel(ctx.download(st.grad_tensors[0]).reshape(R, C), gx) < 1e-5


UNARY = {
    "relu": (lambda x: np.maximum(x, 0), lambda x: (x > 0).astype(float)),
    "elu": (lambda x: np.where(x >= 0, x, np.expm1(x)), lambda x: np.where(x >= 0, 1.0, np.exp(x))),
    "tanh": (np.tanh, lambda x: 1 - np.tanh(x) ** 2),
    "exp": (np.exp, np.exp),
    "abs": (np.abs, np.sign),
    "neg": (lambda x: -x, lambda x: -np.ones_like(x)),
    "log": (lambda x: np.log(np.abs(x) + 0.5), None),
}


@pytest.mark.parametrize("op", list(UNARY))
def test_unary_forward_backward(ctx, op):
    """Each unary op on a [17, 23] input, seed = random upstream gradient."""
    G = api()
    R, C = 17, 23
    graph, meta = new_graph(G.MEAN_SQUARED_ERROR)
    r, c = meta.new_field(), meta.new_field()
    rng = np.random.default_rng(len(op))
    X = rng.standard_normal((R, C)).astype(f32)
    X[np.abs(X) < 1e-3] = 0.5  # keep away from relu / abs kinks
    with graph.define_ops() as ops:
        x = ops.input([r, c])
        if op == "log":  # log(|x| + 0.5): the reference's log backward divides by its output
            ops.log(ops.add(ops.abs(x), ops.constant_f32(0.5)))
        else:
            getattr(ops, op)(x)
    mb = [G.f32_bits(1e-3), R, C]
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    sch = ctx.schedule(graph.lower(meta), mb, [ctx.init_tensor_f32([R, C], X)], st)
    seed = rng.standard_normal((R, C)).astype(f32)
    ctx.upload(st.seed, seed)
    ctx.dispatch_forward(sch)
    ctx.dispatch_backward(sch)
    ctx.sync()
    x64 = X.astype(np.float64)
    fwd, d = UNARY[op]
    assert normwise_rel(ctx.download(st.forward_out).reshape(R, C), fwd(x64)) < 1e-6
    if op == "log":
        exp = seed / (np.abs(x64) + 0.5) * np.sign(x64)
    else:
        exp = seed * d(x64)
    assert normwise_rel(ctx.download(st.grad_tensors[0]).reshape(R, C), exp) < 1e-5


@pytest.mark.parametrize("R,C", [(37, 1024), (37, 1025), (3, 341), (6, 2048), (6, 2049),
                                 (3, 1023), (5, 4097), (1031, 4099), (1024, 4096)],
                         ids=["1k-whole", "1k-partial", "1k-one-partial", "3k-whole",
                              "3k-partial", "3k-one-partial", "2k-and-4k-partial",
                              "streaming-partial", "streaming-whole"])
def test_eltwise_program_whole_and_partial_blocks(ctx, R, C):
    """tanh(x * y + z) and its gradients through elementwise programs at
    sizes on either side of a workgroup's pass (256 threads x U quads: 1024
    elements for the 16-register file, 2048 for the 8-register file, 3072
    for the 4-register file the forward program takes): whole workgroups, a
    partial last workgroup with a partial last quad, and one partial
    workgroup; 1031 x 4099 (4.2 M elements, a partial last quad) and 1024 x
    4096 take the streaming loads and stores of large tensors.  Forward and
    every gradient against float64 numpy."""
    G = api()
    graph, meta = new_graph(G.MEAN_SQUARED_ERROR)
    r, c = meta.new_field(), meta.new_field()
    with graph.define_ops() as ops:
        x = ops.input([r, c])
        y = ops.input([r, c])
        z = ops.input([r, c])
        ops.tanh(ops.add(ops.mul(x, y), z))
    mb = [G.f32_bits(1e-3), R, C]
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    rng = np.random.default_rng(R * C)
    X, Y, Z = (rng.standard_normal((R, C)).astype(f32) for _ in range(3))
    ins = [ctx.init_tensor_f32([R, C], v) for v in (X, Y, Z)]
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    seed = rng.standard_normal((R, C)).astype(f32)
    ctx.upload(st.seed, seed)
    ctx.dispatch_forward(sch)
    ctx.dispatch_backward(sch)
    ctx.sync()
    x, yv, zv, s = (v.astype(np.float64) for v in (X, Y, Z, seed))
    t = np.tanh(x * yv + zv)
    assert normwise_rel(ctx.download(st.forward_out).reshape(R, C), t) < 1e-6
    g = {tt.node: ctx.download(tt) for tt in st.grad_tensors}
    du = s * (1 - t * t)
    assert normwise_rel(g[0].reshape(R, C), du * yv) < 1e-5
    assert normwise_rel(g[1].reshape(R, C), du * x) < 1e-5
    assert normwise_rel(g[2].reshape(R, C), du) < 1e-5


@pytest.mark.parametrize("R,C", [(9, 301), (1100, 4097)], ids=["small", "streaming"])
def test_eltwise_program_wide_expression(ctx, R, C):
    """((a*b + c*d) * (e - f)) / (g*g + 1) with seven inputs: forward and
    every gradient against float64 numpy.  Its programs hold more values at
    once than the tanh chain (more sources than are prefetched, the backward
    reuses many intermediates), so they run on the larger register files;
    1100 x 4097 takes the streaming accesses and a partial last quad."""
    G = api()
    graph, meta = new_graph(G.MEAN_SQUARED_ERROR)
    r, c = meta.new_field(), meta.new_field()
    with graph.define_ops() as ops:
        a, b, cc, d, e, f, g = (ops.input([r, c]) for _ in range(7))
        num = ops.mul(ops.add(ops.mul(a, b), ops.mul(cc, d)), ops.sub(e, f))
        one = ops.constant_f32(1.0)
        ops.div(num, ops.add(ops.mul(g, g), one))
    mb = [G.f32_bits(1e-3), R, C]
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    rng = np.random.default_rng(R + C)
    V = [rng.standard_normal((R, C)).astype(f32) for _ in range(7)]
    ins = [ctx.init_tensor_f32([R, C], v) for v in V]
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    seed = rng.standard_normal((R, C)).astype(f32)
    ctx.upload(st.seed, seed)
    ctx.dispatch_forward(sch)
    ctx.dispatch_backward(sch)
    ctx.sync()
    A, B, Cc, D, E, F, Gv, S = (v.astype(np.float64) for v in V + [seed])
    p = A * B + Cc * D
    q = E - F
    den = Gv * Gv + 1.0
    y = p * q / den
    assert normwise_rel(ctx.download(st.forward_out).reshape(R, C), y) < 1e-6
    g = {t.node: ctx.download(t).reshape(R, C) for t in st.grad_tensors}
    u = S / den
    exp = [u * q * B, u * q * A, u * q * D, u * q * Cc, u * p, -u * p,
           -S * p * q / (den * den) * 2.0 * Gv]
    for k, ref in enumerate(exp):
        assert normwise_rel(g[k], ref) < 1e-5, k


@pytest.mark.parametrize("C", [300, 301])
def test_binary_broadcast_and_div_backward(ctx, C):
    """(a / b) * c - bias (row-broadcast sub): forward and every gradient
    against float64 numpy, including the negated column reduction.  The
    elementwise kernel runs float4 quads: C = 300 reads the bias four columns
    at a time; C = 301 takes the element-wise row broadcast, with quads that
    cross rows and a one-element last quad (9 x 301 elements)."""
    G = api()
    R = 9
    graph, meta = new_graph(G.MEAN_SQUARED_ERROR)
    r, c = meta.new_field(), meta.new_field()
    with graph.define_ops() as ops:
        a = ops.input([r, c])
        b = ops.input([r, c])
        cc = ops.input([r, c])
        bias = ops.input([c])
        ops.sub(ops.mul(ops.div(a, b), cc), bias)
    mb = [G.f32_bits(1e-3), R, C]
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    rng = np.random.default_rng(3)
    A = rng.standard_normal((R, C)).astype(f32)
    Bv = (rng.uniform(0.5, 2.0, (R, C)) * rng.choice([-1, 1], (R, C))).astype(f32)
    Cc = rng.standard_normal((R, C)).astype(f32)
    bias = rng.standard_normal(C).astype(f32)
    ins = [ctx.init_tensor_f32([R, C], A), ctx.init_tensor_f32([R, C], Bv),
           ctx.init_tensor_f32([R, C], Cc), ctx.init_tensor_f32([C], bias)]
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    seed = rng.standard_normal((R, C)).astype(f32)
    ctx.upload(st.seed, seed)
    ctx.dispatch_forward(sch)
    ctx.dispatch_backward(sch)
    ctx.sync()
    a, b, c2, s = (v.astype(np.float64) for v in (A, Bv, Cc, seed))
    assert normwise_rel(ctx.download(st.forward_out).reshape(R, C), a / b * c2 - bias) < 1e-6
    g = {t.node: ctx.download(t) for t in st.grad_tensors}
    assert normwise_rel(g[0].reshape(R, C), s * c2 / b) < 1e-5
    assert normwise_rel(g[1].reshape(R, C), -s * c2 * a / b ** 2) < 1e-5
    assert normwise_rel(g[2].reshape(R, C), s * a / b) < 1e-5
    assert normwise_rel(g[3], -s.sum(0)) < 1e-5
