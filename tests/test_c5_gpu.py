"""BASELINE config c5 at its real size through the planner: the 8-layer MLP
(batch 2048, 1024 -> 4096 x7 -> 1000, GELU-tanh, softmax cross-entropy,
Adam lr 1e-3) lowered as one graph and run forward, loss, backward and
optimiser through the C ABI, against the CPU oracle on the same inputs.

Inputs follow the configuration (generator seed 4): X ~ N(0,1), labels
U{0..999}, Kaiming-uniform weights U(-sqrt(6/fan_in), +sqrt(6/fan_in)),
zero biases.  Checks: mean loss within 1e-5; every dW and db within
1e-5*sqrt(4096) normwise; the Adam update bit for bit against the oracle's
Adam applied to the GPU's own gradients (so any difference would be the
update itself, not the gradient feeding it)."""
import math

import numpy as np
import pytest

import oracle as O
from conftest import normwise_rel

pytestmark = pytest.mark.gpu

f32 = np.float32


def test_c5_full_size_step_matches_oracle(gpu_ctx):
    import ferrograd_amd as fa
    from ferrograd_amd import graph as G

    dims, B = [1024] + [4096] * 7 + [1000], 2048
    L = len(dims) - 1
    print(f"c5 full size: dims {dims}, batch {B}", flush=True)
    ctx = G.GpuContext(gpu_ctx)
    graph, meta = G.Graph(G.CROSS_ENTROPY, G.Optim.adam().lower), G.Metadata.new()
    fb = meta.new_field()
    fd = [meta.new_field() for _ in dims]
    w_nodes, b_nodes = [], []
    with graph.define_ops() as ops:
        h = ops.input([fb, fd[0]], trainable=False)
        for l in range(L):
            W = ops.input([fd[l], fd[l + 1]])
            b = ops.input([fd[l + 1]])
            w_nodes.append(W)
            b_nodes.append(b)
            z = ops.bias_add(ops.matmul(h, W), b)
            h = ops.gelu(z) if l < L - 1 else z
        ops.softmax(h)
    mb = [G.f32_bits(1e-3), B] + dims
    st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    X = fa.rng_normal(4, 0, (B, dims[0]))
    y = fa.rng_int(4, 1, (B,), dims[-1])
    Ws = [fa.rng_uniform(4, 10 + l, (dims[l], dims[l + 1]), -math.sqrt(6 / dims[l]),
                         math.sqrt(6 / dims[l])) for l in range(L)]
    bs = [np.zeros(d, f32) for d in dims[1:]]
    ins = [ctx.init_tensor_f32(X.shape, X)]
    for W, b in zip(Ws, bs):
        ins += [ctx.init_tensor_f32(W.shape, W), ctx.init_tensor_f32(b.shape, b)]
    tgt = ctx.new_onehot_init(y)
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    ctx.dispatch_forward(sch)
    ctx.dispatch_loss(sch, tgt)
    ctx.dispatch_backward(sch)
    ctx.sync()
    gmap = {t.node: t for t in st.grad_tensors}
    dW_gpu = [ctx.download(gmap[n]).reshape(W.shape) for n, W in zip(w_nodes, Ws)]
    db_gpu = [ctx.download(gmap[n]) for n in b_nodes]
    loss_gpu = float(ctx.download(st.mean_loss)[0])
    ctx.dispatch_optim(sch)
    ctx.sync()
    print("c5 full size: GPU step done; oracle step", flush=True)

    # Oracle: forward, CE, backward on the same inputs.
    Zs, Hs, inp = [], [], X
    for l in range(L):
        Z, H = O.bias_act(O.gemm(O.NN, inp, Ws[l]), bs[l], O.ACT_NONE if l == L - 1 else O.ACT_GELU)
        Zs.append(Z)
        Hs.append(H)
        inp = H
    _, dZ, _, mean = O.softmax_ce(Zs[-1], y)
    tol = 1e-5 * math.sqrt(4096)
    assert abs(loss_gpu - mean) < 1e-5 * max(1.0, abs(mean)), (loss_gpu, mean)
    for l in range(L - 1, -1, -1):
        prev = Hs[l - 1] if l > 0 else X
        e_w = normwise_rel(dW_gpu[l], O.gemm(O.TN, prev, dZ))
        e_b = normwise_rel(db_gpu[l], O.bias_grad(dZ))
        print(f"layer {l}: dW {e_w:.2e} db {e_b:.2e}", flush=True)
        assert e_w < tol and e_b < tol, (l, e_w, e_b)
        if l > 0:
            dZ = O.act_bwd(O.ACT_GELU, O.gemm(O.NT, dZ, Ws[l]), Zs[l - 1])

    # Adam step 1 on the GPU's own gradients: bit for bit.
    s, r = O.adam_scalars(f32(1e-3), f32(0.9), f32(0.999), 1)
    for k, (p0, g) in enumerate(zip([w for pair in zip(Ws, bs) for w in pair],
                                    [g for pair in zip(dW_gpu, db_gpu) for g in pair])):
        p = p0.copy()
        O.adam_(p, np.ascontiguousarray(g, f32).reshape(p.shape).copy(), np.zeros_like(p),
                np.zeros_like(p), f32(0.9), f32(0.999), f32(1e-8), s, r)
        assert np.array_equal(ctx.download(ins[k + 1]).reshape(p.shape), p), k
    st.plan.close()
