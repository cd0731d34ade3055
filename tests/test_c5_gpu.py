"""BASELINE config c5 at its real size through the planner: the 8-layer MLP
(batch 2048, 1024 -> 4096 x7 -> 1000, GELU-tanh, softmax cross-entropy,
Adam lr 1e-3) lowered as one graph and run forward, loss, backward and
optimiser through the C ABI, against the CPU oracle on the same inputs.

Inputs follow the configuration (generator seed 4): X ~ N(0,1), labels
U{0..999}, Kaiming-uniform weights U(-sqrt(6/fan_in), +sqrt(6/fan_in)),
zero biases.  Checks: mean loss within 1e-5; every dW and db, and the data
input's gradient dX (ferrograd gives every Input a gradient,
crates/fused_gpu/src/dispatch/backend/kernel/backward.rs:93-106), within
1e-5*sqrt(K) normwise; the Adam update bit for bit against the oracle's
Adam applied to the GPU's own gradients (so any difference would be the
update itself, not the gradient feeding it).

The second test pins the path that bench.py times: the whole step captured
as one hipGraph (fg_plan_capture_step) runs other kernels than eager steps
do (the final softmax elided into the loss, the Adam step counter advanced
on the device), so two steps of a captured plan are compared bit for bit with
two eager steps of an identical plan: every parameter, every gradient
(dX of the data input included), Adam m and v, the mean loss, the per-row
losses and the probabilities -- for fp32 and for bf16 tensors.

The last test runs the step with bf16 tensors against the oracle's 16-bit
composition at the same full size."""
import math

import numpy as np
import pytest

import oracle as O
from conftest import normwise_rel

pytestmark = pytest.mark.gpu

f32 = np.float32
DIMS, BATCH = [1024] + [4096] * 7 + [1000], 2048


def build_c5(gpu_ctx, kind="f32"):
    """The c5 graph, its plan and its bound inputs (host copies kept); kind
    "bf16" builds every tensor in bfloat16 (inputs rounded once from the
    same fp32 draws)."""
    import ferrograd_amd as fa
    from ferrograd_amd import graph as G

    dims, B = DIMS, BATCH
    L = len(dims) - 1
    ctx = G.GpuContext(gpu_ctx)
    graph, meta = G.Graph(G.CROSS_ENTROPY, G.Optim.adam().lower), G.Metadata.new()
    fb = meta.new_field()
    fd = [meta.new_field() for _ in dims]
    w_nodes, b_nodes = [], []
    with graph.define_ops() as ops:
        x_node = h = ops.input([fb, fd[0]], kind, trainable=False)
        for l in range(L):
            W = ops.input([fd[l], fd[l + 1]], kind)
            b = ops.input([fd[l + 1]], kind)
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
    def dev(a):
        if kind == "bf16":
            return ctx.init_tensor_bf16(a.shape, O.from_f32(O.BF16, a))
        return ctx.init_tensor_f32(a.shape, a)

    ins = [dev(X)]
    for W, b in zip(Ws, bs):
        ins += [dev(W), dev(b)]
    tgt = ctx.new_onehot_init(y)
    sch = ctx.schedule(graph.lower(meta), mb, ins, st)
    return dict(ctx=ctx, st=st, sch=sch, ins=ins, tgt=tgt, X=X, y=y, Ws=Ws, bs=bs,
                x_node=x_node, w_nodes=w_nodes, b_nodes=b_nodes)


def free_c5(c):
    c["st"].plan.close()
    for t in c["ins"] + [c["tgt"]]:
        t.free()


def test_c5_full_size_step_matches_oracle(gpu_ctx):
    L = len(DIMS) - 1
    print(f"c5 full size: dims {DIMS}, batch {BATCH}", flush=True)
    c = build_c5(gpu_ctx)
    ctx, st, sch, ins = c["ctx"], c["st"], c["sch"], c["ins"]
    X, y, Ws, bs = c["X"], c["y"], c["Ws"], c["bs"]
    ctx.dispatch_forward(sch)
    ctx.dispatch_loss(sch, c["tgt"])
    ctx.dispatch_backward(sch)
    ctx.sync()
    gmap = {t.node: t for t in st.grad_tensors}
    assert c["x_node"] in gmap, "the data input has no gradient tensor"
    dX_gpu = ctx.download(gmap[c["x_node"]]).reshape(X.shape)
    dW_gpu = [ctx.download(gmap[n]).reshape(W.shape) for n, W in zip(c["w_nodes"], Ws)]
    db_gpu = [ctx.download(gmap[n]) for n in c["b_nodes"]]
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
        up = O.gemm(O.NT, dZ, Ws[l])
        if l > 0:
            dZ = O.act_bwd(O.ACT_GELU, up, Zs[l - 1])
        else:
            # dX = dZ1 . W0^T: K = 4096 (the width of layer 0's output).
            e_x = normwise_rel(dX_gpu, up)
            print(f"data input: dX {e_x:.2e}", flush=True)
            assert e_x < 1e-5 * math.sqrt(DIMS[1]), e_x

    # Adam step 1 on the GPU's own gradients: bit for bit.
    s, r = O.adam_scalars(f32(1e-3), f32(0.9), f32(0.999), 1)
    for k, (p0, g) in enumerate(zip([w for pair in zip(Ws, bs) for w in pair],
                                    [g for pair in zip(dW_gpu, db_gpu) for g in pair])):
        p = p0.copy()
        O.adam_(p, np.ascontiguousarray(g, f32).reshape(p.shape).copy(), np.zeros_like(p),
                np.zeros_like(p), f32(0.9), f32(0.999), f32(1e-8), s, r)
        assert np.array_equal(ctx.download(ins[k + 1]).reshape(p.shape), p), k
    # The data input is frozen: the optimiser leaves it as it was.
    assert np.array_equal(ctx.download(ins[0]).reshape(X.shape), X)
    free_c5(c)


@pytest.mark.parametrize("kind", ["f32", "bf16"])
def test_c5_captured_step_matches_eager_bit_for_bit(gpu_ctx, kind):
    """Two c5 plans from identical inputs: one runs two eager steps (forward,
    loss, backward, optimiser as separate calls), the other captures the
    whole step once and replays it twice.  After each step every parameter,
    gradient (dX included), Adam m and v, the mean loss, the per-row losses
    and the probabilities agree bit for bit.  With bf16 tensors (the step
    bench.py times beside the fp32 one) the step runs other kernels: the
    16-bit dW + dX pairs, K-split GEMMs with their summing kernels, Adam as
    one launch after the backward."""
    from ferrograd_amd._lib import call

    snaps = []
    for captured in (False, True):
        print(f"c5 {kind} {'captured' if captured else 'eager'} plan", flush=True)
        c = build_c5(gpu_ctx, kind)
        ctx, st, sch = c["ctx"], c["st"], c["sch"]
        if captured:
            call("fg_plan_bind_target", sch.plan.handle, c["tgt"].data_ptr(), c["tgt"].nbytes)
            call("fg_plan_capture_step", sch.plan.handle)
        steps = []
        for step in range(2):
            if captured:
                call("fg_plan_launch_step", sch.plan.handle)
            else:
                ctx.dispatch_forward(sch)
                ctx.dispatch_loss(sch, c["tgt"])
                ctx.dispatch_backward(sch)
                ctx.dispatch_optim(sch)
            ctx.sync()
            snap = {"params": [ctx.download(t).copy() for t in c["ins"]],
                    "grads": {t.node: ctx.download(t).copy() for t in st.grad_tensors},
                    "state": [ctx.download(t).copy() for t in st.state],
                    "mean": ctx.download(st.mean_loss).copy(),
                    "row_loss": ctx.download(st.loss_t).copy(),
                    "probs": ctx.download(st.forward_out).copy()}
            print(f"  step {step + 1}: mean loss {float(snap['mean'][0]):.6f}", flush=True)
            steps.append(snap)
        snaps.append((steps, c["x_node"], len(st.state)))
        free_c5(c)
    (eager, x_node, n_state), (capt, _, _) = snaps
    assert n_state == 2 * 2 * (len(DIMS) - 1)  # m and v for every W and b
    for step, (e, g) in enumerate(zip(eager, capt)):
        assert np.array_equal(e["mean"], g["mean"]), step
        assert np.array_equal(e["row_loss"], g["row_loss"]), step
        assert np.array_equal(e["probs"], g["probs"]), step
        for k, (a, b) in enumerate(zip(e["params"], g["params"])):
            assert np.array_equal(a, b), (step, "param", k)
        assert e["grads"].keys() == g["grads"].keys() and x_node in e["grads"]
        for node in e["grads"]:
            assert np.array_equal(e["grads"][node], g["grads"][node]), (step, "grad", node)
        for k, (a, b) in enumerate(zip(e["state"], g["state"])):
            assert np.array_equal(a, b), (step, "adam state", k)
    # The two steps did move the parameters (the comparison is not vacuous).
    assert not np.array_equal(eager[0]["params"][1], eager[1]["params"][1])


def test_c5_bf16_full_size_step_matches_oracle(gpu_ctx):
    """The c5 step with every tensor in bfloat16 (the step bench.py times
    beside the fp32 one), at its real size, against the oracle's 16-bit
    composition in the same node order: each GEMM sums in fp32 and rounds
    once, bias-add and GELU nodes are each rounded (forward), the loss takes
    the widened logits and dlogits are rounded, act' is applied to the
    rounded data gradient and rounded again, column sums are rounded once.
    The GPU sums in another order, so a value that falls on a rounding
    boundary may land one unit in the last place (ulp, 2^-7 relative) away
    and carry that into later layers: every gradient must agree within two
    ulps normwise, as the 2-layer 16-bit step does (the composition through
    eight layers measured at most 1.3 ulps, at the first layer's dW and the
    data input's dX), the mean loss within two ulps; Adam step 1 on the
    GPU's own gradients (fp32 update, the parameter rounded once) bit for
    bit."""
    from ferrograd_amd import graph as G

    L = len(DIMS) - 1
    dt = O.BF16
    ulp = 2.0 ** -7
    print(f"c5 bf16 full size: dims {DIMS}, batch {BATCH}", flush=True)
    c = build_c5(gpu_ctx, "bf16")
    ctx, st, sch, ins = c["ctx"], c["st"], c["sch"], c["ins"]
    X16 = O.from_f32(dt, c["X"])
    W16 = [O.from_f32(dt, W) for W in c["Ws"]]
    b16 = [O.from_f32(dt, b) for b in c["bs"]]
    y = c["y"]
    ctx.dispatch_forward(sch)
    ctx.dispatch_loss(sch, c["tgt"])
    ctx.dispatch_backward(sch)
    ctx.sync()
    gmap = {t.node: t for t in st.grad_tensors}

    def f(t):
        return G.bf16_to_f32(ctx.download(t))

    dX_gpu = f(gmap[c["x_node"]]).reshape(X16.shape)
    dW_gpu = [f(gmap[n]).reshape(W.shape) for n, W in zip(c["w_nodes"], W16)]
    db_gpu = [f(gmap[n]) for n in c["b_nodes"]]
    loss_gpu = float(ctx.download(st.mean_loss)[0])
    ctx.dispatch_optim(sch)
    ctx.sync()
    print("c5 bf16 full size: GPU step done; oracle step", flush=True)

    Zs, Hs, inp = [], [], X16
    for l in range(L):
        if l < L - 1:
            H, Z = O.gemm_x16(dt, O.NN, inp, W16[l], bias=b16[l], act=O.ACT_GELU, want_z=True)
        else:
            Z = O.gemm_x16(dt, O.NN, inp, W16[l], bias=b16[l])
            H = Z
        Zs.append(Z)
        Hs.append(H)
        inp = H
    _, d, _, mean = O.softmax_ce(O.to_f32(dt, Zs[-1]), y)
    dZ = O.from_f32(dt, d)
    print(f"loss: gpu {loss_gpu:.6f} oracle {mean:.6f}", flush=True)
    assert abs(loss_gpu - mean) <= 2 * ulp * max(1.0, abs(mean)), (loss_gpu, mean)
    for l in range(L - 1, -1, -1):
        prev = Hs[l - 1] if l > 0 else X16
        dW = O.to_f32(dt, O.gemm_x16(dt, O.TN, prev, dZ))
        db = O.to_f32(dt, O.from_f32(dt, O.to_f32(dt, dZ).astype(np.float64).sum(0).astype(f32)))
        e_w, e_b = normwise_rel(dW_gpu[l], dW), normwise_rel(db_gpu[l], db)
        print(f"layer {l}: dW {e_w / ulp:.2f} ulp, db {e_b / ulp:.2f} ulp", flush=True)
        assert e_w <= 2 * ulp and e_b <= 2 * ulp, (l, e_w, e_b)
        if l > 0:
            dZ = O.gemm_bwd_x16(dt, O.NT, dZ, W16[l], act=O.ACT_GELU, Zs=Zs[l - 1])
        else:
            e_x = normwise_rel(dX_gpu, O.to_f32(dt, O.gemm_bwd_x16(dt, O.NT, dZ, W16[0])))
            print(f"data input: dX {e_x / ulp:.2f} ulp", flush=True)
            assert e_x <= 2 * ulp, e_x

    s, r = O.adam_scalars(f32(1e-3), f32(0.9), f32(0.999), 1)
    for k, (p16, g) in enumerate(zip([w for pair in zip(W16, b16) for w in pair],
                                     [g for pair in zip(dW_gpu, db_gpu) for g in pair])):
        p = O.to_f32(dt, p16).reshape(-1).copy()
        O.adam_(p, np.ascontiguousarray(g, f32).reshape(-1).copy(), np.zeros_like(p),
                np.zeros_like(p), f32(0.9), f32(0.999), f32(1e-8), s, r)
        got = ctx.download(ins[k + 1]).reshape(-1)
        assert np.array_equal(got, O.from_f32(dt, p)), k
    free_c5(c)
