"""GPU tests of the compiled elementwise kernels (ferrograd_amd/csrc/
fg_elt_jit.cpp): a plan's elementwise programs compiled at run time with
hipRTC must give the same bits as the interpreter of k_eltwise_prog.hip.

Each case builds the same graph twice from the same inputs, once with every
program interpreted (FG_ELTWISE_INTERPRET) and once with every program
compiled (FG_ELTWISE_COMPILE_ALL), runs forward, loss and backward, and
compares the forward output, loss, seed and every gradient bit for bit.  The
process-wide launch counts (fg_eltwise_stats) show which path ran.  The
cases cover every op the planner emits (all unary ops and their derivatives,
the four binary ops, max / select of the losses, label comparison of CE),
fp16 / bf16 loads, stores and rounding, row-broadcast and scalar sources,
partial quads, and the streaming accesses of large tensors; the graphs'
numerics against float64 are checked by tests/test_graph_gpu.py and
tests/test_graph_x16_gpu.py on the default path.  The last test captures an
Adam step whose programs are compiled, and replays it against eager steps
on the interpreter.
"""
import numpy as np
import pytest

import ferrograd_amd as fa

pytestmark = pytest.mark.gpu

f32 = np.float32


def api():
    from ferrograd_amd import graph as G
    return G


@pytest.fixture(scope="module")
def ctx(gpu_ctx):
    from ferrograd_amd.graph import GpuContext
    return GpuContext(gpu_ctx)


def _tanh_chain(ops, x):
    return ops.tanh(ops.add(ops.mul(x[0], x[1]), x[2]))


def _wide(ops, x):
    a, b, c, d, e, f, g = x
    num = ops.mul(ops.add(ops.mul(a, b), ops.mul(c, d)), ops.sub(e, f))
    return ops.div(num, ops.add(ops.mul(g, g), ops.constant_f32(1.0)))


def _broadcast_div(ops, x):
    return ops.sub(ops.mul(ops.div(x[0], x[1]), x[2]), x[3])


def _unary_mix(ops, x):
    v = x[0]
    t = ops.add(ops.relu(v), ops.gelu(v))
    t = ops.add(t, ops.elu(v))
    t = ops.add(t, ops.tanh(v))
    t = ops.add(t, ops.exp(ops.mul(v, ops.constant_f32(0.25))))
    t = ops.sub(t, ops.abs(v))
    t = ops.add(t, ops.neg(ops.log(ops.add(ops.abs(v), ops.constant_f32(0.5)))))
    return t


def _loss_input(ops, x):
    return ops.add(ops.mul(ops.tanh(x[0]), ops.constant_f32(0.4)), ops.constant_f32(0.5))


# name: (build, number of inputs, R, C, loss, element type); the broadcast
# cases take input 3 as a row vector.
CASES = {
    "tanh-partial": (_tanh_chain, 3, 37, 1025, "MEAN_SQUARED_ERROR", "f32"),
    "tanh-streaming": (_tanh_chain, 3, 1031, 4099, "MEAN_SQUARED_ERROR", "f32"),
    "wide-small": (_wide, 7, 9, 301, "MEAN_SQUARED_ERROR", "f32"),
    "wide-streaming": (_wide, 7, 1100, 4097, "MEAN_SQUARED_ERROR", "f32"),
    "broadcast-quads": (_broadcast_div, 4, 9, 300, "MEAN_SQUARED_ERROR", "f32"),
    "broadcast-elements": (_broadcast_div, 4, 9, 301, "MEAN_SQUARED_ERROR", "f32"),
    "unary-mix": (_unary_mix, 1, 67, 513, "MEAN_SQUARED_ERROR", "f32"),
    "mse": (_loss_input, 1, 33, 1001, "MEAN_SQUARED_ERROR", "f32"),
    "bce": (_loss_input, 1, 33, 1001, "BINARY_CROSS_ENTROPY", "f32"),
    "ce": (_loss_input, 1, 33, 1001, "CROSS_ENTROPY", "f32"),
    "tanh-f16": (_tanh_chain, 3, 33, 1001, "MEAN_SQUARED_ERROR", "f16"),
    "tanh-bf16": (_tanh_chain, 3, 33, 1001, "MEAN_SQUARED_ERROR", "bf16"),
    "wide-bf16": (_wide, 7, 65, 2049, "MEAN_SQUARED_ERROR", "bf16"),
}


def run_case(ctx, name, mode):
    G = api()
    build, n_in, R, C, loss, kind = CASES[name]
    prev = fa.eltwise_mode(mode)
    try:
        graph, meta = G.Graph(getattr(G, loss), G.Optim.sgd().lower), G.Metadata.new()
        r, c = meta.new_field(), meta.new_field()
        row = name.startswith("broadcast")
        with graph.define_ops() as ops:
            xs = [ops.input([c] if row and k == 3 else [r, c], kind) for k in range(n_in)]
            build(ops, xs)
        mb = [G.f32_bits(1e-3), R, C]
        st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
        rng = np.random.default_rng(R * C + n_in)
        init = {"f32": ctx.init_tensor_f32, "f16": ctx.init_tensor_f16,
                "bf16": ctx.init_tensor_bf16}[kind]
        ins = []
        for k in range(n_in):
            shape = (C,) if row and k == 3 else (R, C)
            v = rng.standard_normal(shape).astype(f32)
            if name.startswith("broadcast") and k == 1:  # divisors away from zero
                v = (np.abs(v) + 0.5) * np.sign(v + 0.1)
            ins.append(init(shape, v))
        sch = ctx.schedule(graph.lower(meta), mb, ins, st)
        before = fa.eltwise_stats()
        ctx.dispatch_forward(sch)
        if loss == "CROSS_ENTROPY":
            ctx.dispatch_loss(sch, ctx.new_onehot_init(rng.integers(0, C, R)))
        elif loss == "BINARY_CROSS_ENTROPY" or name in ("mse",):
            ctx.dispatch_loss(sch, init((R, C), rng.uniform(0, 1, (R, C)).astype(f32)))
        else:
            ctx.upload(st.seed, rng.standard_normal(R * C).astype(f32))
        ctx.dispatch_backward(sch)
        ctx.sync()
        after = fa.eltwise_stats()
        out = [ctx.download(st.forward_out).copy(), ctx.download(st.seed).copy()]
        if loss != "MEAN_SQUARED_ERROR" or name == "mse":
            out.append(ctx.download(st.loss_t).copy())
        out += [ctx.download(t).copy() for t in st.grad_tensors]
        st.plan.close()
        return out, {k: after[k] - before[k] for k in after}
    finally:
        fa.eltwise_mode(prev)


@pytest.mark.parametrize("name", list(CASES))
def test_compiled_programs_match_interpreter(ctx, name):
    interp, di = run_case(ctx, name, fa.ELTWISE_INTERPRET)
    comp, dc = run_case(ctx, name, fa.ELTWISE_COMPILE_ALL)
    assert di["interpreted_launches"] > 0 and di["compiled_launches"] == 0, di
    assert dc["compiled_launches"] > 0 and dc["interpreted_launches"] == 0, dc
    assert len(interp) == len(comp)
    for k, (a, b) in enumerate(zip(interp, comp)):
        assert a.dtype == b.dtype and a.shape == b.shape
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), (
            name, k, int(np.sum(a.view(np.uint8) != b.view(np.uint8))))


def _unary_out(ctx, op, X, mode):
    G = api()
    prev = fa.eltwise_mode(mode)
    try:
        graph, meta = G.Graph(G.MEAN_SQUARED_ERROR, G.Optim.sgd().lower), G.Metadata.new()
        r, c = meta.new_field(), meta.new_field()
        with graph.define_ops() as ops:
            getattr(ops, op)(ops.input([r, c]))
        mb = [G.f32_bits(1e-3), 1, X.size]
        st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
        sch = ctx.schedule(graph.lower(meta), mb, [ctx.init_tensor_f32((1, X.size), X)], st)
        ctx.dispatch_forward(sch)
        ctx.sync()
        out = ctx.download(st.forward_out).copy()
        st.plan.close()
        return out
    finally:
        fa.eltwise_mode(prev)


def _ulp_err(r, ref):
    """|r - ref| in units of the fp32 spacing at ref (subnormal spacing
    below the normal range); exact matches of inf / nan count 0."""
    ref32 = ref.astype(np.float32)
    same = (r == ref32) | (np.isnan(r) & np.isnan(ref))
    sp = np.spacing(np.abs(ref32).astype(np.float32)).astype(np.float64)
    err = np.abs(r.astype(np.float64) - ref) / sp
    return np.where(same, 0.0, err)


@pytest.mark.parametrize("op,bound", [("exp", 2.0), ("log", 2.0), ("tanh", 3.0)])
def test_exp_log_tanh_accuracy(ctx, op, bound):
    """The elementwise exp / log / tanh (fg_elt_ops.h, built on the
    hardware's base-2 exponential and logarithm) against float64 over their
    whole ranges -- subnormal and overflowing results, the special values --
    within the stated ulp bound, and the same bits interpreted and compiled."""
    rng = np.random.default_rng(5)
    n = 1 << 20
    if op == "exp":
        X = np.concatenate([rng.uniform(-110, 90, n), rng.uniform(-1e-3, 1e-3, n // 4),
                            [0.0, -0.0, np.inf, -np.inf, np.nan, 88.72283, 88.72284, -103.97, -87.3]])
        ref = lambda x: np.exp(x)
    elif op == "log":
        X = np.concatenate([10.0 ** rng.uniform(-45, 38.5, n), rng.uniform(0.999, 1.001, n // 4),
                            [0.0, -0.0, -1.0, np.inf, np.nan, 1.0, 1e-45, 1.1754944e-38]])
        ref = lambda x: np.log(x)
    else:
        X = np.concatenate([rng.uniform(-10, 10, n), rng.uniform(-0.6, 0.6, n),
                            rng.uniform(-1e-4, 1e-4, n // 4),
                            [0.0, -0.0, np.inf, -np.inf, np.nan, 0.55, -0.55, 0.5499999]])
        ref = lambda x: np.tanh(x)
    X = X.astype(f32)
    with np.errstate(all="ignore"):
        exp64 = ref(X.astype(np.float64))
    a = _unary_out(ctx, op, X, fa.ELTWISE_INTERPRET)
    b = _unary_out(ctx, op, X, fa.ELTWISE_COMPILE_ALL)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), op
    with np.errstate(all="ignore"):
        err = _ulp_err(a, exp64)
    worst = int(np.argmax(err))
    assert err.max() <= bound, (op, float(err.max()), float(X[worst]), float(a[worst]),
                                float(exp64[worst]))


def test_programs_compile_once_per_process(ctx):
    """A second plan with the same programs reuses the compiled kernels."""
    run_case(ctx, "tanh-partial", fa.ELTWISE_COMPILE_ALL)
    _, d = run_case(ctx, "tanh-partial", fa.ELTWISE_COMPILE_ALL)
    assert d["compiled"] == 0 and d["compiled_launches"] > 0, d


def test_default_mode_compiles_only_large_programs(ctx):
    """FG_ELTWISE_COMPILE_LARGE: the 37 x 1025 programs stay on the
    interpreter, the 1031 x 4099 ones (over 2^20 elements) are compiled."""
    _, small = run_case(ctx, "tanh-partial", fa.ELTWISE_COMPILE_LARGE)
    _, large = run_case(ctx, "tanh-streaming", fa.ELTWISE_COMPILE_LARGE)
    assert small["compiled_launches"] == 0 and small["interpreted_launches"] > 0, small
    assert large["compiled_launches"] > 0 and large["interpreted_launches"] == 0, large


def test_captured_step_with_compiled_programs(ctx):
    """p = tanh(x * w + b) (b a row vector), MSE, Adam: three replays of a
    step captured with compiled programs match three eager steps on the
    interpreter bit for bit (parameters and per-element loss).  The capture compiles
    the programs before it starts, so no program is interpreted inside it."""
    G = api()
    R, C = 129, 1027
    runs = []
    for captured in (False, True):
        prev = fa.eltwise_mode(fa.ELTWISE_COMPILE_ALL if captured else fa.ELTWISE_INTERPRET)
        try:
            graph, meta = G.Graph(G.MEAN_SQUARED_ERROR, G.Optim.adam().lower), G.Metadata.new()
            r, c = meta.new_field(), meta.new_field()
            with graph.define_ops() as ops:
                x, w, b = ops.input([r, c]), ops.input([r, c]), ops.input([c])
                ops.tanh(ops.bias_add(ops.mul(x, w), b))
            mb = [G.f32_bits(1e-2), R, C]
            st = ctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
            rng = np.random.default_rng(11)
            X, W = (rng.standard_normal((R, C)).astype(f32) for _ in range(2))
            bv = rng.standard_normal(C).astype(f32)
            ins = [ctx.init_tensor_f32((R, C), X), ctx.init_tensor_f32((R, C), W),
                   ctx.init_tensor_f32((C,), bv)]
            tgt = ctx.init_tensor_f32((R, C), rng.uniform(-1, 1, (R, C)).astype(f32))
            sch = ctx.schedule(graph.lower(meta), mb, ins, st)
            if captured:
                s0 = fa.eltwise_stats()
                ctx.capture_step(sch, tgt)
                s1 = fa.eltwise_stats()
                # a program met uncompiled inside the capture would have
                # been recorded as an interpreter launch
                assert s1["interpreted_launches"] == s0["interpreted_launches"], (s0, s1)
            hist = []
            for _ in range(3):
                if captured:
                    ctx.launch_step(sch)
                else:
                    ctx.dispatch_forward(sch)
                    ctx.dispatch_loss(sch, tgt)
                    ctx.dispatch_backward(sch)
                    ctx.dispatch_optim(sch)
                ctx.sync()
                hist.append([ctx.download(t).copy() for t in ins] +
                            [ctx.download(st.loss_t).copy()])
            st.plan.close()
        finally:
            fa.eltwise_mode(prev)
        runs.append(hist)
    for step, (a, b) in enumerate(zip(*runs)):
        for k, (u, v) in enumerate(zip(a, b)):
            assert np.array_equal(u.view(np.uint8), v.view(np.uint8)), (step, k)
