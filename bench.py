#!/usr/bin/env python3
"""Benchmark of ferrograd's fused training path on one MI355X.

Headline ("c5"): one full training step of the
8-layer MLP -- batch 2048, fp32, 1024 -> 4096 x7 -> 1000, GELU (tanh) after
layers 1-7, softmax cross-entropy, Adam (lr 1e-3) -- with inputs and
parameters resident in HBM.  value = training steps per second.

Also measured in the same run (HIP events on the stream the kernels run on):
  * the dominant kernel of the step, the hidden-layer forward GEMM
    (2048 x 4096 x 4096, bias + GELU epilogue) -> roofline vs fp32 MFMA peak;
  * c2: 4096^3 GEMM forward (bias + ReLU) and its dA / dB backward;
  * c3: fused softmax + CE forward/backward over [8192, 32000];
  * c4: multi-tensor Adam over 64 x 4 Mi parameters;
  * c1: the 2-layer MLP step (latency bound: steps/s, launches, us/launch);
  * the same c2 GEMMs and c5 step with bfloat16 tensors;
and the CPU restatement (oracle/) timed on the host cores on a bounded
sample of the same workload (one full c5 step on the same inputs), which
also gives a parity check of the step's loss and gradients.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "MLP train steps/sec on 1 MI355X; GEMM TFLOP/s; softmax/Adam HBM GB/s"
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
PEAK_BF16_MFMA_TFLOPS = 2500.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def event_time_ms(fn, reps: int, warm_ms: float = 0.0) -> float:
    """Average duration of fn() over reps launches, timed with HIP events on
    torch's current stream (the stream the library context enqueues on).
    fn() runs once untimed first, then repeatedly for warm_ms of wall time:
    after an idle spell the GPU's clocks take some tens of milliseconds to
    rise, which reads as a slower kernel (about 7 % on the 4096^3 GEMMs)."""
    import torch

    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < warm_ms:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / reps


class MLPStep:
    """An MLP training step built as a ferrograd graph and run through the
    planner: matmul -> bias_add -> act per hidden layer, softmax +
    CROSS_ENTROPY, then the optimiser.  Weights Kaiming-uniform
    U(-sqrt(6/fan_in), +sqrt(6/fan_in)), biases 0, labels U{0..classes-1},
    all from the device generator keyed by `seed`.  X is an Input whose
    gradient is computed (ferrograd trains every Input) but which the
    optimiser does not update.

    c5: X ~ N(0,1), 1024 -> 4096 x7 -> 1000, GELU, Adam lr 1e-3, seed 4.
    c1: X ~ U[0,1), 784 -> 256 -> 10, ReLU, SGD lr 0.01, seed 0."""

    def __init__(self, ctx, dims, batch, act="gelu", optim="adam", lr=1e-3, seed=4,
                 x_dist="normal", dtype="f32"):
        import torch

        from ferrograd_amd import graph as G

        self.G, self.ctx, self.dims, self.B = G, ctx, dims, batch
        self.gctx = G.GpuContext(ctx)
        opt = G.Optim.adam() if optim == "adam" else G.Optim.sgd()
        graph, meta = G.Graph(G.CROSS_ENTROPY, opt.lower), G.Metadata.new()
        fb = meta.new_field()
        fd = [meta.new_field() for _ in dims]
        L = len(dims) - 1
        with graph.define_ops() as ops:
            h = ops.input([fb, fd[0]], dtype, trainable=False)
            self.w_nodes, self.b_nodes = [], []
            for l in range(L):
                W = ops.input([fd[l], fd[l + 1]], dtype)
                b = ops.input([fd[l + 1]], dtype)
                self.w_nodes.append(W)
                self.b_nodes.append(b)
                z = ops.bias_add(ops.matmul(h, W), b)
                h = (ops.gelu(z) if act == "gelu" else ops.relu(z)) if l < L - 1 else z
            ops.softmax(h)
        mb = [G.f32_bits(lr), batch] + list(dims)
        self.st = self.gctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
        self.X = torch.empty((batch, dims[0]), device="cuda")
        self.labels = torch.empty((batch,), device="cuda", dtype=torch.int32)
        if x_dist == "normal":
            ctx.rng_normal(seed, 0, 0.0, 1.0, self.X, self.X.numel())
        else:
            ctx.rng_uniform(seed, 0, 0.0, 1.0, self.X, self.X.numel())
        ctx.rng_int(seed, 1, dims[-1], self.labels, batch)
        self.W = [torch.empty((dims[l], dims[l + 1]), device="cuda") for l in range(L)]
        self.b = [torch.zeros((dims[l + 1],), device="cuda") for l in range(L)]
        for l, w in enumerate(self.W):
            bound = math.sqrt(6.0 / dims[l])
            ctx.rng_uniform(seed, 10 + l, -bound, bound, w, w.numel())
        if dtype != "f32":  # same draws, rounded to the 16-bit type
            tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
            self.X = self.X.to(tdt)
            self.W = [w.to(tdt) for w in self.W]
            self.b = [b.to(tdt) for b in self.b]
        ins = [self.X]
        for w, b in zip(self.W, self.b):
            ins += [w, b]
        self.sch = self.gctx.schedule(graph.lower(meta), mb, ins, self.st)
        gmap = {t.node: t for t in self.st.grad_tensors}
        self.dW = [gmap[n] for n in self.w_nodes]
        self.db = [gmap[n] for n in self.b_nodes]
        self.describe = self.sch.plan.describe()

    def launches_per_step(self) -> int:
        """Kernel dispatches of one step as planned (forward, loss, backward
        from the fused CE seed, optimiser)."""
        for line in self.describe.splitlines():
            if line.startswith("kernels per step: "):
                return int(line.split()[3])
        raise RuntimeError("plan description has no kernel count")

    def forward(self):
        self.gctx.dispatch_forward(self.sch)

    def loss(self):
        self.gctx.dispatch_loss(self.sch, self.labels)

    def backward(self):
        self.gctx.dispatch_backward(self.sch)

    def step_eager(self):
        self.forward()
        self.loss()
        self.backward()
        self.gctx.dispatch_optim(self.sch)

    def capture(self):
        self.gctx.capture_step(self.sch, self.labels)

    def step_graph(self):
        self.gctx.launch_step(self.sch)

    def mean_loss(self) -> float:
        return float(self.gctx.download(self.st.mean_loss)[0])

    def download(self, t):
        return self.gctx.download(t)

    def gemm_flops(self) -> int:
        """Algorithmic GEMM flops of one step: forward, dW, and dX for every
        layer including the data input (2*M*N*K per GEMM)."""
        return 2 * self.B * sum(self.dims[l] * self.dims[l + 1]
                                for l in range(len(self.dims) - 1)) * 3

    def num_params(self) -> int:
        return sum(w.numel() for w in self.W) + sum(b.numel() for b in self.b)


def gemm_components(ctx, reps: int):
    """c2 (4096^3) forward + dA + dB, and the c5 hidden-layer forward GEMM."""
    import torch

    import ferrograd_amd as fa

    out = {}
    n = 4096
    g = torch.Generator(device="cuda").manual_seed(1)
    A = torch.randn((n, n), device="cuda", generator=g)
    Bm = torch.randn((n, n), device="cuda", generator=g)
    bias = 0.1 * torch.randn((n,), device="cuda", generator=g)
    dC = torch.randn((n, n), device="cuda", generator=g)
    C, Z, dA, dB = (torch.empty((n, n), device="cuda") for _ in range(4))
    flops = 2.0 * n * n * n
    t_f = event_time_ms(lambda: ctx.gemm(fa.NN, n, n, n, A, n, Bm, n, C, n, bias=bias,
                                         act=fa.ACT_RELU, Z=Z, ldz=n), reps, warm_ms=200)
    t_a = event_time_ms(lambda: ctx.gemm_bwd(fa.NT, n, n, n, dC, n, Bm, n, dA, n,
                                             act=fa.ACT_RELU, Zs=Z, ldzs=n), reps, warm_ms=200)
    t_b = event_time_ms(lambda: ctx.gemm(fa.TN, n, n, n, A, n, dC, n, dB, n), reps, warm_ms=200)
    out["c2_gemm_4096"] = {
        "fwd_ms": t_f, "dA_ms": t_a, "dB_ms": t_b,
        "fwd_tflops": flops / t_f / 1e9, "dA_tflops": flops / t_a / 1e9,
        "dB_tflops": flops / t_b / 1e9,
        "fwd_bwd_tflops": 3 * flops / (t_f + t_a + t_b) / 1e9,
    }
    del A, Bm, bias, dC, C, Z, dA, dB
    # c5 hidden layer forward: [2048,4096] x [4096,4096] + bias, GELU.
    M, N, K = 2048, 4096, 4096
    X = torch.randn((M, K), device="cuda", generator=g)
    W = torch.randn((K, N), device="cuda", generator=g)
    b = torch.randn((N,), device="cuda", generator=g)
    H, Zh = torch.empty((M, N), device="cuda"), torch.empty((M, N), device="cuda")
    t = event_time_ms(lambda: ctx.gemm(fa.NN, M, N, K, X, K, W, N, H, N, bias=b,
                                       act=fa.ACT_GELU, Z=Zh, ldz=N), reps, warm_ms=200)
    out["c5_hidden_fwd_gemm"] = {"ms": t, "flops_per_launch": 2 * M * N * K,
                                 "tflops": 2.0 * M * N * K / t / 1e9,
                                 # X, W, bias read once; H and Z written once.
                                 "bytes": 4 * (M * K + K * N + N + 2 * M * N)}
    return out


def softmax_component(ctx, reps: int):
    import torch

    R, C = 8192, 32000
    x = torch.empty((R, C), device="cuda")
    lab = torch.empty((R,), device="cuda", dtype=torch.int32)
    ctx.rng_normal(2, 0, 0.0, 2.0, x, R * C)
    ctx.rng_int(2, 1, C, lab, R)
    d = torch.empty_like(x)
    loss, mean = torch.empty(R, device="cuda"), torch.empty(1, device="cuda")
    am = torch.empty(R, device="cuda", dtype=torch.int32)
    t = event_time_ms(lambda: ctx.softmax_ce(x, C, lab, R, C, 1.0, row_loss=loss,
                                             mean_loss=mean, dlogits=d, ldd=C, argmax=am),
                      reps, warm_ms=200)
    nbytes = 2 * R * C * 4 + R * 4 * 3  # logits in, dlogits out, labels/loss/argmax
    return {"c3_softmax_ce_8192x32000": {"ms": t, "bytes": nbytes, "gbs": nbytes / t / 1e6,
                                         "frac_hbm": nbytes / t / 1e6 / PEAK_HBM_GBS}}


def adam_component(ctx, reps: int):
    import torch

    import ferrograd_amd as fa

    nt, n = 64, 4 * 1024 * 1024
    P = [torch.empty(n, device="cuda") for _ in range(nt)]
    G = [torch.empty(n, device="cuda") for _ in range(nt)]
    M = [torch.zeros(n, device="cuda") for _ in range(nt)]
    V = [torch.zeros(n, device="cuda") for _ in range(nt)]
    for i in range(nt):
        ctx.rng_normal(3, i, 0.0, 0.02, P[i], n)
        ctx.rng_normal(3, 1000 + i, 0.0, 1e-3, G[i], n)
    mt = fa.MultiTensor(ctx, P, G, M, V)
    step = [0]

    def one():
        step[0] += 1
        mt.adam(1e-3, 0.9, 0.999, 1e-8, step[0])

    t = event_time_ms(one, reps, warm_ms=200)
    mt.close()
    nbytes = 28 * nt * n
    return {"c4_adam_64x4Mi": {"ms": t, "bytes": nbytes, "gbs": nbytes / t / 1e6,
                               "frac_hbm": nbytes / t / 1e6 / PEAK_HBM_GBS}}


def copy_component(reps: int):
    """Context for the HBM-bound kernels: a plain device copy of 1 GiB
    (torch's copy kernel), read + write bytes per second."""
    import torch

    a = torch.ones(256 * 1024 * 1024, device="cuda")
    b = torch.empty_like(a)
    t = event_time_ms(lambda: b.copy_(a), reps, warm_ms=200)
    nbytes = 2 * a.numel() * 4
    del a, b
    return {"hbm_copy_1gib": {"ms": t, "bytes": nbytes, "gbs": nbytes / t / 1e6,
                              "frac_hbm": nbytes / t / 1e6 / PEAK_HBM_GBS}}


def c5_bf16_component(ctx, steps: int = 10):
    """The c5 step with every tensor in bfloat16 (16-bit MFMA GEMMs, fp32
    sums and optimiser state): captured steps/s and effective TFLOP/s."""
    import torch

    dims = [1024] + [4096] * 7 + [1000]
    tr = MLPStep(ctx, dims, 2048, dtype="bf16")
    tr.step_eager()
    tr.capture()
    tr.step_graph()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        tr.step_graph()
    torch.cuda.synchronize()
    ms = 1000.0 * (time.perf_counter() - t0) / steps
    return {"c5_bf16_step": {"steps_per_s": 1000.0 / ms, "ms_per_step": ms,
                             "effective_tflops": tr.gemm_flops() / (ms * 1e-3) / 1e12,
                             "loss": tr.mean_loss(), "steps_timed": steps}}


def gemm_bf16_component(ctx, reps: int):
    """c2-shaped 4096^3 GEMMs in bfloat16: forward (bias + ReLU), dA, dB."""
    import torch

    import ferrograd_amd as fa

    n = 4096
    g = torch.Generator(device="cuda").manual_seed(1)
    A, Bm, dC = (torch.randn((n, n), device="cuda", generator=g).to(torch.bfloat16)
                 for _ in range(3))
    bias = (0.1 * torch.randn((n,), device="cuda", generator=g)).to(torch.bfloat16)
    C, Z, dA, dB = (torch.empty((n, n), device="cuda", dtype=torch.bfloat16) for _ in range(4))
    bf = fa.DTYPE_BF16
    flops = 2.0 * n * n * n
    t_f = event_time_ms(lambda: ctx.gemm_x16(bf, fa.NN, n, n, n, A, n, Bm, n, C, n, bias=bias,
                                             act=fa.ACT_RELU, Z=Z, ldz=n), reps, warm_ms=200)
    t_a = event_time_ms(lambda: ctx.gemm_bwd_x16(bf, fa.NT, n, n, n, dC, n, Bm, n, dA, n,
                                                 act=fa.ACT_RELU, Zs=Z, ldzs=n), reps, warm_ms=200)
    t_b = event_time_ms(lambda: ctx.gemm_x16(bf, fa.TN, n, n, n, A, n, dC, n, dB, n), reps,
                        warm_ms=200)
    tf = lambda t: flops / t / 1e9
    return {"c2_gemm_4096_bf16": {"fwd_tflops": tf(t_f), "dA_tflops": tf(t_a),
                                  "dB_tflops": tf(t_b), "peak_tflops": PEAK_BF16_MFMA_TFLOPS,
                                  "fwd_ms": t_f, "dA_ms": t_a, "dB_ms": t_b}}


def c1_component(ctx, steps: int = 2000):
    """c1: the 2-layer MLP step (batch 64, 784 -> 256 -> 10, ReLU, softmax-CE,
    SGD lr 0.01), latency bound: steps/s of the captured step, launches per
    step and the average time per launch."""
    import torch

    tr = MLPStep(ctx, [784, 256, 10], 64, act="relu", optim="sgd", lr=0.01, seed=0,
                 x_dist="uniform")
    for _ in range(3):
        tr.step_eager()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        tr.step_eager()
    torch.cuda.synchronize()
    eager_ms = 1000.0 * (time.perf_counter() - t0) / steps
    tr.capture()
    tr.step_graph()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        tr.step_graph()
    torch.cuda.synchronize()
    ms = 1000.0 * (time.perf_counter() - t0) / steps
    n = tr.launches_per_step()
    return {"c1_mlp_step": {"steps_per_s": 1000.0 / ms, "ms_per_step": ms,
                            "eager_ms_per_step": eager_ms, "launches_per_step": n,
                            "us_per_launch": 1000.0 * ms / n, "loss": tr.mean_loss(),
                            "steps_timed": steps}}


def only_gemm_c5_hidden(ctx, reps):
    """The c5 hidden-layer forward GEMM, 2048x4096x4096 + bias + GELU."""
    import torch

    import ferrograd_amd as fa

    M, N, K = 2048, 4096, 4096
    X, W = torch.randn((M, K), device="cuda"), torch.randn((K, N), device="cuda")
    b = torch.randn((N,), device="cuda")
    H, Z = torch.empty((M, N), device="cuda"), torch.empty((M, N), device="cuda")
    for _ in range(reps):
        ctx.gemm(fa.NN, M, N, K, X, K, W, N, H, N, bias=b, act=fa.ACT_GELU, Z=Z, ldz=N)


def only_softmax_ce_c3(ctx, reps):
    """The c3 fused softmax + CE over [8192, 32000]."""
    import torch

    R, C = 8192, 32000
    x = torch.empty((R, C), device="cuda")
    lab = torch.empty((R,), device="cuda", dtype=torch.int32)
    ctx.rng_normal(2, 0, 0.0, 2.0, x, R * C)
    ctx.rng_int(2, 1, C, lab, R)
    d = torch.empty_like(x)
    loss = torch.empty(R, device="cuda")
    for _ in range(reps):
        ctx.softmax_ce(x, C, lab, R, C, 1.0, row_loss=loss, dlogits=d, ldd=C)


def only_adam_c4(ctx, reps):
    """The c4 multi-tensor Adam over 64 x 4 Mi parameters."""
    import torch

    import ferrograd_amd as fa

    nt, n = 64, 4 * 1024 * 1024
    P = [torch.zeros(n, device="cuda") for _ in range(nt)]
    G = [torch.full((n,), 1e-3, device="cuda") for _ in range(nt)]
    M = [torch.zeros(n, device="cuda") for _ in range(nt)]
    V = [torch.zeros(n, device="cuda") for _ in range(nt)]
    mt = fa.MultiTensor(ctx, P, G, M, V)
    for step in range(1, reps + 1):
        mt.adam(1e-3, 0.9, 0.999, 1e-8, step)
    torch.cuda.synchronize()
    mt.close()


def only_copy_256mib(ctx, reps):
    """Calibration for the HBM counters: a plain device copy of 256 MiB
    (reads 256 MiB, writes 256 MiB per launch)."""
    import torch

    a = torch.ones(64 * 1024 * 1024, device="cuda")
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)


def only_c5_step(ctx, reps, dtype="f32"):
    """The c5 training step as a captured hipGraph, replayed (for kernel
    traces of the step alone)."""
    tr = MLPStep(ctx, [1024] + [4096] * 7 + [1000], 2048, dtype=dtype)
    tr.capture()
    for _ in range(reps):
        tr.step_graph()


def only_c5_step_bf16(ctx, reps):
    """The c5 step with bfloat16 tensors, captured and replayed."""
    only_c5_step(ctx, reps, dtype="bf16")


def only_gemm_bf16_c2(ctx, reps):
    """The c2-shaped 4096^3 bf16 GEMMs: forward (bias + ReLU), dA, dB."""
    import torch

    import ferrograd_amd as fa

    n, bf = 4096, fa.DTYPE_BF16
    g = torch.Generator(device="cuda").manual_seed(1)
    A, Bm, dC = (torch.randn((n, n), device="cuda", generator=g).to(torch.bfloat16)
                 for _ in range(3))
    bias = (0.1 * torch.randn((n,), device="cuda", generator=g)).to(torch.bfloat16)
    C, Z, dA, dB = (torch.empty((n, n), device="cuda", dtype=torch.bfloat16) for _ in range(4))
    for _ in range(reps):
        ctx.gemm_x16(bf, fa.NN, n, n, n, A, n, Bm, n, C, n, bias=bias, act=fa.ACT_RELU, Z=Z, ldz=n)
        ctx.gemm_bwd_x16(bf, fa.NT, n, n, n, dC, n, Bm, n, dA, n, act=fa.ACT_RELU, Zs=Z, ldzs=n)
        ctx.gemm_x16(bf, fa.TN, n, n, n, A, n, dC, n, dB, n)


def only_c1_step(ctx, reps):
    print(json.dumps(c1_component(ctx, steps=max(reps, 10))), flush=True)


ONLY = {
    "c1_step": only_c1_step,
    "c5_step": only_c5_step,
    "c5_step_bf16": only_c5_step_bf16,
    "gemm_bf16_c2": only_gemm_bf16_c2,
    "gemm_c5_hidden": only_gemm_c5_hidden,
    "softmax_ce_c3": only_softmax_ce_c3,
    "adam_c4": only_adam_c4,
    "copy_256mib": only_copy_256mib,
}


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed counter summary
    (profiles/traffic.json, produced from two rocprofv3 --pmc passes,
    FETCH_SIZE and WRITE_SIZE, scaled by what the same counters read for a
    plain 256 MiB copy); None when the summary is absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f)[kernel]["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def cpu_baseline_c5(host, dims, batch, threads):
    """One full c5 training step (forward, CE, backward incl. dX, Adam) with
    the CPU restatement, on the same initial inputs as the GPU run."""
    import numpy as np

    import oracle as O

    O.set_num_threads(threads)
    X, y, W = host["X"], host["y"], host["W"]
    L = len(W)
    b = [np.zeros(dims[l + 1], np.float32) for l in range(L)]
    t0 = time.perf_counter()
    Zs, Hs = [], []
    inp = X
    for l in range(L):
        last = l == L - 1
        Z, H = O.bias_act(O.gemm(O.NN, inp, W[l]), b[l], O.ACT_NONE if last else O.ACT_GELU)
        Zs.append(Z)
        Hs.append(H)
        inp = H
    row_loss, dZ, _, mean = O.softmax_ce(Zs[-1], y)
    dW, db = [None] * L, [None] * L
    for l in range(L - 1, -1, -1):
        prev = Hs[l - 1] if l > 0 else X
        dW[l] = O.gemm(O.TN, prev, dZ)
        db[l] = O.bias_grad(dZ)
        up = O.gemm(O.NT, dZ, W[l])
        dZ = O.act_bwd(O.ACT_GELU, up, Zs[l - 1]) if l > 0 else up
    s, r = O.adam_scalars(np.float32(1e-3), np.float32(0.9), np.float32(0.999), 1)
    Wn = []
    for l in range(L):
        for p, g in ((W[l].copy(), dW[l]), (b[l].copy(), db[l])):
            m, v = np.zeros_like(p), np.zeros_like(p)
            O.adam_(p, g, m, v, np.float32(0.9), np.float32(0.999), np.float32(1e-8), s, r)
            Wn.append(p)
    dt = time.perf_counter() - t0
    return dt, {"mean_loss": mean, "dW": dW, "db": db, "params": Wn}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-components", action="store_true",
                    help="skip the c2/c3/c4 component measurements")
    ap.add_argument("--reps", type=int, default=20, help="launches per kernel timing")
    ap.add_argument("--only", choices=sorted(ONLY), default=None,
                    help="run only this kernel --reps times (for rocprofv3 counter passes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested).", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import ferrograd_amd as fa

    if args.only:
        ctx, _stream = fa.torch_context(0)
        ONLY[args.only](ctx, args.reps)
        torch.cuda.synchronize()
        log(f"ran {args.only} x{args.reps}")
        return 0

    ctx, _stream = fa.torch_context(0)
    log(f"device {ctx.arch}, {ctx.cu_count} CUs")
    dims = [1024] + [4096] * 7 + [1000]
    batch = 2048
    tr = MLPStep(ctx, dims, batch)
    log("plan:\n" + tr.describe)
    torch.cuda.synchronize()
    host = None
    if not args.no_cpu:
        host = {"X": tr.X.cpu().numpy(), "y": tr.labels.cpu().numpy().view(np.uint32),
                "W": [w.cpu().numpy() for w in tr.W]}
    # First step (from the initial state) doubles as the parity sample.
    tr.step_eager()
    torch.cuda.synchronize()
    first = {"mean_loss": tr.mean_loss(),
             "dW": [tr.download(t).reshape(w.shape) for t, w in zip(tr.dW, tr.W)],
             "db": [tr.download(t) for t in tr.db], "W": [w.cpu().numpy() for w in tr.W]}
    for _ in range(max(0, args.warmup - 1)):
        tr.step_eager()
    torch.cuda.synchronize()
    # Eager launches (host-driven, one call per kernel).
    t0 = time.perf_counter()
    for _ in range(args.steps):
        tr.step_eager()
    torch.cuda.synchronize()
    eager_ms = 1000.0 * (time.perf_counter() - t0) / args.steps
    # The whole step captured once into a hipGraph and replayed.
    tr.capture()
    tr.step_graph()
    torch.cuda.synchronize()
    log(f"warmup done ({args.warmup} eager steps, eager {eager_ms:.3f} ms/step); "
        f"timing {args.steps} captured steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        tr.step_graph()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = 1000.0 * elapsed / args.steps
    steps_per_s = args.steps / elapsed
    log(f"c5 step: {ms_per_step:.3f} ms ({steps_per_s:.2f} steps/s); loss {tr.mean_loss():.4f}")

    # Per-phase breakdown (events).
    phases = {
        "eager_step_ms": eager_ms,
        "forward_ms": event_time_ms(tr.forward, 5),
        "loss_backward_ms": event_time_ms(lambda: (tr.loss(), tr.backward()), 5),
    }
    step_flops = tr.gemm_flops()

    comps = gemm_components(ctx, args.reps)
    hid = comps["c5_hidden_fwd_gemm"]
    roofline = {
        "bound": "mfma",
        "kernel": "gemm_f32_pipe NN 2048x4096x4096 + bias + GELU (c5 hidden-layer forward)",
        "achieved": hid["tflops"],
        "peak": PEAK_FP32_MFMA_TFLOPS,
        "unit": "TFLOP/s",
        "frac": hid["tflops"] / PEAK_FP32_MFMA_TFLOPS,
        "traffic": measured_traffic("gemm_c5_hidden"),
        "traffic_unit": "HBM bytes per launch (rocprofv3 FETCH_SIZE/WRITE_SIZE, copy-calibrated)",
        "algorithmic_bytes": hid["bytes"],
    }
    if not args.no_components:
        comps.update(softmax_component(ctx, args.reps))
        comps.update(adam_component(ctx, 10))
        comps.update(c1_component(ctx))
        comps.update(gemm_bf16_component(ctx, args.reps))
        comps.update(c5_bf16_component(ctx))
        comps.update(copy_component(args.reps))
    log("components: " + json.dumps(comps))

    cpu = None
    parity = None
    if host is not None:
        threads = min(16, os.cpu_count() or 1)
        log(f"CPU baseline: one c5 step on {threads} threads")
        dt, ref = cpu_baseline_c5(host, dims, batch, threads)
        cpu = {"value": 1.0 / dt, "unit": "steps/s", "cores": threads, "kind": "port",
               "sample": "one full c5 training step (forward, CE, backward incl. dX, Adam) "
                         "on the same inputs, oracle/ C restatement with OpenMP"}

        def rel(a, b):
            b = np.asarray(b, np.float64)
            return float(np.max(np.abs(np.asarray(a, np.float64) - b)) /
                         max(float(np.max(np.abs(b))), 1e-30))

        parity = {
            "loss_rel": abs(first["mean_loss"] - ref["mean_loss"]) / max(1.0, abs(ref["mean_loss"])),
            "dW_max_rel": max(rel(a, b) for a, b in zip(first["dW"], ref["dW"])),
            "db_max_rel": max(rel(a, b) for a, b in zip(first["db"], ref["db"])),
            # Adam's first step is p - lr*g/(|g|+eps), i.e. nearly -lr*sign(g):
            # where a gradient entry is within rounding noise of zero its sign
            # (and so a 2*lr step) can differ, so report the fraction of
            # parameters off by more than 1e-5 relative.
            "W_after_adam_mismatch_frac": float(np.mean(np.concatenate([
                (np.abs(a.astype(np.float64) - b) > 1e-5 * np.max(np.abs(b))).ravel()
                for a, b in zip(first["W"], ref["params"][0::2])]))),
            "tolerance_gemm": 1e-5 * math.sqrt(4096),
        }
        log("parity vs CPU: " + json.dumps(parity))

    result = {
        "metric": METRIC,
        "value": steps_per_s,
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (counter-based SplitMix64 generator, seed 4; random-init weights)",
        "config": {
            "workload": "c5: 8-layer MLP training step, batch 2048, 1024->4096x7->1000, "
                        "GELU-tanh, softmax-CE, Adam lr 1e-3 (dX of the data input computed, "
                        "as ferrograd trains every Input)",
            "global_batch": batch,
            "dims": dims,
            "parallelism": "single GPU",
            "gemm_flops_per_step": step_flops,
            "params": tr.num_params(),
        },
        "step_effective_tflops": step_flops / (ms_per_step * 1e-3) / 1e12,
        "phases_ms": phases,
        "roofline": roofline,
        "components": comps,
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
