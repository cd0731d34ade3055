#!/usr/bin/env python3
"""Benchmark of ferrograd's fused training path on one MI355X.

Headline ("c5"): one full training step of the
8-layer MLP -- batch 2048, fp32, 1024 -> 4096 x7 -> 1000, GELU (tanh) after
layers 1-7, softmax cross-entropy, Adam (lr 1e-3) -- with inputs and
parameters resident in HBM.  value = training steps per second.

Also measured in the same run (HIP events on the stream the kernels run on):
  * the dominant kernel of the step, the hidden-layer forward GEMM
    (2048 x 4096 x 4096, bias + GELU epilogue) -> roofline vs fp32 MFMA peak;
  * c2: 4096^3 GEMM forward (bias + ReLU) and its backward through the
    ReLU mask (dA, dB, dbias);
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
            self.x_node = h = ops.input([fb, fd[0]], dtype, trainable=False)
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
        self.dX = gmap[self.x_node]
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


def c2_inputs(ctx, n: int = 4096):
    """BASELINE c2 inputs from the library's generator, seed 1: A, B ~ N(0,1)
    (tensor ids 0, 1), bias ~ N(0, 0.1^2) (id 2; the configuration's
    "N(0,0.1)" read as a standard deviation of 0.1), dC ~ N(0,1) (id 3)."""
    import torch

    A, Bm, dC = (torch.empty((n, n), device="cuda") for _ in range(3))
    bias = torch.empty((n,), device="cuda")
    ctx.rng_normal(1, 0, 0.0, 1.0, A, n * n)
    ctx.rng_normal(1, 1, 0.0, 1.0, Bm, n * n)
    ctx.rng_normal(1, 2, 0.0, 0.1, bias, n)
    ctx.rng_normal(1, 3, 0.0, 1.0, dC, n * n)
    return A, Bm, bias, dC


def gemm_components(ctx, reps: int, want_host: bool = False):
    """c2 (4096^3): forward C = ReLU(A.B + bias), then the backward through
    the ReLU mask, dZ = dC*[Z>0], dA = dZ.B^T, dB = A^T.dZ, dbias =
    colsum(dZ) (fg_linear_bwd_f32; the forward output C gives the mask, so
    the forward stores no Z).  The backward is timed both ways: dZ
    materialised by one pass that also sums its columns, then plain GEMMs
    (the figure reported), and the mask applied as the GEMMs load dC (no dZ
    buffer).  Also the c5 hidden-layer forward GEMM.
    Returns (timings, sample): with want_host the sample holds the inputs
    and outputs (the parity sample of the CPU leg), else it is None."""
    import torch

    import ferrograd_amd as fa

    out = {}
    n = 4096
    A, Bm, bias, dC = c2_inputs(ctx, n)
    C, dA, dB, dZ = (torch.empty((n, n), device="cuda") for _ in range(4))
    db = torch.empty((n,), device="cuda")
    flops = 2.0 * n * n * n

    def fwd():
        ctx.gemm(fa.NN, n, n, n, A, n, Bm, n, C, n, bias=bias, act=fa.ACT_RELU)

    def bwd(dX=None, dW=None, dbias=None, mat=True):
        ctx.linear_bwd(fa.ACT_RELU, n, n, n, A, n, Bm, n, C, n, dC, n, dX=dX, lddx=n, dW=dW,
                       lddw=n, dbias=dbias, dZ=dZ if mat else None, lddz=n)

    t_f = event_time_ms(fwd, reps, warm_ms=200)
    # The mask pass alone (dZ and dbias), then each GEMM on dZ, then all.
    t_m = event_time_ms(lambda: bwd(dbias=db), reps, warm_ms=200)
    t_a = event_time_ms(lambda: ctx.gemm_bwd(fa.NT, n, n, n, dZ, n, Bm, n, dA, n), reps,
                        warm_ms=200)
    t_b = event_time_ms(lambda: ctx.gemm(fa.TN, n, n, n, A, n, dZ, n, dB, n), reps, warm_ms=200)
    t_bwd = event_time_ms(lambda: bwd(dX=dA, dW=dB, dbias=db), reps, warm_ms=200)
    t_pro = event_time_ms(lambda: bwd(dX=dA, dW=dB, dbias=db, mat=False), reps, warm_ms=200)
    out["c2_gemm_4096"] = {
        "fwd_ms": t_f, "mask_dbias_ms": t_m, "dA_ms": t_a, "dB_ms": t_b, "bwd_ms": t_bwd,
        "bwd_prologue_ms": t_pro,
        "fwd_tflops": flops / t_f / 1e9, "dA_tflops": flops / t_a / 1e9,
        "dB_tflops": flops / t_b / 1e9,
        "mask_pass_gbs": 12 * n * n / t_m / 1e6,
        "fwd_bwd_ms": t_f + t_bwd,
        "fwd_bwd_tflops": 3 * flops / (t_f + t_bwd) / 1e9,
        "backward": "one pass dZ = dC*[C>0] with dbias = colsum(dZ), then dA = dZ.B^T (NT) "
                    "and dB = A^T.dZ (TN); bwd_prologue_ms: the mask applied as the GEMMs "
                    "load dC instead (no dZ buffer)",
    }
    sample = None
    if want_host:
        bwd(dX=dA, dW=dB, dbias=db)  # the reported path's outputs for the parity sample
        torch.cuda.synchronize()
        sample = {k: v.cpu().numpy() for k, v in (("A", A), ("B", Bm), ("bias", bias),
                                                   ("dC", dC), ("C", C), ("dA", dA),
                                                   ("dB", dB), ("db", db))}
    del A, Bm, bias, dC, C, dA, dB, db, dZ
    g = torch.Generator(device="cuda").manual_seed(1)
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
    return out, sample


def c5_gemm_kernels(ctx):
    """The GEMMs of the c5 step on its shapes and epilogues (random
    operands, library generator): key -> (description, launch closure,
    algorithmic bytes per launch, flops per launch, launches per step).  A
    hidden layer runs the forward and the dW + dX pair (fg_matmul_bwd_f32:
    one launch); dX and dW are also timed alone.  The first layer and the
    head complete the step's 24 GEMMs."""
    import torch

    import ferrograd_amd as fa

    M, N, K = 2048, 4096, 4096
    X, W, dZ, Zs = (torch.empty(shape, device="cuda") for shape in
                    ((M, K), (K, N), (M, N), (M, K)))
    b, db = torch.empty((N,), device="cuda"), torch.empty((N,), device="cuda")
    for i, t in enumerate((X, W, dZ, Zs, b)):
        ctx.rng_normal(4, 500 + i, 0.0, 1.0, t, t.numel())
    H, Z, dX, dW = (torch.empty(shape, device="cuda") for shape in
                    ((M, N), (M, N), (M, K), (K, N)))
    F, C = 1024, 1000  # the first layer's input width, the head's classes
    X0, W0, W7, b7, D7 = (torch.empty(shape, device="cuda") for shape in
                          ((M, F), (F, N), (K, C), (C,), (M, C)))
    for i, t in enumerate((X0, W0, W7, b7, D7)):
        ctx.rng_normal(4, 520 + i, 0.0, 1.0, t, t.numel())
    L7, dW7, db7, dX7, dX0, dW0 = (torch.empty(shape, device="cuda") for shape in
                                   ((M, C), (K, C), (C,), (M, K), (M, F), (F, N)))
    dx_bytes = 4 * (M * N + K * N + 2 * M * K)
    dw_bytes = 4 * (M * K + M * N + K * N + N)
    return {
        "gemm_c5_fwd": ("NN 2048x4096x4096 + bias + GELU, Z stored (forward)",
                        lambda: ctx.gemm(fa.NN, M, N, K, X, K, W, N, H, N, bias=b,
                                         act=fa.ACT_GELU, Z=Z, ldz=N),
                        4 * (M * K + K * N + N + 2 * M * N), 2 * M * N * K, 6),
        "gemm_c5_bwd_pair": ("TN 4096x4096x2048 + fused dbias and NT 2048x4096x4096 * GELU'(Z) "
                             "in one launch (dW, db and dX of a hidden layer)",
                             lambda: ctx.matmul_bwd(M, N, K, X, K, W, N, dZ, N, dX, K, dW, N,
                                                    dbias=db, act=fa.ACT_GELU, Zs=Zs, ldzs=K),
                             # dZ is read by both GEMMs
                             dx_bytes + dw_bytes, 4 * M * N * K, 6),
        "gemm_c5_dx": ("NT 2048x4096x4096 * GELU'(Z) (dX of a hidden layer, alone)",
                       lambda: ctx.gemm_bwd(fa.NT, M, K, N, dZ, N, W, N, dX, K,
                                            act=fa.ACT_GELU, Zs=Zs, ldzs=K),
                       dx_bytes, 2 * M * N * K, 0),
        "gemm_c5_dw": ("TN 4096x4096x2048 + fused dbias (dW, db of a hidden layer, alone)",
                       lambda: ctx.gemm_dw(K, N, M, X, K, dZ, N, dW, N, colsum=db),
                       dw_bytes, 2 * M * N * K, 0),
        # The step's other GEMMs: the 1024-wide first layer and the 1000-wide head.
        "gemm_c5_fwd_first": ("NN 2048x4096x1024 + bias + GELU, Z stored (first layer)",
                              lambda: ctx.gemm(fa.NN, M, N, F, X0, F, W0, N, H, N, bias=b,
                                               act=fa.ACT_GELU, Z=Z, ldz=N),
                              4 * (M * F + F * N + N + 2 * M * N), 2 * M * N * F, 1),
        "gemm_c5_fwd_head": ("NN 2048x1000x4096 + bias (head)",
                             lambda: ctx.gemm(fa.NN, M, C, K, X, K, W7, C, L7, C, bias=b7),
                             4 * (M * K + K * C + C + M * C), 2 * M * C * K, 1),
        "gemm_c5_dw_head": ("TN 4096x1000x2048 + fused dbias (head dW, db)",
                            lambda: ctx.gemm_dw(K, C, M, X, K, D7, C, dW7, C, colsum=db7),
                            4 * (M * K + M * C + K * C + C), 2 * M * C * K, 1),
        "gemm_c5_dx_head": ("NT 2048x4096x1000 * GELU'(Z) (head dX, K tail)",
                            lambda: ctx.gemm_bwd(fa.NT, M, K, C, D7, C, W7, C, dX7, K,
                                                 act=fa.ACT_GELU, Zs=Zs, ldzs=K),
                            4 * (M * C + K * C + 2 * M * K), 2 * M * C * K, 1),
        "gemm_c5_pair_first": ("TN 1024x4096x2048 + fused dbias and NT 2048x1024x4096 in one "
                               "launch (first layer's dW, db and the data input's dX)",
                               lambda: ctx.matmul_bwd(M, N, F, X0, F, W0, N, dZ, N, dX0, F, dW0,
                                                      N, dbias=db),
                               4 * (2 * M * N + F * N + M * F) + 4 * (M * F + M * N + F * N + N),
                               4 * M * N * F, 1),
    }


def c5_gemm_shares(ctx, reps: int, step_ms: float):
    """The c5 step's GEMMs timed with HIP events on the step's own shapes
    and epilogues: the hidden layers' forward NN 2048x4096x4096 + bias +
    GELU (+Z), 6 launches per step, and backward pair (dW TN
    4096x4096x2048 with the fused dbias beside dX NT 2048x4096x4096 with the
    GELU derivative, one launch), 6 per step; the first layer's forward and
    pair and the head's forward, dW and dX, one each; share = launches per
    step * time / step time.  Hidden dX and dW alone (share None: the step
    does not launch them alone) for comparison."""
    out = {}
    for key, (what, fn, nbytes, flops, per_step) in c5_gemm_kernels(ctx).items():
        t = event_time_ms(fn, reps, warm_ms=200)
        out[key] = {"what": what, "ms": t, "tflops": flops / t / 1e9,
                    "frac": flops / t / 1e9 / PEAK_FP32_MFMA_TFLOPS, "per_step": per_step,
                    "step_share": per_step * t / step_ms if per_step else None,
                    "flops_per_launch": flops, "algorithmic_bytes": nbytes}
    return out


def softmax_component(ctx, reps: int, want_host: bool = False):
    """c3: fused softmax + CE forward / backward over [8192, 32000] (library
    generator, seed 2: logits N(0, 2^2) id 0, labels U{0..31999} id 1).  With
    want_host, also returns inputs and outputs as the CPU leg's sample."""
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
    out = {"c3_softmax_ce_8192x32000": {"ms": t, "bytes": nbytes, "gbs": nbytes / t / 1e6,
                                        "frac_hbm": nbytes / t / 1e6 / PEAK_HBM_GBS}}
    if not want_host:
        return out
    import numpy as np
    torch.cuda.synchronize()
    sample = {"x": x.cpu().numpy(), "y": lab.cpu().numpy().view(np.uint32),
              "row_loss": loss.cpu().numpy(), "mean": float(mean.cpu()[0]),
              "d": d.cpu().numpy(), "argmax": am.cpu().numpy().view(np.uint32)}
    return out, sample


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


def eltwise_tanh_plan(ctx, R: int, C: int):
    """The planner's forward of y = tanh(a * b + c) over R x C fp32 inputs
    a, b, c ~ N(0,1) (library generator, seed 7): one elementwise-program
    launch.  Returns (tensors, schedule, context, inputs to keep alive)."""
    import numpy as np
    import torch

    from ferrograd_amd import graph as G

    gctx = G.GpuContext(ctx)
    graph, meta = G.Graph(G.MEAN_SQUARED_ERROR, G.Optim.sgd().lower), G.Metadata.new()
    fr, fc = meta.new_field(), meta.new_field()
    with graph.define_ops() as ops:
        a, b, c = (ops.input([fr, fc], trainable=False) for _ in range(3))
        ops.tanh(ops.add(ops.mul(a, b), c))
    mb = [G.f32_bits(1e-3), R, C]
    st = gctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    xs = [torch.empty((R, C), device="cuda") for _ in range(3)]
    for i, x in enumerate(xs):
        ctx.rng_normal(7, i, 0.0, 1.0, x, x.numel())
    ins = [G.Tensor(x.data_ptr(), x.numel() * 4, x.shape, np.float32, owner=x) for x in xs]
    sch = gctx.schedule(graph.lower(meta), mb, ins, st)
    assert "forward: 1 launches" in st.plan.describe()
    return st, sch, gctx, (xs, ins)


def hbm_kernels_component(ctx, reps: int):
    """The other HBM-bound kernels of the path, in GB/s of algorithmic bytes
    (each launch timed with HIP events after 200 ms of the same launches):
    * eltwise: a fused elementwise program, the planner's forward of
      y = tanh(a * b + c) over 8192 x 8192 fp32 -- one launch reading a, b,
      c and writing the three node values the plan keeps (a * b, a * b + c
      and y, its forward_saved tensors): 24 B per element; the default path
      runs the program's compiled kernel (fg_eltwise_set_mode: programs of
      2^20 elements or more), eltwise_..._interp the same program on the
      interpreter;
    * act_bwd: dZ = dH * GELU'(Z) over 2^28 elements (12 B per element);
    * sgd: the multi-tensor SGD over c4's 64 x 4 Mi parameters, gradients
      zeroed after the update (read p, g; write p, g: 16 B per parameter)."""
    import torch

    import ferrograd_amd as fa

    out = {}
    R = C = 8192
    st, sch, gctx, keep = eltwise_tanh_plan(ctx, R, C)
    nbytes = 24 * R * C
    for key, mode in (("eltwise_fwd_8192x8192", fa.ELTWISE_COMPILE_LARGE),
                      ("eltwise_fwd_8192x8192_interp", fa.ELTWISE_INTERPRET)):
        prev = fa.eltwise_mode(mode)
        try:
            t = event_time_ms(lambda: gctx.dispatch_forward(sch), reps, warm_ms=200)
        finally:
            fa.eltwise_mode(prev)
        out[key] = {"ms": t, "bytes": nbytes, "gbs": nbytes / t / 1e6,
                    "frac_hbm": nbytes / t / 1e6 / PEAK_HBM_GBS}
    st.plan.close()
    del keep

    n = 1 << 28
    dH, Z, dZ = (torch.empty(n, device="cuda") for _ in range(3))
    ctx.rng_normal(7, 10, 0.0, 1.0, dH, n)
    ctx.rng_normal(7, 11, 0.0, 1.0, Z, n)
    t = event_time_ms(lambda: ctx.act_bwd(fa.ACT_GELU, n, dH, Z, dZ), reps, warm_ms=200)
    nbytes = 12 * n
    out["act_bwd_gelu_2p28"] = {"ms": t, "bytes": nbytes, "gbs": nbytes / t / 1e6,
                                "frac_hbm": nbytes / t / 1e6 / PEAK_HBM_GBS}
    del dH, Z, dZ

    nt, n = 64, 4 * 1024 * 1024
    P = [torch.empty(n, device="cuda") for _ in range(nt)]
    Gr = [torch.empty(n, device="cuda") for _ in range(nt)]
    for i in range(nt):
        ctx.rng_normal(3, i, 0.0, 0.02, P[i], n)
    mt = fa.MultiTensor(ctx, P, Gr)
    t = event_time_ms(lambda: mt.sgd(1e-3, True), reps, warm_ms=200)
    mt.close()
    nbytes = 16 * nt * n
    out["sgd_64x4Mi"] = {"ms": t, "bytes": nbytes, "gbs": nbytes / t / 1e6,
                         "frac_hbm": nbytes / t / 1e6 / PEAK_HBM_GBS}
    return out


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


def hbm_roof_component(reps: int):
    """The practical HBM roof of the access patterns the bandwidth-bound
    kernels use, from the measurement kernels of ferrograd_amd/csrc/probe/
    k_hbm_roof.hip (16-byte non-temporal accesses, one 4 KiB chunk per block
    pass): a read-only stream of 1 GiB, a 1 GiB copy, 3 streams read and 3
    written (the elementwise program's count) and 4 read and 3 written
    (Adam's) over 256 MiB each, and the softmax + CE kernel's row structure
    on c3's 8192 x 32000 (one workgroup per 128 KB row: read it all, reduce,
    write it all).  Bytes counted = bytes moved."""
    import ctypes

    import torch

    from ferrograd_amd import _build

    lib = ctypes.CDLL(_build.ROOF_LIB)
    u64, vp = ctypes.c_uint64, ctypes.c_void_p
    stream = vp(torch.cuda.current_stream().cuda_stream)
    out = {}

    def rec(key, fn, nbytes):
        t = event_time_ms(fn, reps, warm_ms=200)
        out[key] = {"ms": t, "bytes": nbytes, "gbs": nbytes / t / 1e6,
                    "frac_hbm": nbytes / t / 1e6 / PEAK_HBM_GBS}

    def check(rc):
        if rc != 0:
            raise RuntimeError("HBM roof kernel launch failed")

    n = 256 * 1024 * 1024
    a = torch.ones(n, device="cuda")
    part = torch.empty(lib.fg_roof_blocks(u64(n)), device="cuda")
    rec("read_1gib", lambda: check(lib.fg_roof_read(stream, vp(a.data_ptr()), u64(n),
                                                   vp(part.data_ptr()))), 4 * n)
    b = torch.empty_like(a)
    rec("copy_1gib", lambda: check(lib.fg_roof_copy(stream, vp(a.data_ptr()), vp(b.data_ptr()),
                                                   u64(n))), 8 * n)
    del a, b, part
    n = 64 * 1024 * 1024
    x = [torch.full((n,), 0.5, device="cuda") for _ in range(6)]
    p = [vp(t.data_ptr()) for t in x]
    rec("s3r3w_256mib", lambda: check(lib.fg_roof_s3r3w(stream, *p, u64(n))), 24 * n)
    rec("s4r3w_256mib", lambda: check(lib.fg_roof_s4r3w(stream, *p[:4], u64(n))), 28 * n)
    del x, p
    # The softmax + CE row structure on c3's shape (a read and a write per
    # element): 512 and 1024 threads per 128 KB row.
    R, C = 8192, 32000
    xs, ys = torch.ones((R, C), device="cuda"), torch.empty((R, C), device="cuda")
    for wide, key in ((0, "rows512_8192x32000"), (1, "rows1024_8192x32000")):
        rec(key, lambda: check(lib.fg_roof_rows(stream, vp(xs.data_ptr()), vp(ys.data_ptr()),
                                                R, C, wide)), 8 * R * C)
    return {"hbm_roof": out}


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


def c1_component(ctx, steps: int = 2000, want_host: bool = True):
    """c1: the 2-layer MLP step (batch 64, 784 -> 256 -> 10, ReLU, softmax-CE,
    SGD lr 0.01), latency bound: steps/s of the captured step, launches per
    step and the average time per launch.  With want_host, also returns the
    inputs and the first step's loss, gradients and SGD result (the parity
    sample for the CPU leg) as a second value."""
    import torch

    tr = MLPStep(ctx, [784, 256, 10], 64, act="relu", optim="sgd", lr=0.01, seed=0,
                 x_dist="uniform")
    sample = None
    if want_host:
        import numpy as np
        sample = {"X": tr.X.cpu().numpy(), "y": tr.labels.cpu().numpy().view(np.uint32),
                  "W": [w.cpu().numpy() for w in tr.W]}
        tr.forward()
        tr.loss()
        tr.backward()
        torch.cuda.synchronize()
        sample["mean_loss"] = tr.mean_loss()
        sample["dW"] = [tr.download(t).reshape(w.shape) for t, w in zip(tr.dW, tr.W)]
        sample["db"] = [tr.download(t) for t in tr.db]
        tr.gctx.dispatch_optim(tr.sch)
        torch.cuda.synchronize()
        sample["W_after"] = [w.cpu().numpy() for w in tr.W]
        sample["b_after"] = [b.cpu().numpy() for b in tr.b]
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
    out = {"c1_mlp_step": {"steps_per_s": 1000.0 / ms, "ms_per_step": ms,
                           "eager_ms_per_step": eager_ms, "launches_per_step": n,
                           "us_per_launch": 1000.0 * ms / n, "loss": tr.mean_loss(),
                           "steps_timed": steps}}
    return (out, sample) if want_host else out


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


def only_eltwise(ctx, reps, mode=None):
    """The elementwise program tanh(a * b + c) over 8192 x 8192 fp32 (its
    compiled kernel, the default; or on the interpreter)."""
    import ferrograd_amd as fa

    prev = fa.eltwise_mode(fa.ELTWISE_COMPILE_LARGE if mode is None else mode)
    try:
        st, sch, gctx, keep = eltwise_tanh_plan(ctx, 8192, 8192)
        for _ in range(reps):
            gctx.dispatch_forward(sch)
        gctx.sync()
        st.plan.close()
    finally:
        fa.eltwise_mode(prev)


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


def only_gemm_bf16_c5_hidden(ctx, reps):
    """The c5 step's hidden-layer GEMMs with bf16 tensors (for counter
    passes): forward NN 2048x4096x4096 + bias + GELU with Z stored, dX NT
    2048x4096x4096 * GELU'(Z), dW TN 4096x4096x2048 with the fused dbias;
    N(0,1) operands."""
    import torch

    import ferrograd_amd as fa

    M, N, K, bf = 2048, 4096, 4096, fa.DTYPE_BF16
    g = torch.Generator(device="cuda").manual_seed(4)

    def rnd(*shape):
        return torch.randn(shape, device="cuda", generator=g).to(torch.bfloat16)

    X, W, dZ, Zs, b = rnd(M, K), rnd(K, N), rnd(M, N), rnd(M, K), rnd(N)
    H, Z, dX, dW, db = (torch.empty(sh, device="cuda", dtype=torch.bfloat16)
                        for sh in ((M, N), (M, N), (M, K), (K, N), (N,)))
    for _ in range(reps):
        ctx.gemm_x16(bf, fa.NN, M, N, K, X, K, W, N, H, N, bias=b, act=fa.ACT_GELU, Z=Z, ldz=N)
        ctx.gemm_bwd_x16(bf, fa.NT, M, K, N, dZ, N, W, N, dX, K, act=fa.ACT_GELU, Zs=Zs, ldzs=K)
        ctx.gemm_dw_x16(bf, K, N, M, X, K, dZ, N, dW, N, colsum=db)


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


def only_gemm_bf16_data(ctx, reps):
    """The plain bf16 NN GEMM at 4096^3, ours and torch.mm's (hipBLASLt),
    each 3 + `reps` times on N(0,1) operands and then on zero operands (for a counter pass of MFMA busy cycles and the clock: the
    matrix units' power, and so the clock, depend on the data)."""
    import torch

    import ferrograd_amd as fa

    n, bf = 4096, fa.DTYPE_BF16
    g = torch.Generator(device="cuda").manual_seed(1)
    C = torch.empty((n, n), device="cuda", dtype=torch.bfloat16)
    flops = 2.0 * n * n * n
    out = {}
    for data in ("normal", "zeros"):
        if data == "normal":
            A, Bm = (torch.randn((n, n), device="cuda", generator=g).to(torch.bfloat16)
                     for _ in range(2))
        else:
            A, Bm = (torch.zeros((n, n), device="cuda", dtype=torch.bfloat16) for _ in range(2))
        for who, fn in (("ours", lambda: ctx.gemm_x16(bf, fa.NN, n, n, n, A, n, Bm, n, C, n)),
                        ("torch_mm", lambda: torch.mm(A, Bm, out=C))):
            for _ in range(3):  # untimed: library set-up, first-touch costs
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            e1.synchronize()
            ms = e0.elapsed_time(e1) / reps
            out[f"{who}_{data}"] = {"ms": ms, "tflops": flops / ms / 1e9}
    print(json.dumps({"gemm_bf16_4096_nn_by_data": out}), flush=True)


def only_gemm_c2(ctx, reps):
    """The c2 GEMMs: forward (bias + ReLU) and the masked backward (dA, dB +
    dbias) through fg_linear_bwd_f32."""
    import torch

    import ferrograd_amd as fa

    n = 4096
    A, Bm, bias, dC = c2_inputs(ctx, n)
    C, dA, dB, dZ = (torch.empty((n, n), device="cuda") for _ in range(4))
    db = torch.empty((n,), device="cuda")
    for _ in range(reps):
        ctx.gemm(fa.NN, n, n, n, A, n, Bm, n, C, n, bias=bias, act=fa.ACT_RELU)
        ctx.linear_bwd(fa.ACT_RELU, n, n, n, A, n, Bm, n, C, n, dC, n, dX=dA, lddx=n, dW=dB,
                       lddw=n, dbias=db, dZ=dZ, lddz=n)


def only_c5_gemm(key):
    def run(ctx, reps):
        fn = c5_gemm_kernels(ctx)[key][1]
        for _ in range(reps):
            fn()
    run.__doc__ = f"The c5 step's {key} GEMM alone (for counter passes)."
    return run


def only_c1_step(ctx, reps):
    print(json.dumps(c1_component(ctx, steps=max(reps, 10), want_host=False)), flush=True)


ONLY = {
    "c1_step": only_c1_step,
    "c5_step": only_c5_step,
    "c5_step_bf16": only_c5_step_bf16,
    "gemm_bf16_c2": only_gemm_bf16_c2,
    "gemm_bf16_c5_hidden": only_gemm_bf16_c5_hidden,
    "gemm_bf16_data": only_gemm_bf16_data,
    "gemm_c2": only_gemm_c2,
    "gemm_c5_hidden": only_gemm_c5_hidden,
    "gemm_c5_fwd": only_c5_gemm("gemm_c5_fwd"),
    "gemm_c5_bwd_pair": only_c5_gemm("gemm_c5_bwd_pair"),
    "gemm_c5_dx": only_c5_gemm("gemm_c5_dx"),
    "gemm_c5_dw": only_c5_gemm("gemm_c5_dw"),
    "gemm_c5_fwd_first": only_c5_gemm("gemm_c5_fwd_first"),
    "gemm_c5_fwd_head": only_c5_gemm("gemm_c5_fwd_head"),
    "gemm_c5_dw_head": only_c5_gemm("gemm_c5_dw_head"),
    "gemm_c5_dx_head": only_c5_gemm("gemm_c5_dx_head"),
    "gemm_c5_pair_first": only_c5_gemm("gemm_c5_pair_first"),
    "softmax_ce_c3": only_softmax_ce_c3,
    "adam_c4": only_adam_c4,
    "copy_256mib": only_copy_256mib,
    "eltwise_8192": only_eltwise,
    "eltwise_8192_interp": lambda ctx, reps: only_eltwise(ctx, reps, 0),
    "hbm_roof": lambda ctx, reps: print(json.dumps(hbm_roof_component(reps)), flush=True),
    "hbm_kernels": lambda ctx, reps: print(json.dumps(hbm_kernels_component(ctx, reps)),
                                           flush=True),
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


# ----------------------------------------------------------- CPU baselines
# The CPU restatement (oracle/, C with OpenMP) timed on the host cores on the
# same inputs as the GPU run (copied from the device, so both sides consume
# identical bits), and the parity of each configuration: normwise relative
# error max|gpu - cpu| / max|cpu| per tensor against the tolerances of the
# configurations (GEMM 1e-5*sqrt(K), elementwise / softmax / optimiser 1e-5;
# argmax, labels and the optimiser updates bit-exact).

def cpu_threads() -> int:
    """Threads of the CPU legs: the job's CPU share -- OMP_NUM_THREADS when
    set (one GPU's share of the GPU box's cores), else the CPUs this process
    may run on."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    return len(os.sched_getaffinity(0))


def cpu_time_s(fn, repeats: int = 5) -> float:
    """Median wall time of fn() over `repeats` runs after one warm-up run."""
    fn()
    ts = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def rel_err(a, b) -> float:
    import numpy as np
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    if b.size == 0:
        return 0.0
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1e-30))


def oracle_mlp_grads(X, y, W, b, act):
    """Forward, softmax-CE and backward (dX of the data included) of an MLP
    with the CPU restatement: (mean loss, dW list, db list, dX)."""
    import oracle as O

    L = len(W)
    Zs, Hs, inp = [], [], X
    for l in range(L):
        Z, H = O.bias_act(O.gemm(O.NN, inp, W[l]), b[l], O.ACT_NONE if l == L - 1 else act)
        Zs.append(Z)
        Hs.append(H)
        inp = H
    _, dZ, _, mean = O.softmax_ce(Zs[-1], y)
    dW, db = [None] * L, [None] * L
    for l in range(L - 1, -1, -1):
        prev = Hs[l - 1] if l > 0 else X
        dW[l] = O.gemm(O.TN, prev, dZ)
        db[l] = O.bias_grad(dZ)
        up = O.gemm(O.NT, dZ, W[l])
        dZ = O.act_bwd(act, up, Zs[l - 1]) if l > 0 else up
    return mean, dW, db, dZ


def cpu_c1(sample, threads):
    """c1 on the CPU: the whole step (forward, CE, backward incl. dX, SGD),
    single-threaded and on `threads` threads; parity of the GPU's first step
    (loss, gradients; SGD bit-exact on the GPU's own gradients)."""
    import numpy as np

    import oracle as O

    X, y, W = sample["X"], sample["y"], sample["W"]
    b = [np.zeros(w.shape[1], np.float32) for w in W]

    def step():
        mean, dW, db, _ = oracle_mlp_grads(X, y, W, b, O.ACT_RELU)
        for p, g in zip(W + b, dW + db):
            O.sgd_(p.copy().reshape(-1), g.copy().reshape(-1), np.float32(0.01), True)
        return mean, dW, db

    O.set_num_threads(1)
    t1 = cpu_time_s(step, 20)
    O.set_num_threads(threads)
    tn = cpu_time_s(step, 20)
    mean, dW, db = step()
    sgd_exact = True
    for p0, g, got in zip(W + b, sample["dW"] + sample["db"], sample["W_after"] + sample["b_after"]):
        w = p0.copy().reshape(-1)
        O.sgd_(w, np.ascontiguousarray(g, np.float32).reshape(-1).copy(), np.float32(0.01), True)
        sgd_exact &= bool(np.array_equal(w, got.reshape(-1)))
    tol = 1e-5 * math.sqrt(784)
    err = {"loss": abs(sample["mean_loss"] - mean) / max(1.0, abs(mean)),
           "dW": max(rel_err(a, r) for a, r in zip(sample["dW"], dW)),
           "db": max(rel_err(a, r) for a, r in zip(sample["db"], db))}
    return {"cpu_steps_per_s_1thread": 1.0 / t1, "cpu_steps_per_s": 1.0 / tn,
            "cpu_ms_per_step_1thread": 1e3 * t1, "cpu_ms_per_step": 1e3 * tn,
            "cores": threads, "kind": "port", "max_rel_err": err, "tolerance": tol,
            "sgd_bit_exact": sgd_exact,
            "parity_ok": bool(err["loss"] < 1e-5 and err["dW"] < tol and err["db"] < tol
                              and sgd_exact)}


def cpu_c2(sample, threads):
    """c2 on the CPU: forward ReLU(A.B + bias) and the masked backward (dA,
    dB, dbias) on `threads` threads (412 GFLOP), each timed as the median of
    5 runs after a warm-up run.  The CPU backward takes the GPU forward's
    mask ([C_gpu > 0]; a sign that fp32 rounding decides differently would
    otherwise flip single terms), and the flipped signs are counted."""
    import numpy as np

    import oracle as O

    O.set_num_threads(threads)
    A, B, bias, dC = sample["A"], sample["B"], sample["bias"], sample["dC"]
    Cg = sample["C"]
    out = {}

    def fwd():
        out["C"] = O.bias_act(O.gemm(O.NN, A, B), bias, O.ACT_RELU)[1]

    def bwd():
        dZ = O.act_bwd(O.ACT_RELU, dC, Cg)
        out["dA"], out["dB"], out["db"] = O.gemm(O.NT, dZ, B), O.gemm(O.TN, A, dZ), O.bias_grad(dZ)

    t_f = cpu_time_s(fwd, 5)
    t_b = cpu_time_s(bwd, 5)
    C, dA, dB, db = out["C"], out["dA"], out["dB"], out["db"]
    flops = 3 * 2.0 * A.shape[0] * A.shape[1] * B.shape[1]
    tol = 1e-5 * math.sqrt(A.shape[1])
    err = {"C": rel_err(Cg, C), "dA": rel_err(sample["dA"], dA), "dB": rel_err(sample["dB"], dB),
           "dbias": rel_err(sample["db"], db)}
    return {"cpu_ms": 1e3 * (t_f + t_b), "cpu_fwd_ms": 1e3 * t_f, "cpu_bwd_ms": 1e3 * t_b,
            "cpu_tflops": flops / (t_f + t_b) / 1e12, "cores": threads, "kind": "port",
            "timing": "median of 5 after a warm-up run, forward and backward each",
            "mask_sign_flips": int(np.count_nonzero((Cg > 0) != (C > 0))),
            "max_rel_err": err, "tolerance": tol,
            "parity_ok": bool(max(err.values()) < tol)}


def cpu_c3(sample, threads):
    """c3 on the CPU: softmax + CE forward and backward over [8192, 32000]
    (median of 5 after a warm-up) on `threads` threads; argmax bit-exact."""
    import numpy as np

    import oracle as O

    O.set_num_threads(threads)
    x, y = sample["x"], sample["y"]
    t = cpu_time_s(lambda: O.softmax_ce(x, y), 5)
    rl, d, am, mean = O.softmax_ce(x, y)
    err = {"row_loss": rel_err(sample["row_loss"], rl),
           "mean_loss": abs(float(sample["mean"]) - mean) / max(1.0, abs(mean)),
           "dlogits": rel_err(sample["d"], d)}
    am_exact = int(np.count_nonzero(sample["argmax"] == am))
    nbytes = 2 * x.size * 4
    return {"cpu_ms": 1e3 * t, "cpu_gbs": nbytes / t / 1e9, "cores": threads, "kind": "port",
            "max_rel_err": err, "tolerance": 1e-5, "argmax_exact": am_exact,
            "rows": int(x.shape[0]),
            "parity_ok": bool(max(err.values()) < 1e-5 and am_exact == x.shape[0])}


def adam_sample_run(ctx, nt: int = 8, steps: int = 10, threads: int = 1):
    """c4's parity and CPU sample: the first `nt` of its 64 tensors (4 Mi
    parameters each), `steps` Adam steps with fresh gradients each step
    (library generator, seed 3: parameters N(0, 0.02^2) ids 0..63, step s's
    gradients N(0, 1e-3^2) ids 1000 + 64(s-1) + i), on the GPU and with the
    CPU restatement on the same bits; the CPU's update is timed (`threads`
    threads) and scaled to the 64 tensors."""
    import numpy as np
    import torch

    import ferrograd_amd as fa
    import oracle as O

    O.set_num_threads(threads)
    n = 4 * 1024 * 1024
    P = [torch.empty(n, device="cuda") for _ in range(nt)]
    G = [torch.empty(n, device="cuda") for _ in range(nt)]
    M = [torch.zeros(n, device="cuda") for _ in range(nt)]
    V = [torch.zeros(n, device="cuda") for _ in range(nt)]
    for i in range(nt):
        ctx.rng_normal(3, i, 0.0, 0.02, P[i], n)
    hp = [p.cpu().numpy() for p in P]
    hm = [np.zeros(n, np.float32) for _ in range(nt)]
    hv = [np.zeros(n, np.float32) for _ in range(nt)]
    mt = fa.MultiTensor(ctx, P, G, M, V)
    t_cpu = 0.0
    for step in range(1, steps + 1):
        for i in range(nt):
            ctx.rng_normal(3, 1000 + 64 * (step - 1) + i, 0.0, 1e-3, G[i], n)
        hg = [g.cpu().numpy() for g in G]
        mt.adam(1e-3, 0.9, 0.999, 1e-8, step)
        sc, r = O.adam_scalars(np.float32(1e-3), np.float32(0.9), np.float32(0.999), step)
        t0 = time.perf_counter()
        for i in range(nt):
            O.adam_(hp[i], hg[i], hm[i], hv[i], np.float32(0.9), np.float32(0.999),
                    np.float32(1e-8), sc, r)
        t_cpu += time.perf_counter() - t0
    torch.cuda.synchronize()
    exact = all(np.array_equal(a.cpu().numpy(), b) for X, H in ((P, hp), (M, hm), (V, hv))
                for a, b in zip(X, H))
    err = max(rel_err(a.cpu().numpy(), b) for a, b in zip(P, hp))
    mt.close()
    per_step_64 = t_cpu / steps * (64 / nt)
    return {"cpu_ms_per_step": 1e3 * per_step_64, "cpu_gbs": 28 * 64 * n / per_step_64 / 1e9,
            "cores": threads, "kind": "port",
            "sample": f"{nt} of 64 tensors x {steps} steps, fresh gradients each step; time "
                      f"scaled to 64 tensors",
            "max_rel_err": {"params": err}, "tolerance": 1e-5, "bit_exact_p_m_v": exact,
            "parity_ok": bool(exact)}


def cpu_c5(host, first, dims, threads):
    """c5 on the CPU: one full training step (forward, CE, backward incl. dX,
    Adam) on the same initial inputs; parity of the GPU's first step (loss,
    every dW / db, the data input's dX) and Adam bit-exact on the GPU's own
    gradients."""
    import numpy as np

    import oracle as O

    O.set_num_threads(threads)
    X, y, W = host["X"], host["y"], host["W"]
    L = len(W)
    b = [np.zeros(dims[l + 1], np.float32) for l in range(L)]
    s, r = O.adam_scalars(np.float32(1e-3), np.float32(0.9), np.float32(0.999), 1)
    t0 = time.perf_counter()
    mean, dW, db, dX = oracle_mlp_grads(X, y, W, b, O.ACT_GELU)
    for p0, g in zip(W + b, dW + db):
        p = p0.copy()
        O.adam_(p, g, np.zeros_like(p), np.zeros_like(p), np.float32(0.9), np.float32(0.999),
                np.float32(1e-8), s, r)
    dt = time.perf_counter() - t0
    # Adam on the GPU's own gradients: the update itself, bit for bit.
    adam_exact = True
    for p0, g, got in zip(W + b, first["dW"] + first["db"], first["W"] + first["b"]):
        p = p0.copy()
        g = np.ascontiguousarray(g, np.float32).reshape(p.shape).copy()
        O.adam_(p, g, np.zeros_like(p), np.zeros_like(p), np.float32(0.9), np.float32(0.999),
                np.float32(1e-8), s, r)
        adam_exact &= bool(np.array_equal(p, got.reshape(p.shape)))
    tol = 1e-5 * math.sqrt(4096)
    err = {"loss": abs(first["mean_loss"] - mean) / max(1.0, abs(mean)),
           "dW": max(rel_err(a, r_) for a, r_ in zip(first["dW"], dW)),
           "db": max(rel_err(a, r_) for a, r_ in zip(first["db"], db)),
           "dX": rel_err(first["dX"], dX)}
    return dt, {"max_rel_err": err, "tolerance_gemm": tol, "adam_bit_exact_on_gpu_grads":
                adam_exact, "parity_ok": bool(err["loss"] < 1e-5 and err["dW"] < tol and
                                              err["db"] < tol and err["dX"] < tol and
                                              adam_exact)}


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
             "db": [tr.download(t) for t in tr.db], "W": [w.cpu().numpy() for w in tr.W],
             "dX": tr.download(tr.dX).reshape(tuple(tr.X.shape)),
             "b": [b.cpu().numpy() for b in tr.b]}
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

    want_cpu = not args.no_cpu
    comps, c2_sample = gemm_components(ctx, args.reps, want_host=want_cpu and
                                       not args.no_components)
    # The dominant kernel of the step by time share (6 launches of each of
    # the three hidden-layer GEMMs per step).
    shares = c5_gemm_shares(ctx, args.reps, ms_per_step)
    comps["c5_step_gemms"] = shares
    dom_key = max((k for k in shares if shares[k]["step_share"]),
                  key=lambda k: shares[k]["step_share"])
    dom = shares[dom_key]
    kernel_name = "gemm_pair_big" if dom_key == "gemm_c5_bwd_pair" else "gemm_f32_pipe"
    roofline = {
        "bound": "mfma",
        "kernel": kernel_name + " " + dom["what"] + " -- the c5 step's largest kernel time share",
        "achieved": dom["tflops"],
        "peak": PEAK_FP32_MFMA_TFLOPS,
        "unit": "TFLOP/s",
        "frac": dom["frac"],
        "traffic": measured_traffic(dom_key),
        "traffic_unit": "HBM bytes per launch (rocprofv3 FETCH_SIZE/WRITE_SIZE, copy-calibrated)",
        "algorithmic_bytes": dom["algorithmic_bytes"],
        "step_share": dom["step_share"],
        "others": {k: {"tflops": v["tflops"], "frac": v["frac"], "step_share": v["step_share"]}
                   for k, v in shares.items() if k != dom_key},
    }
    samples = {}
    if not args.no_components:
        r = softmax_component(ctx, args.reps, want_host=want_cpu)
        if want_cpu:
            r, samples["c3"] = r
        comps.update(r)
        comps.update(adam_component(ctx, 10))
        comps.update(hbm_kernels_component(ctx, args.reps))
        r = c1_component(ctx, want_host=want_cpu)
        if want_cpu:
            r, samples["c1"] = r
        comps.update(r)
        comps.update(gemm_bf16_component(ctx, args.reps))
        comps.update(c5_bf16_component(ctx))
        comps.update(copy_component(args.reps))
        comps.update(hbm_roof_component(args.reps))
    log("components: " + json.dumps(comps))

    cpu = None
    parity = None
    if want_cpu:
        threads = cpu_threads()
        log(f"CPU legs on {threads} threads (os.cpu_count() = {os.cpu_count()}, "
            f"affinity {len(os.sched_getaffinity(0))}, OMP_NUM_THREADS = "
            f"{os.environ.get('OMP_NUM_THREADS')})")
        parity = {}
        if not args.no_components:
            c1c = cpu_c1(samples.pop("c1"), threads)
            comps["c1_mlp_step"]["cpu"] = c1c
            parity["c1"] = c1c["parity_ok"]
            log("c1 CPU: " + json.dumps(c1c))
            c2c = cpu_c2(c2_sample, threads)
            c2_sample = None
            comps["c2_gemm_4096"]["cpu"] = c2c
            parity["c2"] = c2c["parity_ok"]
            log("c2 CPU: " + json.dumps(c2c))
            c3c = cpu_c3(samples.pop("c3"), threads)
            comps["c3_softmax_ce_8192x32000"]["cpu"] = c3c
            parity["c3"] = c3c["parity_ok"]
            log("c3 CPU: " + json.dumps(c3c))
            c4c = adam_sample_run(ctx, threads=threads)
            comps["c4_adam_64x4Mi"]["cpu"] = c4c
            parity["c4"] = c4c["parity_ok"]
            log("c4 CPU: " + json.dumps(c4c))
        log(f"CPU baseline: one c5 step on {threads} threads")
        dt, c5p = cpu_c5(host, first, dims, threads)
        cpu = {"value": 1.0 / dt, "unit": "steps/s", "cores": threads, "kind": "port",
               "sample": "one full c5 training step (forward, CE, backward incl. dX, Adam) "
                         "on the same inputs, oracle/ C restatement with OpenMP",
               "nproc": os.cpu_count()}
        parity["c5"] = c5p["parity_ok"]
        parity["c5_detail"] = c5p
        parity["all_ok"] = all(v for k, v in parity.items() if not k.endswith("_detail"))
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
    if parity is not None and not parity["all_ok"]:
        log("PARITY FAILED: " + json.dumps({k: v for k, v in parity.items()
                                              if not k.endswith("_detail")}))
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
