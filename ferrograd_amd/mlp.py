"""Fused MLP training step (Linear -> act -> ... -> Linear -> softmax-CE ->
optimiser) as a fixed launch sequence of the gfx950 kernels.

This is the launch plan the graph lowering produces for ferrograd's MLP
graphs (matmul -> bias add -> activation per layer, softmax + CE loss,
multi-tensor optimiser); it is kept as a direct class too because the
benchmarks use it with preallocated device tensors.

Per step (L layers, batch B):
  forward : L GEMMs (NN) with bias + activation fused in the epilogue; the
            pre-activation Z_l is saved for backward
  loss    : 1 fused softmax + CE launch writing dlogits = p - onehot
            (the reference's CE gradient, kernel/loss.rs:12-165, unscaled)
            and the per-row losses, plus the mean-loss reduction
  backward: per layer dW_l = H_{l-1}^T dZ_l (TN), db_l = colsum(dZ_l), and
            dZ_{l-1} = (dZ_l W_l^T) * act'(Z_{l-1}) (NT with the activation
            derivative fused in the epilogue); optionally dX for the data
            input (every Input is trainable in ferrograd,
            backward.rs:95-106)
  optim   : 1 multi-tensor Adam or SGD launch over all W_l, b_l
"""
from __future__ import annotations

from typing import List, Optional, Sequence

from . import ACT_GELU, ACT_NONE, ACT_RELU, NN, NT, TN, Context, MultiTensor  # noqa: F401


class MLPTrainStep:
    """Device buffers are torch tensors (plain device memory); every
    computation is a library kernel."""

    def __init__(self, ctx: Context, dims: Sequence[int], batch: int, act: int,
                 optim: str = "adam", lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8,
                 data_grad: bool = True):
        import torch

        self.ctx = ctx
        self.dims = list(dims)
        self.L = len(dims) - 1
        self.B = batch
        self.act = act
        self.optim = optim
        self.lr, self.betas, self.eps = lr, betas, eps
        self.data_grad = data_grad
        self.step_count = 0
        dev = dict(device="cuda", dtype=torch.float32)
        B = batch
        self.X = torch.empty((B, dims[0]), **dev)
        self.labels = torch.empty((B,), device="cuda", dtype=torch.int32)
        self.W = [torch.empty((dims[l], dims[l + 1]), **dev) for l in range(self.L)]
        self.b = [torch.zeros((dims[l + 1],), **dev) for l in range(self.L)]
        self.dW = [torch.empty_like(w) for w in self.W]
        self.db = [torch.empty_like(b) for b in self.b]
        # Z_l pre-activations (l < L-1 saved for backward; the last is the logits).
        self.Z = [torch.empty((B, dims[l + 1]), **dev) for l in range(self.L)]
        self.H = [torch.empty((B, dims[l + 1]), **dev) for l in range(self.L - 1)]
        wmax = max(dims[1:])
        self.dZbuf = [torch.empty((B * wmax,), **dev) for _ in range(2)]
        self.dX = torch.empty((B, dims[0]), **dev) if data_grad else None
        self.row_loss = torch.empty((B,), **dev)
        self.loss = torch.empty((1,), **dev)
        params = self.W + self.b
        grads = self.dW + self.db
        if optim == "adam":
            self.m = [torch.zeros_like(p) for p in params]
            self.v = [torch.zeros_like(p) for p in params]
            self.mt = MultiTensor(ctx, params, grads, self.m, self.v)
        elif optim == "sgd":
            self.mt = MultiTensor(ctx, params, grads)
        else:
            raise ValueError(optim)
        # bias-grad partials live in the context workspace: size it now so
        # the step never allocates.
        ctx.reserve_workspace(64 << 20)

    # ------------------------------------------------------------ phases
    def forward(self) -> None:
        c, B, d = self.ctx, self.B, self.dims
        inp = self.X
        for l in range(self.L):
            last = l == self.L - 1
            out = self.Z[l] if last else self.H[l]
            c.gemm(NN, B, d[l + 1], d[l], inp, d[l], self.W[l], d[l + 1], out, d[l + 1],
                   bias=self.b[l], act=ACT_NONE if last else self.act,
                   Z=None if last else self.Z[l], ldz=d[l + 1])
            inp = out

    def loss_and_grad(self) -> None:
        C = self.dims[-1]
        self.ctx.softmax_ce(self.Z[-1], C, self.labels, self.B, C, 1.0, row_loss=self.row_loss,
                            mean_loss=self.loss, dlogits=self.dZbuf[0], ldd=C)

    def backward(self) -> None:
        c, B, d = self.ctx, self.B, self.dims
        cur = 0
        for l in range(self.L - 1, -1, -1):
            dZ = self.dZbuf[cur]
            prev = self.H[l - 1] if l > 0 else self.X
            c.gemm(TN, d[l], d[l + 1], B, prev, d[l], dZ, d[l + 1], self.dW[l], d[l + 1])
            c.bias_grad(B, d[l + 1], dZ, d[l + 1], self.db[l])
            if l > 0:
                nxt = self.dZbuf[cur ^ 1]
                c.gemm_bwd(NT, B, d[l], d[l + 1], dZ, d[l + 1], self.W[l], d[l + 1], nxt, d[l],
                           act=self.act, Zs=self.Z[l - 1], ldzs=d[l])
                cur ^= 1
            elif self.data_grad:
                c.gemm_bwd(NT, B, d[0], d[1], dZ, d[1], self.W[0], d[1], self.dX, d[0])

    def optimise(self) -> None:
        self.step_count += 1
        if self.optim == "adam":
            self.mt.adam(self.lr, self.betas[0], self.betas[1], self.eps, self.step_count)
        else:
            self.mt.sgd(self.lr, zero_grad=True)

    def step(self) -> None:
        self.forward()
        self.loss_and_grad()
        self.backward()
        self.optimise()

    # ---------------------------------------------------------- accounting
    def gemm_flops(self) -> int:
        """Algorithmic GEMM flops of one step (2*M*N*K per GEMM)."""
        B, d = self.B, self.dims
        s = sum(d[l] * d[l + 1] for l in range(self.L))
        f = 2 * B * s * 3
        if not self.data_grad:
            f -= 2 * B * d[0] * d[1]
        return f

    def num_params(self) -> int:
        return sum(w.numel() for w in self.W) + sum(b.numel() for b in self.b)

    def close(self) -> None:
        self.mt.close()
