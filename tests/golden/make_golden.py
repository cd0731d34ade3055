"""Writes the golden fixtures under tests/golden/ (run in the build container).

The reference (ferrograd) is Rust with no CPU implementation and no golden
vectors for this path beyond the closed-form tests re-hosted in
tests/test_oracle.py, so these fixtures come from independent library
routines evaluated in float64:

* GEMM: numpy float64 matmul on odd shapes (17x29 by 29x33) for the three
  operand layouts;
* GELU (tanh form) and its derivative: torch.nn.functional.gelu(
  approximate="tanh") and torch.autograd in float64;
* softmax + cross-entropy: torch.log_softmax / F.cross_entropy(reduction=
  "none") in float64 plus numpy argmax (first occurrence) on rows with ties;
* Adam: torch.optim.Adam (float64 and float32) over 10 steps;
* a small Linear-GELU-Linear-CE step: torch.autograd in float64.

Inputs are drawn with numpy's PCG64 generator from fixed seeds.  Usage:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))


def gemm_fixture():
    rng = np.random.default_rng(101)
    M, K, N = 17, 29, 33
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    C = A.astype(np.float64) @ B.astype(np.float64)
    np.savez_compressed(os.path.join(HERE, "gemm_17x29x33.npz"), A=A, B=B, bias=bias, C=C)


def gelu_fixture():
    z = np.concatenate([np.linspace(-6, 6, 241), [0.0, 1.0, -1.0, 3.0, -3.0, 1e-4, -1e-4]])
    zt = torch.tensor(z, dtype=torch.float64, requires_grad=True)
    y = F.gelu(zt, approximate="tanh")
    (g,) = torch.autograd.grad(y.sum(), zt)
    relu_y = torch.relu(torch.tensor(z))
    np.savez_compressed(os.path.join(HERE, "gelu_tanh.npz"), z=z, y=y.detach().numpy(),
                        dy=g.numpy(), relu=relu_y.numpy())


def softmax_ce_fixture():
    rng = np.random.default_rng(202)
    R, C = 9, 37
    x = (2.0 * rng.standard_normal((R, C))).astype(np.float32)
    # Ties for argmax: row 3 has its maximum at columns 5 and 20, row 4 is
    # constant, row 5 has the max at the last column.
    x[3, 5] = x[3, 20] = 9.0
    x[4, :] = 0.25
    x[5, C - 1] = 11.0
    labels = rng.integers(0, C, size=R).astype(np.uint32)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    loss = F.cross_entropy(xt, torch.tensor(labels.astype(np.int64)), reduction="none")
    (d,) = torch.autograd.grad(loss.sum(), xt)
    p = torch.softmax(torch.tensor(x, dtype=torch.float64), dim=1)
    np.savez_compressed(os.path.join(HERE, "softmax_ce_9x37.npz"), x=x, labels=labels,
                        loss=loss.detach().numpy(), dlogits=d.numpy(), p=p.numpy(),
                        argmax=np.argmax(x, axis=1).astype(np.uint32))


def adam_fixture():
    rng = np.random.default_rng(303)
    n, steps = 1000, 10
    p0 = (0.02 * rng.standard_normal(n)).astype(np.float32)
    grads = (1e-3 * rng.standard_normal((steps, n))).astype(np.float32)
    out = {}
    for name, dt in (("f64", torch.float64), ("f32", torch.float32)):
        p = torch.tensor(p0, dtype=dt, requires_grad=True)
        opt = torch.optim.Adam([p], lr=1e-3, betas=(0.9, 0.999), eps=1e-8, foreach=False)
        for s in range(steps):
            p.grad = torch.tensor(grads[s], dtype=dt)
            opt.step()
        out[name] = p.detach().numpy().astype(np.float64)
    np.savez_compressed(os.path.join(HERE, "adam_10steps.npz"), p0=p0, grads=grads,
                        p_f64=out["f64"], p_f32=out["f32"])


def mlp_fixture():
    """Linear(12->16) - GELU(tanh) - Linear(16->5) - CE (sum over rows)."""
    rng = np.random.default_rng(404)
    B, I, H, O = 8, 12, 16, 5
    X = rng.standard_normal((B, I)).astype(np.float32)
    W1 = (0.5 * rng.standard_normal((I, H))).astype(np.float32)
    b1 = (0.1 * rng.standard_normal(H)).astype(np.float32)
    W2 = (0.5 * rng.standard_normal((H, O))).astype(np.float32)
    b2 = (0.1 * rng.standard_normal(O)).astype(np.float32)
    y = rng.integers(0, O, size=B).astype(np.uint32)
    t = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True)
         for k, v in dict(X=X, W1=W1, b1=b1, W2=W2, b2=b2).items()}
    h = F.gelu(t["X"] @ t["W1"] + t["b1"], approximate="tanh")
    logits = h @ t["W2"] + t["b2"]
    loss = F.cross_entropy(logits, torch.tensor(y.astype(np.int64)), reduction="sum")
    grads = torch.autograd.grad(loss, [t[k] for k in ("X", "W1", "b1", "W2", "b2")])
    np.savez_compressed(os.path.join(HERE, "mlp_gelu_ce.npz"), X=X, W1=W1, b1=b1, W2=W2, b2=b2,
                        y=y, loss_sum=float(loss.detach()),
                        dX=grads[0].numpy(), dW1=grads[1].numpy(), db1=grads[2].numpy(),
                        dW2=grads[3].numpy(), db2=grads[4].numpy())


if __name__ == "__main__":
    gemm_fixture()
    gelu_fixture()
    softmax_ce_fixture()
    adam_fixture()
    mlp_fixture()
    print("fixtures written to", HERE)
