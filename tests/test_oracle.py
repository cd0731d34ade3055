"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Each check is chosen so that a plausible slip in the oracle (a dropped term,
a transposed operand, a wrong constant or index) fails it:

* the reference's own closed-form GPU tests, re-hosted exactly
  (crates/ferrograd/tests/std_wgsl.rs, tests/optim.rs);
* float64 library routines on golden fixtures (numpy matmul; torch GELU-tanh,
  cross-entropy and Adam; torch autograd for a small MLP step), written by
  tests/golden/make_golden.py;
* closed forms and invariants (Adam's first step, uniform softmax rows,
  softmax rows summing to one, dlogits rows summing to zero).
"""
import math

import numpy as np
import pytest

import oracle as O
from conftest import golden, normwise_rel

f32 = np.float32


# ------------------------------------------------------------------- GEMM
def full(shape, v):
    return np.full(shape, v, dtype=np.float32)


def test_gemm_matmul_add_closed_form():
    """std_wgsl.rs:268-373: a@b + c with a=3 [32,16], b=2 [16,64], c=1; seed 1."""
    M, N, K = 32, 64, 16
    A, B, Cc = full((M, K), 3), full((K, N), 2), full((M, N), 1)
    X = O.gemm(O.NN, A, B)
    assert np.all(X + Cc == 97.0)
    seed = full((M, N), 1)
    assert np.all(O.gemm(O.NT, seed, B) == 128.0)  # dA = seed . B^T
    assert np.all(O.gemm(O.TN, A, seed) == 96.0)   # dB = A^T . seed


def test_gemm_matmul_sub_closed_form():
    """std_wgsl.rs:523-653: a@b - c@d, M32 N64 K128."""
    M, N, K = 32, 64, 128
    A, B, C, D = full((M, K), 3), full((K, N), 2), full((M, K), 1), full((K, N), 0.5)
    X, Y = O.gemm(O.NN, A, B), O.gemm(O.NN, C, D)
    assert np.all(X == 768.0) and np.all(Y == 64.0) and np.all(X - Y == 704.0)
    seed = full((M, N), 1)
    assert np.all(O.gemm(O.NT, seed, B) == 128.0)
    assert np.all(O.gemm(O.TN, A, seed) == 96.0)
    assert np.all(O.gemm(O.NT, -seed, D) == -32.0)
    assert np.all(O.gemm(O.TN, C, -seed) == -32.0)


def test_gemm_matmul_chain3_closed_form():
    """std_wgsl.rs:376-520: ((c@(a@b))@d) + e, M32 N64 K128 H256."""
    M, N, K, H = 32, 64, 128, 256
    a, b, c, d = full((M, K), 3), full((K, N), 2), full((H, M), 1), full((N, H), 0.5)
    X = O.gemm(O.NN, a, b)
    Y = O.gemm(O.NN, c, X)
    Z = O.gemm(O.NN, Y, d)
    X_VAL = 3 * 2 * K
    Y_VAL = 1 * X_VAL * M
    Z_VAL = Y_VAL * 0.5 * N
    assert np.all(X == X_VAL) and np.all(Y == Y_VAL) and np.all(Z == Z_VAL)
    seed = full((H, H), 1)
    dY = O.gemm(O.NT, seed, d)          # dZ . d^T
    assert np.all(dY == 0.5 * H)
    dd = O.gemm(O.TN, Y, seed)          # Y^T . dZ
    assert np.all(dd == Y_VAL * H)
    dX = O.gemm(O.TN, c, dY)            # c^T . dY
    assert np.all(dX == 0.5 * H * 1 * H)
    dc = O.gemm(O.NT, dY, X)            # dY . X^T
    assert np.all(dc == 0.5 * H * X_VAL * N)
    db = O.gemm(O.TN, a, dX)
    assert np.all(db == 3 * (0.5 * H * H) * M)
    da = O.gemm(O.NT, dX, b)
    assert np.all(da == (0.5 * H * H) * 2 * N)


@pytest.mark.parametrize("layout", [O.NN, O.NT, O.TN])
def test_gemm_vs_float64_fixture(layout):
    g = golden("gemm_17x29x33.npz")
    A, B, C64 = g["A"], g["B"], g["C"]
    if layout == O.NN:
        C = O.gemm(O.NN, A, B)
    elif layout == O.NT:
        C = O.gemm(O.NT, A, np.ascontiguousarray(B.T))
    else:
        C = O.gemm(O.TN, np.ascontiguousarray(A.T), B)
    K = A.shape[1]
    assert normwise_rel(C, C64) < 1e-6 * math.sqrt(K)
    # A transposed operand would be wrong by O(1), far outside this bound.
    assert normwise_rel(O.gemm(O.NN, A, np.ascontiguousarray(B[::-1])), C64) > 0.1


def test_gemm_edge_shapes_match_float64():
    rng = np.random.default_rng(7)
    for (M, N, K) in [(1, 1, 1), (64, 10, 784), (3, 1000, 5), (257, 3, 513)]:
        A = rng.standard_normal((M, K)).astype(f32)
        B = rng.standard_normal((K, N)).astype(f32)
        assert normwise_rel(O.gemm(O.NN, A, B), A.astype(np.float64) @ B) < 1e-6 * math.sqrt(K)


# ------------------------------------------------------------ activations
def test_gelu_tanh_vs_torch_fixture():
    g = golden("gelu_tanh.npz")
    z = g["z"].astype(f32)
    y = O.act(O.ACT_GELU, z)
    ref = g["y"]
    # fp32 result of the float64 evaluation at the fp32-rounded input.
    zr = z.astype(np.float64)
    assert np.max(np.abs(y - ref) / np.maximum(np.abs(ref), 1.0)) < 2e-6 + 1e-6 * np.max(np.abs(zr - g["z"]))
    dy = np.array([O.act_grad_scalar(O.ACT_GELU, v) for v in z])
    assert np.max(np.abs(dy - g["dy"])) < 1e-5


def test_gelu_special_values():
    # gelu(0) = 0; gelu(x) - gelu(-x) = x (tanh is odd); gelu'(0) = 0.5.
    assert O.act(O.ACT_GELU, np.zeros(1, f32))[0] == 0.0
    x = np.linspace(0.1, 5, 50).astype(f32)
    d = O.act(O.ACT_GELU, x).astype(np.float64) - O.act(O.ACT_GELU, -x)
    assert np.max(np.abs(d - x)) < 1e-6 * 5
    assert abs(O.act_grad_scalar(O.ACT_GELU, 0.0) - 0.5) < 1e-7


def test_relu_and_mask_convention():
    z = np.array([-2.0, -1e-30, 0.0, 1e-30, 3.0], dtype=f32)
    assert np.array_equal(O.act(O.ACT_RELU, z), np.maximum(z, 0))
    g = [O.act_grad_scalar(O.ACT_RELU, v) for v in z]
    assert g == [0.0, 0.0, 0.0, 1.0, 1.0]  # [z > 0], zero at z == 0


def test_act_bwd_and_bias_grad():
    rng = np.random.default_rng(8)
    Z = rng.standard_normal((33, 17)).astype(f32)
    dH = rng.standard_normal((33, 17)).astype(f32)
    relu = O.act_bwd(O.ACT_RELU, dH, Z)
    assert np.array_equal(relu, np.where(Z > 0, dH, 0).astype(f32))
    db = O.bias_grad(dH)
    assert np.max(np.abs(db - dH.astype(np.float64).sum(0))) < 1e-6


def test_bias_act_broadcast():
    C = np.zeros((3, 4), f32)
    b = np.array([1, -2, 3, -4], f32)
    Z, H = O.bias_act(C, b, O.ACT_RELU)
    assert np.array_equal(Z, np.tile(b, (3, 1)))
    assert np.array_equal(H, np.tile(np.maximum(b, 0), (3, 1)))


# -------------------------------------------------------- softmax and CE
def test_softmax_ce_vs_torch_fixture():
    g = golden("softmax_ce_9x37.npz")
    loss, d, am, mean = O.softmax_ce(g["x"], g["labels"])
    assert np.max(np.abs(loss - g["loss"]) / np.maximum(np.abs(g["loss"]), 1)) < 2e-6
    assert np.max(np.abs(d - g["dlogits"])) < 1e-6
    assert np.array_equal(am, g["argmax"])           # first occurrence on ties
    assert am[3] == 5 and am[4] == 0 and am[5] == 36
    assert abs(mean - g["loss"].mean()) < 1e-5


def test_softmax_uniform_rows_closed_form():
    """std_wgsl.rs:97-187 (uniform rows of 64 -> 1/64; backward of seed 1 -> 0)
    and :190-265 (softmax(2/x) over 32 columns, + 2 -> 2 + 1/32)."""
    x = full((16, 64), 3.0 * 2.0 * 32 - 1)  # c - a@b is constant per row
    y = O.softmax(x)
    assert np.all(y == f32(1 / 64))
    assert np.all(O.softmax_bwd(y, np.ones_like(y)) == 0.0)
    y2 = O.softmax(full((16, 32), 2.0 / 3.0))
    assert np.all(y2 + f32(2) == f32(2 + 1 / 32))


def test_softmax_ce_invariants():
    rng = np.random.default_rng(9)
    x = (2 * rng.standard_normal((50, 1000))).astype(f32)
    lab = rng.integers(0, 1000, 50).astype(np.uint32)
    loss, d, am, mean = O.softmax_ce(x, lab)
    x64 = x.astype(np.float64)
    m = x64.max(1, keepdims=True)
    lse = (m + np.log(np.exp(x64 - m).sum(1, keepdims=True)))[:, 0]
    assert np.max(np.abs(loss - (lse - x64[np.arange(50), lab]))) < 1e-5
    assert np.max(np.abs(d.astype(np.float64).sum(1))) < 1e-5
    p = np.exp(x64 - lse[:, None])
    assert np.max(np.abs(d[np.arange(50), lab] - (p[np.arange(50), lab] - 1))) < 1e-6
    assert np.array_equal(am, np.argmax(x, 1))
    sm = O.softmax(x).astype(np.float64)
    assert np.max(np.abs(sm.sum(1) - 1)) < 1e-5


def test_softmax_bwd_matches_jacobian():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((4, 7)).astype(f32)
    dy = rng.standard_normal((4, 7)).astype(f32)
    y = O.softmax(x).astype(np.float64)
    dx = O.softmax_bwd(y.astype(f32), dy)
    for r in range(4):
        J = np.diag(y[r]) - np.outer(y[r], y[r])
        assert np.max(np.abs(dx[r] - J @ dy[r])) < 1e-6


# --------------------------------------------------------------- optimisers
def test_sgd_reference_values():
    """tests/optim.rs:10-104: after forward/backward of c + a*b with seed 1 and
    lr 1e-3, weights become 3 - 2e-3, 2 - 3e-3, 1 - 1e-3 and grads are zeroed."""
    lr = f32(1e-3)
    for w0, g0 in ((3.0, 2.0), (2.0, 3.0), (1.0, 1.0)):
        w = full(1024, w0)
        g = full(1024, g0)
        O.sgd_(w, g, lr)
        assert np.all(w == f32(w0) - f32(g0 * 1e-3))
        assert np.all(g == 0.0)


def test_adam_first_step_closed_form():
    rng = np.random.default_rng(11)
    p0 = (0.02 * rng.standard_normal(4096)).astype(f32)
    g = (1e-3 * rng.standard_normal(4096)).astype(f32)
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    b1, b2, eps, lr = f32(0.9), f32(0.999), f32(1e-8), f32(1e-3)
    s, r = O.adam_scalars(lr, b1, b2, 1)
    O.adam_(p, g.copy(), m, v, b1, b2, eps, s, r)
    g64 = g.astype(np.float64)
    expect = p0 - 1e-3 * g64 / (np.abs(g64) + 1e-8)
    assert np.max(np.abs(p - expect)) / np.max(np.abs(p0)) < 1e-6


def test_adam_vs_torch_fixture():
    g = golden("adam_10steps.npz")
    p = g["p0"].copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    b1, b2, eps, lr = f32(0.9), f32(0.999), f32(1e-8), f32(1e-3)
    for s in range(10):
        ss, r = O.adam_scalars(lr, b1, b2, s + 1)
        O.adam_(p, np.ascontiguousarray(g["grads"][s]), m, v, b1, b2, eps, ss, r)
    assert normwise_rel(p, g["p_f64"]) < 1e-5
    assert normwise_rel(p, g["p_f32"]) < 1e-5


# ----------------------------------------------------------- composition
def test_mlp_step_composition_vs_torch_autograd():
    """Linear-GELU-Linear-CE forward and backward from oracle pieces vs torch."""
    g = golden("mlp_gelu_ce.npz")
    X, W1, b1, W2, b2, y = g["X"], g["W1"], g["b1"], g["W2"], g["b2"], g["y"]
    Z1, H1 = O.bias_act(O.gemm(O.NN, X, W1), b1, O.ACT_GELU)
    Z2, _ = O.bias_act(O.gemm(O.NN, H1, W2), b2, O.ACT_NONE)
    loss, dZ2, _, mean = O.softmax_ce(Z2, y)
    assert abs(float(loss.astype(np.float64).sum()) - float(g["loss_sum"])) < 1e-5 * abs(float(g["loss_sum"]))
    dW2 = O.gemm(O.TN, H1, dZ2)
    db2 = O.bias_grad(dZ2)
    dZ1 = O.act_bwd(O.ACT_GELU, O.gemm(O.NT, dZ2, W2), Z1)
    dW1 = O.gemm(O.TN, X, dZ1)
    db1 = O.bias_grad(dZ1)
    dX = O.gemm(O.NT, dZ1, W1)
    for got, key in ((dW2, "dW2"), (db2, "db2"), (dW1, "dW1"), (db1, "db1"), (dX, "dX")):
        assert normwise_rel(got, g[key]) < 1e-5, key
