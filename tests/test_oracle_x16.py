"""Pins the oracle's 16-bit storage types (conversions and the 16-bit GEMM)
against independent implementations: numpy's IEEE binary16 conversion,
torch's bfloat16 conversion, and exact integer arithmetic.

The reference stores F16 / BF16 tensors as 16-bit words converted by the
`half` crate at its upload / download boundary
(crates/fused_gpu/src/dispatch/mod.rs:614-645, backend/mod.rs:335-427).
"""
import numpy as np
import pytest
import torch

import oracle

F16, BF16 = oracle.F16, oracle.BF16


def _bf16_torch(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def _round_ref(dtype, x64: np.ndarray) -> np.ndarray:
    """Independent rounding of float64 values (exactly representable in
    float32 here) to 16-bit words."""
    if dtype == F16:
        with np.errstate(over="ignore"):
            return x64.astype(np.float16).view(np.uint16)
    return _bf16_torch(x64.astype(np.float32))


def _widen_ref(dtype, bits: np.ndarray) -> np.ndarray:
    if dtype == F16:
        return bits.view(np.float16).astype(np.float64)
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.fixture(scope="module")
def patterns():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=1_000_000, dtype=np.uint64).astype(np.uint32)
    # Near the binary16 range ends and exact ties, where a dropped rounding
    # step or an off-by-one exponent shows.
    edge = np.array([0x477FE000, 0x477FEFFF, 0x477FF000, 0x477FF001, 0x38800000, 0x387FFFFF,
                     0x33000000, 0x33000001, 0x32FFFFFF, 0x33800000, 0x00000001, 0x7F7FFFFF,
                     0x7F800000, 0xFF800000, 0x80000000, 0x00000000, 0x3F800000, 0x3F801000,
                     0x3F803000, 0x3F808000, 0x3F818000], dtype=np.uint32)
    return np.concatenate([bits, edge, edge | np.uint32(0x80000000)]).view(np.float32)


def test_f16_conversion_matches_numpy(patterns):
    x = patterns
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    got = oracle.from_f32(F16, x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all(np.isnan(oracle.to_f32(F16, got[nan])))


def test_f16_ties_round_to_even():
    codes = np.arange(0x0000, 0x7BFF, dtype=np.uint16)  # finite, positive, with a successor
    lo = codes.view(np.float16).astype(np.float64)
    hi = (codes + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)  # exact in float32
    got = oracle.from_f32(F16, mid)
    want = np.where(codes % 2 == 0, codes, codes + 1).astype(np.uint16)
    assert np.array_equal(got, want)


def test_bf16_conversion_matches_torch(patterns):
    x = patterns
    got = oracle.from_f32(BF16, x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], _bf16_torch(x)[~nan])
    assert np.all(np.isnan(oracle.to_f32(BF16, got[nan])))


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_widen_every_code(dtype):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    with np.errstate(invalid="ignore"):  # signalling-NaN codes
        got = oracle.to_f32(dtype, codes).astype(np.float64)
        ref = _widen_ref(dtype, codes)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], ref[~nan])
    # Every non-NaN code survives the round trip.
    back = oracle.from_f32(dtype, got.astype(np.float32))
    assert np.array_equal(back[~nan], codes[~nan])


def _quarter_ints(rng, shape):
    return rng.integers(-8, 9, size=shape).astype(np.float64) / 4.0


@pytest.mark.parametrize("dtype", [F16, BF16])
@pytest.mark.parametrize("layout", [oracle.NN, oracle.NT, oracle.TN])
def test_gemm_x16_exact_integers(dtype, layout):
    """Inputs k/4 (|k| <= 8) make every product and partial sum exact in
    fp32, so the 16-bit results are fixed by the rounding of each node value
    alone: matmul, bias add, ReLU."""
    rng = np.random.default_rng(11 + layout + 3 * dtype)
    M, N, K = 37, 29, 300
    a = _quarter_ints(rng, (M, K))
    b = _quarter_ints(rng, (K, N))
    bias = _quarter_ints(rng, (N,))
    A = a if layout != oracle.TN else a.T
    B = b if layout != oracle.NT else b.T
    A16 = _round_ref(dtype, np.ascontiguousarray(A))
    B16 = _round_ref(dtype, np.ascontiguousarray(B))
    b16 = _round_ref(dtype, bias)
    exact = (np.rint(a * 4).astype(np.int64) @ np.rint(b * 4).astype(np.int64)) / 16.0
    v = _widen_ref(dtype, _round_ref(dtype, exact))
    z16 = _round_ref(dtype, v + bias[None, :])
    h16 = _round_ref(dtype, np.maximum(_widen_ref(dtype, z16), 0.0))
    C, Z = oracle.gemm_x16(dtype, layout, A16, B16, bias=b16, act=oracle.ACT_RELU, want_z=True)
    assert np.array_equal(Z, z16)
    assert np.array_equal(C, h16)
    # Plain product and accumulation into an existing C.
    C0 = _round_ref(dtype, _quarter_ints(rng, (M, N)))
    got = oracle.gemm_x16(dtype, layout, A16, B16, C=C0)
    want = _round_ref(dtype, v + _widen_ref(dtype, C0))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_gemm_bwd_x16_relu_mask(dtype):
    rng = np.random.default_rng(5)
    M, N, K = 20, 24, 64
    a, b = _quarter_ints(rng, (M, K)), _quarter_ints(rng, (N, K))
    zs = _quarter_ints(rng, (M, N))
    A16, B16, Z16 = (_round_ref(dtype, x) for x in (a, b, zs))
    exact = (np.rint(a * 4).astype(np.int64) @ np.rint(b * 4).astype(np.int64).T) / 16.0
    v = _widen_ref(dtype, _round_ref(dtype, exact))
    want = _round_ref(dtype, np.where(zs > 0, v, 0.0))  # a mask: +0 where zs <= 0
    got = oracle.gemm_bwd_x16(dtype, oracle.NT, A16, B16, act=oracle.ACT_RELU, Zs=Z16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_gemm_x16_random_vs_float64(dtype):
    """Random operands: the fp32 sum differs from the exact one by far less
    than a 16-bit rounding step, so nearly every element rounds identically
    and none is off by more than one unit in the last place."""
    rng = np.random.default_rng(3)
    M, N, K = 33, 47, 129
    A16 = _round_ref(dtype, rng.standard_normal((M, K)))
    B16 = _round_ref(dtype, rng.standard_normal((K, N)))
    exact = _widen_ref(dtype, A16) @ _widen_ref(dtype, B16)
    want = _round_ref(dtype, exact.astype(np.float32).astype(np.float64))
    got = oracle.gemm_x16(dtype, oracle.NN, A16, B16)
    diff = np.abs(got.astype(np.int32) - want.astype(np.int32))
    assert diff.max() <= 1
    assert np.mean(diff != 0) < 0.01


# GELU-tanh with the reference's constants (crates/ferrograd-nn/src/op/
# unary.rs:493-494), evaluated independently of the C oracle: numpy float64
# for the value, complex-step differentiation of the same float64 form for
# the derivative (f'(x) = Im f(x + ih) / h, exact to float64 rounding for
# tiny h, with no closed form of the derivative involved).
_C0, _C1 = 0.7978846, 0.044715


def _gelu64(x):
    return 0.5 * x * (1.0 + np.tanh(_C0 * (x + _C1 * x * x * x)))


def _gelu_grad64(x):
    h = 1e-30
    return np.imag(_gelu64(x.astype(np.complex128) + 1j * h)) / h


def _sixty_fourths(rng, shape):
    """Multiples of 1/64 in [-1/2, 1/2] (exact in both 16-bit types):
    products are multiples of 1/4096, and sums over K = 64 stay exact in fp32
    (at most 16 significant bits) yet need more bits than either 16-bit type
    holds, and are of order one, where GELU curves."""
    return rng.integers(-32, 33, size=shape).astype(np.float64) / 64.0


def _round_f32(dtype, x64):
    """A float64 value rounded to float32, then to the 16-bit type (the
    oracle evaluates activations in double and stores them through float)."""
    return _round_ref(dtype, x64.astype(np.float32).astype(np.float64))


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_gemm_x16_gelu_rounds_each_node_once(dtype):
    """Forward matmul -> bias add -> GELU on 16-bit tensors: exact-integer
    operands fix the product, so the result is set by the rounding points:
    the matmul node, the bias-add node (Z) and the GELU node are each rounded
    once to the storage type.  The inputs are chosen so that GELU of an
    unrounded pre-activation, or of a product whose rounding was dropped,
    gives other bits on some elements (asserted), so either mistake fails."""
    rng = np.random.default_rng(21 + dtype)
    M, N, K = 37, 29, 64
    a, b, bias = _sixty_fourths(rng, (M, K)), _sixty_fourths(rng, (K, N)), _sixty_fourths(rng, (N,))
    A16, B16, b16 = _round_ref(dtype, a), _round_ref(dtype, b), _round_ref(dtype, bias)
    exact = (np.rint(a * 64).astype(np.int64) @ np.rint(b * 64).astype(np.int64)) / 4096.0
    v = _widen_ref(dtype, _round_ref(dtype, exact))
    z16 = _round_ref(dtype, v + bias[None, :])
    want = _round_f32(dtype, _gelu64(_widen_ref(dtype, z16)))
    C, Z = oracle.gemm_x16(dtype, oracle.NN, A16, B16, bias=b16, act=oracle.ACT_GELU, want_z=True)
    assert np.array_equal(Z, z16)
    assert np.array_equal(C, want)
    # The plausible mistakes differ on these inputs.
    no_z_round = _round_f32(dtype, _gelu64(v + bias[None, :]))
    no_v_round = _round_f32(dtype, _gelu64(_widen_ref(dtype, _round_ref(dtype, exact + bias))))
    assert np.count_nonzero(no_z_round != want) > 0
    assert np.count_nonzero(no_v_round != want) > 0


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_gemm_bwd_x16_gelu_grad_rounds_once(dtype):
    """Data gradient through GELU on 16-bit tensors: dX = round(round(dC.W^T)
    * GELU'(Z)), the product in fp32 and one rounding of the result.  A
    dropped rounding of the matmul node, or an extra rounding of GELU'(Z) to
    the storage type before the multiply, gives other bits on some elements
    of these inputs (asserted)."""
    rng = np.random.default_rng(31 + dtype)
    M, N, K = 24, 40, 64
    a, w = _sixty_fourths(rng, (M, K)), _sixty_fourths(rng, (N, K))
    Z16 = _round_ref(dtype, rng.normal(0.0, 2.0, (M, N)))
    A16, W16 = _round_ref(dtype, a), _round_ref(dtype, w)
    exact = (np.rint(a * 64).astype(np.int64) @ np.rint(w * 64).astype(np.int64).T) / 4096.0
    v32 = _widen_ref(dtype, _round_ref(dtype, exact)).astype(np.float32)
    g32 = _gelu_grad64(_widen_ref(dtype, Z16)).astype(np.float32)
    want = _round_ref(dtype, (v32 * g32).astype(np.float64))
    got = oracle.gemm_bwd_x16(dtype, oracle.NT, A16, W16, act=oracle.ACT_GELU, Zs=Z16)
    assert np.array_equal(got, want)
    no_v_round = _round_ref(dtype, (exact.astype(np.float32) * g32).astype(np.float64))
    g16 = _widen_ref(dtype, _round_ref(dtype, g32.astype(np.float64))).astype(np.float32)
    extra_g_round = _round_ref(dtype, (v32 * g16).astype(np.float64))
    assert np.count_nonzero(no_v_round != want) > 0
    assert np.count_nonzero(extra_g_round != want) > 0


def test_gelu_reference_forms_agree_with_torch():
    """The float64 forms above against torch's tanh GELU and its autograd
    derivative (torch's constant sqrt(2/pi) differs from the reference's
    0.7978846 by 5e-8 relative, hence the tolerance)."""
    x = np.linspace(-8.0, 8.0, 4001)
    t = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    y = torch.nn.functional.gelu(t, approximate="tanh")
    y.sum().backward()
    assert np.allclose(_gelu64(x), y.detach().numpy(), rtol=1e-6, atol=1e-7)
    assert np.allclose(_gelu_grad64(x), t.grad.numpy(), rtol=1e-6, atol=1e-7)
