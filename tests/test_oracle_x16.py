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
