"""GPU parity of the 16-bit (fp16 / bf16) kernels against the CPU oracle,
through the C ABI.

Bar: on operands whose products and partial sums are exact in fp32
(multiples of 1/4 of magnitude <= 2), the GPU's 16-bit words equal the
oracle's bit for bit -- the result is then fixed by the rounding of each
node value, whatever the MFMA summation order.  On random operands every
element is within the rounding steps of the oracle's -- the fp32 sums differ
in order only, by at most 2 K u sum|a b|, and each node value then rounds
once -- with at most 1 % of the elements differing at all.
"""
import sys

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

F16, BF16 = O.F16, O.BF16
DT_IDS = {F16: "f16", BF16: "bf16"}


def _torch():
    import torch
    return torch


def dev16(bits):
    torch = _torch()
    a = np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)
    return torch.from_numpy(a.copy()).cuda()


def host16(t):
    _torch().cuda.synchronize()
    return t.cpu().numpy().view(np.uint16)


def empty16(shape):
    torch = _torch()
    return torch.zeros(shape, dtype=torch.int16, device="cuda")


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def quarter_ints(rng, shape, dtype):
    return O.from_f32(dtype, (rng.integers(-8, 9, size=shape) / 4.0).astype(np.float32))


def normal16(rng, shape, dtype, scale=1.0):
    return O.from_f32(dtype, (scale * rng.standard_normal(shape)).astype(np.float32))


def ulp_of(bits, dtype):
    """Unit in the last place of the storage type at each value."""
    r = O.to_f32(dtype, bits).astype(np.float64)
    mant = 10 if dtype == F16 else 7
    tiny = 2.0 ** -14 if dtype == F16 else 2.0 ** -126
    return np.exp2(np.floor(np.log2(np.maximum(np.abs(r), tiny))) - mant)


def ulp_diff(got, ref, dtype):
    """|got - ref| in units in the last place of the storage type at ref."""
    g = O.to_f32(dtype, got).astype(np.float64)
    r = O.to_f32(dtype, ref).astype(np.float64)
    return np.abs(g - r) / ulp_of(ref, dtype)


def sum_error_bound(dtype, layout, A, B):
    """Rigorous bound on the difference of two fp32 evaluations of the same
    dot products in different orders: 2 K u sum_k |a_ik b_kj| (u = 2^-24)."""
    a = np.abs(O.to_f32(dtype, A).astype(np.float64))
    b = np.abs(O.to_f32(dtype, B).astype(np.float64))
    a = a.T if layout == O.TN else a
    b = b.T if layout == O.NT else b
    K = a.shape[1]
    return 2.0 * K * 2.0 ** -24 * (a @ b)


def check_epilogue(dtype, gotV, gotC, gotZ, refV, refC, refZ, act, esum):
    """The fp32 sums differ from the oracle's in order only (bounded by
    esum); each node value then rounds once: V within esum + ulp(V), Z within
    that + ulp(Z), C within 1.2 times that + ulp(C) (|GELU'| < 1.13); at most
    1 % of the elements differ at all."""
    f = lambda b: O.to_f32(dtype, b).astype(np.float64)
    tv = esum + ulp_of(refV, dtype)
    if gotV is not None:
        assert np.all(np.abs(f(gotV) - f(refV)) <= tv)
    tz = tv + ulp_of(refZ, dtype)
    assert np.all(np.abs(f(gotZ) - f(refZ)) <= tz)
    tc = (1.2 * tz + ulp_of(refC, dtype)) if act != O.ACT_NONE else tz
    assert np.all(np.abs(f(gotC) - f(refC)) <= tc)
    for got, ref in ((gotV, refV), (gotZ, refZ), (gotC, refC)):
        if got is not None:
            assert np.mean(got != ref) < 0.01


def storage_shapes(layout, M, N, K):
    a = (K, M) if layout == O.TN else (M, K)
    b = (N, K) if layout == O.NT else (K, N)
    return a, b


LAYOUTS = [O.NN, O.NT, O.TN]
LAYOUT_IDS = ["NN", "NT", "TN"]
SHAPES = [(37, 29, 300), (64, 256, 784), (64, 10, 256), (300, 260, 100), (128, 1000, 512),
          (512, 512, 512), (1, 1, 1), (257, 513, 40)]


@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
@pytest.mark.parametrize("layout", LAYOUTS, ids=LAYOUT_IDS)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_gemm_x16_exact_bits(gpu_ctx, dtype, layout, shape):
    M, N, K = shape
    note(f"gemm_x16 exact {DT_IDS[dtype]} layout={layout} {M}x{N}x{K}")
    rng = np.random.default_rng(100 + M + N + K + layout)
    sa, sb = storage_shapes(layout, M, N, K)
    A, B = quarter_ints(rng, sa, dtype), quarter_ints(rng, sb, dtype)
    bias = quarter_ints(rng, (N,), dtype)
    refC, refZ = O.gemm_x16(dtype, layout, A, B, bias=bias, act=O.ACT_RELU, want_z=True)
    dC, dZ = empty16((M, N)), empty16((M, N))
    gpu_ctx.gemm_x16(dtype, layout, M, N, K, dev16(A), sa[1], dev16(B), sb[1], dC, N,
                     bias=dev16(bias), act=O.ACT_RELU, Z=dZ, ldz=N)
    assert np.array_equal(host16(dZ), refZ)
    assert np.array_equal(host16(dC), refC)
    # Accumulation into an existing C, no epilogue.
    C0 = quarter_ints(rng, (M, N), dtype)
    dC = dev16(C0)
    gpu_ctx.gemm_x16(dtype, layout, M, N, K, dev16(A), sa[1], dev16(B), sb[1], dC, N,
                     accumulate=True)
    assert np.array_equal(host16(dC), O.gemm_x16(dtype, layout, A, B, C=C0))


@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
@pytest.mark.parametrize("case", [(O.NN, 4096, 2048, 64), (O.NT, 4096, 4096, 64),
                                  (O.TN, 4096, 4096, 48), (O.NN, 2050, 4000, 96),
                                  (O.NT, 4096, 4000, 96), (O.TN, 4000, 4096, 96),
                                  (O.NN, 2050, 4000, 128), (O.NT, 4096, 4000, 192),
                                  (O.TN, 4000, 4096, 128), (O.NT, 2048, 1024, 1000),
                                  (O.NT, 2050, 1030, 1000), (O.NT, 2048, 1024, 40),
                                  (O.NN, 2048, 4096, 1000), (O.TN, 4096, 4096, 1001)],
                         ids=["NN-4096x2048x64", "NT-4096x4096x64", "TN-4096x4096x48",
                              "NN-2050x4000x96", "NT-4096x4000x96", "TN-4000x4096x96",
                              "NN-2050x4000x128", "NT-4096x4000x192", "TN-4000x4096x128",
                              "NT-2048x1024x1000", "NT-2050x1030x1000", "NT-2048x1024x40",
                              "NN-2048x4096x1000", "TN-4096x4096x1001"])
def test_gemm_x16_exact_bits_large_tiles(gpu_ctx, dtype, case):
    """Shapes large enough for the 256-wide tile configurations the
    dispatcher picks for full-chip GEMMs (8-wave 256x256 and 256x128 at
    BK 64, 256x256 at BK 32, 128x128), on the pipelined path (K a
    multiple of 32 or 64; edge tiles in M and N) and off it (K = 48, and
    NT with K = 1000 or 40 on the 256x128 tiles of the any-shape kernel)."""
    layout, M, N, K = case
    note(f"gemm_x16 exact large {DT_IDS[dtype]} layout={layout} {M}x{N}x{K}")
    rng = np.random.default_rng(M + K + layout)
    sa, sb = storage_shapes(layout, M, N, K)
    A, B = quarter_ints(rng, sa, dtype), quarter_ints(rng, sb, dtype)
    bias = quarter_ints(rng, (N,), dtype)
    refC = O.gemm_x16(dtype, layout, A, B, bias=bias, act=O.ACT_RELU)
    dC = empty16((M, N))
    gpu_ctx.gemm_x16(dtype, layout, M, N, K, dev16(A), sa[1], dev16(B), sb[1], dC, N,
                     bias=dev16(bias), act=O.ACT_RELU)
    assert np.array_equal(host16(dC), refC)


@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
def test_gemm_bwd_x16_head_shape_exact_bits(gpu_ctx, dtype):
    """The data gradient of a 1000-wide head, NT 2048x4096x1000 with the
    ReLU derivative (K not a multiple of the tile depth), on operands whose
    sums are exact in fp32: bit for bit on a sample of rows."""
    M, N, K = 2048, 4096, 1000
    note(f"gemm_bwd_x16 head shape {DT_IDS[dtype]}")
    rng = np.random.default_rng(1000 + dtype)
    A, B = quarter_ints(rng, (M, K), dtype), quarter_ints(rng, (N, K), dtype)
    Zs = quarter_ints(rng, (M, N), dtype)
    rows = np.sort(rng.choice(M, size=64, replace=False))
    ref = O.gemm_bwd_x16(dtype, O.NT, A[rows], B, act=O.ACT_RELU, Zs=Zs[rows])
    dC = empty16((M, N))
    gpu_ctx.gemm_bwd_x16(dtype, O.NT, M, N, K, dev16(A), K, dev16(B), K, dC, N,
                         act=O.ACT_RELU, Zs=dev16(Zs), ldzs=N)
    assert np.array_equal(host16(dC)[rows], ref)


@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
@pytest.mark.parametrize("layout", LAYOUTS, ids=LAYOUT_IDS)
def test_gemm_bwd_x16_exact_bits(gpu_ctx, dtype, layout):
    M, N, K = 130, 200, 96
    note(f"gemm_bwd_x16 exact {DT_IDS[dtype]} layout={layout}")
    rng = np.random.default_rng(7 + layout)
    sa, sb = storage_shapes(layout, M, N, K)
    A, B = quarter_ints(rng, sa, dtype), quarter_ints(rng, sb, dtype)
    Zs = quarter_ints(rng, (M, N), dtype)
    ref = O.gemm_bwd_x16(dtype, layout, A, B, act=O.ACT_RELU, Zs=Zs)
    dC = empty16((M, N))
    gpu_ctx.gemm_bwd_x16(dtype, layout, M, N, K, dev16(A), sa[1], dev16(B), sb[1], dC, N,
                         act=O.ACT_RELU, Zs=dev16(Zs), ldzs=N)
    assert np.array_equal(host16(dC), ref)


@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
@pytest.mark.parametrize("layout", LAYOUTS, ids=LAYOUT_IDS)
@pytest.mark.parametrize("act", [O.ACT_NONE, O.ACT_GELU], ids=["none", "gelu"])
def test_gemm_x16_random_within_one_ulp(gpu_ctx, dtype, layout, act):
    M, N, K = 300, 520, 1000
    note(f"gemm_x16 random {DT_IDS[dtype]} layout={layout} act={act}")
    rng = np.random.default_rng(31 + layout + act)
    sa, sb = storage_shapes(layout, M, N, K)
    A, B = normal16(rng, sa, dtype), normal16(rng, sb, dtype, 1.0 / np.sqrt(K))
    bias = normal16(rng, (N,), dtype, 0.1)
    refC, refZ = O.gemm_x16(dtype, layout, A, B, bias=bias, act=act, want_z=True)
    refV = O.gemm_x16(dtype, layout, A, B)
    dC, dZ, dV = empty16((M, N)), empty16((M, N)), empty16((M, N))
    gpu_ctx.gemm_x16(dtype, layout, M, N, K, dev16(A), sa[1], dev16(B), sb[1], dC, N,
                     bias=dev16(bias), act=act, Z=dZ, ldz=N)
    gpu_ctx.gemm_x16(dtype, layout, M, N, K, dev16(A), sa[1], dev16(B), sb[1], dV, N)
    check_epilogue(dtype, host16(dV), host16(dC), host16(dZ), refV, refC, refZ, act,
                   sum_error_bound(dtype, layout, A, B))


@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
def test_gemm_x16_unaligned_leading_dims(gpu_ctx, dtype):
    """Leading dimensions that are not multiples of 8 take the element-load
    variant; results still match bit for bit on exact operands."""
    M, N, K = 70, 45, 33
    note(f"gemm_x16 unaligned {DT_IDS[dtype]}")
    rng = np.random.default_rng(9)
    lda, ldb, ldc = K + 3, N + 5, N + 1
    A = quarter_ints(rng, (M, lda), dtype)
    B = quarter_ints(rng, (K, ldb), dtype)
    ref = O.gemm_x16(dtype, O.NN, A[:, :K], B[:, :N])
    dC = empty16((M, ldc))
    gpu_ctx.gemm_x16(dtype, O.NN, M, N, K, dev16(A), lda, dev16(B), ldb, dC, ldc)
    assert np.array_equal(host16(dC)[:, :N], ref)


@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
def test_gemm_x16_c5_hidden_shape_sampled(gpu_ctx, dtype):
    """The c5 hidden-layer forward shape 2048x4096x4096 with bias + GELU,
    checked on a sample of 64 rows against the oracle."""
    M, N, K = 2048, 4096, 4096
    note(f"gemm_x16 c5 hidden {DT_IDS[dtype]}")
    rng = np.random.default_rng(4)
    A = normal16(rng, (M, K), dtype)
    B = normal16(rng, (K, N), dtype, 1.0 / np.sqrt(K))
    bias = normal16(rng, (N,), dtype, 0.1)
    dC, dZ = empty16((M, N)), empty16((M, N))
    gpu_ctx.gemm_x16(dtype, O.NN, M, N, K, dev16(A), K, dev16(B), N, dC, N, bias=dev16(bias),
                     act=O.ACT_GELU, Z=dZ, ldz=N)
    rows = np.sort(rng.choice(M, size=64, replace=False))
    refC, refZ = O.gemm_x16(dtype, O.NN, A[rows], B, bias=bias, act=O.ACT_GELU, want_z=True)
    refV = O.gemm_x16(dtype, O.NN, A[rows], B)
    check_epilogue(dtype, None, host16(dC)[rows], host16(dZ)[rows], refV, refC, refZ,
                   O.ACT_GELU, sum_error_bound(dtype, O.NN, A[rows], B))


@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
@pytest.mark.parametrize("case", [
    # (layout, M, N, K, mode): 64 output tiles of 256x128 over a long K, the
    # shapes of a batch-2048 MLP's 1000-wide head and 1024-wide data gradient
    (O.NN, 2048, 1000, 4096, "fwd"),
    (O.NT, 2048, 1024, 4096, "bwd"),
    (O.NN, 1024, 1024, 2048, "fwd"),   # 128x128 tiles, BK 32
], ids=lambda c: f"{['NN', 'NT', 'TN'][c[0]]}-{c[1]}x{c[2]}x{c[3]}-{c[4]}")
def test_gemm_x16_split_k(dtype, case):
    """Few output tiles and a long K: the 16-bit GEMM splits K into fp32 slots
    of the context's workspace (when reserved) and a second kernel sums them
    in slot order and applies the epilogue.  On operands whose sums are exact
    in fp32 (multiples of 1/4; ReLU, whose mask is exact, and C += with no
    epilogue) the split result equals the oracle bit for bit -- every slice
    offset and slot index is pinned; on random operands with GELU a sample
    of rows is within the rounding bounds, as the unsplit kernel's result on
    a context without workspace is."""
    torch = _torch()
    import ferrograd_amd as fa
    layout, M, N, K, mode = case
    note(f"gemm_x16 split-K {DT_IDS[dtype]} {case}")
    split = fa.Context(0, torch.cuda.current_stream().cuda_stream)
    plain = fa.Context(0, torch.cuda.current_stream().cuda_stream)
    try:
        split.reserve_workspace(64 << 20)
        rng = np.random.default_rng(M + N + K + layout)
        sa, sb = storage_shapes(layout, M, N, K)
        rows = np.sort(rng.choice(M, size=48, replace=False))
        rows_a = (lambda X: X[rows]) if layout != O.TN else (lambda X: X[:, rows])
        for exact in (True, False):
            act = O.ACT_RELU if exact else O.ACT_GELU
            if exact:
                A, B = quarter_ints(rng, sa, dtype), quarter_ints(rng, sb, dtype)
                bias, Zs = quarter_ints(rng, (N,), dtype), quarter_ints(rng, (M, N), dtype)
            else:
                A, B = normal16(rng, sa, dtype), normal16(rng, sb, dtype, 1.0 / np.sqrt(K))
                bias, Zs = normal16(rng, (N,), dtype, 0.1), normal16(rng, (M, N), dtype)
            outs = []
            for c in (split, plain):
                dC, dZ = empty16((M, N)), empty16((M, N))
                if mode == "fwd":
                    c.gemm_x16(dtype, layout, M, N, K, dev16(A), sa[1], dev16(B), sb[1], dC, N,
                               bias=dev16(bias), act=act, Z=dZ, ldz=N)
                else:
                    c.gemm_bwd_x16(dtype, layout, M, N, K, dev16(A), sa[1], dev16(B), sb[1], dC,
                                   N, act=act, Zs=dev16(Zs), ldzs=N)
                c.sync()
                outs.append((host16(dC)[rows], host16(dZ)[rows]))
            if mode == "fwd":
                refC, refZ = O.gemm_x16(dtype, layout, rows_a(A), B, bias=bias, act=act,
                                        want_z=True)
                refV = O.gemm_x16(dtype, layout, rows_a(A), B)
            else:
                refC = O.gemm_bwd_x16(dtype, layout, rows_a(A), B, act=act, Zs=Zs[rows])
            for k, (gC, gZ) in enumerate(outs):
                if exact:
                    assert np.array_equal(gC, refC), ("split", "plain")[k]
                    if mode == "fwd":
                        assert np.array_equal(gZ, refZ), ("split", "plain")[k]
                elif mode == "fwd":
                    check_epilogue(dtype, None, gC, gZ, refV, refC, refZ, act,
                                   sum_error_bound(dtype, layout, rows_a(A), B))
                else:
                    # dC = round(round(v) * gelu'(z)): within 1.2 (esum + ulp(v)) + ulp(dC)
                    f = lambda b: O.to_f32(dtype, b).astype(np.float64)
                    v = O.gemm_x16(dtype, layout, rows_a(A), B)
                    t = 1.2 * (sum_error_bound(dtype, layout, rows_a(A), B) + ulp_of(v, dtype)) \
                        + ulp_of(refC, dtype)
                    assert np.all(np.abs(f(gC) - f(refC)) <= t)
                    assert np.mean(gC != refC) < 0.01
        # C += op(A).op(B), no epilogue, on exact operands (the summing
        # kernel's accumulate path)
        A, B = quarter_ints(rng, sa, dtype), quarter_ints(rng, sb, dtype)
        C0 = quarter_ints(rng, (M, N), dtype)
        dC = dev16(C0)
        split.gemm_x16(dtype, layout, M, N, K, dev16(A), sa[1], dev16(B), sb[1], dC, N,
                       accumulate=True)
        split.sync()
        ref = O.gemm_x16(dtype, layout, rows_a(A), B, C=C0[rows])
        assert np.array_equal(host16(dC)[rows], ref)
    finally:
        split.close()
        plain.close()


@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
@pytest.mark.parametrize("case", [
    (2048, 4096, 4096, O.ACT_GELU, False),  # hidden layer: one launch (gemm16_pair_big)
    (2048, 4096, 1024, O.ACT_NONE, True),   # 1024-wide layer: two launches
    (300, 260, 100, O.ACT_RELU, False),     # small, unaligned tiles: two launches
], ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}-act{c[3]}{'-acc' if c[4] else ''}")
def test_matmul_bwd_x16_matches_separate_calls(dtype, case):
    """fg_matmul_bwd_x16 (dW + dbias and dX with act', one launch where the
    two kernels pair) against fg_gemm_dw_x16 and fg_gemm_bwd_x16 on one
    context and workspace: every output equal bit for bit."""
    torch = _torch()
    import ferrograd_amd as fa
    M, N, K, act, acc = case
    note(f"matmul_bwd_x16 {DT_IDS[dtype]} {case}")
    rng = np.random.default_rng(M + 3 * N + 7 * K)
    X, W = normal16(rng, (M, K), dtype), normal16(rng, (K, N), dtype, 1.0 / np.sqrt(K))
    dZ, Zs = normal16(rng, (M, N), dtype), normal16(rng, (M, K), dtype)
    dX0, dW0, db0 = (normal16(rng, sh, dtype) for sh in ((M, K), (K, N), (N,)))
    own = fa.Context(0, torch.cuda.current_stream().cuda_stream)
    try:
        own.reserve_workspace(1 << 20)
        gX, gW, gdZ, gZs = dev16(X), dev16(W), dev16(dZ), dev16(Zs)
        outs = []
        for fused in (True, False):
            gx, gw, gb = dev16(dX0), dev16(dW0), dev16(db0)
            if fused:
                own.matmul_bwd_x16(dtype, M, N, K, gX, K, gW, N, gdZ, N, gx, K, gw, N, dbias=gb,
                                   act=act, Zs=gZs, ldzs=K, accumulate=acc)
            else:
                own.gemm_dw_x16(dtype, K, N, M, gX, K, gdZ, N, gw, N, accumulate=acc, colsum=gb,
                                colsum_accumulate=acc)
                own.gemm_bwd_x16(dtype, O.NT, M, K, N, gdZ, N, gW, N, gx, K, act=act, Zs=gZs,
                                 ldzs=K, accumulate=acc)
            own.sync()
            outs.append([host16(gx), host16(gw), host16(gb)])
        for a, b in zip(*outs):
            assert np.array_equal(a, b)
    finally:
        own.sync()
        own.close()


@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
@pytest.mark.parametrize("acc", [False, True], ids=["write", "accumulate"])
def test_gemm_dw_x16_split_k_with_column_sums(dtype, acc):
    """The weight gradient of a 1000-wide head, TN 4096x1000x2048 with the
    fused bias gradient: its 128 tiles split K in two when the workspace
    holds the slots and the slices' column sums (each slice's first tile row
    leaves N fp32 sums, added in slot order by the summing kernel).  On
    operands whose sums are exact in fp32 both dW and dbias equal the oracle
    bit for bit, split (64 MiB workspace) and unsplit (none), written and
    accumulated."""
    torch = _torch()
    import ferrograd_amd as fa
    M, N, K = 4096, 1000, 2048
    note(f"gemm_dw_x16 split-K colsum {DT_IDS[dtype]} acc={acc}")
    rng = np.random.default_rng(77 + dtype + acc)
    A, B = quarter_ints(rng, (K, M), dtype), quarter_ints(rng, (K, N), dtype)
    C0, b0 = quarter_ints(rng, (M, N), dtype), quarter_ints(rng, (N,), dtype)
    rows = np.sort(rng.choice(M, size=64, replace=False))
    refC = O.gemm_x16(dtype, O.TN, A[:, rows], B, C=C0[rows] if acc else None)
    colsum = O.to_f32(dtype, B).astype(np.float64).sum(0)
    refb = O.from_f32(dtype, (colsum + (O.to_f32(dtype, b0) if acc else 0)).astype(np.float32))
    split = fa.Context(0, torch.cuda.current_stream().cuda_stream)
    plain = fa.Context(0, torch.cuda.current_stream().cuda_stream)
    try:
        split.reserve_workspace(64 << 20)
        for c in (split, plain):
            dC, db = (dev16(C0), dev16(b0)) if acc else (empty16((M, N)), empty16((N,)))
            c.gemm_dw_x16(dtype, M, N, K, dev16(A), M, dev16(B), N, dC, N, accumulate=acc,
                          colsum=db, colsum_accumulate=acc)
            c.sync()
            assert np.array_equal(host16(dC)[rows], refC)
            assert np.array_equal(host16(db), refb)
    finally:
        split.close()
        plain.close()


def test_gemm_x16_rejects_fp32_dtype(gpu_ctx):
    import ferrograd_amd as fa

    dC = empty16((4, 4))
    with pytest.raises(fa.FgError):
        gpu_ctx.gemm_x16(fa.DTYPE_F32, O.NN, 4, 4, 4, dC, 4, dC, 4, dC, 4)


# ------------------------------------------------------- softmax, bias grad
@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
@pytest.mark.parametrize("shape", [(64, 10), (300, 1000), (33, 4096), (17, 1001), (8, 40000)],
                         ids=lambda s: "x".join(map(str, s)))
def test_softmax_ce_x16(gpu_ctx, dtype, shape):
    """Logits and dlogits of the 16-bit type; fp32 arithmetic inside.  The
    oracle runs on the widened logits; dlogits are compared after rounding
    (within one unit in the last place), losses to 1e-5, argmax exactly."""
    torch = _torch()
    R, C = shape
    note(f"softmax_ce x16 {DT_IDS[dtype]} {R}x{C}")
    rng = np.random.default_rng(R + C)
    X = normal16(rng, (R, C), dtype, 2.0)
    labels = rng.integers(0, C, size=R).astype(np.uint32)
    row_ref, d_ref, am_ref, mean_ref = O.softmax_ce(O.to_f32(dtype, X), labels)
    dX, dD = dev16(X), empty16((R, C))
    dl = torch.from_numpy(labels.view(np.int32).copy()).cuda()
    row = torch.empty(R, device="cuda")
    mean = torch.empty(1, device="cuda")
    am = torch.empty(R, dtype=torch.int32, device="cuda")
    gpu_ctx.softmax_ce(dX, C, dl, R, C, 1.0, row_loss=row, mean_loss=mean, dlogits=dD, ldd=C,
                       argmax=am, dtype=dtype)
    torch.cuda.synchronize()
    assert np.array_equal(am.cpu().numpy().view(np.uint32), am_ref)
    assert np.max(np.abs(row.cpu().numpy() - row_ref) / np.maximum(1.0, np.abs(row_ref))) < 1e-5
    assert abs(float(mean.cpu()[0]) - mean_ref) <= 1e-5 * max(1.0, abs(mean_ref))
    # p - 1 at the label can cancel: allow one unit of the type plus the
    # fp32 noise of p itself.
    ref16 = O.from_f32(dtype, d_ref)
    err = np.abs(O.to_f32(dtype, host16(dD)).astype(np.float64) - O.to_f32(dtype, ref16))
    assert np.all(err <= ulp_of(ref16, dtype) + 2.5e-7)


@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
@pytest.mark.parametrize("shape", [(64, 10), (50, 4096), (9, 1003)],
                         ids=lambda s: "x".join(map(str, s)))
def test_softmax_fwd_bwd_x16(gpu_ctx, dtype, shape):
    R, C = shape
    note(f"softmax x16 {DT_IDS[dtype]} {R}x{C}")
    rng = np.random.default_rng(2 * R + C)
    X = normal16(rng, (R, C), dtype)
    dY = normal16(rng, (R, C), dtype)
    y_ref = O.softmax(O.to_f32(dtype, X))
    dY_ = empty16((R, C))
    gpu_ctx.softmax(dev16(X), R, C, dY_, dtype=dtype)
    Y = host16(dY_)
    assert ulp_diff(Y, O.from_f32(dtype, y_ref), dtype).max() <= 1.0
    dx_ref = O.softmax_bwd(O.to_f32(dtype, Y), O.to_f32(dtype, dY))
    dX = empty16((R, C))
    gpu_ctx.softmax_bwd(dev16(Y), dev16(dY), R, C, dX, dtype=dtype)
    got = O.to_f32(dtype, host16(dX)).astype(np.float64)
    # The row dot product may cancel: bound the error by the row's scale.
    scale = np.max(np.abs(O.to_f32(dtype, Y) * O.to_f32(dtype, dY)), axis=1, keepdims=True)
    eps = 2.0 ** -10 if dtype == F16 else 2.0 ** -7
    assert np.all(np.abs(got - dx_ref) <= eps * np.abs(dx_ref) + 1e-5 * C * scale + 1e-30)


@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
@pytest.mark.parametrize("shape", [(2048, 4096), (64, 10), (333, 257)],
                         ids=lambda s: "x".join(map(str, s)))
def test_bias_grad_x16_exact(gpu_ctx, dtype, shape):
    """Column sums of k/4 values are exact in fp32: the 16-bit result is the
    rounded exact sum, bit for bit; with accumulate, round(old + sum)."""
    M, N = shape
    note(f"bias_grad x16 {DT_IDS[dtype]} {M}x{N}")
    rng = np.random.default_rng(M + N)
    dZ = quarter_ints(rng, (M, N), dtype)
    exact = O.to_f32(dtype, dZ).astype(np.float64).sum(axis=0)
    out = empty16((N,))
    gpu_ctx.bias_grad(M, N, dev16(dZ), N, out, dtype=dtype)
    assert np.array_equal(host16(out), O.from_f32(dtype, exact.astype(np.float32)))
    old = quarter_ints(rng, (N,), dtype)
    out = dev16(old)
    gpu_ctx.bias_grad(M, N, dev16(dZ), N, out, accumulate=True, dtype=dtype)
    want = O.from_f32(dtype, (exact + O.to_f32(dtype, old)).astype(np.float32))
    assert np.array_equal(host16(out), want)


@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
@pytest.mark.parametrize("shape", [(4096, 4096, 64), (1024, 4096, 192), (4000, 1000, 128),
                                   (1024, 1024, 32), (512, 512, 96), (37, 29, 300),
                                   (64, 10, 256), (0, 64, 128), (64, 64, 0),
                                   (1024, 4096, 1000), (1024, 4096, 999)],
                         ids=lambda s: "x".join(map(str, s)))
def test_gemm_dw_x16_fused_bias_grad(gpu_ctx, dtype, shape):
    """dW = A^T.dZ and dbias = column sums of dZ in one call (TN layout): on
    k/4 operands every fp32 sum is exact in any order, so both 16-bit results
    equal the oracle's bit for bit, with and without accumulation.  The
    shapes take the pipelined kernels that sum the columns in the GEMM
    (8-wave 256x256 and 256x128 tiles at BK 64 with edge tiles, 4-wave
    128x128 at BK 32, 8-wave 256x128 with a K tail of 40 or 39 rows) and
    the fallback of GEMM + separate reduction (unaligned, N = 10, no rows,
    K = 0)."""
    M, N, K = shape  # dW is M x N; the reduction runs over K rows
    note(f"gemm_dw_x16 {DT_IDS[dtype]} M={M} N={N} K={K}")
    rng = np.random.default_rng(7 + M + 3 * N + K)
    A, dZ = quarter_ints(rng, (K, M), dtype), quarter_ints(rng, (K, N), dtype)
    exact = O.to_f32(dtype, dZ).astype(np.float64).sum(axis=0)
    # Device operands are never empty (K = 0 reads nothing from them).
    dA = dev16(A if K > 0 else quarter_ints(rng, (1, max(M, 1)), dtype))
    ddZ = dev16(dZ if K > 0 else quarter_ints(rng, (1, N), dtype))
    C, db = empty16((max(M, 1), N)), empty16((N,))
    gpu_ctx.gemm_dw_x16(dtype, M, N, K, dA, max(M, 1), ddZ, N, C, N, colsum=db)
    assert np.array_equal(host16(db), O.from_f32(dtype, exact.astype(np.float32)))
    if M > 0:
        assert np.array_equal(host16(C), O.gemm_x16(dtype, O.TN, A, dZ))
    C0, old = quarter_ints(rng, (max(M, 1), N), dtype), quarter_ints(rng, (N,), dtype)
    C, db = dev16(C0), dev16(old)
    gpu_ctx.gemm_dw_x16(dtype, M, N, K, dA, max(M, 1), ddZ, N, C, N,
                        accumulate=True, colsum=db, colsum_accumulate=True)
    want = O.from_f32(dtype, (exact + O.to_f32(dtype, old)).astype(np.float32))
    assert np.array_equal(host16(db), want)
    if M > 0:
        assert np.array_equal(host16(C), O.gemm_x16(dtype, O.TN, A, dZ, C=C0))


# ------------------------------------------------------------ optimisers
@pytest.mark.parametrize("dtype", [F16, BF16], ids=lambda d: DT_IDS[d])
def test_sgd_adam_x16_bit_exact(gpu_ctx, dtype):
    """16-bit parameters and gradients, fp32 Adam state, a list mixing
    16-bit and fp32 tensors: the update runs in fp32 exactly as the oracle's
    (bit-exact) and the parameter is rounded to its type once."""
    import ferrograd_amd as fa

    torch = _torch()
    note(f"optimisers x16 {DT_IDS[dtype]}")
    rng = np.random.default_rng(77)
    sizes = [1000, 4099, 3]
    kinds = [dtype, fa.DTYPE_F32, dtype]
    p0 = [(0.02 * rng.standard_normal(n)).astype(np.float32) for n in sizes]
    g0 = [(1e-3 * rng.standard_normal(n)).astype(np.float32) for n in sizes]

    def to_dev(x, k):
        return dev16(O.from_f32(k, x)) if k != fa.DTYPE_F32 else torch.from_numpy(x).cuda()

    def widen(t, k):
        return O.to_f32(k, host16(t)) if k != fa.DTYPE_F32 else t.cpu().numpy()

    # SGD (zeroes the gradient).
    P = [to_dev(x, k) for x, k in zip(p0, kinds)]
    G = [to_dev(x, k) for x, k in zip(g0, kinds)]
    mt = fa.MultiTensor(gpu_ctx, P, G, sizes=sizes, dtypes=kinds)
    mt.sgd(0.01)
    torch.cuda.synchronize()
    for t, g, x, gx, k in zip(P, G, p0, g0, kinds):
        w = widen(to_dev(x, k), k).copy()
        gg = widen(to_dev(gx, k), k).copy()
        O.sgd_(w, gg, 0.01)
        want = O.from_f32(k, w) if k != fa.DTYPE_F32 else w
        got = host16(t) if k != fa.DTYPE_F32 else t.cpu().numpy()
        assert np.array_equal(got, want)
        assert not np.any(widen(g, k))
    mt.close()
    # Adam, three steps.
    P = [to_dev(x, k) for x, k in zip(p0, kinds)]
    G = [to_dev(x, k) for x, k in zip(g0, kinds)]
    M = [torch.zeros(n, device="cuda") for n in sizes]
    V = [torch.zeros(n, device="cuda") for n in sizes]
    mt = fa.MultiTensor(gpu_ctx, P, G, M, V, sizes=sizes, dtypes=kinds)
    ref_p = [widen(to_dev(x, k), k).copy() for x, k in zip(p0, kinds)]
    ref_g = [widen(to_dev(x, k), k).copy() for x, k in zip(g0, kinds)]
    ref_m = [np.zeros(n, np.float32) for n in sizes]
    ref_v = [np.zeros(n, np.float32) for n in sizes]
    for step in (1, 2, 3):
        mt.adam(1e-3, 0.9, 0.999, 1e-8, step)
        # The device derives the scalars from the fp32 arguments.
        f32 = np.float32
        ss, inv = O.adam_scalars(f32(1e-3), f32(0.9), f32(0.999), step)
        for i, k in enumerate(kinds):
            O.adam_(ref_p[i], ref_g[i], ref_m[i], ref_v[i], f32(0.9), f32(0.999), f32(1e-8), ss,
                    inv)
            if k != fa.DTYPE_F32:  # the stored parameter is rounded each step
                ref_p[i] = O.to_f32(k, O.from_f32(k, ref_p[i]))
    torch.cuda.synchronize()
    for i, k in enumerate(kinds):
        assert np.array_equal(widen(P[i], k), ref_p[i])
        assert np.array_equal(M[i].cpu().numpy(), ref_m[i])
        assert np.array_equal(V[i].cpu().numpy(), ref_v[i])
    mt.close()
