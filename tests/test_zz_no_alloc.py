"""fg_bias_grad_noalloc -- the bias-gradient reduction that allocates nothing
(its partial sums live in the library's fixed per-GPU scratch array) --
against fg_bias_grad, the entry point it varies, through the C ABI.

The two run the same launches, so their outputs are compared bit for bit
(integer-exact bar for the same arithmetic in the same order).  Two calls in
a row, the second on a smaller input, show that what the first call left in
the shared scratch does not reach the second's result."""
import numpy as np
import pytest

from conftest import normwise_rel

pytestmark = pytest.mark.gpu

f32 = np.float32


def _call(name, *args):
    from ferrograd_amd._lib import call
    call(name, *args)


def _bias_grads(ctx, dtype, dZ_host, accumulate, init):
    """(noalloc result, fg_bias_grad result) as host arrays of dZ's dtype."""
    import torch
    M, N = dZ_host.shape
    tdt = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}[dtype]
    dZ = torch.from_numpy(dZ_host).cuda().to(tdt)
    outs = []
    for name in ("fg_bias_grad_noalloc", "fg_bias_grad"):
        db = torch.from_numpy(init).cuda().to(tdt)
        _call(name, ctx.handle, dtype, M, N, dZ.data_ptr(), N, db.data_ptr(), int(accumulate))
        outs.append(db)
    torch.cuda.synchronize()
    return [o.float().cpu().numpy() for o in outs], dZ.float().cpu().numpy()


@pytest.mark.parametrize("dtype", [0, 1, 2], ids=["f32", "f16", "bf16"])
def test_noalloc_bias_grad_matches_bias_grad_twice(gpu_ctx, dtype):
    rng = np.random.default_rng(11 + dtype)
    for (M, N), acc in (((2048, 4096), False), ((64, 10), True)):
        print(f"noalloc bias_grad dtype={dtype} M={M} N={N} accumulate={acc}", flush=True)
        dZ = rng.standard_normal((M, N)).astype(f32)
        init = rng.standard_normal(N).astype(f32)
        (got, ref), dZ_used = _bias_grads(gpu_ctx, dtype, dZ, acc, init)
        assert np.array_equal(got, ref), (M, N)
        # And the value itself: float64 column sums (of the stored dZ).
        exp = dZ_used.astype(np.float64).sum(axis=0)
        if acc:
            exp = exp + init.astype(np.float64)
        tol = 1e-5 if dtype == 0 else 1e-2
        assert normwise_rel(got, exp) < tol


def test_noalloc_bias_grad_rejects_too_many_columns(gpu_ctx):
    """N beyond the fixed scratch is refused before any launch."""
    from ferrograd_amd._lib import FgError
    N = (1 << 20) + 1
    with pytest.raises(FgError) as e:
        # Device pointers are never touched: the size check comes first.
        _call("fg_bias_grad_noalloc", gpu_ctx.handle, 0, 64, N, 256, N, 256, 0)
    assert e.value.code == 9  # FG_ERR_OUT_OF_BOUNDS
    assert "scratch" in str(e.value)


def test_noalloc_bias_grad_under_graph_capture_on_fresh_context(gpu_ctx):
    """The case the entry point is for: a context that has never allocated a
    workspace calls fg_bias_grad_noalloc inside a hipGraph capture (global
    capture mode, so any allocation or synchronising call in the capture
    fails it).  The graph is replayed twice, with eager work and a
    synchronisation between the replays, and each result is compared bit for
    bit with fg_bias_grad run afterwards (which then grows the workspace)."""
    import torch

    import ferrograd_amd as fa

    M, N = 2048, 4096
    rng = np.random.default_rng(23)
    dZ = torch.from_numpy(rng.standard_normal((M, N)).astype(f32)).cuda()
    db = torch.empty(N, device="cuda")
    s = torch.cuda.Stream()
    fresh = fa.Context(0, s.cuda_stream)
    try:
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        print("noalloc under capture: capturing", flush=True)
        with torch.cuda.graph(g, stream=s, capture_error_mode="global"):
            _call("fg_bias_grad_noalloc", fresh.handle, 0, M, N, dZ.data_ptr(), N,
                  db.data_ptr(), 0)
        ref = torch.empty(N, device="cuda")
        for rep in range(2):
            db.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            got = db.cpu().numpy().copy()
            with torch.cuda.stream(s):
                _call("fg_bias_grad", fresh.handle, 0, M, N, dZ.data_ptr(), N,
                      ref.data_ptr(), 0)
            torch.cuda.synchronize()
            print(f"noalloc under capture: replay {rep} compared", flush=True)
            assert np.array_equal(got, ref.cpu().numpy()), rep
            dZ.mul_(-0.5)  # eager work between replays; the next replay reads it
    finally:
        fresh.sync()
        fresh.close()
