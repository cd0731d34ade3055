"""bpat files from and into device memory, and plan checkpoints (inputs plus
Adam state), through the C ABI."""
import math

import numpy as np
import pytest

import ferrograd_amd as fa
from ferrograd_amd import io as fio

pytestmark = pytest.mark.gpu

H = fio.BpatHeader


@pytest.fixture(scope="module")
def gctx(gpu_ctx):
    from ferrograd_amd.graph import GpuContext
    return GpuContext(gpu_ctx)


@pytest.mark.parametrize("header", [H.BpatV1, H.BpatV2f32, H.BpatV2f16, H.BpatV2bf16])
def test_device_tensors_round_trip(gctx, tmp_path, header):
    import torch
    rng = np.random.default_rng(5)
    host = [rng.standard_normal((33, 17)).astype(np.float32),
            rng.standard_normal((1000,)).astype(np.float32)]
    dev = [torch.from_numpy(a).cuda() for a in host]
    dev.append(torch.from_numpy(host[0]).cuda().to(torch.bfloat16))
    p = tmp_path / "d.bpat"
    fio.save_tensors(p, gctx, dev, header)
    loaded = fio.load_tensors(p, gctx)
    assert [t.shape for t in loaded] == [(33, 17), (1000,), (33, 17)]
    with fio.BpatFile(p) as f:
        ref = [f.read_f32(i) for i in range(3)]
    for t, r in zip(loaded, ref):
        got = gctx.download(t)
        if header == H.BpatV2f16:
            got = got.astype(np.float32)
        elif header == H.BpatV2bf16:
            got = (got.astype(np.uint32) << 16).view(np.float32)
        assert np.array_equal(got.reshape(r.shape), r)
    # fp32 files keep fp32 data exactly; the bf16 tensor round-trips exactly
    # through every format (its values are bf16, which all of them hold).
    if header in (H.BpatV1, H.BpatV2f32):
        assert np.array_equal(ref[0], host[0]) and np.array_equal(ref[1], host[1])
    want_bf16 = dev[2].float().cpu().numpy()
    if header != H.BpatV2f16:
        assert np.array_equal(ref[2], want_bf16)
    # Upload into existing device memory as another element type.
    out = torch.empty(1000, device="cuda", dtype=torch.float16)
    with fio.BpatFile(p) as f:
        f.upload(gctx, 1, out, fa.DTYPE_F16)
    assert np.array_equal(out.cpu().numpy(), ref[1].astype(np.float16))


def _mlp(gctx, seed):
    from ferrograd_amd import graph as G
    dims, B = [64, 96, 10], 32
    graph, meta = G.Graph(G.CROSS_ENTROPY, G.Optim.adam().lower), G.Metadata.new()
    fb = meta.new_field()
    fd = [meta.new_field() for _ in dims]
    with graph.define_ops() as ops:
        h = ops.input([fb, fd[0]], trainable=False)
        for l in range(2):
            W = ops.input([fd[l], fd[l + 1]])
            b = ops.input([fd[l + 1]])
            z = ops.bias_add(ops.matmul(h, W), b)
            h = ops.gelu(z) if l == 0 else z
        ops.softmax(h)
    mb = [G.f32_bits(1e-2), B] + dims
    st = gctx.alloc_tensors(graph, graph.compute_saved_nodes(), mb)
    X = fa.rng_normal(3, 0, (B, dims[0]))
    y = fa.rng_int(3, 1, (B,), dims[-1])
    ins = [gctx.init_tensor_f32(X.shape, X)]
    for l in range(2):
        bound = math.sqrt(6 / dims[l])
        W = fa.rng_uniform(seed, 10 + l, (dims[l], dims[l + 1]), -bound, bound)
        ins += [gctx.init_tensor_f32(W.shape, W), gctx.init_tensor_f32((dims[l + 1],),
                                                                       np.zeros(dims[l + 1]))]
    sch = gctx.schedule(graph.lower(meta), mb, ins, st)
    return sch, ins, gctx.new_onehot_init(y)


def _step(gctx, sch, tgt):
    gctx.dispatch_forward(sch)
    gctx.dispatch_loss(sch, tgt)
    gctx.dispatch_backward(sch)
    gctx.dispatch_optim(sch)
    gctx.sync()


def test_plan_checkpoint_resumes_bit_exactly(gctx, tmp_path):
    """Two Adam steps, checkpoint, a third step; a fresh plan (other initial
    weights) that loads the checkpoint and takes one step ends bit-identical
    (parameters, and the step count drives the bias corrections)."""
    sch_a, ins_a, tgt_a = _mlp(gctx, 4)
    _step(gctx, sch_a, tgt_a)
    _step(gctx, sch_a, tgt_a)
    p = tmp_path / "ckpt.bpat"
    fio.save_checkpoint(sch_a, p)
    with fio.BpatFile(p) as f:
        # 5 inputs, m and v of the 4 updated ones, the step count.
        assert f.count == 5 + 8 + 1
        assert float(f.read_f32(f.count - 1)[0]) == 2.0
    _step(gctx, sch_a, tgt_a)
    sch_b, ins_b, tgt_b = _mlp(gctx, 9)
    fio.load_checkpoint(sch_b, p)
    _step(gctx, sch_b, tgt_b)
    for ta, tb in zip(ins_a, ins_b):
        assert np.array_equal(gctx.download(ta), gctx.download(tb))
    # A checkpoint of another graph is rejected.
    q = tmp_path / "other.bpat"
    fio.save_tensors(q, gctx, [ins_a[0]], H.BpatV2f32)
    with pytest.raises(fa.FgError):
        fio.load_checkpoint(sch_b, q)
