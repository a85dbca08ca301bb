"""HIP graph capture of the entry points that allocate nothing.

The fused MGN kernels (fp16 and bf16, with or without LayerNorm, the gather
front end) take their launch status word from a static device array and need
no workspace, so a caller may capture them into a graph (torch.cuda.CUDAGraph
drives hipStreamBeginCapture on its capture stream).  Every replay must equal
the eager call on the inputs the buffers hold at replay time, bit for bit;
the replays are interleaved with eager work, synchronisations and new input
values.  The queue-chained implementations (a new queue epoch per launch) and
the calls that use the per-stream workspace refuse capture with
GP_ERR_INVALID_ARG before enqueueing anything.
"""
import pytest
import torch

import gpipes
from gpipes.synth import bert_params, mgn_params, normal_fp16

pytestmark = pytest.mark.gpu


def to_dev(p, dev):
    return {k: (None if v is None else v.to(dev)) for k, v in p.items()}


def mgn_call(x, p, out, impl="fused"):
    gpipes.mgn_mlp_out(x, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"], p["gamma"], p["beta"], out,
                       impl=impl)


@pytest.mark.parametrize("K,ln,dtype", [(384, True, torch.float16), (256, True, torch.float16),
                                        (384, False, torch.float16), (384, True, torch.bfloat16)])
def test_fused_mgn_graph_replays_match_eager(cuda, K, ln, dtype):
    M = 20000
    p = to_dev(mgn_params(K, seed=K, layernorm=ln, affine_random=True, dtype=dtype), cuda)
    xs = [normal_fp16(M, K, seed=s, device=cuda, dtype=dtype) for s in (1, 2)]
    outs = [torch.empty((M, 128), dtype=dtype, device=cuda) for _ in range(2)]
    mgn_call(xs[0], p, outs[0])  # the first call sets up the device's status words outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        mgn_call(xs[0], p, outs[0])
        mgn_call(xs[1], p, outs[1])
    for r in range(4):
        # new inputs in place, eager work in between, then one replay
        xs[0].copy_(normal_fp16(M, K, seed=10 + r, device=cuda, dtype=dtype))
        xs[1].copy_(normal_fp16(M, K, seed=20 + r, device=cuda, dtype=dtype))
        want = [torch.empty_like(o) for o in outs]
        mgn_call(xs[0], p, want[0])
        mgn_call(xs[1], p, want[1])
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            assert torch.equal(o.view(torch.int16), w.view(torch.int16)), f"replay {r}"
    gpipes.pipeline_check()


def test_gather_graph_replays_match_eager(cuda):
    E, N = 30000, 5000
    p = to_dev(mgn_params(384, seed=3, affine_random=True), cuda)
    nf = normal_fp16(N, 128, seed=4, device=cuda)
    ef = normal_fp16(E, 128, seed=5, device=cuda)
    gen = torch.Generator().manual_seed(6)
    src = torch.randint(0, N, (E,), generator=gen).to(cuda)
    dst = torch.randint(0, N, (E,), generator=gen).to(cuda)
    out = torch.empty((E, 128), dtype=torch.float16, device=cuda)

    def call(o):
        gpipes.mgn_edge_gather_out(nf, ef, src, dst, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"],
                                   p["gamma"], p["beta"], o)

    call(out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(out)
    for r in range(3):
        nf.copy_(normal_fp16(N, 128, seed=30 + r, device=cuda))
        want = torch.empty_like(out)
        call(want)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {r}"


@pytest.mark.parametrize("impl", ["pipelined", "pipelined_split_ln"])
def test_queue_chained_refuses_capture(cuda, impl):
    M, K = 1000, 384
    p = to_dev(mgn_params(K, seed=7), cuda)
    x = normal_fp16(M, K, seed=8, device=cuda)
    out = torch.zeros((M, 128), dtype=torch.float16, device=cuda)
    mgn_call(x, p, out, impl=impl)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    err = None
    with torch.cuda.graph(g):
        try:
            mgn_call(x, p, out, impl=impl)
        except gpipes.GpipesError as e:
            err = e
    assert err is not None and err.code == -1 and "graph" in str(err)
    # the stream is usable afterwards, eagerly
    out2 = torch.zeros_like(out)
    mgn_call(x, p, out2, impl=impl)
    gpipes.pipeline_check()
    assert torch.equal(out, out2)


def test_workspace_call_refuses_capture(cuda):
    M, H, FF = 256, 128, 512
    p = to_dev(bert_params(H, FF, seed=9), cuda)
    x = normal_fp16(M, H, seed=10, device=cuda)
    out = torch.empty_like(x)

    def call():
        gpipes.bert_ffn_out(x, p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"], out)

    call()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    err = None
    with torch.cuda.graph(g):
        try:
            call()
        except gpipes.GpipesError as e:
            err = e
    assert err is not None and err.code == -1


def test_linear_stage_graph_replays_match_eager(cuda):
    """The whole-matrix GEMM stage (part-buffer prefetch) allocates nothing and
    sets its LDS limit once per device, so it can be captured too."""
    M, K = 5000, 384
    x = normal_fp16(M, K, seed=11, device=cuda)
    w = (normal_fp16(K, 128, seed=12, device=cuda).float() / 20).half()
    b = normal_fp16(1, 128, seed=13, device=cuda)[0]
    out = torch.empty((M, 128), dtype=torch.float16, device=cuda)
    gpipes.linear_out(x, w, b, act="gelu_tanh", out=out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gpipes.linear_out(x, w, b, act="gelu_tanh", out=out)
    for r in range(3):
        x.copy_(normal_fp16(M, K, seed=40 + r, device=cuda))
        want = gpipes.linear_out(x, w, b, act="gelu_tanh")
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {r}"


def test_nerf_noalloc_graph_replays_match_eager(cuda):
    """gp_nerf_full_out_noalloc under capture: the graph holds the weight-packing kernel and
    the fused NeRF kernel, both on the static scratch.  Between replays x, d and the
    weights change in place; every replay must equal the eager (workspace) call on the new
    contents bit for bit, so the replay re-packs the weights it finds."""
    from gpipes.synth import nerf_inputs, nerf_params
    M = 5000
    ws, bs = nerf_params(64, 27, 1, 3, seed=40, device=cuda)
    x, d = nerf_inputs(M, seed=41, device=cuda)
    out_r = torch.empty((M, 1), dtype=torch.float16, device=cuda)
    out_rgb = torch.empty((M, 3), dtype=torch.float16, device=cuda)
    wb = [t for pair in zip(ws, bs) for t in pair]
    gpipes.nerf_full_out_noalloc(x, d, *wb, out_r, out_rgb, rgb_act="sigmoid")  # first call: symbol lookup
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gpipes.nerf_full_out_noalloc(x, d, *wb, out_r, out_rgb, rgb_act="sigmoid")
    for r in range(3):
        ws2, bs2 = nerf_params(64, 27, 1, 3, seed=50 + r, device=cuda)
        for t, n in zip(ws + bs, ws2 + bs2):
            t.copy_(n)
        x2, d2 = nerf_inputs(M, seed=60 + r, device=cuda)
        x.copy_(x2)
        d.copy_(d2)
        want_r, want_rgb = gpipes.nerf_full(x, d, *wb, rgb_act="sigmoid")
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_r.view(torch.int16), want_r.view(torch.int16)), f"replay {r} density"
        assert torch.equal(out_rgb.view(torch.int16), want_rgb.view(torch.int16)), f"replay {r} colour"
