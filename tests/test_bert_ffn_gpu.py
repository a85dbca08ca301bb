"""GPU parity of the wide GEMM stage (gp_gemm_out) and the BERT FFN block
(gp_bert_ffn_out): LayerNorm(Linear2(act(Linear1(x))) + x).

Checked against the golden fixtures (torch.nn modules in float64) and the CPU
oracle at the fp16 I/O bar (max-abs 2e-2, relative-L2 5e-3).  At the full
BERT-large size (M = 65,536) the oracle checks every row, and two
size-independent properties are asserted beside it: every row is computed independently,
so the rows of a small batch are bit-identical to the same rows inside a large
(chunked) batch; and with gamma = 1, beta = 0 every output row has mean 0 and
variance var / (var + eps) of its pre-LayerNorm row (~1).
"""
import numpy as np
import pytest
import torch

import gpipes
import oracle
from conftest import load_golden
from gpipes.synth import bert_params, normal_fp16

pytestmark = pytest.mark.gpu

ACT_ID = {"relu": oracle.ACT_RELU, "gelu_tanh": oracle.ACT_GELU_TANH, "none": oracle.ACT_NONE,
          "sigmoid": oracle.ACT_SIGMOID}


def assert_parity(got, want, what):
    max_abs, rel = oracle.errors(got, want)
    print(f"[parity] {what}: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= oracle.MAX_ABS_TOL and rel <= oracle.REL_L2_TOL, (what, max_abs, rel)


def f(t):
    return None if t is None else t.detach().float().cpu().numpy()


def dev(p, cuda):
    return {k: (None if v is None else v.to(cuda)) for k, v in p.items()}


def ffn(x, p, act, eps):
    return gpipes.bert_ffn(x, p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"], eps=eps, act=act)


def oracle_ffn(x, p, act, eps):
    return oracle.bert_ffn(f(x), f(p["w1"]), f(p["b1"]), f(p["w2"]), f(p["b2"]), f(p["gamma"]), f(p["beta"]),
                           act=ACT_ID[act], eps=eps)


# ------------------------------------------------------------------ golden fixtures
@pytest.mark.parametrize("name", ["bert_ffn_relu.npz", "bert_ffn_gelu.npz"])
@pytest.mark.parametrize("impl", ["fused", "pipelined"])
def test_bert_ffn_golden(cuda, name, impl):
    z = load_golden(name)
    p = {k: torch.from_numpy(z[k]).to(cuda) for k in ("w1", "b1", "w2", "b2", "gamma", "beta")}
    if impl == "pipelined" and tuple(p["w1"].shape) != (128, 512):
        pytest.skip("the pipelined layout is built for the app's shape H 128, FF 512")
    y = gpipes.bert_ffn(torch.from_numpy(z["x"]).to(cuda), p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"],
                        eps=float(z["eps"]), act=str(z["act"]), impl=impl)
    if impl == "pipelined":
        gpipes.pipeline_check()
    assert_parity(f(y), z["expected"], f"golden {name} {impl}")


def test_bert_ffn_reference_signature(cuda):
    """bert_ffn(x, w1, b1, w2, b2, ga, be) with the reference app's defaults
    (apps/bert_ffn/pipelined/val.py:8-22: M = 64 x 512, H 128, FF 512, ReLU)."""
    M = 64 * 512
    p = dev(bert_params(128, 512, seed=3, init="torch"), cuda)
    x = normal_fp16(M, 128, seed=4, device=cuda)
    y = gpipes.bert_ffn(x, p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"])
    assert_parity(f(y), oracle_ffn(x, p, "relu", 1e-5), "reference app shape")


# ------------------------------------------------------------------ shapes vs oracle
@pytest.mark.parametrize("M,H,FF,act", [
    (1, 128, 512, "relu"), (300, 128, 512, "relu"), (257, 256, 1024, "gelu_tanh"), (129, 512, 2048, "gelu_tanh"),
    (1000, 1024, 4096, "gelu_tanh"), (77, 1024, 128, "relu"), (513, 128, 384, "gelu_tanh"),
])
def test_bert_ffn_vs_oracle(cuda, M, H, FF, act):
    p = dev(bert_params(H, FF, seed=M + H, init="bert", affine_random=True), cuda)
    x = normal_fp16(M, H, seed=M, device=cuda)
    eps = 1e-12 if act == "gelu_tanh" else 1e-5
    assert_parity(f(ffn(x, p, act, eps)), oracle_ffn(x, p, act, eps), f"bert_ffn M={M} H={H} FF={FF} {act}")


def test_bert_ffn_no_affine_no_bias(cuda):
    M, H, FF = 200, 256, 512
    p = dev(bert_params(H, FF, seed=5, init="torch"), cuda)
    x = normal_fp16(M, H, seed=6, device=cuda)
    y = gpipes.bert_ffn(x, p["w1"], None, p["w2"], None, None, None, eps=1e-12, act="gelu_tanh")
    want = oracle.bert_ffn(f(x), f(p["w1"]), None, f(p["w2"]), None, None, None, act=oracle.ACT_GELU_TANH,
                           eps=1e-12)
    assert_parity(f(y), want, "no biases, no affine")


# ------------------------------------------------------------------ LayerNorm in GEMM2's epilogue
@pytest.mark.parametrize("M,H,FF", [(300, 128, 512), (257, 256, 1024), (1000, 512, 2048), (20000, 1024, 4096),
                                    (70000, 1024, 128), (100000, 512, 256)])
def test_bert_ffn_ln_epilogue_matches_separate_launches(cuda, M, H, FF):
    """gp_bert_ffn_out computes the LayerNorm in GEMM2's epilogue: within a wave
    at H = 128, from per-wave partial statistics exchanged between waves and
    workgroups above (M = 20,000 at H = 1024 is two row chunks, two launches of
    one exchange epoch; M = 70,000 at H = 1024, FF = 128 runs a 65,536-row chunk
    as four rounds of 256 tiles in one launch, then a partial round; M = 100,000
    at H = 512 four rounds, the last one partial).  Against GEMM2 + residual written out and the
    LayerNorm launch reading it back, the pre-LayerNorm rows are the same fp16
    values and only the summation order of the statistics differs, so every
    output agrees to one fp16 rounding step and almost all bit for bit.  The
    step has an absolute floor of 2^-18 (3.8e-6): where gamma * t + beta
    cancels to about 1e-6 (fp16 subnormals, 6e-8 apart), the fp32 statistics'
    relative difference of order 1e-7, times |gamma * t| (a few units), moves
    the result by a few subnormal steps, up to about 1e-6."""
    print(f"[ln-epilogue] M={M} H={H} FF={FF}", flush=True)
    p = dev(bert_params(H, FF, seed=H, init="bert", affine_random=True), cuda)
    x = normal_fp16(M, H, seed=7, device=cuda)
    y = ffn(x, p, "gelu_tanh", 1e-12)
    h = gpipes.gemm_out(x, p["w1"], p["b1"], act="gelu_tanh")
    pre = gpipes.gemm_out(h, p["w2"], p["b2"], r=x)
    sep = gpipes.layer_norm_out(pre, p["gamma"], p["beta"], eps=1e-12)
    gpipes.pipeline_check()
    yf, sf = y.float(), sep.float()
    step = torch.maximum(yf.abs(), sf.abs()) * 2.0 ** -10 + 2.0 ** -18
    assert bool(((yf - sf).abs() <= step).all()), float((yf - sf).abs().max())
    same = (y.view(torch.int16) == sep.view(torch.int16)).float().mean().item()
    print(f"[ln-epilogue] bit-identical fraction {same:.5f}", flush=True)
    assert same >= 0.99
    rows = np.r_[0:min(M, 64), max(0, M - 64):M]
    assert_parity(f(y)[rows], oracle_ffn(x[rows], p, "gelu_tanh", 1e-12), f"LN epilogue M={M} H={H}")


def test_bert_ffn_ln_exchange_reused_across_shapes(cuda):
    """The exchange area of the LayerNorm epilogue is one per stream and is reused
    by calls of any shape: a call with fewer row blocks writes its partial
    statistics, then calls with more row blocks and another width must still
    find their counters clean (a regression test: with the statistics placed
    right after the launch's own counters, the second call's counters held the
    first call's statistics and its waits ran out)."""
    H, FF = 1024, 1024
    p = dev(bert_params(H, FF, seed=11, init="bert", affine_random=True), cuda)
    p2 = dev(bert_params(256, 512, seed=12, init="bert", affine_random=True), cuda)
    for M, q, width in [(77, p, H), (1000, p, H), (3000, p2, 256), (600, p, H), (1000, p, H)]:
        print(f"[ln-exchange] M={M} H={width}", flush=True)
        x = normal_fp16(M, width, seed=M, device=cuda)
        y = ffn(x, q, "gelu_tanh", 1e-12)
        gpipes.pipeline_check()
        rows = np.r_[0:min(M, 40), max(0, M - 40):M]
        assert_parity(f(y)[rows], oracle_ffn(x[rows], q, "gelu_tanh", 1e-12), f"reused exchange M={M} H={width}")


def test_bert_ffn_h128_tile_heights_agree(cuda):
    """At H = 128 a launch with fewer than 256 rows per CU runs its GEMM2 +
    LayerNorm on 128-row tiles, a larger one on 256-row tiles: the same
    products in the same order per row, so the rows of a small call equal the
    same rows of a large one bit for bit (both against the oracle too)."""
    M = 80000
    p = dev(bert_params(128, 512, seed=13, init="torch", affine_random=True), cuda)
    x = normal_fp16(M, 128, seed=14, device=cuda)
    big = ffn(x, p, "relu", 1e-5)
    for r0, n in ((0, 300), (40000, 5000), (M - 1000, 1000)):
        small = ffn(x[r0:r0 + n].contiguous(), p, "relu", 1e-5)
        assert torch.equal(small.view(torch.int16), big[r0:r0 + n].view(torch.int16)), (r0, n)
    rows = np.r_[0:100, 40000:40100, M - 100:M]
    assert_parity(f(big)[rows], oracle_ffn(x[rows], p, "relu", 1e-5), "H 128, 256-row tiles")


# ------------------------------------------------------------------ full size (config 2)
def test_bert_large_full_size(cuda):
    """M = 65,536 (128 x 512 tokens), H 1024, FF 4096, GELU(tanh), eps 1e-12: four
    16,384-row chunks.  Oracle on every row (about 2 s on the box's cores), bit
    identity of a small batch with the same rows of the large one, and the
    LayerNorm row statistics."""
    M, H, FF = 65536, 1024, 4096
    p = dev(bert_params(H, FF, seed=0, init="bert"), cuda)
    x = normal_fp16(M, H, seed=0, device=cuda)
    y = ffn(x, p, "gelu_tanh", 1e-12)
    torch.cuda.synchronize()
    assert_parity(f(y), oracle_ffn(x, p, "gelu_tanh", 1e-12), f"BERT-large all {M} rows")
    small = ffn(x[:1000].contiguous(), p, "gelu_tanh", 1e-12)
    assert torch.equal(small.view(torch.int16), y[:1000].view(torch.int16))
    tail = ffn(x[16000:17000].contiguous(), p, "gelu_tanh", 1e-12)  # crosses a chunk edge in the big batch
    assert torch.equal(tail.view(torch.int16), y[16000:17000].view(torch.int16))
    yf = y.float()
    assert torch.isfinite(yf).all()
    assert yf.mean(dim=1).abs().max().item() < 1e-2
    assert (yf.var(dim=1, unbiased=False) - 1).abs().max().item() < 2e-2


# ------------------------------------------------------------------ wide GEMM stage
@pytest.mark.parametrize("M,N,K", [(1, 128, 64), (255, 256, 128), (257, 384, 1024), (1000, 4096, 1024),
                                   (513, 1024, 4096), (64, 128, 4096)])
@pytest.mark.parametrize("act", ["none", "relu", "gelu_tanh", "sigmoid"])
def test_gemm_vs_oracle(cuda, M, N, K, act):
    g = torch.Generator().manual_seed(M * 7 + N + K)
    x = torch.randn((M, K), generator=g).to(torch.float16)
    w = (torch.randn((K, N), generator=g) / np.sqrt(K)).to(torch.float16)
    b = (torch.randn((N,), generator=g) * 0.5).to(torch.float16)
    y = gpipes.gemm_out(x.to(cuda), w.to(cuda), b.to(cuda), act=act)
    assert_parity(f(y), oracle.linear(f(x), f(w), f(b), ACT_ID[act]), f"gemm M={M} N={N} K={K} {act}")


@pytest.mark.parametrize("M,N,K", [(300, 128, 512), (1000, 1024, 4096)])
def test_gemm_residual(cuda, M, N, K):
    g = torch.Generator().manual_seed(M + N)
    x = torch.randn((M, K), generator=g).to(torch.float16)
    w = (torch.randn((K, N), generator=g) / np.sqrt(K)).to(torch.float16)
    b = (torch.randn((N,), generator=g) * 0.5).to(torch.float16)
    r = torch.randn((M, N), generator=g).to(torch.float16)
    y = gpipes.gemm_out(x.to(cuda), w.to(cuda), b.to(cuda), r.to(cuda))
    assert_parity(f(y), oracle.linear(f(x), f(w), f(b)) + f(r), f"gemm+residual M={M} N={N} K={K}")
    y0 = gpipes.gemm_out(x.to(cuda), w.to(cuda), None, r.to(cuda))
    assert_parity(f(y0), oracle.linear(f(x), f(w), None) + f(r), f"gemm+residual no bias M={M}")


def test_gemm_weight_paths_agree(cuda):
    """Below 8e10 FLOP per call the GEMM reads the weights in their own [K, N]
    layout (transposing LDS reads); above, it reads a transposed copy.  The
    two compute the same products in the same order: a call above the limit
    and the same rows in calls below it are bit-identical, and both match the
    oracle on sampled rows."""
    M, N, K = 16384, 2048, 1280  # 2 M N K = 8.6e10: the transposed copy
    g = torch.Generator().manual_seed(17)
    x = torch.randn((M, K), generator=g).to(torch.float16).to(cuda)
    w = (torch.randn((K, N), generator=g) / np.sqrt(K)).to(torch.float16).to(cuda)
    b = (torch.randn((N,), generator=g) * 0.5).to(torch.float16).to(cuda)
    y = gpipes.gemm_out(x, w, b, act="gelu_tanh")
    parts = torch.cat([gpipes.gemm_out(x[r:r + 2048].contiguous(), w, b, act="gelu_tanh") for r in range(0, M, 2048)])
    assert torch.equal(y.view(torch.int16), parts.view(torch.int16))
    rows = np.r_[0:32, 8000:8032, M - 32:M]
    xs = f(x[torch.from_numpy(rows).to(cuda)])
    assert_parity(f(y[torch.from_numpy(rows).to(cuda)]), oracle.linear(xs, f(w), f(b), ACT_ID["gelu_tanh"]),
                  "gemm transposed-copy path, sampled rows")


def test_gemm_identity_weight_is_exact(cuda):
    """x . I (+ 0) passes every fp16 value through the fp32 accumulator unchanged."""
    M, K = 700, 256
    x = normal_fp16(M, K, seed=9, device=cuda)
    x = torch.where(x.abs() < 2.0 ** -14, torch.zeros_like(x), x)  # no fp16 subnormals
    eye = torch.eye(K, dtype=torch.float16, device=cuda)
    y = gpipes.gemm_out(x, eye)
    assert torch.equal(y.view(torch.int16), x.view(torch.int16))
    # a column permutation is exact as well: catches a transposed or shuffled operand
    perm = torch.randperm(K, generator=torch.Generator().manual_seed(1)).to(cuda)
    y = gpipes.gemm_out(x, eye[:, perm].contiguous())
    assert torch.equal(y.view(torch.int16), x[:, perm].contiguous().view(torch.int16))


# ------------------------------------------------------------------ the reference app's queue-chained layout
@pytest.mark.parametrize("act", ["relu", "gelu_tanh"])
@pytest.mark.parametrize("M", [1, 127, 129, 1000, 64 * 512, 100003])
def test_bert_ffn_pipelined_vs_oracle(cuda, act, M):
    """impl="pipelined" (gp_bert_ffn_impl_out): the app's layout of
    apps/bert_ffn/pipelined/bert_ffn_pl.cuh:79-162 at its shape (H 128, FF 512),
    four W1 column slices feeding two W2 + residual + LayerNorm workers through
    ring queues, against the oracle over every row; partial last tiles (any M)
    travel as the queues' row counts."""
    print(f"[bert-ffn-pipelined] act={act} M={M}", flush=True)
    p = dev(bert_params(128, 512, seed=M, init="torch", affine_random=True), cuda)
    x = normal_fp16(M, 128, seed=M + 1, device=cuda)
    y = gpipes.bert_ffn(x, p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"], eps=1e-5, act=act,
                        impl="pipelined")
    gpipes.pipeline_check()
    assert_parity(f(y), oracle_ffn(x, p, act, 1e-5), f"pipelined {act} M={M}")


def test_bert_ffn_pipelined_null_params(cuda):
    """No biases, no affine (gamma 1, beta 0), in the queue-chained layout."""
    M = 1500
    p = dev(bert_params(128, 512, seed=3, init="torch"), cuda)
    x = normal_fp16(M, 128, seed=4, device=cuda)
    y = gpipes.bert_ffn(x, p["w1"], None, p["w2"], None, None, None, eps=1e-5, act="relu", impl="pipelined")
    gpipes.pipeline_check()
    want = oracle.bert_ffn(f(x), f(p["w1"]), None, f(p["w2"]), None, None, None, act=oracle.ACT_RELU, eps=1e-5)
    assert_parity(f(y), want, "pipelined without biases or affine")


def test_bert_ffn_pipelined_deterministic_and_agrees_with_fused(cuda):
    """Two calls, and a call on a second stream, are bit-identical (each tile's
    arithmetic does not depend on which pipeline ran it); the fused (GEMM) form
    sums in another order and agrees at the fp16 bar."""
    M = 64 * 512
    p = dev(bert_params(128, 512, seed=8, init="torch", affine_random=True), cuda)
    x = normal_fp16(M, 128, seed=9, device=cuda)
    args = (x, p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"])
    a = gpipes.bert_ffn(*args, eps=1e-5, act="relu", impl="pipelined")
    b = gpipes.bert_ffn(*args, eps=1e-5, act="relu", impl="pipelined")
    s2 = torch.cuda.Stream()
    with torch.cuda.stream(s2):
        c = gpipes.bert_ffn(*args, eps=1e-5, act="relu", impl="pipelined")
        gpipes.pipeline_check()
    torch.cuda.synchronize()
    gpipes.pipeline_check()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(a.view(torch.int16), c.view(torch.int16))
    fused = gpipes.bert_ffn(*args, eps=1e-5, act="relu")
    assert_parity(f(a), f(fused).astype(np.float64), "pipelined vs fused")


def test_bert_ffn_pipelined_rejects_other_shapes(cuda):
    p = dev(bert_params(256, 1024, seed=1, init="torch"), cuda)
    x = normal_fp16(300, 256, seed=2, device=cuda)
    with pytest.raises(gpipes.GpipesError) as ei:
        gpipes.bert_ffn(x, p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"], impl="pipelined")
    assert ei.value.code == -2


def test_bert_ffn_pipelined_refuses_capture(cuda):
    """The queue-chained launch takes a new queue epoch per call, which a graph
    replay would repeat: under capture it fails with GP_ERR_INVALID_ARG and the
    stream stays usable."""
    p = dev(bert_params(128, 512, seed=5, init="torch"), cuda)
    x = normal_fp16(512, 128, seed=6, device=cuda)
    out = torch.zeros_like(x)
    args = (x, p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"], out)
    gpipes.bert_ffn_out(*args, impl="pipelined")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    err = None
    with torch.cuda.graph(g):
        try:
            gpipes.bert_ffn_out(*args, impl="pipelined")
        except gpipes.GpipesError as e:
            err = e
    assert err is not None and err.code == -1 and "graph" in str(err)
    out2 = torch.zeros_like(out)
    gpipes.bert_ffn_out(*args[:-1], out2, impl="pipelined")
    gpipes.pipeline_check()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))
