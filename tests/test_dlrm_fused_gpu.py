"""GPU parity of the fused DLRM kernels (dlrm_fused.hip).  Every chain of
gp_mlp_out / gp_mlp_dtype_out shaped K0 -> 512 -> 256 -> 128 with K0 <= 32,
identity or ReLU after the first two layers, runs as one kernel whose
activations never leave the CU (the reference's
apps/dlrm_botmlp/pipelined/dlrm_botmlp_pl.cuh:79-173 runs the same tower as
one queue-chained kernel); a chain ending K -> 256 -> 1 (K 256, 512 or 1024,
the DLRM top MLP's tail with its click head, dlrm_topmlp_pl.cuh:185-224) runs
its last two layers as one kernel.

Checked against the CPU oracle at the fp16 I/O bar (max-abs 2e-2, rel-L2
5e-3; bf16: 8x) over every row, for input widths that fill one or two MFMA
k-blocks, widths that are not a multiple of 8 (element-wise input reads,
masked tails), ragged row counts (partial last tiles, several tiles per
workgroup), other activations and null biases.  Rows are independent and run
the same instruction stream wherever they sit, so the rows of a small call are
bit-identical to the same rows of a large one, and an input or output that is
not 16-byte aligned (routed through the workspace) gives bit-identical results.
"""
import numpy as np
import pytest
import torch

import gpipes
import oracle
from gpipes.synth import dlrm_params, normal_fp16, padded_uniform

pytestmark = pytest.mark.gpu

ACT = {"relu": oracle.ACT_RELU, "sigmoid": oracle.ACT_SIGMOID, "none": oracle.ACT_NONE,
       "gelu_tanh": oracle.ACT_GELU_TANH}
BF = torch.bfloat16


def f(t):
    return None if t is None else t.detach().float().cpu().numpy()


def to(ts, dev):
    return [None if t is None else t.to(dev) for t in ts]


def check(got, want, what, bf16=False):
    max_abs, rel = oracle.errors(got, want)
    print(f"[parity] {what}: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    tol_abs = oracle.BF16_MAX_ABS_TOL if bf16 else oracle.MAX_ABS_TOL
    tol_rel = oracle.BF16_REL_L2_TOL if bf16 else oracle.REL_L2_TOL
    assert max_abs <= tol_abs and rel <= tol_rel, (what, max_abs, rel)


def run(cuda, M, K0, acts=("relu",) * 3, seed=0, bias=True, dtype=torch.float16, x=None):
    widths = [K0, 512, 256, 128]
    ws, bs = dlrm_params(widths, seed=seed + K0, init="xavier")
    if not bias:
        bs = [None] * 3
    ws = [w.to(dtype) for w in ws]
    bs = [None if b is None else b.to(dtype) for b in bs]
    if x is None:
        x = normal_fp16(M, K0, seed=seed + M, dtype=dtype)
    y = gpipes.mlp_out(x.to(cuda), to(ws, cuda), to(bs, cuda), list(acts))
    want = oracle.mlp(f(x), [f(w) for w in ws], [f(b) for b in bs], [ACT[a] for a in acts])
    return y, want, x, ws, bs


@pytest.mark.parametrize("K0", [1, 8, 13, 16, 17, 24, 32])
@pytest.mark.parametrize("M", [1, 255, 257, 3000])
def test_dlrm_bottom_fused_vs_oracle(cuda, K0, M):
    print(f"[dlrm-fused] K0={K0} M={M}", flush=True)
    y, want, *_ = run(cuda, M, K0)
    assert y.shape == (M, 128)
    check(f(y), want, f"dlrm bottom K0={K0} M={M}")


@pytest.mark.parametrize("acts", [("none", "relu", "sigmoid"), ("relu", "none", "gelu_tanh"),
                                  ("none", "none", "none"), ("relu", "relu", "none")])
def test_dlrm_bottom_fused_activations(cuda, acts):
    print(f"[dlrm-fused] acts={acts}", flush=True)
    y, want, *_ = run(cuda, 1000, 16, acts=acts, seed=5)
    check(f(y), want, f"dlrm bottom acts={acts}")


def test_dlrm_bottom_fused_null_biases(cuda):
    y, want, *_ = run(cuda, 700, 13, bias=False, seed=9)
    check(f(y), want, "dlrm bottom without biases")


@pytest.mark.parametrize("K0", [13, 32])
def test_dlrm_bottom_fused_bf16(cuda, K0):
    print(f"[dlrm-fused] bf16 K0={K0}", flush=True)
    y, want, *_ = run(cuda, 3000, K0, dtype=BF, seed=3)
    assert y.dtype == BF
    check(f(y), want, f"dlrm bottom bf16 K0={K0}", bf16=True)


def test_dlrm_bottom_fused_rows_independent(cuda):
    """A ragged M with several tiles per workgroup (1,101 tiles of 256 rows
    over at most 256 workgroups): every row against the oracle, and rows of
    small calls (the first, a middle and the last partial tile) bit-identical
    to the same rows of the large call."""
    M = 256 * 1100 + 77
    print(f"[dlrm-fused] rows independent M={M}", flush=True)
    x = padded_uniform(M, 13, 16, seed=4)
    y, want, x, ws, bs = run(cuda, M, 16, x=x, seed=1)
    check(f(y), want, f"dlrm bottom all {M} rows")
    wd, bd = to(ws, cuda), to(bs, cuda)
    xd = x.to(cuda)
    for a, b in ((0, 300), (131000, 132000), (M - 77 - 256, M)):
        small = gpipes.mlp_out(xd[a:b].contiguous(), wd, bd, ["relu"] * 3)
        assert torch.equal(small.view(torch.int16), y[a:b].view(torch.int16)), (a, b)


def test_dlrm_bottom_fused_unaligned_bit_exact(cuda):
    """x and out at a 2-byte offset (not 16-byte aligned) go through the
    workspace: the result equals the aligned call bit for bit."""
    M, K0 = 999, 16
    y, want, x, ws, bs = run(cuda, M, K0, seed=7)
    wd, bd = to(ws, cuda), to(bs, cuda)
    xbuf = torch.zeros(M * K0 + 8, dtype=torch.float16, device=cuda)
    xu = xbuf[1:1 + M * K0].view(M, K0)
    xu.copy_(x.to(cuda))
    obuf = torch.zeros(M * 128 + 8, dtype=torch.float16, device=cuda)
    ou = obuf[1:1 + M * 128].view(M, 128)
    gpipes.mlp_out(xu, wd, bd, ["relu"] * 3, out=ou)
    torch.cuda.synchronize()
    assert torch.equal(ou.view(torch.int16), y.view(torch.int16))
    assert float(obuf[0]) == 0.0 and float(obuf[1 + M * 128]) == 0.0


def test_dlrm_bottom_generic_chain_beside_fused(cuda):
    """K0 = 33 is past the fused kernel's limit and runs as one GEMM launch
    per layer; both paths meet the bar against the oracle on the same rows."""
    for K0 in (32, 33):
        y, want, *_ = run(cuda, 2000, K0, seed=11)
        check(f(y), want, f"dlrm bottom K0={K0}")


def test_dlrm_bottom_fused_back_to_back_weights(cuda):
    """Consecutive calls with other weights re-pack the weight stream: each
    call meets the bar against its own oracle, on one stream and on a second
    stream (its own workspace)."""
    s2 = torch.cuda.Stream()
    for i in range(3):
        y, want, *_ = run(cuda, 513, 16, seed=20 + i)
        check(f(y), want, f"dlrm bottom back-to-back {i}")
    with torch.cuda.stream(s2):
        y, want, *_ = run(cuda, 513, 16, seed=30)
    torch.cuda.synchronize()
    check(f(y), want, "dlrm bottom second stream")


# ------------------------------------------------------------------ top MLP tail: K -> 256 -> 1
def run_tail(cuda, M, widths, acts, seed=0, bias=True, dtype=torch.float16, x=None):
    ws, bs = dlrm_params(widths, seed=seed + widths[0], init="xavier")
    if not bias:
        bs = [None] * len(ws)
    ws = [w.to(dtype) for w in ws]
    bs = [None if b is None else b.to(dtype) for b in bs]
    if x is None:
        x = normal_fp16(M, widths[0], seed=seed + M, dtype=dtype)
    y = gpipes.mlp_out(x.to(cuda), to(ws, cuda), to(bs, cuda), list(acts))
    want = oracle.mlp(f(x), [f(w) for w in ws], [f(b) for b in bs], [ACT[a] for a in acts])
    return y, want, x, ws, bs


@pytest.mark.parametrize("K", [256, 512, 1024])
@pytest.mark.parametrize("M", [1, 255, 257, 3000])
def test_dlrm_tail_fused_vs_oracle(cuda, K, M):
    """A chain ending K -> 256 -> 1 (K 256, 512, 1024) runs its last two layers
    as the fused tail kernel: here the whole chain is the tail."""
    print(f"[dlrm-tail] K={K} M={M}", flush=True)
    y, want, *_ = run_tail(cuda, M, [K, 256, 1], ["relu", "sigmoid"])
    assert y.shape == (M, 1)
    check(f(y), want, f"tail K={K} M={M}")


@pytest.mark.parametrize("acts", [("none", "none"), ("relu", "gelu_tanh"), ("none", "relu"), ("relu", "none")])
def test_dlrm_tail_fused_activations(cuda, acts):
    print(f"[dlrm-tail] acts={acts}", flush=True)
    y, want, *_ = run_tail(cuda, 1000, [512, 256, 1], acts, seed=4)
    check(f(y), want, f"tail acts={acts}")


def test_dlrm_tail_fused_null_biases(cuda):
    y, want, *_ = run_tail(cuda, 900, [512, 256, 1], ["relu", "sigmoid"], bias=False, seed=6)
    check(f(y), want, "tail without biases")


@pytest.mark.parametrize("dtype", [torch.float16, BF])
def test_dlrm_top_mlp_with_fused_tail(cuda, dtype):
    """The DLRM top MLP 480 -> 1024 -> 1024 -> 512 -> 256 -> 1: three GEMM
    launches, then the tail kernel reading the 512-wide activations from the
    workspace."""
    print(f"[dlrm-tail] top MLP {dtype}", flush=True)
    y, want, *_ = run_tail(cuda, 3000, [480, 1024, 1024, 512, 256, 1], ["relu"] * 4 + ["sigmoid"], seed=8,
                           dtype=dtype)
    assert y.dtype == dtype
    check(f(y), want, f"top MLP {dtype}", bf16=dtype == BF)


def test_dlrm_tail_fused_two_chunks_rows_independent(cuda):
    """M = 300,077: two row chunks (262,144 + 37,933; the weights are packed once,
    with the first), several tiles per workgroup and a partial last tile.  Every
    row against the oracle; rows of small calls bit-identical to the same rows
    of the large call."""
    M = 300077
    print(f"[dlrm-tail] two chunks M={M}", flush=True)
    y, want, x, ws, bs = run_tail(cuda, M, [512, 256, 1], ["relu", "sigmoid"], seed=10)
    check(f(y), want, f"tail all {M} rows")
    wd, bd, xd = to(ws, cuda), to(bs, cuda), x.to(cuda)
    for a, b in ((0, 300), (262000, 262400), (M - 77 - 256, M)):
        small = gpipes.mlp_out(xd[a:b].contiguous(), wd, bd, ["relu", "sigmoid"])
        assert torch.equal(small.view(torch.int16), y[a:b].view(torch.int16)), (a, b)


def test_dlrm_tail_fused_unaligned_bit_exact(cuda):
    """x at a 2-byte offset (copied into the workspace first) and out at a
    2-byte offset (written in place, one 2-byte store per row): the result
    equals the aligned call bit for bit."""
    M, K = 777, 512
    y, want, x, ws, bs = run_tail(cuda, M, [K, 256, 1], ["relu", "sigmoid"], seed=12)
    wd, bd = to(ws, cuda), to(bs, cuda)
    xbuf = torch.zeros(M * K + 8, dtype=torch.float16, device=cuda)
    xu = xbuf[1:1 + M * K].view(M, K)
    xu.copy_(x.to(cuda))
    obuf = torch.zeros(M + 8, dtype=torch.float16, device=cuda)
    ou = obuf[1:1 + M].view(M, 1)
    gpipes.mlp_out(xu, wd, bd, ["relu", "sigmoid"], out=ou)
    torch.cuda.synchronize()
    assert torch.equal(ou.view(torch.int16), y.view(torch.int16))
    assert float(obuf[0]) == 0.0 and float(obuf[1 + M]) == 0.0


def test_dlrm_fused_randomized_sweep(cuda):
    """Twenty seeded random cases per kernel: input width, row count (partial
    last tiles, one to several tiles per workgroup), activations, null biases
    and element type, each against the oracle over every row."""
    rng = np.random.default_rng(2024)
    hidden = ["none", "relu"]
    heads = ["none", "relu", "sigmoid", "gelu_tanh"]
    for i in range(20):
        K0 = int(rng.integers(1, 33))
        M = int(rng.integers(1, 70000))
        acts = (hidden[rng.integers(2)], hidden[rng.integers(2)], heads[rng.integers(4)])
        bias = bool(rng.integers(2))
        dtype = BF if rng.integers(4) == 0 else torch.float16
        print(f"[dlrm-fused] sweep {i}: K0={K0} M={M} acts={acts} bias={bias} {dtype}", flush=True)
        y, want, *_ = run(cuda, M, K0, acts=acts, seed=100 + i, bias=bias, dtype=dtype)
        check(f(y), want, f"sweep {i}", bf16=dtype == BF)
    for i in range(20):
        K = int(rng.choice([256, 512, 1024]))
        M = int(rng.integers(1, 70000))
        acts = (hidden[rng.integers(2)], heads[rng.integers(4)])
        bias = bool(rng.integers(2))
        dtype = BF if rng.integers(4) == 0 else torch.float16
        print(f"[dlrm-tail] sweep {i}: K={K} M={M} acts={acts} bias={bias} {dtype}", flush=True)
        y, want, *_ = run_tail(cuda, M, [K, 256, 1], acts, seed=200 + i, bias=bias, dtype=dtype)
        check(f(y), want, f"tail sweep {i}", bf16=dtype == BF)
