"""GPU parity of the MGN MLP kernels against the CPU oracle (oracle/oracle.c).

Bar (fp16 I/O, fp32 accumulate): max-abs <= 2e-2 and relative-L2 <= 5e-3
against the fp32 oracle on identical fp16-rounded inputs, over every row up to
the full headline size.  Size-independent properties are checked beside it:
permutation equivariance (bit-exact), per-row LayerNorm moments, determinism,
and untouched memory past the output.
"""
import numpy as np
import pytest
import torch

import gpipes
import oracle
from gpipes.synth import mgn_params, normal_fp16
from conftest import load_golden

pytestmark = pytest.mark.gpu

TOL = dict(max_abs=oracle.MAX_ABS_TOL, rel=oracle.REL_L2_TOL)


def to_dev(p, dev):
    return {k: (None if v is None else v.to(dev)) for k, v in p.items()}


def run_gpu(x, p, impl="fused", eps=1e-5):
    return gpipes.mgn_mlp(x, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"], p["gamma"], p["beta"],
                          eps=eps, impl=impl)


def run_oracle(x16, p, eps=1e-5):
    f = lambda t: None if t is None else t.detach().cpu().float().numpy()  # noqa: E731
    return oracle.mgn_mlp(f(x16), f(p["w1"]), f(p["b1"]), f(p["w2"]), f(p["b2"]), f(p["w3"]), f(p["b3"]),
                          f(p["gamma"]), f(p["beta"]), eps=eps)


def assert_parity(got, want, what=""):
    max_abs, rel = oracle.errors(got, want)
    print(f"[parity] {what}: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= TOL["max_abs"] and rel <= TOL["rel"], (what, max_abs, rel)


GOLDEN = [("mgn_edge_ln.npz", 384), ("mgn_edge_ln_affine.npz", 384), ("mgn_edge_linears.npz", 384),
          ("mgn_node_ln.npz", 256)]


@pytest.mark.parametrize("name,K", GOLDEN)
@pytest.mark.parametrize("M", [1, 7, 64, 65, 256])
def test_golden_fixtures(cuda, name, K, M):
    z = load_golden(name)
    p = {k: torch.from_numpy(z[k]).to(cuda) if k in z else None
         for k in ("w1", "b1", "w2", "b2", "w3", "b3", "gamma", "beta")}
    x = torch.from_numpy(z["x"][:M]).to(cuda)
    got = run_gpu(x, p, eps=float(z["eps"])).float().cpu().numpy()
    assert_parity(got, z["expected"][:M], f"{name} M={M}")


@pytest.mark.parametrize("K", [384, 256, 128])
@pytest.mark.parametrize("ln", [True, False])
@pytest.mark.parametrize("M", [1, 63, 64, 65, 129, 1000, 16384 * 3 + 17])
def test_random_shapes(cuda, K, ln, M):
    p = mgn_params(K, seed=K + M, layernorm=ln, affine_random=True)
    x = normal_fp16(M, K, seed=M)
    got = run_gpu(x.to(cuda), to_dev(p, cuda)).float().cpu().numpy()
    assert_parity(got, run_oracle(x, p), f"K={K} ln={ln} M={M}")


def test_config0_shape(cuda):
    """The CPU-reference shape: edge MLP, M = 16384, gamma = 1, beta = 0."""
    M, K = 16384, 384
    p = mgn_params(K, seed=0)
    x = normal_fp16(M, K, seed=0)
    got = run_gpu(x.to(cuda), to_dev(p, cuda)).float().cpu().numpy()
    assert_parity(got, run_oracle(x, p), "config0")


def test_reference_entry_points(cuda):
    M, K = 3000, 384
    p = to_dev(mgn_params(K, seed=5, affine_random=True), cuda)
    x = normal_fp16(M, K, seed=6).to(cuda)
    a = gpipes.mgn_fullmlp(x, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"], p["gamma"], p["beta"])
    out = torch.empty_like(a)
    gpipes.mgn_fullmlp_out(x, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"], p["gamma"], p["beta"], out)
    assert torch.equal(a, out)
    assert_parity(a.float().cpu().numpy(), run_oracle(x, p), "mgn_fullmlp")
    pl = dict(p, gamma=None, beta=None)
    c = gpipes.mgn_linears(x, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"])
    assert_parity(c.float().cpu().numpy(), run_oracle(x, pl), "mgn_linears")


def test_no_write_past_output(cuda):
    M, K = 1000, 384
    p = to_dev(mgn_params(K, seed=7), cuda)
    x = normal_fp16(M, K, seed=8).to(cuda)
    big = torch.full((M + 64, 128), 7.0, dtype=torch.float16, device=cuda)
    out = big[:M]
    gpipes.mgn_mlp_out(x, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"], p["gamma"], p["beta"], out)
    torch.cuda.synchronize()
    assert torch.all(big[M:] == 7.0)
    assert_parity(out.float().cpu().numpy(), run_oracle(x, p), "guarded")


def test_nondefault_stream_and_repeat(cuda):
    M, K = 20000, 384
    p = to_dev(mgn_params(K, seed=9), cuda)
    x = normal_fp16(M, K, seed=10).to(cuda)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        outs = [run_gpu(x, p) for _ in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


@pytest.mark.parametrize("which", ["edge", "node"])
def test_full_size_all_rows_and_invariants(cuda, which):
    """Headline sizes: edge M=1,048,576 K=384; node M=262,144 K=256.  The
    oracle runs over every row (a few tenths of a second on the box's cores)."""
    M, K = (1048576, 384) if which == "edge" else (262144, 256)
    p = to_dev(mgn_params(K, seed=11), cuda)
    x = normal_fp16(M, K, seed=12, device=cuda)
    y = run_gpu(x, p)
    assert_parity(y.float().cpu().numpy(), run_oracle(x.cpu(), p), f"{which} all {M} rows")
    # every row: LayerNorm with gamma=1, beta=0 has mean 0 and variance v/(v+eps) ~ 1
    yf = y.float()
    mean = yf.mean(dim=1)
    var = yf.var(dim=1, unbiased=False)
    assert float(mean.abs().max()) < 5e-3
    assert float((var - 1).abs().max()) < 2e-2
    # permutation equivariance: rows move with their inputs, bit-exact
    perm = torch.randperm(M, device=cuda, generator=torch.Generator(device=cuda).manual_seed(14))
    yp = run_gpu(x[perm].contiguous(), p)
    assert torch.equal(yp, y[perm])
