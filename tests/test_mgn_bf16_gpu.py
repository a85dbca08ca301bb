"""GPU parity of the bf16 MGN MLP (gp_mgn_mlp_dtype_out, fused kernel) against
the CPU oracle and the bf16 golden fixtures.

Bar (bf16 I/O, fp32 accumulate): the fp16 bar scaled by the ratio of the unit
roundoffs (2^-8 / 2^-11 = 8): max-abs <= 0.16 and relative-L2 <= 0.04
against the fp32 oracle on identical bf16 inputs (oracle.BF16_*_TOL).  The
kernel rounds the two hidden activations and the output to bf16; the oracle
keeps them in fp32.  At the full edge size the oracle checks a row sample;
per-row LayerNorm moments, permutation equivariance and determinism cover
every row.
"""
import numpy as np
import pytest
import torch

import gpipes
import oracle
from gpipes.synth import mgn_params, normal_fp16
from conftest import bf16_to_f32, load_golden
from test_mgn_gpu import run_gpu, run_oracle, to_dev

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
KEYS = ("w1", "b1", "w2", "b2", "w3", "b3", "gamma", "beta")


def assert_parity_bf16(got, want, what=""):
    max_abs, rel = oracle.errors(got, want)
    print(f"[parity bf16] {what}: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= oracle.BF16_MAX_ABS_TOL and rel <= oracle.BF16_REL_L2_TOL, (what, max_abs, rel)


def from_bits(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(BF).to(dev)


@pytest.mark.parametrize("name", ["mgn_edge_ln_bf16.npz", "mgn_node_ln_bf16.npz"])
@pytest.mark.parametrize("M", [1, 7, 64, 65, 256])
def test_golden_fixtures(cuda, name, M):
    z = load_golden(name)
    p = {k: from_bits(z[k], cuda) for k in KEYS}
    x = from_bits(z["x"][:M], cuda)
    got = run_gpu(x, p, eps=float(z["eps"]))
    assert got.dtype == BF
    assert_parity_bf16(got.float().cpu().numpy(), z["expected"][:M], f"{name} M={M}")
    # the fixture's inputs through the fp32 oracle, too
    want = oracle.mgn_mlp(bf16_to_f32(z["x"][:M]), *(bf16_to_f32(z[k]) for k in KEYS), eps=float(z["eps"]))
    assert_parity_bf16(got.float().cpu().numpy(), want, f"{name} M={M} oracle")


@pytest.mark.parametrize("K", [384, 256, 128])
@pytest.mark.parametrize("ln", [True, False])
@pytest.mark.parametrize("M", [1, 65, 1000, 16384 * 3 + 17])
def test_random_shapes(cuda, K, ln, M):
    p = mgn_params(K, seed=K + M + 1, layernorm=ln, affine_random=True, dtype=BF)
    x = normal_fp16(M, K, seed=M + 2, dtype=BF)
    got = run_gpu(x.to(cuda), to_dev(p, cuda)).float().cpu().numpy()
    assert_parity_bf16(got, run_oracle(x, p), f"K={K} ln={ln} M={M}")


def test_bf16_is_not_fp16_reinterpreted(cuda):
    """The same weights and inputs in both types give outputs within the bf16
    bar of each other, far from what reading bf16 bits as fp16 would give."""
    M, K = 4096, 384
    p32 = mgn_params(K, seed=3, affine_random=True, dtype=torch.float32)
    x32 = normal_fp16(M, K, seed=4, dtype=torch.float32)
    yb = run_gpu(x32.to(BF).to(cuda), to_dev({k: v.to(BF) for k, v in p32.items()}, cuda)).float().cpu().numpy()
    yh = run_gpu(x32.half().to(cuda), to_dev({k: v.half() for k, v in p32.items()}, cuda)).float().cpu().numpy()
    assert_parity_bf16(yb, yh, "bf16 vs fp16 path")


def test_rejects(cuda):
    M, K = 64, 384
    p = to_dev(mgn_params(K, seed=5, dtype=BF), cuda)
    x = normal_fp16(M, K, seed=6, dtype=BF).to(cuda)
    with pytest.raises(gpipes.GpipesError) as ei:
        run_gpu(x, p, impl="pipelined")
    assert ei.value.code == -1  # bf16 runs on the fused kernel only
    ph = to_dev(mgn_params(K, seed=5), cuda)
    with pytest.raises(RuntimeError):
        run_gpu(x, ph)  # fp16 weights with a bf16 input


def test_nondefault_stream_and_repeat(cuda):
    M, K = 20000, 384
    p = to_dev(mgn_params(K, seed=9, dtype=BF), cuda)
    x = normal_fp16(M, K, seed=10, dtype=BF).to(cuda)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        outs = [run_gpu(x, p) for _ in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


def test_full_size_all_rows_and_invariants(cuda):
    """Edge MLP at the headline size, M = 1,048,576, in bf16; the oracle runs over every row."""
    M, K = 1048576, 384
    p = to_dev(mgn_params(K, seed=11, dtype=BF), cuda)
    x = normal_fp16(M, K, seed=12, device=cuda, dtype=BF)
    y = run_gpu(x, p)
    assert_parity_bf16(y.float().cpu().numpy(), run_oracle(x.cpu(), p), f"edge bf16 all {M} rows")
    yf = y.float()
    assert float(yf.mean(dim=1).abs().max()) < 8 * 5e-3
    assert float((yf.var(dim=1, unbiased=False) - 1).abs().max()) < 8 * 2e-2
    perm = torch.randperm(M, device=cuda, generator=torch.Generator(device=cuda).manual_seed(14))
    yp = run_gpu(x[perm].contiguous(), p)
    assert torch.equal(yp, y[perm])
