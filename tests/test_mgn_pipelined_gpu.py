"""GPU parity of the stage-chained MGN MLP (ring queues between stage
workgroups, the reference's pipelined layout) against the CPU oracle.

Same bar as the fused kernel: max-abs <= 2e-2, relative-L2 <= 5e-3.  After
every launch gpipes.pipeline_check() confirms that no queue wait hit its
spin bound.
"""
import pytest
import torch

import gpipes
import oracle
from gpipes.synth import mgn_params, normal_fp16
from conftest import load_golden
from test_mgn_gpu import GOLDEN, assert_parity, run_gpu, run_oracle, to_dev

pytestmark = pytest.mark.gpu

IMPLS = ["pipelined", "pipelined_split_ln"]


def run_checked(x, p, impl, eps=1e-5):
    y = run_gpu(x, p, impl=impl, eps=eps)
    gpipes.pipeline_check()
    return y


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("name,K", GOLDEN)
@pytest.mark.parametrize("M", [1, 65, 256])
def test_golden_fixtures(cuda, impl, name, K, M):
    z = load_golden(name)
    if impl == "pipelined_split_ln" and "gamma" not in z:
        pytest.skip("the split-LayerNorm layout exists only with LayerNorm")
    p = {k: torch.from_numpy(z[k]).to(cuda) if k in z else None
         for k in ("w1", "b1", "w2", "b2", "w3", "b3", "gamma", "beta")}
    x = torch.from_numpy(z["x"][:M]).to(cuda)
    got = run_checked(x, p, impl, eps=float(z["eps"])).float().cpu().numpy()
    assert_parity(got, z["expected"][:M], f"{impl} {name} M={M}")


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("K", [384, 256, 128])
# 64 and 192: a last tile whose second 64-row half (the second layer-1
# worker's share in the default layout) is empty
@pytest.mark.parametrize("M", [64, 127, 128, 129, 192, 5000, 16384 * 3 + 17])
def test_random_shapes(cuda, impl, K, M):
    for ln in (True, False):
        if impl == "pipelined_split_ln" and not ln:
            continue
        p = mgn_params(K, seed=K + M, layernorm=ln, affine_random=True)
        x = normal_fp16(M, K, seed=M)
        got = run_checked(x.to(cuda), to_dev(p, cuda), impl).float().cpu().numpy()
        assert_parity(got, run_oracle(x, p), f"{impl} K={K} ln={ln} M={M}")


def test_split_needs_layernorm(cuda):
    p = to_dev(mgn_params(384, seed=1, layernorm=False), cuda)
    x = normal_fp16(100, 384, seed=2).to(cuda)
    with pytest.raises(gpipes.GpipesError):
        run_gpu(x, p, impl="pipelined_split_ln")


@pytest.mark.parametrize("impl", IMPLS)
def test_full_size_edge(cuda, impl):
    """Headline edge size through the queue pipelines: every row vs the
    oracle, and a second launch bit-identical to the first (the tile-to-pipeline
    assignment may change between launches; the per-row arithmetic may not)."""
    M, K = 1048576, 384
    p = to_dev(mgn_params(K, seed=11), cuda)
    x = normal_fp16(M, K, seed=12, device=cuda)
    y = run_checked(x, p, impl)
    assert_parity(y.float().cpu().numpy(), run_oracle(x.cpu(), p), f"{impl} edge all {M} rows")
    y2 = run_checked(x, p, impl)
    assert torch.equal(y, y2)
