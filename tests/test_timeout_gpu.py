"""Device-side timeouts are reported, and kernels still end normally.

The host lowers the poll bound of every device-side wait with the test hook
gp_set_wait_limit, so that the waits of the next launch run out while every
wave still reaches the end of the kernel; gp_pipeline_check must then return
GP_ERR_TIMEOUT (-5).  With the default bound restored the next launch on the
same stream must check clean and match the CPU oracle (the status words are
epoch-tagged, so a failure never leaks into a later launch).

The fused kernels must not store anything computed after a timed-out wait:
every row of an aborted launch's output is either untouched or bit-identical
to the row of a normal launch.
"""
import numpy as np
import pytest
import torch

import gpipes
from gpipes.synth import mgn_params, normal_fp16
from test_mgn_gpu import assert_parity, run_gpu, run_oracle, to_dev

pytestmark = pytest.mark.gpu

TIMEOUT = -5
SENTINEL = 0x7E00  # fp16 NaN bit pattern: rows the kernel never stored keep it


@pytest.fixture
def restore_limit():
    yield
    gpipes.set_wait_limit(0)


def expect_timeout():
    with pytest.raises(gpipes.GpipesError) as ei:
        gpipes.pipeline_check()
    assert ei.value.code == TIMEOUT, str(ei.value)


def untouched_or_equal(got, ref):
    """Rows of `got` are either all sentinel or bit-identical to `ref`."""
    g = got.view(torch.int16).cpu().numpy()
    r = ref.view(torch.int16).cpu().numpy()
    untouched = np.all(g == np.int16(SENTINEL), axis=1)
    equal = np.all(g == r, axis=1)
    return bool(np.all(untouched | equal)), int(untouched.sum())


@pytest.mark.parametrize("K,ln", [(384, True), (384, False), (256, True)])
def test_fused_timeout_reported(cuda, restore_limit, K, ln):
    M = 64 * 256 * 3 + 5  # three tiles per workgroup and a partial one
    print(f"[timeout] fused K={K} ln={ln} M={M}", flush=True)
    p = to_dev(mgn_params(K, seed=K, layernorm=ln, affine_random=True), cuda)
    x = normal_fp16(M, K, seed=1).to(cuda)
    ref = run_gpu(x, p)
    gpipes.pipeline_check()  # a normal launch checks clean

    out = torch.full((M, 128), SENTINEL, dtype=torch.int16, device=cuda).view(torch.float16)
    gpipes.set_wait_limit(1)
    gpipes.mgn_mlp_out(x, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"], p["gamma"], p["beta"], out)
    expect_timeout()
    ok, n_untouched = untouched_or_equal(out, ref)
    print(f"[timeout] rows left untouched: {n_untouched} of {M}", flush=True)
    assert ok, "an aborted launch stored rows that differ from a normal launch"

    gpipes.set_wait_limit(0)
    y = run_gpu(x, p)
    gpipes.pipeline_check()
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))
    idx = np.linspace(0, M - 1, 1500).astype(np.int64)
    assert_parity(y.float().cpu().numpy()[idx], run_oracle(x.cpu()[idx], p), f"after timeout K={K}")


def test_gemm_ln_exchange_timeout_reported(cuda, restore_limit):
    """GEMM2's LayerNorm epilogue at H = 1024: each row's partial statistics come
    from 16 waves of four workgroups.  With a one-poll bound the waits give up;
    the call reports GP_ERR_TIMEOUT.  A wave stores its 128 features of a row
    only after its own wait succeeded, so a row may be partly stored: every
    element is either untouched or equal to a normal call's."""
    from gpipes.synth import bert_params
    M, H, FF = 16384, 1024, 1024
    print(f"[timeout] bert_ffn LayerNorm exchange M={M} H={H} FF={FF}", flush=True)
    p = {k: (None if v is None else v.to(cuda)) for k, v in bert_params(H, FF, seed=2, init="bert").items()}
    x = normal_fp16(M, H, seed=3).to(cuda)

    def call(out):
        return gpipes.bert_ffn_out(x, p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"], out, eps=1e-12,
                                   act="gelu_tanh")

    ref = call(torch.empty_like(x))
    gpipes.pipeline_check()
    out = torch.full((M, H), SENTINEL, dtype=torch.int16, device=cuda).view(torch.float16)
    gpipes.set_wait_limit(1)
    call(out)
    expect_timeout()
    g = out.view(torch.int16)
    untouched = g == SENTINEL
    print(f"[timeout] elements left untouched: {int(untouched.sum())} of {M * H}", flush=True)
    assert bool((untouched | (g == ref.view(torch.int16))).all()), "an aborted launch stored values that differ"

    gpipes.set_wait_limit(0)
    y = call(torch.empty_like(x))
    gpipes.pipeline_check()
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


def test_gather_timeout_reported(cuda, restore_limit):
    E, N = 64 * 256 * 2 + 33, 5000
    print(f"[timeout] gather E={E} N={N}", flush=True)
    p = to_dev(mgn_params(384, seed=3, affine_random=True), cuda)
    g = torch.Generator().manual_seed(4)
    nf = normal_fp16(N, 128, seed=5).to(cuda)
    ef = normal_fp16(E, 128, seed=6).to(cuda)
    src = torch.randint(0, N, (E,), generator=g).to(cuda)
    dst = torch.randint(0, N, (E,), generator=g).to(cuda)
    args = (nf, ef, src, dst, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"], p["gamma"], p["beta"])
    ref = gpipes.mgn_edge_gather(*args)
    gpipes.pipeline_check()

    out = torch.full((E, 128), SENTINEL, dtype=torch.int16, device=cuda).view(torch.float16)
    gpipes.set_wait_limit(1)
    gpipes.mgn_edge_gather_out(*args, out)
    expect_timeout()
    ok, _ = untouched_or_equal(out, ref)
    assert ok, "an aborted gather launch stored rows that differ from a normal launch"

    gpipes.set_wait_limit(0)
    y = gpipes.mgn_edge_gather(*args)
    gpipes.pipeline_check()
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("impl", ["pipelined", "pipelined_split_ln"])
def test_pipelined_timeout_reported(cuda, restore_limit, impl):
    M, K = 128 * 300 + 7, 384
    print(f"[timeout] {impl} M={M}", flush=True)
    p = to_dev(mgn_params(K, seed=11, affine_random=True), cuda)
    x = normal_fp16(M, K, seed=12).to(cuda)
    gpipes.set_wait_limit(1)
    run_gpu(x, p, impl=impl)
    expect_timeout()
    gpipes.set_wait_limit(0)
    y = run_gpu(x, p, impl=impl)
    gpipes.pipeline_check()
    idx = np.linspace(0, M - 1, 1500).astype(np.int64)
    assert_parity(y.float().cpu().numpy()[idx], run_oracle(x.cpu()[idx], p), f"{impl} after timeout")


@pytest.mark.parametrize("route", ["ident", "broadcast", "split", "drain", "reload"])
def test_route_timeout_reported(cuda, restore_limit, route):
    M = 128 * 200 + 3
    print(f"[timeout] route {route} M={M}", flush=True)
    x = normal_fp16(M, 128, seed=21).to(cuda)
    gpipes.set_wait_limit(1)
    gpipes.pipe_route(x, route)
    expect_timeout()
    gpipes.set_wait_limit(0)
    out, out2 = gpipes.pipe_route(x, route)
    gpipes.pipeline_check()
    assert torch.equal(out.view(torch.int16), x.view(torch.int16))
    if out2 is not None:
        assert torch.equal(out2.view(torch.int16), x.view(torch.int16))


def test_check_without_launch(cuda):
    """A stream that has had no reporting launch is an argument error, not a pass."""
    s = torch.cuda.Stream(device=cuda)
    with torch.cuda.stream(s):
        with pytest.raises(gpipes.GpipesError) as ei:
            gpipes.pipeline_check()
    assert ei.value.code == -1


def test_wait_limit_bounds():
    with pytest.raises(gpipes.GpipesError):
        gpipes.set_wait_limit(-1)
    with pytest.raises(gpipes.GpipesError):
        gpipes.set_wait_limit(1 << 31)
    gpipes.set_wait_limit(0)
