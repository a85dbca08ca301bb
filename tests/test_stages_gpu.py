"""GPU parity of the library's stage functions run over whole matrices, and
of the ring-queue identity pipelines.

Integer / byte work (copies through queues, concat) and fp16 addition are
checked bit-exactly; floating-point stages against the CPU oracle at the fp16
I/O bar (max-abs 2e-2, relative-L2 5e-3).
"""
import numpy as np
import pytest
import torch

import gpipes
import oracle
from conftest import load_golden

pytestmark = pytest.mark.gpu


def assert_parity(got, want, what):
    max_abs, rel = oracle.errors(got, want)
    print(f"[parity] {what}: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= oracle.MAX_ABS_TOL and rel <= oracle.REL_L2_TOL, (what, max_abs, rel)


def h(shape, scale=1.0, seed=0, lo=None, hi=None):
    g = torch.Generator().manual_seed(seed)
    if lo is not None:
        t = torch.rand(shape, generator=g) * (hi - lo) + lo
    else:
        t = torch.randn(shape, generator=g) * scale
    return t.to(torch.float16)


def f(t):
    return None if t is None else t.float().cpu().numpy()


# ------------------------------------------------------------------ LayerNorm
@pytest.mark.parametrize("D", [128, 256, 512, 1024])
@pytest.mark.parametrize("M", [1, 127, 128, 1000])
def test_layer_norm(cuda, D, M):
    x = h((M, D), 2.0, seed=D + M) + 0.5
    gm, bt = h((D,), lo=0.5, hi=1.5, seed=1), h((D,), lo=-0.5, hi=0.5, seed=2)
    for eps in (1e-5, 1e-12):
        y = gpipes.layer_norm_out(x.to(cuda), gm.to(cuda), bt.to(cuda), eps=eps)
        assert_parity(f(y), oracle.layer_norm(f(x), f(gm), f(bt), eps), f"LN D={D} M={M} eps={eps}")


def test_layer_norm_reference_row(cuda):
    z = load_golden("layer_norm_row.npz")
    y = gpipes.layer_norm_out(torch.from_numpy(z["x"]).to(cuda), eps=float(z["eps"]))
    assert_parity(f(y), z["expected"], "LN reference row")


# ------------------------------------------------------------------ add / concat
@pytest.mark.parametrize("M,N", [(1, 8), (129, 128), (1000, 1024), (300, 40)])
def test_add_bit_exact(cuda, M, N):
    a, b = h((M, N), 3.0, seed=1), h((M, N), 3.0, seed=2)
    c = gpipes.add_out(a.to(cuda), b.to(cuda)).cpu()
    want = (a.float() + b.float()).to(torch.float16)  # one rounding of the exact sum
    assert torch.equal(c.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("M,N0,N1", [(1, 8, 8), (130, 256, 64), (1000, 256, 32), (77, 128, 128)])
def test_concat_bit_exact(cuda, M, N0, N1):
    a, b = h((M, N0), seed=3), h((M, N1), seed=4)
    c = gpipes.concat_out(a.to(cuda), b.to(cuda)).cpu()
    assert torch.equal(c.view(torch.int16), torch.cat([a, b], dim=1).view(torch.int16))


# ------------------------------------------------------------------ GEMM stages
@pytest.mark.parametrize("K", [128, 256, 384])
@pytest.mark.parametrize("act", ["none", "relu", "gelu_tanh", "sigmoid"])
@pytest.mark.parametrize("M", [1, 200, 4099])
def test_linear(cuda, K, act, M):
    x = h((M, K), seed=K + M)
    w = h((K, 128), 1.0 / np.sqrt(K), seed=7)
    b = h((128,), 0.5, seed=8)
    y = gpipes.linear_out(x.to(cuda), w.to(cuda), b.to(cuda), act=act)
    want = oracle.linear(f(x), f(w), f(b), gpipes.ACTS[act])
    assert_parity(f(y), want, f"linear K={K} act={act} M={M}")


@pytest.mark.parametrize("K", [128, 384])
@pytest.mark.parametrize("M", [63, 64, 65, 127, 129, 191, 192, 193, 100003])
def test_linear_tile_edges(cuda, K, M):
    """The memory-fed stage copies tiles in 64-row parts through a ring of three
    part buffers, the next tile's parts under this tile's MFMAs: tiles whose
    second part is partial or empty, and (M = 100,003) several tiles per
    workgroup, with nothing written past the output rows."""
    x = h((M, K), seed=K + 3 * M)
    w = h((K, 128), 1.0 / np.sqrt(K), seed=17)
    b = h((128,), 0.5, seed=18)
    big = torch.full((M + 64, 128), 7.0, dtype=torch.float16, device=cuda)
    y = gpipes.linear_out(x.to(cuda), w.to(cuda), b.to(cuda), act="relu", out=big[:M])
    torch.cuda.synchronize()
    assert torch.all(big[M:] == 7.0)
    rows = np.unique(np.concatenate([np.arange(min(M, 300)), np.arange(max(0, M - 300), M),
                                     np.random.default_rng(M).integers(0, M, 2000)]))
    assert_parity(f(y)[rows], oracle.linear(f(x)[rows], f(w), f(b), gpipes.ACTS["relu"]),
                  f"linear edges K={K} M={M}")


@pytest.mark.parametrize("K", [128, 384])
def test_linear_accumulator_input(cuda, K):
    """pipe_gemm: no bias, an accumulator tile added (the K-split chaining form)."""
    M = 777
    x, w, acc = h((M, K), seed=1), h((K, 128), 1.0 / np.sqrt(K), seed=2), h((M, 128), seed=3)
    y = gpipes.linear_out(x.to(cuda), w.to(cuda), None, acc.to(cuda))
    assert_parity(f(y), oracle.linear(f(x), f(w), None) + f(acc), f"linear+acc K={K}")


def test_linear_k_split_chain(cuda):
    """Two 128-wide stages chained through the accumulator equal one 256-wide product."""
    M = 777
    x = h((M, 256), seed=5)
    w = h((256, 128), 1.0 / 16, seed=6)
    p1 = gpipes.linear_out(x[:, :128].contiguous().to(cuda), w[:128].contiguous().to(cuda))
    p2 = gpipes.linear_out(x[:, 128:].contiguous().to(cuda), w[128:].contiguous().to(cuda), None, p1)
    assert_parity(f(p2), oracle.linear(f(x), f(w), None), "K-split chain")


@pytest.mark.parametrize("K", [128, 256, 384])
def test_linear_layer_norm(cuda, K):
    M = 1030
    x, w = h((M, K), seed=K), h((K, 128), 1.0 / np.sqrt(K), seed=9)
    b, gm, bt = h((128,), 0.3, seed=10), h((128,), lo=0.5, hi=1.5, seed=11), h((128,), lo=-0.5, hi=0.5, seed=12)
    y = gpipes.linear_layer_norm_out(x.to(cuda), w.to(cuda), b.to(cuda), gm.to(cuda), bt.to(cuda), eps=1e-5)
    want = oracle.layer_norm(oracle.linear(f(x), f(w), f(b)), f(gm), f(bt), 1e-5)
    assert_parity(f(y), want, f"linear+LN K={K}")


# ------------------------------------------------------------------ ring-queue pipelines
@pytest.mark.parametrize("M", [1, 128, 129, 100003, 1048576])
@pytest.mark.parametrize("max_pipes", [1, 3, 0])
def test_pipe_ident_bit_exact(cuda, M, max_pipes):
    x = torch.randn((M, 128), device=cuda, generator=torch.Generator(device=cuda).manual_seed(M)).to(torch.float16)
    y = gpipes.pipe_ident(x, max_pipes=max_pipes)
    gpipes.pipeline_check()
    assert torch.equal(y.view(torch.int16), x.view(torch.int16))


def test_pipe_ident_back_to_back(cuda):
    """Epoch-tagged counters: repeated launches on one arena need no reset."""
    x = torch.randn((50000, 128), device=cuda).to(torch.float16)
    for i in range(5):
        y = gpipes.pipe_ident(x, max_pipes=[0, 2, 7, 1, 0][i])
        gpipes.pipeline_check()
        assert torch.equal(y.view(torch.int16), x.view(torch.int16)), i


@pytest.mark.parametrize("route", ["ident", "broadcast", "split", "drain", "reload"])
@pytest.mark.parametrize("M", [1, 129, 100003, 1048576])
@pytest.mark.parametrize("max_pipes", [1, 0, 5])
def test_pipe_route_bit_exact(cuda, route, M, max_pipes):
    """Queue topologies: 1:1 over striped input chunks (read_striped_input), one producer /
    two consumers, split / merge, the broadcast whose second consumer is a NullWriter
    (it must keep the two-consumer queue draining, or the launch times out), and a one-slot
    queue of 64-row entries whose consumer re-reads the same 16 KiB every tile (payload
    loads served by its L1 would return the slot's previous round)."""
    x = torch.randn((M, 128), device=cuda, generator=torch.Generator(device=cuda).manual_seed(M + 1)).to(torch.float16)
    out, out2 = gpipes.pipe_route(x, route, max_pipes=max_pipes)
    gpipes.pipeline_check()
    assert torch.equal(out.view(torch.int16), x.view(torch.int16))
    if route == "broadcast":
        assert torch.equal(out2.view(torch.int16), x.view(torch.int16))


@pytest.mark.parametrize("M", [1, 128, 129, 100003, 128 * 20000])
@pytest.mark.parametrize("max_pipes", [1, 0, 5])
def test_pipe_handoff_checksums(cuda, M, max_pipes):
    """Queue hand-off benchmark route: every tile's checksum, computed by the consumer from
    the payload the producer generated, equals the closed form (handoff_checksums is pinned
    against a brute-force sum in test_capi.py)."""
    got = gpipes.pipe_handoff(M, max_pipes=max_pipes)
    gpipes.pipeline_check()
    want = gpipes.handoff_checksums(M)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want)


def test_pipe_handoff_back_to_back(cuda):
    """Repeated hand-off launches over the arena the copy routes use."""
    x = torch.randn((5000, 128), device=cuda).to(torch.float16)
    for i, mp in enumerate([0, 1, 0, 3]):
        got = gpipes.pipe_handoff(128 * 3000 + 77, max_pipes=mp)
        gpipes.pipeline_check()
        assert np.array_equal(got.cpu().numpy().view(np.uint32), gpipes.handoff_checksums(128 * 3000 + 77)), i
        out, _ = gpipes.pipe_route(x, "ident")
        gpipes.pipeline_check()
        assert torch.equal(out, x), i


def test_arena_shared_by_different_queue_layouts(cuda):
    """Launches with different queue layouts on one stream share the arena."""
    from gpipes.synth import mgn_params, normal_fp16
    x = torch.randn((70000, 128), device=cuda).to(torch.float16)
    p = {k: (None if v is None else v.to(cuda)) for k, v in mgn_params(384, seed=2).items()}
    xe = normal_fp16(5000, 384, seed=3, device=cuda)
    ref = gpipes.mgn_mlp(xe, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"], p["gamma"], p["beta"],
                         impl="pipelined")
    gpipes.pipeline_check()
    for route in ["split", "ident", "reload", "broadcast", "drain", "split", "reload", "ident"]:
        out, _ = gpipes.pipe_route(x, route)
        gpipes.pipeline_check()
        assert torch.equal(out, x), route
        y = gpipes.mgn_mlp(xe, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"], p["gamma"], p["beta"],
                           impl="pipelined")
        gpipes.pipeline_check()
        assert torch.equal(y, ref), route
