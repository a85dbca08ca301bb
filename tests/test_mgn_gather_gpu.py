"""GPU parity of the fused gather front end (gp_mgn_edge_gather_out):
out[e] = MgnMlp([nf[src[e]] | ef[e] | nf[dst[e]]]).

Checked against the CPU oracle on the gathered rows (numpy fancy indexing,
then oracle.mgn_mlp), and bit-exactly against the same MLP run on the
materialised [E, 384] input (the layer-1 k-order is identical, so the results
must be identical to the last bit).
"""
import numpy as np
import pytest
import torch

import gpipes
import oracle
from gpipes.synth import mgn_params, normal_fp16
from test_mgn_gpu import assert_parity, to_dev

pytestmark = pytest.mark.gpu


def graph(N, E, seed, idx_dtype, device):
    g = torch.Generator().manual_seed(seed)
    nf = normal_fp16(N, 128, seed=seed)
    ef = normal_fp16(E, 128, seed=seed + 1)
    src = torch.randint(0, N, (E,), generator=g, dtype=idx_dtype)
    dst = torch.randint(0, N, (E,), generator=g, dtype=idx_dtype)
    return nf.to(device), ef.to(device), src.to(device), dst.to(device)


def oracle_gather(nf, ef, src, dst, p, eps=1e-5):
    f = lambda t: None if t is None else t.detach().cpu().float().numpy()  # noqa: E731
    nfh, efh = f(nf), f(ef)
    s, d = src.cpu().numpy().astype(np.int64), dst.cpu().numpy().astype(np.int64)
    N = nfh.shape[0]
    zero = np.zeros((1, 128), np.float32)
    g = lambda idx: np.where(((idx >= 0) & (idx < N))[:, None], nfh[np.clip(idx, 0, N - 1)], zero)  # noqa: E731
    x = np.concatenate([g(s), efh, g(d)], axis=1)
    return oracle.mgn_mlp(x, f(p["w1"]), f(p["b1"]), f(p["w2"]), f(p["b2"]), f(p["w3"]), f(p["b3"]),
                          f(p["gamma"]), f(p["beta"]), eps=eps)


def run(nf, ef, src, dst, p):
    return gpipes.mgn_edge_gather(nf, ef, src, dst, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"],
                                  p["gamma"], p["beta"])


def materialised(nf, ef, src, dst, p):
    x = torch.cat([nf[src.long()], ef, nf[dst.long()]], dim=1).contiguous()
    return gpipes.mgn_mlp(x, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"], p["gamma"], p["beta"])


@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("ln", [True, False])
@pytest.mark.parametrize("N,E", [(1, 1), (5, 63), (7, 64), (1000, 65), (1000, 1000), (3000, 50001)])
def test_gather_vs_oracle_and_materialised(cuda, idx_dtype, ln, N, E):
    p = to_dev(mgn_params(384, seed=N + E, layernorm=ln, affine_random=True), cuda)
    nf, ef, src, dst = graph(N, E, N * 7 + E, idx_dtype, cuda)
    y = run(nf, ef, src, dst, p)
    assert_parity(y.float().cpu().numpy(), oracle_gather(nf, ef, src, dst, p), f"gather N={N} E={E} ln={ln}")
    assert torch.equal(y, materialised(nf, ef, src, dst, p))


@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
def test_out_of_range_indices_gather_zeros(cuda, idx_dtype):
    N, E = 100, 2000
    p = to_dev(mgn_params(384, seed=3, affine_random=True), cuda)
    nf, ef, src, dst = graph(N, E, 4, idx_dtype, cuda)
    src[::7] = -1
    dst[::5] = N
    dst[1::11] = N + 12345
    if idx_dtype == torch.int64:
        src[3::13] = (1 << 32) + 2  # low word valid, high word not
    y = run(nf, ef, src, dst, p)
    assert_parity(y.float().cpu().numpy(), oracle_gather(nf, ef, src, dst, p), "gather out-of-range")


def test_no_write_past_output(cuda):
    N, E = 50, 1000
    p = to_dev(mgn_params(384, seed=5), cuda)
    nf, ef, src, dst = graph(N, E, 6, torch.int64, cuda)
    big = torch.full((E + 64, 128), 7.0, dtype=torch.float16, device=cuda)
    gpipes.mgn_edge_gather_out(nf, ef, src, dst, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"],
                               p["gamma"], p["beta"], big[:E])
    torch.cuda.synchronize()
    assert torch.all(big[E:] == 7.0)


def test_full_size_edges(cuda):
    """Headline sizes: E = 1,048,576 edges over N = 262,144 nodes (the node MLP's batch)."""
    N, E = 262144, 1048576
    p = to_dev(mgn_params(384, seed=11), cuda)
    nf, ef, src, dst = graph(N, E, 12, torch.int64, cuda)
    y = run(nf, ef, src, dst, p)
    assert torch.equal(y, materialised(nf, ef, src, dst, p))
    idx = torch.from_numpy(np.unique(np.random.default_rng(13).integers(0, E, 4096))).to(cuda)
    assert_parity(y[idx].float().cpu().numpy(), oracle_gather(nf, ef[idx], src[idx], dst[idx], p), "gather full")
