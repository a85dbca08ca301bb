"""GPU parity of the bf16 forms of the wide GEMM stage, the BERT FFN block, the
fused bert_addln_ffn chain, the MLP chains, the NeRF MLP and the NerfA trunk
(gp_gemm_dtype_out, gp_bert_ffn_dtype_out, gp_bert_addln_ffn_dtype_out,
gp_mlp_dtype_out, gp_nerf_full_dtype_out, gp_nerf_a_dtype_out; the Python
mirrors follow the tensors' dtype).

The oracle is the same fp32 restatement, run on the bf16 values (exact in
fp32).  The bar is the fp16 bar scaled by the ratio of the unit roundoffs,
oracle.BF16_MAX_ABS_TOL / BF16_REL_L2_TOL (max-abs 0.16, relative-L2 0.04): the
kernels round the activations between GEMMs and the outputs to bf16 where the
oracle keeps fp32.  The bf16 golden fixture (torch.nn in float64 on bf16
parameters) pins the block; on the same values the bf16 and fp16 paths agree
within the bf16 bar; the two weight paths (in place / transposed copy) are
bit-identical in bf16 as in fp16.
"""
import numpy as np
import pytest
import torch

import gpipes
import oracle
from conftest import load_golden
from gpipes.synth import bert_addln_params, bert_params, nerf_a_params, nerf_inputs, nerf_params, normal_fp16

pytestmark = pytest.mark.gpu

ACT_ID = {"relu": oracle.ACT_RELU, "gelu_tanh": oracle.ACT_GELU_TANH, "none": oracle.ACT_NONE,
          "sigmoid": oracle.ACT_SIGMOID}
BF = torch.bfloat16


def assert_bf16_parity(got, want, what):
    max_abs, rel = oracle.errors(got, want)
    print(f"[parity bf16] {what}: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= oracle.BF16_MAX_ABS_TOL and rel <= oracle.BF16_REL_L2_TOL, (what, max_abs, rel)


def f(t):
    return None if t is None else t.detach().float().cpu().numpy()


def to(p, cuda, dtype=BF):
    return {k: (None if v is None else v.to(dtype).to(cuda)) for k, v in p.items()}


# ------------------------------------------------------------------ wide GEMM stage
@pytest.mark.parametrize("M,N,K", [(1, 128, 64), (257, 384, 1024), (1000, 4096, 1024), (513, 1024, 4096)])
@pytest.mark.parametrize("act", ["none", "relu", "gelu_tanh", "sigmoid"])
def test_gemm_bf16_vs_oracle(cuda, M, N, K, act):
    g = torch.Generator().manual_seed(M * 7 + N + K)
    x = torch.randn((M, K), generator=g).to(BF)
    w = (torch.randn((K, N), generator=g) / np.sqrt(K)).to(BF)
    b = (torch.randn((N,), generator=g) * 0.5).to(BF)
    y = gpipes.gemm_out(x.to(cuda), w.to(cuda), b.to(cuda), act=act)
    assert y.dtype == BF
    assert_bf16_parity(f(y), oracle.linear(f(x), f(w), f(b), ACT_ID[act]), f"gemm M={M} N={N} K={K} {act}")


@pytest.mark.parametrize("M,N,K", [(300, 128, 512), (1000, 1024, 4096)])
def test_gemm_bf16_residual(cuda, M, N, K):
    g = torch.Generator().manual_seed(M + N)
    x = torch.randn((M, K), generator=g).to(BF)
    w = (torch.randn((K, N), generator=g) / np.sqrt(K)).to(BF)
    b = (torch.randn((N,), generator=g) * 0.5).to(BF)
    r = torch.randn((M, N), generator=g).to(BF)
    y = gpipes.gemm_out(x.to(cuda), w.to(cuda), b.to(cuda), r.to(cuda))
    assert_bf16_parity(f(y), oracle.linear(f(x), f(w), f(b)) + f(r), f"gemm+residual M={M} N={N} K={K}")


def test_gemm_bf16_weight_paths_agree(cuda):
    """Above 8e10 FLOP the GEMM reads a transposed copy of W, below it W in
    place: the same products in the same order, bit-identical in bf16."""
    M, N, K = 16384, 2048, 1280
    g = torch.Generator().manual_seed(18)
    x = torch.randn((M, K), generator=g).to(BF).to(cuda)
    w = (torch.randn((K, N), generator=g) / np.sqrt(K)).to(BF).to(cuda)
    b = (torch.randn((N,), generator=g) * 0.5).to(BF).to(cuda)
    y = gpipes.gemm_out(x, w, b, act="gelu_tanh")
    parts = torch.cat([gpipes.gemm_out(x[r:r + 2048].contiguous(), w, b, act="gelu_tanh") for r in range(0, M, 2048)])
    assert torch.equal(y.view(torch.int16), parts.view(torch.int16))
    rows = np.r_[0:32, M - 32:M]
    assert_bf16_parity(f(y)[rows], oracle.linear(f(x[rows]), f(w), f(b), oracle.ACT_GELU_TANH), "both weight paths")


def test_gemm_rejects_mixed_dtypes(cuda):
    x = torch.zeros((64, 128), dtype=BF, device=cuda)
    with pytest.raises(RuntimeError, match="bfloat16"):
        gpipes.gemm_out(x, torch.zeros((128, 128), dtype=torch.float16, device=cuda))


# ------------------------------------------------------------------ BERT FFN block
def bert_ffn(x, p, act, eps):
    return gpipes.bert_ffn(x, p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"], eps=eps, act=act)


def test_bert_ffn_bf16_golden(cuda):
    z = load_golden("bert_ffn_gelu_bf16.npz")
    assert str(z["dtype"]) == "bf16"
    t = {k: torch.from_numpy(z[k].view(np.int16)).view(BF).to(cuda) for k in
         ("x", "w1", "b1", "w2", "b2", "gamma", "beta")}
    y = bert_ffn(t["x"], t, str(z["act"]), float(z["eps"]))
    assert_bf16_parity(f(y), z["expected"], "golden bert_ffn_gelu_bf16")


@pytest.mark.parametrize("M,H,FF,act", [(1, 128, 512, "relu"), (300, 128, 512, "relu"), (257, 256, 1024, "gelu_tanh"),
                                        (1000, 1024, 4096, "gelu_tanh"), (20000, 1024, 1024, "gelu_tanh")])
def test_bert_ffn_bf16_vs_oracle(cuda, M, H, FF, act):
    """H 128 keeps the LayerNorm rows in a wave; H 256 and 1024 exchange partial
    statistics between workgroups; M 20,000 is two row chunks."""
    print(f"[bf16 bert_ffn] M={M} H={H} FF={FF} {act}", flush=True)
    p = to(bert_params(H, FF, seed=M + H, init="bert", affine_random=True), cuda)
    x = normal_fp16(M, H, seed=M, device=cuda, dtype=BF)
    eps = 1e-12 if act == "gelu_tanh" else 1e-5
    y = bert_ffn(x, p, act, eps)
    if H > 128:
        gpipes.pipeline_check()  # the LayerNorm exchange reports its waits
    rows = np.r_[0:min(M, 200), max(0, M - 200):M]
    want = oracle.bert_ffn(f(x[rows]), f(p["w1"]), f(p["b1"]), f(p["w2"]), f(p["b2"]), f(p["gamma"]), f(p["beta"]),
                           act=ACT_ID[act], eps=eps)
    assert_bf16_parity(f(y)[rows], want, f"bert_ffn bf16 M={M} H={H} FF={FF}")


def test_bert_ffn_bf16_agrees_with_fp16(cuda):
    """The same values through both element types (bf16 values are exact in
    fp16 at these magnitudes): the results differ only by the bf16 rounding of
    the activations and outputs."""
    M, H, FF = 2000, 1024, 4096
    p16 = to(bert_params(H, FF, seed=5, init="bert", affine_random=True), cuda, BF)
    x16 = normal_fp16(M, H, seed=6, device=cuda, dtype=BF)
    yb = bert_ffn(x16, p16, "gelu_tanh", 1e-12)
    ph = {k: (None if v is None else v.to(torch.float16)) for k, v in p16.items()}
    yh = bert_ffn(x16.to(torch.float16), ph, "gelu_tanh", 1e-12)
    assert_bf16_parity(f(yb), f(yh), "bf16 against fp16 on the same values")


# ------------------------------------------------------------------ bert_addln_ffn (fused)
@pytest.mark.parametrize("M,H,FF,act", [(300, 128, 512, "relu"), (1000, 256, 384, "gelu_tanh")])
def test_bert_addln_bf16_vs_oracle(cuda, M, H, FF, act):
    p = to(bert_addln_params(H, FF, seed=H + FF, init="bert" if act == "gelu_tanh" else "torch",
                             affine_random=True), cuda)
    attn = normal_fp16(M, H, seed=M, device=cuda, dtype=BF)
    x = normal_fp16(M, H, seed=M + 1, device=cuda, dtype=BF)
    eps = 1e-12 if act == "gelu_tanh" else 1e-5
    y = gpipes.bert_addln_ffn(attn, x, p["w0"], p["b0"], p["w1"], p["b1"], p["w2"], p["b2"], p["ga0"], p["be0"],
                              p["ga2"], p["be2"], eps=eps, act=act)
    if H > 128:
        gpipes.pipeline_check()
    want = oracle.bert_addln_ffn(f(attn), f(x), f(p["w0"]), f(p["b0"]), f(p["w1"]), f(p["b1"]), f(p["w2"]),
                                 f(p["b2"]), f(p["ga0"]), f(p["be0"]), f(p["ga2"]), f(p["be2"]), act=ACT_ID[act],
                                 eps=eps)
    assert_bf16_parity(f(y), want, f"bert_addln_ffn bf16 M={M} H={H} FF={FF}")


def test_bert_addln_bf16_pipelined_rejected(cuda):
    p = to(bert_addln_params(128, 512, seed=1, init="torch", affine_random=True), cuda)
    a = normal_fp16(128, 128, seed=1, device=cuda, dtype=BF)
    with pytest.raises(gpipes.GpipesError):
        gpipes.bert_addln_ffn(a, a, p["w0"], p["b0"], p["w1"], p["b1"], p["w2"], p["b2"], p["ga0"], p["be0"],
                              p["ga2"], p["be2"], impl="pipelined")


# ------------------------------------------------------------------ DLRM towers (MLP chain)
@pytest.mark.parametrize("widths,acts", [
    ([13, 512, 256, 128], ["relu"] * 3),                               # the bottom MLP (unaligned input width)
    ([479, 1024, 1024, 512, 256, 1], ["relu"] * 4 + ["sigmoid"]),      # the top MLP with its GEMV click head
    ([256, 384, 200], ["gelu_tanh", "none"]),                          # a narrow, unaligned output
])
def test_mlp_bf16_vs_oracle(cuda, widths, acts):
    """gp_mlp_dtype_out: the bf16 GEMM layers, the GEMV head and the raw
    16-bit padding copies of the chain against the oracle on the bf16 values."""
    from gpipes.synth import dlrm_params
    M = 3000
    ws, bs = dlrm_params(widths, seed=len(widths))
    ws = [w.to(BF).to(cuda) for w in ws]
    bs = [b.to(BF).to(cuda) for b in bs]
    x = normal_fp16(M, widths[0], seed=7, device=cuda, dtype=BF)
    y = gpipes.mlp_out(x, ws, bs, acts)
    assert y.dtype == BF
    want = oracle.mlp(f(x), [f(w) for w in ws], [f(b) for b in bs], [ACT_ID[a] for a in acts])
    assert_bf16_parity(f(y), want, f"mlp bf16 {widths}")


# ------------------------------------------------------------------ NeRF MLP
def nerf_bf16(M, Kx, Kd, Na, Nrgb, seed, cuda):
    """Parameters at 2x the default init (outputs of order 1 through all twelve
    layers) and the positional-encoding inputs, cut or zero-padded to Kx / Kd."""
    ws, bs = nerf_params(Kx, Kd, Na, Nrgb, seed=seed, zero_pad_rows=None)
    ws = [(w.float() * 2).to(BF).to(cuda) for w in ws]
    bs = [(b.float() * 2).to(BF).to(cuda) for b in bs]
    x0, d0 = nerf_inputs(M, seed=seed)
    x = torch.zeros((M, Kx))
    x[:, :min(Kx, 63)] = x0[:, :min(Kx, 63)].float()
    d = torch.zeros((M, Kd))
    d[:, :min(Kd, 27)] = d0[:, :min(Kd, 27)].float()
    return x.to(BF).to(cuda), d.to(BF).to(cuda), ws, bs


@pytest.mark.parametrize("Kx,Kd,Na,Nrgb,act", [
    (64, 27, 1, 3, "sigmoid"),   # the NeRF workload's widths (fused kernel)
    (64, 32, 64, 64, "none"),    # the reference app's padded widths (fused kernel)
    (63, 27, 4, 3, "sigmoid"),   # odd widths: rows copied to 16-byte aligned bases first
    (72, 27, 1, 3, "sigmoid"),   # x wider than 64: one GEMM launch per layer
    (64, 27, 65, 3, "none"),     # density head wider than 64: likewise
])
@pytest.mark.parametrize("M", [257, 4099])
def test_nerf_bf16_vs_oracle(cuda, Kx, Kd, Na, Nrgb, act, M):
    """gp_nerf_full_dtype_out on both of its paths against the oracle on the bf16 values."""
    print(f"[bf16 nerf] M={M} Kx={Kx} Kd={Kd} Na={Na} Nrgb={Nrgb} {act}", flush=True)
    x, d, ws, bs = nerf_bf16(M, Kx, Kd, Na, Nrgb, M + Kx, cuda)
    wb = [t for pair in zip(ws, bs) for t in pair]
    a, r = gpipes.nerf_full(x, d, *wb, rgb_act=act)
    assert a.dtype == BF and r.dtype == BF
    wa, wr = oracle.nerf(f(x), f(d), [f(w) for w in ws], [f(b) for b in bs], ACT_ID[act])
    assert_bf16_parity(f(a), wa, f"nerf alpha bf16 M={M} Kx={Kx} Na={Na}")
    assert_bf16_parity(f(r), wr, f"nerf rgb bf16 M={M} Kx={Kx} Nrgb={Nrgb}")


def test_nerf_bf16_agrees_with_fp16_and_slices(cuda):
    """The same bf16 values through both element types of the fused kernel agree
    within the bf16 bar; a row slice of the batch (tiles at other offsets)
    reproduces its rows bit for bit."""
    M = 70000
    x, d, ws, bs = nerf_bf16(M, 64, 27, 1, 3, 11, cuda)
    wb = [t for pair in zip(ws, bs) for t in pair]
    a, r = gpipes.nerf_full(x, d, *wb, rgb_act="sigmoid")
    h = lambda t: t.to(torch.float16)  # noqa: E731
    ah, rh = gpipes.nerf_full(h(x), h(d), *[h(t) for t in wb], rgb_act="sigmoid")
    assert_bf16_parity(f(a), f(ah), "nerf alpha bf16 against fp16")
    assert_bf16_parity(f(r), f(rh), "nerf rgb bf16 against fp16")
    sa, sr = gpipes.nerf_full(x[1000:5000].contiguous(), d[1000:5000].contiguous(), *wb, rgb_act="sigmoid")
    assert torch.equal(sa.view(torch.int16), a[1000:5000].view(torch.int16))
    assert torch.equal(sr.view(torch.int16), r[1000:5000].view(torch.int16))
    assert ((r.float() >= 0) & (r.float() <= 1)).all()


# ------------------------------------------------------------------ NerfA trunk
@pytest.mark.parametrize("Kx,M", [(64, 300), (60, 4099), (72, 1000)])
def test_nerf_a_bf16_vs_oracle(cuda, Kx, M):
    """gp_nerf_a_dtype_out in bf16 against the oracle on the bf16 values: Kx 64
    and 60 run the NeRF kernel's trunk, Kx 72 (wider than the trunk's 64) the
    GEMM chain; weights at 2x the default init keep every layer's signal
    visible."""
    ws, bs = nerf_a_params(Kx, seed=M + Kx)
    ws = [(w.float() * 2).to(BF).to(cuda) for w in ws]
    bs = [(b.float() * 2).to(BF).to(cuda) for b in bs]
    x = normal_fp16(M, Kx, seed=M, device=cuda, dtype=BF)
    wb = [t for pair in zip(ws, bs) for t in pair]
    y = gpipes.nerf_a(x, *wb)
    assert y.dtype == BF
    want = oracle.nerf_a(f(x), [f(w) for w in ws], [f(b) for b in bs])
    assert_bf16_parity(f(y), want, f"nerf_a bf16 Kx={Kx} M={M}")
    with pytest.raises(gpipes.GpipesError):
        gpipes.nerf_a(x, *wb, impl="pipelined")
