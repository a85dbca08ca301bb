"""GPU parity of the dense MLP chains: gp_mlp_out and the DLRM wrappers
(DlrmMlp, common/mlps.py:23-34) and gp_nerf_full_out (the NeRF MLP,
apps/nerf_full/torch/model.py:5-66).

Checked against the golden fixtures (torch.nn in float64) and the CPU oracle
at the fp16 I/O bar (max-abs 2e-2, relative-L2 5e-3).  At the workload sizes
(DLRM M = 262,144, NeRF M = 1,048,576) the oracle checks every row, and rows
are independent, so a small call must equal the same rows of the large call
bit for bit (for NeRF across the 262,144-row chunk edges).
"""
import numpy as np
import pytest
import torch

import gpipes
import oracle
from conftest import load_golden
from gpipes.synth import (dlrm_params, nerf_inputs, nerf_params, normal_fp16, padded_normal,
                          padded_uniform)

pytestmark = pytest.mark.gpu

ACT = {"relu": oracle.ACT_RELU, "sigmoid": oracle.ACT_SIGMOID, "none": oracle.ACT_NONE,
       "gelu_tanh": oracle.ACT_GELU_TANH}


def assert_parity(got, want, what):
    max_abs, rel = oracle.errors(got, want)
    print(f"[parity] {what}: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= oracle.MAX_ABS_TOL and rel <= oracle.REL_L2_TOL, (what, max_abs, rel)


def f(t):
    return None if t is None else t.detach().float().cpu().numpy()


def to(ts, dev):
    return [None if t is None else t.to(dev) for t in ts]


# ------------------------------------------------------------------ generic chains
@pytest.mark.parametrize("name", ["dlrm_bot.npz", "dlrm_sigmoid_head.npz"])
def test_mlp_golden(cuda, name):
    z = load_golden(name)
    n = sum(1 for k in z if k.startswith("w"))
    ws = [torch.from_numpy(z[f"w{i + 1}"]).to(cuda) for i in range(n)]
    bs = [torch.from_numpy(z[f"b{i + 1}"]).to(cuda) for i in range(n)]
    si = int(z["sigmoid_i"])
    acts = ["sigmoid" if i == si else "relu" for i in range(n)]
    y = gpipes.mlp_out(torch.from_numpy(z["x"]).to(cuda), ws, bs, acts)
    assert_parity(f(y), z["expected"], f"golden {name}")


@pytest.mark.parametrize("widths,acts", [
    ([13, 512, 256, 128], ["relu"] * 3),
    ([16, 512, 256, 128], ["relu"] * 3),
    ([64, 300, 77], ["gelu_tanh", "none"]),
    ([480, 1024, 1024, 512, 256, 1], ["relu"] * 4 + ["sigmoid"]),
    ([200, 128, 5], ["relu", "sigmoid"]),
    ([8, 8], ["none"]),
])
@pytest.mark.parametrize("M", [1, 257, 3000])
def test_mlp_vs_oracle(cuda, widths, acts, M):
    ws, bs = dlrm_params(widths, seed=M + len(widths), init="xavier")
    x = normal_fp16(M, widths[0], seed=M)
    y = gpipes.mlp_out(x.to(cuda), to(ws, cuda), to(bs, cuda), acts)
    want = oracle.mlp(f(x), [f(w) for w in ws], [f(b) for b in bs], [ACT[a] for a in acts])
    assert_parity(f(y), want, f"mlp {widths} M={M}")


@pytest.mark.parametrize("widths,acts,bias", [
    ([64, 128, 1], ["relu", "none"], False),      # one-output head as a GEMV, no bias
    ([64, 256, 1], ["relu", "sigmoid"], True),    # ... with bias and sigmoid
    ([64, 100, 1], ["relu", "sigmoid"], True),    # K = 100 is not a multiple of 8: GEMM head
    ([32, 4104, 1], ["relu", "relu"], True),      # K past 4096: several chunks per lane
])
def test_mlp_one_output_head(cuda, widths, acts, bias):
    ws, bs = dlrm_params(widths, seed=21, init="xavier")
    if not bias:
        bs = [None] * len(bs)
    M = 1027
    x = normal_fp16(M, widths[0], seed=22)
    y = gpipes.mlp_out(x.to(cuda), to(ws, cuda), [None if b is None else b.to(cuda) for b in bs], acts)
    assert y.shape == (M, 1)
    want = oracle.mlp(f(x), [f(w) for w in ws], [None if b is None else f(b) for b in bs], [ACT[a] for a in acts])
    assert_parity(f(y), want, f"mlp head {widths}")


def test_mlp_input_tail_reads_zero(cuda):
    """A 200-wide input is read in place and the GEMM's k-loop runs to 256: the columns
    past 200 must read as zeros, not as the next row's head.  Row 5 starts with +inf, so
    row 4 would turn NaN (inf x zero weight) if its tail read row 5."""
    widths = [200, 128, 5]
    ws, bs = dlrm_params(widths, seed=11, init="xavier")
    x = normal_fp16(64, 200, seed=12)
    x[5, 0] = float("inf")
    y = f(gpipes.mlp_out(x.to(cuda), to(ws, cuda), to(bs, cuda), ["relu", "none"]))
    keep = np.r_[0:5, 6:64]
    assert np.isfinite(y[keep]).all()
    want = oracle.mlp(f(x[keep]), [f(w) for w in ws], [f(b) for b in bs], [oracle.ACT_RELU, oracle.ACT_NONE])
    assert_parity(y[keep], want, "mlp input tail")


def test_mlp_no_bias_and_odd_stride(cuda):
    """Null biases; an input whose row is not 16-byte aligned (width 13) takes the padded path."""
    widths = [13, 256, 40]
    ws, bs = dlrm_params(widths, seed=3)
    x = padded_uniform(999, 13, 13, seed=4)
    y = gpipes.mlp_out(x.to(cuda), to(ws, cuda), [None, None], ["relu", "none"])
    want = oracle.mlp(f(x), [f(w) for w in ws], [None, None], [oracle.ACT_RELU, oracle.ACT_NONE])
    assert_parity(f(y), want, "mlp no bias")


# ------------------------------------------------------------------ DLRM
def test_dlrm_reference_signatures(cuda):
    """dlrm_botmlp(x[M,32], ...) and dlrm_topmlp(x[M,512], ...) -> [M,64] as the reference
    apps call them (apps/dlrm_*/pipelined/val.py), DlrmMlp with ReLU on every layer."""
    M = 2048
    wb, bb = dlrm_params([32, 512, 256, 128], seed=1, init="torch")
    xb = normal_fp16(M, 32, seed=2)
    yb = gpipes.dlrm_botmlp(xb.to(cuda), *[t for pair in zip(to(wb, cuda), to(bb, cuda)) for t in pair])
    assert_parity(f(yb), oracle.mlp(f(xb), [f(w) for w in wb], [f(b) for b in bb], [oracle.ACT_RELU] * 3),
                  "dlrm_botmlp reference shape")
    wt, bt = dlrm_params([512, 1024, 1024, 512, 256, 64], seed=3, init="torch")
    xt = normal_fp16(M, 512, seed=4)
    yt = gpipes.dlrm_topmlp(xt.to(cuda), *[t for pair in zip(to(wt, cuda), to(bt, cuda)) for t in pair])
    assert_parity(f(yt), oracle.mlp(f(xt), [f(w) for w in wt], [f(b) for b in bt], [oracle.ACT_RELU] * 5),
                  "dlrm_topmlp reference shape")


def dlrm_workload(cuda, M):
    wb, bb = dlrm_params([16, 512, 256, 128], seed=0, init="xavier")
    wb[0][13:] = 0  # 13 dense features padded to 16
    wt, bt = dlrm_params([480, 1024, 1024, 512, 256, 1], seed=1, init="xavier")
    wt[0][479:] = 0  # 479 padded to 480
    xb = padded_uniform(M, 13, 16, seed=2, device=cuda)
    xt = padded_normal(M, 479, 480, seed=3, device=cuda)
    return to(wb, cuda), to(bb, cuda), xb, to(wt, cuda), to(bt, cuda), xt


def test_dlrm_full_size(cuda):
    M = 262144
    wb, bb, xb, wt, bt, xt = dlrm_workload(cuda, M)
    yb = gpipes.mlp_out(xb, wb, bb, ["relu"] * 3)
    yt = gpipes.mlp_out(xt, wt, bt, ["relu"] * 4 + ["sigmoid"])
    torch.cuda.synchronize()
    assert_parity(f(yb), oracle.mlp(f(xb), [f(w) for w in wb], [f(b) for b in bb], [oracle.ACT_RELU] * 3),
                  f"DLRM bottom all {M} rows")
    assert_parity(f(yt), oracle.mlp(f(xt), [f(w) for w in wt], [f(b) for b in bt],
                                    [oracle.ACT_RELU] * 4 + [oracle.ACT_SIGMOID]), f"DLRM top all {M} rows")
    small = gpipes.mlp_out(xt[65000:66000].contiguous(), wt, bt, ["relu"] * 4 + ["sigmoid"])
    assert torch.equal(small.view(torch.int16), yt[65000:66000].view(torch.int16))
    assert ((yt.float() >= 0) & (yt.float() <= 1)).all()


# ------------------------------------------------------------------ NeRF
def nerf_call(x, d, ws, bs, rgb_act):
    wb = [t for pair in zip(ws, bs) for t in pair]
    return gpipes.nerf_full(x, d, *wb, rgb_act=rgb_act)


def test_nerf_golden(cuda):
    z = load_golden("nerf_workload.npz")
    ws, bs = nerf_params(64, int(z["Kd"]), int(z["Na"]), int(z["Nrgb"]), seed=int(z["seed"]), device=cuda)
    a, r = nerf_call(torch.from_numpy(z["x"]).to(cuda), torch.from_numpy(z["d"]).to(cuda), ws, bs, "sigmoid")
    assert_parity(f(a), z["alpha"], "nerf golden alpha")
    assert_parity(f(r), z["rgb"], "nerf golden rgb")


@pytest.mark.parametrize("Kd,Na,Nrgb,act,scale", [(27, 1, 3, "sigmoid", 1.0), (32, 64, 64, "none", 1.0),
                                                  (27, 1, 3, "sigmoid", 2.0), (32, 64, 64, "none", 2.0)])
@pytest.mark.parametrize("M", [1, 300, 70000])
def test_nerf_vs_oracle(cuda, Kd, Na, Nrgb, act, scale, M):
    """Reference shapes (view dirs 32, heads 64, no colour activation) and the workload's;
    weights at 2x the default init keep every layer's signal visible in outputs of order 1
    (at the default init the deep layers contract the signal to ~0.1)."""
    ws, bs = nerf_params(64, Kd, Na, Nrgb, seed=M + Kd)
    ws, bs = [(w.float() * scale).half() for w in ws], [(b.float() * scale).half() for b in bs]
    x, d = nerf_inputs(M, seed=M, Kd=Kd)
    a, r = nerf_call(x.to(cuda), d.to(cuda), to(ws, cuda), to(bs, cuda), act)
    rows = np.arange(M) if M <= 300 else np.r_[0:128, 65500:65600, M - 64:M]
    wa, wr = oracle.nerf(f(x[rows]), f(d[rows]), [f(w) for w in ws], [f(b) for b in bs], ACT[act])
    assert_parity(f(a)[rows], wa, f"nerf alpha Kd={Kd} Na={Na} M={M} x{scale}")
    assert_parity(f(r)[rows], wr, f"nerf rgb Kd={Kd} Nrgb={Nrgb} M={M} x{scale}")


def test_nerf_full_size(cuda):
    M = 1048576
    ws, bs = nerf_params(64, 27, 1, 3, seed=0, device=cuda)
    x, d = nerf_inputs(M, seed=0, device=cuda)
    a, r = nerf_call(x, d, ws, bs, "sigmoid")
    torch.cuda.synchronize()
    wa, wr = oracle.nerf(f(x), f(d), [f(w) for w in ws], [f(b) for b in bs], oracle.ACT_SIGMOID)
    assert_parity(f(a), wa, f"NeRF full alpha all {M} samples")
    assert_parity(f(r), wr, f"NeRF full rgb all {M} samples")
    sa, sr = nerf_call(x[261900:262900].contiguous(), d[261900:262900].contiguous(), ws, bs, "sigmoid")
    assert torch.equal(sa.view(torch.int16), a[261900:262900].view(torch.int16))  # across a chunk edge
    assert torch.equal(sr.view(torch.int16), r[261900:262900].view(torch.int16))
    assert torch.isfinite(a.float()).all() and ((r.float() >= 0) & (r.float() <= 1)).all()


def nerf_general_inputs(M, Kx, Kd, seed, device="cpu"):
    """Inputs of any width: the positional encodings (63 and 27 features) cut or zero-padded."""
    x0, d0 = nerf_inputs(M, seed=seed)
    x = torch.zeros((M, Kx), dtype=torch.float16)
    x[:, :min(Kx, 63)] = x0[:, :min(Kx, 63)]
    d = torch.zeros((M, Kd), dtype=torch.float16)
    d[:, :min(Kd, 27)] = d0[:, :min(Kd, 27)]
    return x.to(device), d.to(device)


@pytest.mark.parametrize("Kx,Kd,Na,Nrgb", [
    (60, 24, 1, 3),     # the reference model's defaults (in_x_ch 60, in_d_ch 24)
    (63, 27, 4, 3),     # odd input widths (rows not 16-byte multiples)
    (64, 32, 64, 64),   # the reference pipelined app's padded shapes
    (8, 1, 33, 63),     # narrow inputs, heads of two feature blocks
    (72, 27, 1, 3),     # x wider than 64: one GEMM launch per layer
    (64, 70, 1, 3),     # d wider than 64: likewise
    (64, 27, 65, 3),    # density head wider than 64: likewise
])
@pytest.mark.parametrize("M", [33, 255, 257, 4099])
def test_nerf_widths_vs_oracle(cuda, Kx, Kd, Na, Nrgb, M):
    """Every input / head width the C ABI accepts goes through one of the two paths
    (the fused kernel for Kx, Kd, Na, Nrgb <= 64, the GEMM chain otherwise).  At least
    33 rows: the relative-L2 bar over a single near-zero density value is meaningless
    (M = 1 is covered at the workload widths above)."""
    ws, bs = nerf_params(Kx, Kd, Na, Nrgb, seed=M + Kx, zero_pad_rows=None)
    ws, bs = [(w.float() * 2).half() for w in ws], [(b.float() * 2).half() for b in bs]
    x, d = nerf_general_inputs(M, Kx, Kd, seed=M)
    a, r = nerf_call(x.to(cuda), d.to(cuda), to(ws, cuda), to(bs, cuda), "sigmoid")
    wa, wr = oracle.nerf(f(x), f(d), [f(w) for w in ws], [f(b) for b in bs], oracle.ACT_SIGMOID)
    assert_parity(f(a), wa, f"nerf alpha Kx={Kx} Kd={Kd} Na={Na} M={M}")
    assert_parity(f(r), wr, f"nerf rgb Kx={Kx} Kd={Kd} Nrgb={Nrgb} M={M}")


def test_nerf_null_biases(cuda):
    M = 1000
    ws, bs = nerf_params(64, 27, 1, 3, seed=5)
    bs = [None if i % 2 else b for i, b in enumerate(bs)]
    x, d = nerf_inputs(M, seed=5)
    a, r = nerf_call(x.to(cuda), d.to(cuda), to(ws, cuda), to(bs, cuda), "none")
    wa, wr = oracle.nerf(f(x), f(d), [f(w) for w in ws], [f(b) for b in bs], oracle.ACT_NONE)
    assert_parity(f(a), wa, "nerf null biases alpha")
    assert_parity(f(r), wr, "nerf null biases rgb")


def test_nerf_fused_matches_layer_chain(cuda):
    """The same network through both paths: x zero-padded from 64 to 72 columns (with zero
    weight rows for the padding) takes the per-layer GEMM chain; both agree with each other
    and with the oracle."""
    M = 20000
    ws, bs = nerf_params(64, 27, 1, 3, seed=9, device=cuda)
    x, d = nerf_inputs(M, seed=9, device=cuda)
    x72 = torch.zeros((M, 72), dtype=torch.float16, device=cuda)
    x72[:, :64] = x
    w72 = list(ws)
    w72[0] = torch.cat([ws[0], torch.zeros((8, 256), dtype=torch.float16, device=cuda)])
    w72[5] = torch.cat([ws[5], torch.zeros((8, 256), dtype=torch.float16, device=cuda)])
    a1, r1 = nerf_call(x, d, ws, bs, "sigmoid")
    a2, r2 = nerf_call(x72, d, w72, bs, "sigmoid")
    assert_parity(f(a1), f(a2), "fused vs chain alpha")
    assert_parity(f(r1), f(r2), "fused vs chain rgb")
    rows = np.r_[0:100, M - 100:M]
    wa, wr = oracle.nerf(f(x[rows]), f(d[rows]), [f(w) for w in ws], [f(b) for b in bs], oracle.ACT_SIGMOID)
    assert_parity(f(a2)[rows], wa, "chain alpha")
    assert_parity(f(r2)[rows], wr, "chain rgb")


def test_nerf_unaligned_inputs_bit_exact(cuda):
    """Row slices of [M, 27] or [M, 63] inputs start at addresses that are not 16-byte aligned;
    they are copied into the workspace and give exactly the aligned call's results."""
    M = 5000
    for Kx, Kd in ((64, 27), (63, 27), (64, 32)):
        ws, bs = nerf_params(Kx, Kd, 1, 3, seed=Kx + Kd, device=cuda, zero_pad_rows=None)
        x, d = nerf_general_inputs(M + 7, Kx, Kd, seed=3, device=cuda)
        a1, r1 = nerf_call(x[3:3 + M].clone(), d[3:3 + M].clone(), ws, bs, "sigmoid")
        xs, ds = x[3:3 + M], d[3:3 + M]   # views: 3 rows into the buffers
        a2, r2 = nerf_call(xs, ds, ws, bs, "sigmoid")
        assert torch.equal(a1.view(torch.int16), a2.view(torch.int16)), (Kx, Kd)
        assert torch.equal(r1.view(torch.int16), r2.view(torch.int16)), (Kx, Kd)


def test_nerf_back_to_back_and_streams(cuda):
    """Two calls with different weights on one stream, then one on a side stream: the packed
    weight stream lives in the per-stream workspace and is rebuilt by every call."""
    M = 3000
    x, d = nerf_inputs(M, seed=11, device=cuda)
    p1 = nerf_params(64, 27, 1, 3, seed=12, device=cuda)
    p2 = nerf_params(64, 27, 1, 3, seed=13, device=cuda)
    a1, r1 = nerf_call(x, d, *p1, "sigmoid")
    a2, r2 = nerf_call(x, d, *p2, "sigmoid")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        a3, r3 = nerf_call(x, d, *p1, "sigmoid")
    s.synchronize()
    torch.cuda.synchronize()
    for (a, r), (ws, bs) in (((a1, r1), p1), ((a2, r2), p2)):
        wa, wr = oracle.nerf(f(x), f(d), [f(w) for w in ws], [f(b) for b in bs], oracle.ACT_SIGMOID)
        assert_parity(f(a), wa, "alpha")
        assert_parity(f(r), wr, "rgb")
    assert torch.equal(a1.view(torch.int16), a3.view(torch.int16))
    assert torch.equal(r1.view(torch.int16), r3.view(torch.int16))
