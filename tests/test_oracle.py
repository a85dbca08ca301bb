"""Pin the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against something that is not a retyping of
its own formula:
  * fp16 conversion    -- numpy's IEEE binary16 conversion, all 65536 patterns
  * linear (+act)      -- torch.nn.functional (library) in float64; K != N so a
                          transposed weight fails
  * layer_norm         -- torch.nn.functional.layer_norm in float64, closed
                          forms (constant row -> beta, alternating +-a -> +-1),
                          and the literal row of misc_tests/layer_norm/torch_val.py:88-105
  * mgn_mlp            -- golden fixtures made by torch.nn modules in float64,
                          closed forms (zero weights -> beta; identity weights ->
                          LN(relu(x[:, :128]))), and planted mistakes that must fail
  * bert_ffn           -- golden fixtures made by torch.nn modules in float64
                          (ReLU / eps 1e-5 and GELU(tanh) / eps 1e-12), closed forms
                          (w2 = 0 -> LN(x + b2); constant rows -> beta; GELU(tanh)
                          told apart from erf GELU), planted mistakes (no residual,
                          residual after LN, transposed w2, ReLU for GELU, wrong
                          eps) that must fail
  * bert_addln_ffn     -- golden fixtures made by torch.nn modules in float64 with the
                          structure of apps/bert_addln_ffn/torch/model.py:3-20 (ReLU /
                          eps 1e-5 at the reference app's shape, GELU(tanh) / eps 1e-12 at
                          H 256), the zero-FFN closed form, planted mistakes (be0 passed
                          for be2 and ln0 skipped -- the reference extension's defects --,
                          the second residual taken from x, no first residual, swapped
                          LayerNorm affines, transposed w0) that must fail
  * nerf_a             -- golden fixture made by torch.nn modules in float64 with the
                          structure of apps/nerf_a/torch/model.py:5-38, planted mistakes
                          (skip order, no skip, skip one layer early, no final ReLU,
                          rotated skip rows of w6) that must fail
  * add / concat       -- numpy
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from conftest import bf16_to_f32, load_golden

RNG = np.random.default_rng(1234)


def test_h2f_all_patterns():
    bits = np.arange(65536, dtype=np.uint16)
    got = oracle.h2f(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f2h_round_to_nearest_even():
    vals = np.concatenate([
        RNG.standard_normal(200000).astype(np.float32) * np.float32(10.0),
        (RNG.standard_normal(50000) * 1e-5).astype(np.float32),            # subnormal range
        (RNG.standard_normal(50000) * 3e4).astype(np.float32),             # near overflow
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001, 2.0 ** -26], np.float32),
    ])
    # exact ties between adjacent fp16 values
    h = RNG.integers(0, 0x7bff, 20000).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    vals = np.concatenate([vals, ((lo + hi) / 2).astype(np.float32)])
    got = oracle.f2h(vals)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    nanb = oracle.f2h(np.array([np.nan], np.float32))
    assert np.isnan(nanb.view(np.float16)[0])


@pytest.mark.parametrize("act,tfn", [
    (oracle.ACT_NONE, lambda t: t),
    (oracle.ACT_RELU, torch.relu),
    (oracle.ACT_GELU_TANH, lambda t: F.gelu(t, approximate="tanh")),
    (oracle.ACT_SIGMOID, torch.sigmoid),
])
def test_linear_vs_torch(act, tfn):
    M, K, N = 37, 96, 48
    x = RNG.standard_normal((M, K)).astype(np.float32)
    w = RNG.standard_normal((K, N)).astype(np.float32) / np.sqrt(K)
    b = RNG.standard_normal(N).astype(np.float32)
    got = oracle.linear(x, w, b, act)
    ref = tfn(F.linear(torch.from_numpy(x).double(), torch.from_numpy(w).double().t(),
                       torch.from_numpy(b).double())).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_linear_no_bias_and_k1():
    x = RNG.standard_normal((5, 1)).astype(np.float32)
    w = RNG.standard_normal((1, 7)).astype(np.float32)
    got = oracle.linear(x, w, None)
    np.testing.assert_allclose(got, x @ w, rtol=1e-6)


@pytest.mark.parametrize("eps", [1e-5, 1e-12])
def test_layer_norm_vs_torch(eps):
    M, D = 64, 128
    x = (RNG.standard_normal((M, D)) * 3 + 1.5).astype(np.float32)
    g = RNG.uniform(0.5, 1.5, D).astype(np.float32)
    b = RNG.uniform(-1, 1, D).astype(np.float32)
    got = oracle.layer_norm(x, g, b, eps)
    ref = F.layer_norm(torch.from_numpy(x).double(), [D], torch.from_numpy(g).double(),
                       torch.from_numpy(b).double(), eps).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=2e-5)


def test_layer_norm_closed_forms():
    D = 128
    # constant row: variance 0, output is exactly beta
    beta = RNG.uniform(-1, 1, D).astype(np.float32)
    x = np.full((3, D), 0.375, np.float32)  # sums exactly in fp32
    np.testing.assert_array_equal(oracle.layer_norm(x, np.ones(D, np.float32), beta), np.broadcast_to(beta, x.shape))
    # alternating +-a: mean 0, var a^2 -> +-a/sqrt(a^2+eps)
    for a in (1.0, 0.25, 7.0):
        row = np.where(np.arange(D) % 2 == 0, a, -a).astype(np.float32)[None]
        want = row / np.sqrt(a * a + 1e-5)
        np.testing.assert_allclose(oracle.layer_norm(row), want, rtol=1e-6)


def test_layer_norm_reference_row():
    z = load_golden("layer_norm_row.npz")
    x = z["x"].astype(np.float32)
    got = oracle.layer_norm(x, eps=float(z["eps"]))
    np.testing.assert_allclose(got, z["expected"], rtol=1e-5, atol=2e-5)
    # normalised row: zero mean, variance v / (v + eps) for the input variance v
    v = x[0].astype(np.float64).var()
    assert abs(got[0].mean()) < 1e-5
    assert abs(got[0].var() - v / (v + 1e-5)) < 1e-5


FIXTURES = ["mgn_edge_ln.npz", "mgn_edge_ln_affine.npz", "mgn_edge_linears.npz", "mgn_node_ln.npz"]


def _run_fixture(z, **override):
    p = {k: z[k].astype(np.float32) for k in ("x", "w1", "b1", "w2", "b2", "w3", "b3")}
    p["gamma"] = z["gamma"].astype(np.float32) if "gamma" in z else None
    p["beta"] = z["beta"].astype(np.float32) if "beta" in z else None
    p.update(override)
    return oracle.mgn_mlp(p["x"], p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"],
                          p["gamma"], p["beta"], eps=float(z["eps"]))


@pytest.mark.parametrize("name", FIXTURES)
def test_mgn_mlp_golden(name):
    z = load_golden(name)
    got = _run_fixture(z)
    np.testing.assert_allclose(got, z["expected"], rtol=1e-4, atol=1e-4)
    max_abs, rel = oracle.errors(got, z["expected"])
    assert max_abs < 1e-4 and rel < 1e-5


def test_bf16_decode_matches_torch():
    """The tests' bf16 decoder against torch.bfloat16 over all 65,536 bit patterns."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = bf16_to_f32(bits)
    want = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name", ["mgn_edge_ln_bf16.npz", "mgn_node_ln_bf16.npz"])
def test_mgn_mlp_golden_bf16(name):
    """The oracle on bf16 inputs (exact in fp32) against torch.nn in float64."""
    z = load_golden(name)
    assert str(z["dtype"]) == "bf16"
    zf = {k: (bf16_to_f32(v) if v.dtype == np.uint16 else v) for k, v in z.items()}
    got = _run_fixture(zf)
    max_abs, rel = oracle.errors(got, z["expected"])
    assert max_abs < 1e-4 and rel < 1e-5


@pytest.mark.parametrize("mutant", ["no_relu1", "relu3", "w1_rows_swapped", "b3_dropped", "eps_wrong"])
def test_mgn_mlp_golden_rejects_planted_mistakes(mutant):
    """A plausible oracle mistake must fail the same fixture check."""
    z = load_golden("mgn_edge_ln_affine.npz")
    x = z["x"].astype(np.float32)
    w1, b1 = z["w1"].astype(np.float32), z["b1"].astype(np.float32)
    w2, b2 = z["w2"].astype(np.float32), z["b2"].astype(np.float32)
    w3, b3 = z["w3"].astype(np.float32), z["b3"].astype(np.float32)
    g, bt = z["gamma"].astype(np.float32), z["beta"].astype(np.float32)
    if mutant == "no_relu1":
        h = oracle.linear(x, w1, b1)
        h = oracle.linear(h, w2, b2, oracle.ACT_RELU)
        got = oracle.layer_norm(oracle.linear(h, w3, b3), g, bt)
    elif mutant == "relu3":
        h = oracle.linear(oracle.linear(x, w1, b1, oracle.ACT_RELU), w2, b2, oracle.ACT_RELU)
        got = oracle.layer_norm(oracle.linear(h, w3, b3, oracle.ACT_RELU), g, bt)
    elif mutant == "w1_rows_swapped":
        got = _run_fixture(z, w1=np.roll(w1, 1, axis=0))
    elif mutant == "b3_dropped":
        got = _run_fixture(z, b3=np.zeros_like(b3))
    else:
        got = oracle.layer_norm(oracle.linear(oracle.linear(oracle.linear(x, w1, b1, 1), w2, b2, 1), w3, b3),
                                g, bt, eps=1e-1)
    max_abs, rel = oracle.errors(got, z["expected"])
    assert max_abs > oracle.MAX_ABS_TOL or rel > oracle.REL_L2_TOL, (mutant, max_abs, rel)


def test_mgn_mlp_zero_weights():
    """W = 0: every row becomes LN(b3); with a constant b3 that is exactly beta."""
    K = 384
    x = RNG.standard_normal((9, K)).astype(np.float32)
    z = np.zeros
    b3 = RNG.standard_normal(128).astype(np.float32)
    beta = RNG.uniform(-1, 1, 128).astype(np.float32)
    gamma = RNG.uniform(0.5, 1.5, 128).astype(np.float32)
    args = (x, z((K, 128), np.float32), RNG.standard_normal(128), z((128, 128), np.float32),
            RNG.standard_normal(128), z((128, 128), np.float32))
    out = oracle.mgn_mlp(*args, b3, gamma, beta)
    ref = F.layer_norm(torch.from_numpy(b3).double()[None], [128], torch.from_numpy(gamma).double(),
                       torch.from_numpy(beta).double()).numpy()
    np.testing.assert_allclose(out, np.broadcast_to(ref, out.shape), rtol=1e-5, atol=1e-5)
    out_c = oracle.mgn_mlp(*args, np.full(128, -0.625, np.float32), gamma, beta)
    np.testing.assert_array_equal(out_c, np.broadcast_to(beta, out_c.shape))


def test_mgn_mlp_identity_weights():
    K = 384
    x = RNG.standard_normal((33, K)).astype(np.float32)
    w1 = np.zeros((K, 128), np.float32)
    w1[:128] = np.eye(128)
    eye = np.eye(128, dtype=np.float32)
    zb = np.zeros(128, np.float32)
    out = oracle.mgn_mlp(x, w1, zb, eye, zb, eye, zb, np.ones(128), zb)
    ref = F.layer_norm(torch.relu(torch.from_numpy(x[:, :128]).double()), [128]).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)
    out_nl = oracle.mgn_mlp(x, w1, zb, eye, zb, eye, zb)
    np.testing.assert_array_equal(out_nl, np.maximum(x[:, :128], 0))


def test_add_concat():
    a = RNG.standard_normal((17, 64)).astype(np.float32)
    b = RNG.standard_normal((17, 64)).astype(np.float32)
    np.testing.assert_array_equal(oracle.add(a, b), a + b)
    c = RNG.standard_normal((17, 32)).astype(np.float32)
    np.testing.assert_array_equal(oracle.concat(a, c), np.concatenate([a, c], axis=1))


def test_errors_helper():
    e = np.array([3.0, 4.0])
    assert oracle.errors(e, e) == (0.0, 0.0)
    ma, rel = oracle.errors(np.array([3.0, 4.5]), e)
    assert ma == pytest.approx(0.5) and rel == pytest.approx(0.1)


BERT_FIXTURES = ["bert_ffn_relu.npz", "bert_ffn_gelu.npz"]


def _bert_args(z):
    p = {k: z[k].astype(np.float32) for k in ("x", "w1", "b1", "w2", "b2", "gamma", "beta")}
    act = oracle.ACT_RELU if str(z["act"]) == "relu" else oracle.ACT_GELU_TANH
    return p, act, float(z["eps"])


@pytest.mark.parametrize("name", BERT_FIXTURES)
def test_bert_ffn_golden(name):
    z = load_golden(name)
    p, act, eps = _bert_args(z)
    got = oracle.bert_ffn(p["x"], p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"], act=act, eps=eps)
    max_abs, rel = oracle.errors(got, z["expected"])
    assert max_abs < 2e-4 and rel < 1e-5, (max_abs, rel)


def test_bert_ffn_golden_bf16():
    """The oracle on bf16 inputs (exact in fp32) against torch.nn in float64."""
    z = load_golden("bert_ffn_gelu_bf16.npz")
    assert str(z["dtype"]) == "bf16"
    p = {k: bf16_to_f32(z[k]) for k in ("x", "w1", "b1", "w2", "b2", "gamma", "beta")}
    got = oracle.bert_ffn(p["x"], p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"],
                          act=oracle.ACT_GELU_TANH, eps=float(z["eps"]))
    max_abs, rel = oracle.errors(got, z["expected"])
    assert max_abs < 2e-4 and rel < 1e-5, (max_abs, rel)


@pytest.mark.parametrize("mutant", ["no_residual", "residual_after_ln", "w2_transposed_blocks", "relu_for_gelu",
                                    "eps_1e-5_instead"])
def test_bert_ffn_golden_rejects_planted_mistakes(mutant):
    """Plausible oracle mistakes must fail the GELU / eps 1e-12 fixture at the parity bar."""
    z = load_golden("bert_ffn_gelu.npz")
    p, act, eps = _bert_args(z)
    x, w1, b1, w2, b2, g, bt = (p[k] for k in ("x", "w1", "b1", "w2", "b2", "gamma", "beta"))
    h = oracle.linear(x, w1, b1, act)
    if mutant == "no_residual":
        got = oracle.layer_norm(oracle.linear(h, w2, b2), g, bt, eps)
    elif mutant == "residual_after_ln":
        got = oracle.layer_norm(oracle.linear(h, w2, b2), g, bt, eps) + x
    elif mutant == "w2_transposed_blocks":
        FF, H = w2.shape  # read w2 as if it were stored [H, FF] in blocks
        got = oracle.bert_ffn(x, w1, b1, w2.reshape(H, FF).T.copy(), b2, g, bt, act=act, eps=eps)
    elif mutant == "relu_for_gelu":
        got = oracle.bert_ffn(x, w1, b1, w2, b2, g, bt, act=oracle.ACT_RELU, eps=eps)
    else:
        # eps too large for rows whose pre-LN variance is tiny: make them tiny
        got = oracle.bert_ffn(x * 1e-3, w1, b1, w2, b2, g, bt, act=act, eps=1e-5)
        want = oracle.bert_ffn(x * 1e-3, w1, b1, w2, b2, g, bt, act=act, eps=eps)
        max_abs, rel = oracle.errors(got, want)
        assert max_abs > oracle.MAX_ABS_TOL or rel > oracle.REL_L2_TOL, (mutant, max_abs, rel)
        return
    max_abs, rel = oracle.errors(got, z["expected"])
    assert max_abs > oracle.MAX_ABS_TOL or rel > oracle.REL_L2_TOL, (mutant, max_abs, rel)


def test_bert_ffn_closed_forms():
    M, H, FF = 24, 128, 256
    x = RNG.standard_normal((M, H)).astype(np.float32)
    w1 = RNG.standard_normal((H, FF)).astype(np.float32) * 0.05
    b1 = RNG.standard_normal(FF).astype(np.float32)
    b2 = RNG.standard_normal(H).astype(np.float32)
    g = RNG.uniform(0.5, 1.5, H).astype(np.float32)
    bt = RNG.uniform(-0.5, 0.5, H).astype(np.float32)
    zero_w2 = np.zeros((FF, H), np.float32)
    # w2 = 0: the FFN contributes only b2, so out = LN(x + b2)
    for act in (oracle.ACT_RELU, oracle.ACT_GELU_TANH):
        got = oracle.bert_ffn(x, w1, b1, zero_w2, b2, g, bt, act=act, eps=1e-12)
        ref = F.layer_norm(torch.from_numpy(x + b2).double(), [H], torch.from_numpy(g).double(),
                           torch.from_numpy(bt).double(), 1e-12).numpy()
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    # constant x rows and b2 = 0, w2 = 0: variance 0, output exactly beta
    xc = np.full((3, H), 0.25, np.float32)
    got = oracle.bert_ffn(xc, w1, b1, zero_w2, np.zeros(H, np.float32), g, bt, act=oracle.ACT_RELU)
    np.testing.assert_array_equal(got, np.broadcast_to(bt, got.shape))
    # the hidden activation is GELU(tanh), told apart from exact-erf GELU (which the
    # end-to-end parity bar cannot resolve: the two differ by < 1e-3)
    h = oracle.linear(x, w1, b1, oracle.ACT_GELU_TANH)
    pre = torch.from_numpy(x).double() @ torch.from_numpy(w1).double() + torch.from_numpy(b1).double()
    np.testing.assert_allclose(h, F.gelu(pre, approximate="tanh").numpy(), rtol=1e-5, atol=1e-6)
    assert np.abs(h - F.gelu(pre).numpy()).max() > 1e-5


# ---------------------------------------------------------------------------- DLRM / NeRF chains
ACT_OF = {"relu": oracle.ACT_RELU, "sigmoid": oracle.ACT_SIGMOID, "none": oracle.ACT_NONE}


def _dlrm(z):
    n = sum(1 for k in z if k.startswith("w"))
    ws = [z[f"w{i + 1}"].astype(np.float32) for i in range(n)]
    bs = [z[f"b{i + 1}"].astype(np.float32) for i in range(n)]
    si = int(z["sigmoid_i"])
    acts = [oracle.ACT_SIGMOID if i == si else oracle.ACT_RELU for i in range(n)]
    return ws, bs, acts


@pytest.mark.parametrize("name", ["dlrm_bot.npz", "dlrm_sigmoid_head.npz"])
def test_mlp_golden(name):
    z = load_golden(name)
    ws, bs, acts = _dlrm(z)
    got = oracle.mlp(z["x"], ws, bs, acts)
    max_abs, rel = oracle.errors(got, z["expected"])
    assert max_abs < 1e-4 and rel < 1e-5, (max_abs, rel)


def test_mlp_golden_rejects_sigmoid_on_wrong_layer():
    z = load_golden("dlrm_sigmoid_head.npz")
    ws, bs, _ = _dlrm(z)
    got = oracle.mlp(z["x"], ws, bs, [oracle.ACT_RELU] * 3)
    max_abs, rel = oracle.errors(got, z["expected"])
    assert max_abs > oracle.MAX_ABS_TOL or rel > oracle.REL_L2_TOL


def _nerf_fixture():
    import hashlib
    import torch
    from gpipes.synth import nerf_params
    z = load_golden("nerf_workload.npz")
    ws, bs = nerf_params(64, int(z["Kd"]), int(z["Na"]), int(z["Nrgb"]), seed=int(z["seed"]))
    h = hashlib.sha256()
    for t in ws + bs:
        h.update(t.contiguous().view(torch.int16).numpy().tobytes())
    assert h.hexdigest() == str(z["weights_sha256"]), "nerf_params no longer reproduces the fixture's weights"
    f = lambda ts: [t.float().numpy() for t in ts]  # noqa: E731
    return z, f(ws), f(bs)


def test_nerf_golden():
    z, ws, bs = _nerf_fixture()
    alpha, rgb = oracle.nerf(z["x"], z["d"], ws, bs, oracle.ACT_SIGMOID)
    for got, want in ((alpha, z["alpha"]), (rgb, z["rgb"])):
        max_abs, rel = oracle.errors(got, want)
        assert max_abs < 1e-4 and rel < 1e-5, (max_abs, rel)


def _torch_nerf(x, d, ws, bs, sigmoid):
    """The NeRF MLP built from torch.nn modules in float64 with the module structure of
    apps/nerf_full/torch/model.py:5-66 (an implementation independent of the oracle)."""
    import torch

    def lin(i):
        m = torch.nn.Linear(ws[i].shape[0], ws[i].shape[1]).double()
        with torch.no_grad():
            m.weight.copy_(torch.from_numpy(ws[i]).double().t())
            m.bias.copy_(torch.from_numpy(bs[i]).double())
        return m
    relu = torch.nn.ReLU
    pre = torch.nn.Sequential(lin(0), relu(), lin(1), relu(), lin(2), relu(), lin(3), relu(), lin(4), relu())
    post = torch.nn.Sequential(lin(5), relu(), lin(6), relu(), lin(7), relu())
    rgb = torch.nn.Sequential(lin(10), relu(), lin(11), *([torch.nn.Sigmoid()] if sigmoid else []))
    with torch.no_grad():
        xt, dt = torch.from_numpy(x).double(), torch.from_numpy(d).double()
        enc = post(torch.cat([pre(xt), xt], dim=-1))
        return lin(8)(enc).numpy(), rgb(torch.cat([lin(9)(enc), dt], dim=-1)).numpy()


def _nerf_scaled():
    """Weights 3x the default init, so every layer's signal survives to the outputs."""
    _, ws, bs = _nerf_fixture()
    rng = np.random.default_rng(5)
    x = rng.standard_normal((48, 64)).astype(np.float32)
    d = rng.standard_normal((48, 27)).astype(np.float32)
    return x, d, [w * 3 for w in ws], [b * 3 for b in bs]


def test_nerf_vs_torch_scaled():
    x, d, ws, bs = _nerf_scaled()
    for sig in (False, True):
        a_o, r_o = oracle.nerf(x, d, ws, bs, oracle.ACT_SIGMOID if sig else oracle.ACT_NONE)
        a_t, r_t = _torch_nerf(x, d, ws, bs, sig)
        np.testing.assert_allclose(a_o, a_t, rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(r_o, r_t, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("mutant", ["skip_order", "no_skip", "w9_rows_rotated", "bottleneck_relu", "d_dropped",
                                    "no_sigmoid"])
def test_nerf_rejects_planted_mistakes(mutant):
    """Plausible oracle mistakes must fail against torch.nn at the parity bar."""
    x, d, ws, bs = _nerf_scaled()
    want_alpha, want_rgb = _torch_nerf(x, d, ws, bs, True)
    lin = oracle.linear
    h = x
    for i in range(5):
        h = lin(h, ws[i], bs[i], oracle.ACT_RELU)
    if mutant == "skip_order":
        h = oracle.concat(x, h)
    elif mutant == "no_skip":
        h = oracle.concat(h, np.zeros_like(x))
    else:
        h = oracle.concat(h, x)
    for i in range(5, 8):
        h = lin(h, ws[i], bs[i], oracle.ACT_RELU)
    alpha = lin(h, np.roll(ws[8], 1, axis=0) if mutant == "w9_rows_rotated" else ws[8], bs[8])
    dd = np.zeros_like(d) if mutant == "d_dropped" else d
    f = lin(h, ws[9], bs[9], oracle.ACT_RELU if mutant == "bottleneck_relu" else oracle.ACT_NONE)
    g = lin(oracle.concat(f, dd), ws[10], bs[10], oracle.ACT_RELU)
    rgb = lin(g, ws[11], bs[11], oracle.ACT_NONE if mutant == "no_sigmoid" else oracle.ACT_SIGMOID)
    fails = []
    for got, want in ((alpha, want_alpha), (rgb, want_rgb)):
        max_abs, rel = oracle.errors(got, want)
        fails.append(max_abs > oracle.MAX_ABS_TOL or rel > oracle.REL_L2_TOL)
    assert any(fails), mutant


# ---------------------------------------------------------------------------- bert_addln_ffn / nerf_a
ADDLN_FIXTURES = ["bert_addln_ffn.npz", "bert_addln_ffn_gelu.npz"]
ADDLN_KEYS = ("attn", "x", "w0", "b0", "w1", "b1", "w2", "b2", "ga0", "be0", "ga2", "be2")


def _addln_args(z):
    p = {k: z[k].astype(np.float32) for k in ADDLN_KEYS}
    act = oracle.ACT_RELU if str(z["act"]) == "relu" else oracle.ACT_GELU_TANH
    return p, act, float(z["eps"])


@pytest.mark.parametrize("name", ADDLN_FIXTURES)
def test_bert_addln_ffn_golden(name):
    z = load_golden(name)
    p, act, eps = _addln_args(z)
    got = oracle.bert_addln_ffn(*(p[k] for k in ADDLN_KEYS), act=act, eps=eps)
    max_abs, rel = oracle.errors(got, z["expected"])
    assert max_abs < 2e-4 and rel < 1e-5, (max_abs, rel)


@pytest.mark.parametrize("mutant", ["be0_for_be2", "ln0_skipped", "residual_x_not_h0", "no_attn_residual",
                                    "ln2_affine_swapped", "w0_transposed"])
def test_bert_addln_ffn_rejects_planted_mistakes(mutant):
    """Plausible mistakes (among them the reference extension's own defects,
    bert_addln_ffn_pl_ext.cu:71 and bert_addln_ffn_pl.cuh:227: be0 passed for be2,
    ln0 never run) must fail the fixture at the parity bar."""
    z = load_golden("bert_addln_ffn.npz")
    p, act, eps = _addln_args(z)
    a = dict(p)
    if mutant == "be0_for_be2":
        a["be2"] = p["be0"]
    elif mutant == "ln2_affine_swapped":
        a["ga2"], a["ga0"] = p["ga0"], p["ga2"]
    elif mutant == "w0_transposed":
        a["w0"] = p["w0"].T.copy()
    if mutant == "ln0_skipped":
        h0 = oracle.add(oracle.linear(p["attn"], p["w0"], p["b0"]), p["x"])
        f = oracle.linear(oracle.linear(h0, p["w1"], p["b1"], act), p["w2"], p["b2"])
        got = oracle.layer_norm(oracle.add(f, h0), p["ga2"], p["be2"], eps)
    elif mutant == "residual_x_not_h0":
        h0 = oracle.layer_norm(oracle.add(oracle.linear(p["attn"], p["w0"], p["b0"]), p["x"]), p["ga0"], p["be0"], eps)
        f = oracle.linear(oracle.linear(h0, p["w1"], p["b1"], act), p["w2"], p["b2"])
        got = oracle.layer_norm(oracle.add(f, p["x"]), p["ga2"], p["be2"], eps)
    elif mutant == "no_attn_residual":
        h0 = oracle.layer_norm(oracle.linear(p["attn"], p["w0"], p["b0"]), p["ga0"], p["be0"], eps)
        f = oracle.linear(oracle.linear(h0, p["w1"], p["b1"], act), p["w2"], p["b2"])
        got = oracle.layer_norm(oracle.add(f, h0), p["ga2"], p["be2"], eps)
    else:
        got = oracle.bert_addln_ffn(*(a[k] for k in ADDLN_KEYS), act=act, eps=eps)
    max_abs, rel = oracle.errors(got, z["expected"])
    assert max_abs > oracle.MAX_ABS_TOL or rel > oracle.REL_L2_TOL, (mutant, max_abs, rel)


def test_bert_addln_ffn_closed_forms():
    """w1 = w2 = 0 and b1 = b2 = 0: the FFN adds nothing, so out = LN(LN(attn W0 + b0 + x))
    with unit affines, and LayerNorm of an already normalised row is that row (up to eps):
    out = F.layer_norm(attn W0 + b0 + x)."""
    M, H, FF = 16, 128, 256
    attn = RNG.standard_normal((M, H)).astype(np.float32)
    x = RNG.standard_normal((M, H)).astype(np.float32)
    w0 = RNG.standard_normal((H, H)).astype(np.float32) * 0.1
    b0 = RNG.standard_normal(H).astype(np.float32)
    zw1, zb1 = np.zeros((H, FF), np.float32), np.zeros(FF, np.float32)
    zw2, zb2 = np.zeros((FF, H), np.float32), np.zeros(H, np.float32)
    got = oracle.bert_addln_ffn(attn, x, w0, b0, zw1, zb1, zw2, zb2, eps=1e-12)
    pre = torch.from_numpy(attn).double() @ torch.from_numpy(w0).double() + torch.from_numpy(b0).double() \
        + torch.from_numpy(x).double()
    ref = F.layer_norm(pre, [H], eps=1e-12).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)


def _nerf_a_fixture():
    import hashlib
    from gpipes.synth import nerf_a_params
    z = load_golden("nerf_a.npz")
    ws, bs = nerf_a_params(int(z["Kx"]), seed=int(z["seed"]))
    h = hashlib.sha256()
    for t in ws + bs:
        h.update(t.contiguous().view(torch.int16).numpy().tobytes())
    assert h.hexdigest() == str(z["weights_sha256"]), "nerf_a_params no longer reproduces the fixture's weights"
    f = lambda ts: [t.float().numpy() for t in ts]  # noqa: E731
    return z, f(ws), f(bs)


def test_nerf_a_golden():
    z, ws, bs = _nerf_a_fixture()
    got = oracle.nerf_a(z["x"], ws, bs)
    max_abs, rel = oracle.errors(got, z["expected"])
    assert max_abs < 1e-4 and rel < 1e-5, (max_abs, rel)


@pytest.mark.parametrize("mutant", ["skip_order", "no_skip", "skip_one_layer_early", "last_layer_no_relu",
                                    "w6_skip_rows_rotated"])
def test_nerf_a_rejects_planted_mistakes(mutant):
    """Plausible mistakes must fail the fixture at the parity bar."""
    z, ws, bs = _nerf_a_fixture()
    x = z["x"].astype(np.float32)
    lin = oracle.linear
    h = x
    nskip = 4 if mutant == "skip_one_layer_early" else 5
    for i in range(nskip):
        h = lin(h, ws[i], bs[i], oracle.ACT_RELU)
    if mutant == "skip_order":
        h = oracle.concat(x, h)
    elif mutant == "no_skip":
        h = oracle.concat(h, np.zeros_like(x))
    else:
        h = oracle.concat(h, x)
    if mutant == "skip_one_layer_early":
        h = lin(h, ws[5], bs[5], oracle.ACT_RELU)  # layer 5 never runs
    else:
        w6 = ws[5].copy()
        if mutant == "w6_skip_rows_rotated":
            w6[256:] = np.roll(w6[256:], 1, axis=0)
        h = lin(h, w6, bs[5], oracle.ACT_RELU)
    h = lin(h, ws[6], bs[6], oracle.ACT_RELU)
    h = lin(h, ws[7], bs[7], oracle.ACT_NONE if mutant == "last_layer_no_relu" else oracle.ACT_RELU)
    max_abs, rel = oracle.errors(h, z["expected"])
    assert max_abs > oracle.MAX_ABS_TOL or rel > oracle.REL_L2_TOL, (mutant, max_abs, rel)
