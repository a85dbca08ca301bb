"""GPU parity of the bert_addln_ffn and nerf_a drop-ins against the CPU oracle.

Both implementations of each are checked: the default one (one GEMM launch per
layer with fused epilogues; for nerf_a with Kx <= 64 the NeRF kernel's trunk,
all eight layers in one kernel) and the reference's queue-chained layout
(GP_IMPL_PIPELINED), whose adds (bert_addln_ffn) and skip concatenation
(nerf_a) are stages fed from ring queues.  Bar (fp16 I/O, fp32 accumulate):
max-abs <= 2e-2 and relative-L2 <= 5e-3 against the fp32 oracle on identical
fp16-rounded inputs; after every pipelined launch gpipes.pipeline_check()
confirms that no queue wait hit its bound.
"""
import numpy as np
import pytest
import torch

import gpipes
import oracle
from gpipes.synth import bert_addln_params, nerf_a_params, normal_fp16
from conftest import load_golden
from test_mgn_gpu import assert_parity

pytestmark = pytest.mark.gpu

ADDLN_KEYS = ("w0", "b0", "w1", "b1", "w2", "b2", "ga0", "be0", "ga2", "be2")
ACT_ID = {"relu": oracle.ACT_RELU, "gelu_tanh": oracle.ACT_GELU_TANH}


def f32(t):
    return None if t is None else t.detach().float().cpu().numpy()


def addln_gpu(attn, x, p, act, eps, impl):
    y = gpipes.bert_addln_ffn(attn, x, *(p[k] for k in ADDLN_KEYS), eps=eps, act=act, impl=impl)
    if impl == "pipelined":
        gpipes.pipeline_check()
    return y


def addln_oracle(attn, x, p, act, eps, rows=None):
    sel = (lambda t: t) if rows is None else (lambda t: t[rows])
    return oracle.bert_addln_ffn(sel(f32(attn)), sel(f32(x)), *(f32(p[k]) for k in ADDLN_KEYS), act=ACT_ID[act],
                                 eps=eps)


@pytest.mark.parametrize("impl", ["fused", "pipelined"])
@pytest.mark.parametrize("name", ["bert_addln_ffn.npz", "bert_addln_ffn_gelu.npz"])
@pytest.mark.parametrize("M", [1, 65, 256])
def test_bert_addln_golden(cuda, impl, name, M):
    z = load_golden(name)
    if impl == "pipelined" and z["w1"].shape != (128, 512):
        pytest.skip("the pipelined layout is built for the app's shape H 128, FF 512")
    p = {k: torch.from_numpy(z[k]).to(cuda) for k in ADDLN_KEYS}
    attn, x = (torch.from_numpy(z[k][:M]).to(cuda) for k in ("attn", "x"))
    got = addln_gpu(attn, x, p, str(z["act"]), float(z["eps"]), impl)
    assert_parity(f32(got), z["expected"][:M], f"{impl} {name} M={M}")


@pytest.mark.parametrize("H,FF", [(128, 512), (256, 384), (1024, 4096)])
@pytest.mark.parametrize("act", ["relu", "gelu_tanh"])
@pytest.mark.parametrize("M", [1, 300, 20000])
def test_bert_addln_fused_shapes(cuda, H, FF, act, M):
    p = {k: v.to(cuda) for k, v in bert_addln_params(H, FF, seed=H + M, init="torch" if H == 128 else "bert",
                                                     affine_random=True).items()}
    attn, x = normal_fp16(M, H, seed=M).to(cuda), normal_fp16(M, H, seed=M + 1).to(cuda)
    got = f32(addln_gpu(attn, x, p, act, 1e-5, "fused"))
    rows = np.linspace(0, M - 1, min(M, 1500)).astype(np.int64)
    assert_parity(got[rows], addln_oracle(attn, x, p, act, 1e-5, rows), f"fused H={H} FF={FF} {act} M={M}")


@pytest.mark.parametrize("act", ["relu", "gelu_tanh"])
@pytest.mark.parametrize("M", [1, 127, 128, 129, 1000, 64 * 512, 100003])
def test_bert_addln_pipelined(cuda, act, M):
    """M = 64 x 512 is the reference's val.py / perf.py batch; 100003 gives every
    pipeline several tiles and a partial last tile."""
    p = {k: v.to(cuda) for k, v in bert_addln_params(seed=M, affine_random=True).items()}
    attn, x = normal_fp16(M, 128, seed=M + 2).to(cuda), normal_fp16(M, 128, seed=M + 3).to(cuda)
    got = f32(addln_gpu(attn, x, p, act, 1e-5, "pipelined"))
    rows = np.linspace(0, M - 1, min(M, 2000)).astype(np.int64)
    assert_parity(got[rows], addln_oracle(attn, x, p, act, 1e-5, rows), f"pipelined {act} M={M}")
    assert np.isfinite(got).all()


def test_bert_addln_no_bias_no_affine(cuda):
    M = 700
    p = {k: v.to(cuda) for k, v in bert_addln_params(seed=5).items()}
    for k in ("b0", "b1", "b2", "ga0", "be0", "ga2", "be2"):
        p[k] = None
    attn, x = normal_fp16(M, 128, seed=8).to(cuda), normal_fp16(M, 128, seed=9).to(cuda)
    want = addln_oracle(attn, x, p, "relu", 1e-5)
    for impl in ("fused", "pipelined"):
        assert_parity(f32(addln_gpu(attn, x, p, "relu", 1e-5, impl)), want, f"{impl} no bias / affine")


def test_bert_addln_pipelined_deterministic_and_reentrant(cuda):
    """Back-to-back launches on one arena (epoch-tagged queues) and a second
    stream give bit-identical outputs; the two implementations agree."""
    M = 64 * 512
    p = {k: v.to(cuda) for k, v in bert_addln_params(seed=0).items()}
    attn, x = normal_fp16(M, 128, seed=0).to(cuda), normal_fp16(M, 128, seed=1).to(cuda)
    a = addln_gpu(attn, x, p, "relu", 1e-5, "pipelined")
    b = addln_gpu(attn, x, p, "relu", 1e-5, "pipelined")
    s = torch.cuda.Stream(device=cuda)
    with torch.cuda.stream(s):
        c = addln_gpu(attn, x, p, "relu", 1e-5, "pipelined")
    s.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(a.view(torch.int16), c.view(torch.int16))
    fused = addln_gpu(attn, x, p, "relu", 1e-5, "fused")
    assert_parity(f32(a), f32(fused).astype(np.float64), "pipelined vs fused")


def test_bert_addln_rejects(cuda):
    M = 64
    p = {k: v.to(cuda) for k, v in bert_addln_params(256, 512, seed=1).items()}
    attn, x = normal_fp16(M, 256).to(cuda), normal_fp16(M, 256).to(cuda)
    with pytest.raises(gpipes.GpipesError) as ei:
        gpipes.bert_addln_ffn(attn, x, *(p[k] for k in ADDLN_KEYS), impl="pipelined")
    assert ei.value.code == -2  # the pipelined layout is H 128 / FF 512 only


# ---------------------------------------------------------------------------- nerf_a

def nerf_a_gpu(x, ws, bs, impl):
    wb = [t for pair in zip(ws, bs) for t in pair]
    y = gpipes.nerf_a(x, *wb, impl=impl)
    if impl == "pipelined":
        gpipes.pipeline_check()
    return y


def nerf_a_oracle(x, ws, bs, rows=None):
    xs = f32(x) if rows is None else f32(x)[rows]
    return oracle.nerf_a(xs, [f32(w) for w in ws], [f32(b) for b in bs])


def scaled(ws, bs, s):
    return [(w.float() * s).half() for w in ws], [(b.float() * s).half() for b in bs]


@pytest.mark.parametrize("impl", ["fused", "pipelined"])
@pytest.mark.parametrize("M", [1, 63, 256])
def test_nerf_a_golden(cuda, impl, M):
    z = load_golden("nerf_a.npz")
    ws, bs = nerf_a_params(int(z["Kx"]), seed=int(z["seed"]), device=cuda)
    x = torch.from_numpy(z["x"][:M]).to(cuda)
    assert_parity(f32(nerf_a_gpu(x, ws, bs, impl)), z["expected"][:M], f"nerf_a {impl} M={M}")


@pytest.mark.parametrize("impl,Kx", [("fused", 64), ("fused", 60), ("fused", 63), ("fused", 39), ("fused", 3),
                                     ("fused", 200),
                                     ("pipelined", 64), ("pipelined", 8), ("pipelined", 120), ("pipelined", 128)])
@pytest.mark.parametrize("scale", [1.0, 2.0])
@pytest.mark.parametrize("M", [1, 65, 3000, 70001])
def test_nerf_a_shapes(cuda, impl, Kx, scale, M):
    """Weights x2 keep every layer's contribution visible through the eight ReLU layers."""
    ws, bs = scaled(*nerf_a_params(Kx, seed=M + Kx), scale)
    x = normal_fp16(M, Kx, seed=M)
    got = f32(nerf_a_gpu(x.to(cuda), [w.to(cuda) for w in ws], [b.to(cuda) for b in bs], impl))
    rows = np.linspace(0, M - 1, min(M, 1200)).astype(np.int64)
    assert_parity(got[rows], nerf_a_oracle(x, ws, bs, rows), f"nerf_a {impl} Kx={Kx} x{scale} M={M}")


def test_nerf_a_rejects_unaligned_out(cuda):
    """Every NerfA path writes out in 16-byte stores: an out that starts 2 bytes past an
    aligned base is rejected with GP_ERR_ALIGN for both implementations, and nothing is written."""
    M = 300
    ws, bs = nerf_a_params(64, seed=5, device=cuda)
    x = normal_fp16(M, 64, seed=6).to(cuda)
    buf = torch.full((M * 256 + 8,), 3.0, dtype=torch.float16, device=cuda)
    out = buf[1:1 + M * 256].view(M, 256)
    wb = [t for pair in zip(ws, bs) for t in pair]
    for impl in ("fused", "pipelined"):
        with pytest.raises(gpipes.GpipesError) as e:
            gpipes.nerf_a_out(x, *wb, out, impl=impl)
        assert e.value.code == -3, impl
    torch.cuda.synchronize()
    assert bool((buf == 3.0).all())


def test_nerf_a_no_bias_and_agreement(cuda):
    M = 5000
    ws, bs = scaled(*nerf_a_params(64, seed=3, device=cuda), 2.0)
    x = normal_fp16(M, 64, seed=4).to(cuda)
    nb = [None] * 8
    want = nerf_a_oracle(x, ws, [torch.zeros(256)] * 8)
    a = nerf_a_gpu(x, ws, nb, "fused")
    b = nerf_a_gpu(x, ws, nb, "pipelined")
    assert_parity(f32(a), want, "fused no bias")
    assert_parity(f32(b), want, "pipelined no bias")
    b2 = nerf_a_gpu(x, ws, nb, "pipelined")
    assert torch.equal(b.view(torch.int16), b2.view(torch.int16))


def test_nerf_a_fused_kernel_matches_layer_chain(cuda):
    """Kx <= 64 runs the NeRF kernel's trunk (one kernel for all eight layers),
    wider inputs one GEMM launch per layer: the same network with x
    zero-padded from 64 to 72 columns (zero weight rows for the padding) takes
    the chain, and both agree with each other and with the oracle.  A row slice
    at an odd, unaligned offset (copied to an aligned base first) and a
    second stream reproduce the rows bit for bit."""
    M = 70001
    ws, bs = scaled(*nerf_a_params(64, seed=21, device=cuda), 2.0)
    x = normal_fp16(M, 64, seed=22).to(cuda)
    x72 = torch.zeros((M, 72), dtype=torch.float16, device=cuda)
    x72[:, :64] = x
    w72 = list(ws)
    w72[0] = torch.cat([ws[0], torch.zeros((8, 256), dtype=torch.float16, device=cuda)])
    w72[5] = torch.cat([ws[5], torch.zeros((8, 256), dtype=torch.float16, device=cuda)])
    a = nerf_a_gpu(x, ws, bs, "fused")
    c = nerf_a_gpu(x72, w72, bs, "fused")
    assert_parity(f32(a), f32(c), "nerf_a fused kernel vs GEMM chain")
    rows = np.r_[0:300, 65400:65700, M - 300:M]
    assert_parity(f32(a)[rows], nerf_a_oracle(x, ws, bs, rows), "nerf_a fused kernel vs oracle")
    buf = torch.empty(M * 64 + 1, dtype=torch.float16, device=cuda)
    xs = buf[1:1 + 3001 * 64].view(3001, 64)
    xs.copy_(x[997:3998])
    s = nerf_a_gpu(xs, ws, bs, "fused")
    assert torch.equal(s.view(torch.int16), a[997:3998].view(torch.int16))
    st = torch.cuda.Stream(device=cuda)
    with torch.cuda.stream(st):
        a2 = nerf_a_gpu(x, ws, bs, "fused")
    st.synchronize()
    assert torch.equal(a2.view(torch.int16), a.view(torch.int16))


def test_nerf_a_rejects(cuda):
    M = 64
    ws, bs = nerf_a_params(60, seed=1, device=cuda)
    x = normal_fp16(M, 60).to(cuda)
    with pytest.raises(gpipes.GpipesError) as ei:
        nerf_a_gpu(x, ws, bs, "pipelined")
    assert ei.value.code == -2  # Kx must be a multiple of 8 for the pipelined layout
