"""Generate the golden fixtures under tests/golden/ (run from the repo root).

The reference ships no fixture files and its validation scripts assert nothing
(apps/*/pipelined/val.py only print errors), so the vectors are produced
here from first principles:

* inputs: X ~ N(0,1) and torch.nn default-initialised MgnMlp parameters
  (nn.Linear / nn.LayerNorm built in the order of common/mlps.py:3-20),
  everything rounded to fp16 exactly as the kernels receive it;
* expected outputs: the torch.nn library modules (Linear, ReLU, LayerNorm)
  evaluated in float64 on the fp16-rounded values -- an implementation
  independent of both the C oracle and the HIP kernels.

The BERT FFN fixtures follow the module structure of
apps/bert_ffn/torch/model.py:3-14 (Linear -> activation -> Linear, + x,
LayerNorm), once with the reference app's shape and defaults (H 128, FF 512,
ReLU, eps 1e-5, nn.Linear init) and once with the BERT-large recipe (GELU(tanh),
eps 1e-12, N(0, 0.02) weights, zero biases) at a small width; expected outputs
are again the torch.nn modules in float64.

The DLRM fixtures are DlrmMlp (common/mlps.py:23-34) built from torch.nn
modules in float64; the NeRF fixture follows the module structure of
apps/nerf_full/torch/model.py:5-66.  Its 1.2 MB of weights are not stored:
gpipes.synth.nerf_params regenerates them from the seed, and the fixture
keeps their SHA-256 so a changed generator is detected.

The LayerNorm fixture uses the literal 128-value input row that the
reference's own LayerNorm check types in (misc_tests/layer_norm/torch_val.py:88-105,
repeated over 128 rows there, gamma = 1, beta = 0); its expected output is
F.layer_norm in float64.

The bf16 MGN fixtures are the same MgnMlp with inputs and parameters rounded to
bfloat16 (stored as uint16 bit patterns), expected again from torch.nn in float64;
bert_ffn_gelu_bf16 is the BERT FFN block the same way.

The bert_addln_ffn fixtures follow apps/bert_addln_ffn/torch/model.py:3-20 and the
nerf_a fixture apps/nerf_a/torch/model.py:5-38, each evaluated with torch.nn modules in
float64 (the nerf_a weights are regenerated from the seed, as for NeRF).

Usage: python tests/golden/gen_fixtures.py [fixture names...]   (default: all)
"""
import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "gpu-pipes_amd"))
from gpipes.synth import (bert_addln_params, bert_params, dlrm_params, mgn_params, nerf_a_params,  # noqa: E402
                          nerf_inputs, nerf_params, normal_fp16)

M_FIX = 256

# misc_tests/layer_norm/torch_val.py:88-105 (fp16 in the reference)
LN_ROW = [
    0.0584, -0.0362, -0.0660, 0.0422, 0.0275, -0.0063, 0.0683, 0.0086,
    0.0682, 0.0531, -0.0416, -0.0233, 0.1115, 0.0872, 0.0444, -0.1655,
    -0.0645, -0.0249, -0.1387, 0.0323, 0.0275, 0.0374, -0.0202, -0.1707,
    -0.0095, 0.0696, -0.0305, -0.0340, -0.1326, -0.0438, 0.1910, 0.0103,
    -0.0041, -0.0133, 0.0273, -0.0519, -0.0641, -0.0294, 0.1016, -0.0116,
    0.2269, -0.0229, -0.0088, -0.0543, 0.1884, 0.2455, -0.0098, 0.0155,
    0.0209, 0.0940, -0.0056, 0.2769, 0.0936, 0.0133, -0.1065, 0.1091,
    0.0047, 0.0628, 0.0091, -0.0368, 0.0240, 0.0104, -0.0033, 0.1326,
    -0.1333, 0.2052, 0.0168, 0.1188, -0.2090, -0.1128, -0.1947, -0.1901,
    0.0079, -0.0408, 0.0222, 0.0292, 0.0156, 0.0968, 0.0820, -0.0456,
    -0.1573, 0.0282, -0.0734, 0.0977, -0.0263, -0.2069, 0.0491, 0.1038,
    -0.0596, -0.1426, 0.0345, -0.1094, 0.0271, -0.1213, 0.1202, -0.0337,
    -0.0151, -0.0343, -0.0700, -0.2043, -0.0188, 0.0386, 0.0837, 0.0340,
    -0.0264, 0.0816, -0.0600, -0.0872, -0.0091, 0.0435, -0.0995, 0.0306,
    0.1932, 0.0959, 0.0385, -0.0917, 0.0891, 0.1542, 0.0395, 0.1276,
    0.0145, -0.0723, 0.0550, 0.0746, -0.0141, 0.0147, 0.2205, -0.0380,
]


def torch_mgn_f64(x16, p, eps):
    """MgnMlp forward with torch.nn library modules in float64."""
    K = x16.shape[1]
    seq = [torch.nn.Linear(K, 128), torch.nn.ReLU(), torch.nn.Linear(128, 128), torch.nn.ReLU(),
           torch.nn.Linear(128, 128)]
    if p["gamma"] is not None:
        seq.append(torch.nn.LayerNorm(128, eps=eps))
    net = torch.nn.Sequential(*seq).double()
    with torch.no_grad():
        for idx, (w, b) in zip((0, 2, 4), (("w1", "b1"), ("w2", "b2"), ("w3", "b3"))):
            net[idx].weight.copy_(p[w].double().t())
            net[idx].bias.copy_(p[b].double())
        if p["gamma"] is not None:
            net[5].weight.copy_(p["gamma"].double())
            net[5].bias.copy_(p["beta"].double())
        return net(x16.double())


def make_mgn_fixture(name, K, layernorm, seed, affine_random, eps=1e-5):
    p = mgn_params(K, seed=seed, layernorm=layernorm, affine_random=affine_random)
    x = normal_fp16(M_FIX, K, seed=seed + 1000)
    y = torch_mgn_f64(x, p, eps)
    arrs = {"x": x.numpy(), "expected": y.numpy().astype(np.float64), "eps": np.float64(eps)}
    for k, v in p.items():
        if v is not None:
            arrs[k] = v.numpy()
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **arrs)
    return path


def bf16_bits(t):
    """bfloat16 tensor -> its uint16 bit patterns (numpy has no bfloat16)."""
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def make_mgn_bf16_fixture(name, K, seed, eps=1e-5):
    """MgnMlp with bf16 inputs and parameters (stored as uint16 bit patterns,
    key `dtype` = "bf16"); expected = torch.nn modules in float64 on the
    bf16 values."""
    p = mgn_params(K, seed=seed, layernorm=True, affine_random=True, dtype=torch.bfloat16)
    x = normal_fp16(M_FIX, K, seed=seed + 1000, dtype=torch.bfloat16)
    y = torch_mgn_f64(x, p, eps)
    arrs = {"x": bf16_bits(x), "expected": y.numpy().astype(np.float64), "eps": np.float64(eps),
            "dtype": np.array("bf16")}
    for k, v in p.items():
        arrs[k] = bf16_bits(v)
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **arrs)
    return path


def torch_bert_ffn_f64(x16, p, act, eps):
    """BERT FFN block, LayerNorm(Linear2(act(Linear1(x))) + x), with torch.nn
    library modules in float64 (the module structure of
    apps/bert_ffn/torch/model.py:3-14, activation and eps as given)."""
    H, FF = p["w1"].shape
    a = torch.nn.ReLU() if act == "relu" else torch.nn.GELU(approximate="tanh")
    ffn = torch.nn.Sequential(torch.nn.Linear(H, FF), a, torch.nn.Linear(FF, H)).double()
    ln = torch.nn.LayerNorm(H, eps=eps).double()
    with torch.no_grad():
        ffn[0].weight.copy_(p["w1"].double().t())
        ffn[0].bias.copy_(p["b1"].double())
        ffn[2].weight.copy_(p["w2"].double().t())
        ffn[2].bias.copy_(p["b2"].double())
        ln.weight.copy_(p["gamma"].double())
        ln.bias.copy_(p["beta"].double())
        xd = x16.double()
        return ln(ffn(xd) + xd)


def make_bert_fixture(name, M, H, FF, act, eps, init, seed, affine_random):
    p = bert_params(H, FF, seed=seed, init=init, affine_random=affine_random)
    x = normal_fp16(M, H, seed=seed + 1000)
    y = torch_bert_ffn_f64(x, p, act, eps)
    arrs = {"x": x.numpy(), "expected": y.numpy().astype(np.float32), "eps": np.float64(eps),
            "act": np.array(act)}
    for k, v in p.items():
        arrs[k] = v.numpy()
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **arrs)
    return path


def make_bert_bf16_fixture(name, M, H, FF, act, eps, seed):
    """The BERT FFN block with bf16 inputs and parameters (stored as uint16 bit
    patterns, key `dtype` = "bf16"); expected = torch.nn modules in float64 on
    the bf16 values."""
    p = {k: v.to(torch.bfloat16) for k, v in bert_params(H, FF, seed=seed, init="bert", affine_random=True).items()}
    x = normal_fp16(M, H, seed=seed + 1000, dtype=torch.bfloat16)
    y = torch_bert_ffn_f64(x, p, act, eps)
    arrs = {"x": bf16_bits(x), "expected": y.numpy().astype(np.float64), "eps": np.float64(eps),
            "act": np.array(act), "dtype": np.array("bf16")}
    for k, v in p.items():
        arrs[k] = bf16_bits(v)
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **arrs)
    return path


def torch_dlrm_f64(x16, ws, bs, sigmoid_i=None):
    """DlrmMlp(widths, sigmoid_i) (common/mlps.py:23-34) with torch.nn modules in float64."""
    mods = []
    for i, (w, b) in enumerate(zip(ws, bs)):
        lin = torch.nn.Linear(w.shape[0], w.shape[1]).double()
        with torch.no_grad():
            lin.weight.copy_(w.double().t())
            lin.bias.copy_(b.double())
        mods += [lin, torch.nn.Sigmoid() if i == sigmoid_i else torch.nn.ReLU()]
    with torch.no_grad():
        return torch.nn.Sequential(*mods)(x16.double())


def make_dlrm_fixture(name, M, widths, sigmoid_i, init, seed):
    ws, bs = dlrm_params(widths, seed=seed, init=init)
    x = normal_fp16(M, widths[0], seed=seed + 1000)
    y = torch_dlrm_f64(x, ws, bs, sigmoid_i)
    arrs = {"x": x.numpy(), "expected": y.numpy().astype(np.float32),
            "sigmoid_i": np.int64(-1 if sigmoid_i is None else sigmoid_i)}
    for i, (w, b) in enumerate(zip(ws, bs)):
        arrs[f"w{i + 1}"], arrs[f"b{i + 1}"] = w.numpy(), b.numpy()
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **arrs)
    return path


def torch_nerf_f64(x16, d16, ws, bs, sigmoid):
    """The NeRF MLP with the module structure of apps/nerf_full/torch/model.py:5-66
    (hidden 256, skip after the fifth layer, view directions), torch.nn in float64;
    sigmoid adds the workload's colour activation."""
    def lin(i):
        m = torch.nn.Linear(ws[i].shape[0], ws[i].shape[1]).double()
        with torch.no_grad():
            m.weight.copy_(ws[i].double().t())
            m.bias.copy_(bs[i].double())
        return m
    relu = torch.nn.ReLU
    preskip = torch.nn.Sequential(lin(0), relu(), lin(1), relu(), lin(2), relu(), lin(3), relu(), lin(4), relu())
    postskip = torch.nn.Sequential(lin(5), relu(), lin(6), relu(), lin(7), relu())
    alpha, bottleneck = lin(8), lin(9)
    rgb = torch.nn.Sequential(lin(10), relu(), lin(11), *([torch.nn.Sigmoid()] if sigmoid else []))
    with torch.no_grad():
        x, d = x16.double(), d16.double()
        enc = postskip(torch.cat([preskip(x), x], dim=-1))
        return alpha(enc), rgb(torch.cat([bottleneck(enc), d], dim=-1))


def weights_digest(ws, bs):
    h = hashlib.sha256()
    for t in list(ws) + list(bs):
        h.update(t.contiguous().view(torch.int16).numpy().tobytes())
    return h.hexdigest()


def make_nerf_fixture(name, M, seed, Kd, Na, Nrgb, sigmoid):
    """Inputs and expected outputs; the 1.2 MB of weights are regenerated from the
    seed by gpipes.synth.nerf_params and checked against the stored digest."""
    ws, bs = nerf_params(64, Kd, Na, Nrgb, seed=seed)
    x, d = nerf_inputs(M, seed=seed + 1000, Kx=64, Kd=Kd)
    alpha, rgb = torch_nerf_f64(x, d, ws, bs, sigmoid)
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, x=x.numpy(), d=d.numpy(), alpha=alpha.numpy().astype(np.float32),
                        rgb=rgb.numpy().astype(np.float32), seed=np.int64(seed), Kd=np.int64(Kd), Na=np.int64(Na),
                        Nrgb=np.int64(Nrgb), sigmoid=np.int64(sigmoid), weights_sha256=np.array(weights_digest(ws, bs)))
    return path


def torch_bert_addln_f64(attn16, x16, p, act, eps):
    """The add + LayerNorm + FFN block with the module structure of
    apps/bert_addln_ffn/torch/model.py:3-20 (y0w0, ln0, ffn, ln2; forward
    ln2(ffn(h) + h) with h = ln0(y0w0(attn) + x)), torch.nn in float64."""
    H, FF = p["w1"].shape
    a = torch.nn.ReLU() if act == "relu" else torch.nn.GELU(approximate="tanh")
    y0w0 = torch.nn.Linear(H, H).double()
    ln0 = torch.nn.LayerNorm(H, eps=eps).double()
    ffn = torch.nn.Sequential(torch.nn.Linear(H, FF), a, torch.nn.Linear(FF, H)).double()
    ln2 = torch.nn.LayerNorm(H, eps=eps).double()
    with torch.no_grad():
        y0w0.weight.copy_(p["w0"].double().t())
        y0w0.bias.copy_(p["b0"].double())
        ffn[0].weight.copy_(p["w1"].double().t())
        ffn[0].bias.copy_(p["b1"].double())
        ffn[2].weight.copy_(p["w2"].double().t())
        ffn[2].bias.copy_(p["b2"].double())
        ln0.weight.copy_(p["ga0"].double())
        ln0.bias.copy_(p["be0"].double())
        ln2.weight.copy_(p["ga2"].double())
        ln2.bias.copy_(p["be2"].double())
        h = ln0(y0w0(attn16.double()) + x16.double())
        return ln2(ffn(h) + h)


def make_bert_addln_fixture(name, M, H, FF, act, eps, init, seed):
    p = bert_addln_params(H, FF, seed=seed, init=init, affine_random=True)
    attn = normal_fp16(M, H, seed=seed + 1000)
    x = normal_fp16(M, H, seed=seed + 2000)
    y = torch_bert_addln_f64(attn, x, p, act, eps)
    arrs = {"attn": attn.numpy(), "x": x.numpy(), "expected": y.numpy().astype(np.float32), "eps": np.float64(eps),
            "act": np.array(act)}
    for k, v in p.items():
        arrs[k] = v.numpy()
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **arrs)
    return path


def torch_nerf_a_f64(x16, ws, bs):
    """NerfA with the module structure of apps/nerf_a/torch/model.py:5-38 (preskip:
    five Linear + ReLU; resid = cat([preskip(x), x]); postskip: three Linear + ReLU),
    torch.nn in float64."""
    def lin(i):
        m = torch.nn.Linear(ws[i].shape[0], ws[i].shape[1]).double()
        with torch.no_grad():
            m.weight.copy_(ws[i].double().t())
            m.bias.copy_(bs[i].double())
        return m
    relu = torch.nn.ReLU
    preskip = torch.nn.Sequential(*[m for i in range(5) for m in (lin(i), relu())])
    postskip = torch.nn.Sequential(*[m for i in range(5, 8) for m in (lin(i), relu())])
    with torch.no_grad():
        x = x16.double()
        return postskip(torch.cat([preskip(x), x], dim=-1))


def make_nerf_a_fixture(name, M, seed, Kx):
    """Inputs and expected outputs; the weights are regenerated from the seed by
    gpipes.synth.nerf_a_params and checked against the stored digest."""
    ws, bs = nerf_a_params(Kx, seed=seed)
    x = normal_fp16(M, Kx, seed=seed + 1000)
    y = torch_nerf_a_f64(x, ws, bs)
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, x=x.numpy(), expected=y.numpy().astype(np.float32), seed=np.int64(seed),
                        Kx=np.int64(Kx), weights_sha256=np.array(weights_digest(ws, bs)))
    return path


def make_ln_fixture():
    row = torch.tensor(LN_ROW, dtype=torch.float16)
    x = row.repeat(128, 1)
    y = torch.nn.functional.layer_norm(x.double(), [128], weight=torch.ones(128, dtype=torch.float64),
                                       bias=torch.zeros(128, dtype=torch.float64), eps=1e-5)
    path = os.path.join(HERE, "layer_norm_row.npz")
    np.savez_compressed(path, x=x.numpy(), expected=y.numpy(), eps=np.float64(1e-5))
    return path


FIXTURES = {
    "mgn_edge_ln": lambda: make_mgn_fixture("mgn_edge_ln", 384, True, seed=0, affine_random=False),
    "mgn_edge_ln_affine": lambda: make_mgn_fixture("mgn_edge_ln_affine", 384, True, seed=1, affine_random=True),
    "mgn_edge_linears": lambda: make_mgn_fixture("mgn_edge_linears", 384, False, seed=2, affine_random=False),
    "mgn_node_ln": lambda: make_mgn_fixture("mgn_node_ln", 256, True, seed=3, affine_random=True),
    "layer_norm_row": make_ln_fixture,
    # the reference app's shape and defaults (H 128, FF 512, ReLU, eps 1e-5)
    "bert_ffn_relu": lambda: make_bert_fixture("bert_ffn_relu", 256, 128, 512, "relu", 1e-5, "torch", seed=10,
                                               affine_random=False),
    # DlrmMlp at the reference's bottom-MLP shape, and a narrow chain with a sigmoid head
    "dlrm_bot": lambda: make_dlrm_fixture("dlrm_bot", 64, [32, 512, 256, 128], None, "torch", seed=20),
    "dlrm_sigmoid_head": lambda: make_dlrm_fixture("dlrm_sigmoid_head", 64, [24, 256, 128, 1], 2, "xavier", seed=21),
    # the NeRF MLP at the workload's shape (view dirs 27, density 1, colour 3 + sigmoid)
    "nerf_workload": lambda: make_nerf_fixture("nerf_workload", 64, seed=22, Kd=27, Na=1, Nrgb=3, sigmoid=True),
    # the BERT-large recipe (GELU(tanh), eps 1e-12, N(0, 0.02) weights) at a small width
    "bert_ffn_gelu": lambda: make_bert_fixture("bert_ffn_gelu", 128, 256, 512, "gelu_tanh", 1e-12, "bert", seed=11,
                                               affine_random=True),
    # the reference app bert_addln_ffn at its shape (H 128, FF 512, ReLU, eps 1e-5, nn.Linear
    # init), with distinct LayerNorm affines, and the BERT-large recipe at a small width
    "bert_addln_ffn": lambda: make_bert_addln_fixture("bert_addln_ffn", 256, 128, 512, "relu", 1e-5, "torch",
                                                      seed=30),
    "bert_addln_ffn_gelu": lambda: make_bert_addln_fixture("bert_addln_ffn_gelu", 128, 256, 512, "gelu_tanh", 1e-12,
                                                           "bert", seed=31),
    # NerfA at the reference app's input width (64)
    "nerf_a": lambda: make_nerf_a_fixture("nerf_a", 256, seed=32, Kx=64),
    # MgnMlp in bfloat16 (edge and node widths)
    "mgn_edge_ln_bf16": lambda: make_mgn_bf16_fixture("mgn_edge_ln_bf16", 384, seed=40),
    "mgn_node_ln_bf16": lambda: make_mgn_bf16_fixture("mgn_node_ln_bf16", 256, seed=41),
    # the BERT-large recipe in bfloat16 at a small width
    "bert_ffn_gelu_bf16": lambda: make_bert_bf16_fixture("bert_ffn_gelu_bf16", 128, 256, 512, "gelu_tanh", 1e-12,
                                                         seed=42),
}


def main():
    """Regenerate the fixtures named on the command line (default: all) and
    update their entries of MANIFEST.json."""
    names = sys.argv[1:] or list(FIXTURES)
    paths = [FIXTURES[n]() for n in names]
    mpath = os.path.join(HERE, "MANIFEST.json")
    with open(mpath) as f:
        manifest = json.load(f)
    for pth in paths:
        with open(pth, "rb") as f:
            manifest[os.path.basename(pth)] = hashlib.sha256(f.read()).hexdigest()
    with open(os.path.join(HERE, "MANIFEST.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print(json.dumps(manifest, indent=1))


if __name__ == "__main__":
    main()
