"""Deterministic synthetic inputs for the MGN MLP, BERT FFN, DLRM and NeRF workloads.

Parameters follow torch.nn defaults, which is what the workload definition
asks for: Linear weights Kaiming-uniform(a=sqrt(5)) = U(+-1/sqrt(fan_in)),
biases U(+-1/sqrt(fan_in)), LayerNorm gamma = 1, beta = 0; X ~ N(0, 1).
Weights are returned in the kernel layout [K, N] (nn.Linear.weight.t()),
all fp16, as apps/mgn_fullmlp/pipelined/val.py:15-21 feeds them.
"""
import torch


def mgn_params(K, seed=0, layernorm=True, device="cpu", affine_random=False, dtype=torch.float16):
    """Parameters of MgnMlp(K, [128, 128, 128], layernorm) in kernel layout,
    rounded to `dtype` (float16 or bfloat16)."""
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        l1 = torch.nn.Linear(K, 128)
        l2 = torch.nn.Linear(128, 128)
        l3 = torch.nn.Linear(128, 128)
        lnm = torch.nn.LayerNorm(128) if layernorm else None
        if lnm is not None and affine_random:
            with torch.no_grad():
                lnm.weight.uniform_(0.5, 1.5)
                lnm.bias.uniform_(-0.5, 0.5)

    def h(t):
        return t.detach().to(dtype).contiguous().to(device)

    p = {
        "w1": h(l1.weight.t()), "b1": h(l1.bias),
        "w2": h(l2.weight.t()), "b2": h(l2.bias),
        "w3": h(l3.weight.t()), "b3": h(l3.bias),
        "gamma": h(lnm.weight) if lnm is not None else None,
        "beta": h(lnm.bias) if lnm is not None else None,
    }
    return p


def bert_params(H, FF, seed=0, init="bert", device="cpu", affine_random=False):
    """Parameters of the BERT FFN block (Linear(H, FF), Linear(FF, H), LayerNorm(H))
    in kernel layout.  init="bert": weights ~ N(0, 0.02), biases 0 (the BERT-large
    workload); init="torch": nn.Linear defaults, as apps/bert_ffn/torch/model.py:3-11
    builds them.  LayerNorm gamma = 1, beta = 0 unless affine_random."""
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        l1 = torch.nn.Linear(H, FF)
        l2 = torch.nn.Linear(FF, H)
        lnm = torch.nn.LayerNorm(H)
        with torch.no_grad():
            if init == "bert":
                for lin in (l1, l2):
                    lin.weight.normal_(0.0, 0.02)
                    lin.bias.zero_()
            elif init != "torch":
                raise ValueError(f"unknown init {init!r}")
            if affine_random:
                lnm.weight.uniform_(0.5, 1.5)
                lnm.bias.uniform_(-0.5, 0.5)

    def h(t):
        return t.detach().to(torch.float16).contiguous().to(device)

    return {"w1": h(l1.weight.t()), "b1": h(l1.bias), "w2": h(l2.weight.t()), "b2": h(l2.bias),
            "gamma": h(lnm.weight), "beta": h(lnm.bias)}


def normal_fp16(M, K, seed=0, device="cpu", dtype=torch.float16):
    """X ~ N(0, 1) rounded to fp16 (or `dtype`), generated on `device` with a seeded generator."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn((M, K), generator=g, device=dev, dtype=torch.float32).to(dtype)


def dlrm_params(widths, seed=0, init="xavier", device="cpu"):
    """Parameters of DlrmMlp(widths) (common/mlps.py:23-34) in kernel layout:
    init="xavier" draws the weights Xavier-uniform (the DLRM workload), "torch"
    keeps nn.Linear's defaults; biases keep nn.Linear's default init."""
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        lins = [torch.nn.Linear(widths[i], widths[i + 1]) for i in range(len(widths) - 1)]
        with torch.no_grad():
            if init == "xavier":
                for lin in lins:
                    torch.nn.init.xavier_uniform_(lin.weight)
            elif init != "torch":
                raise ValueError(f"unknown init {init!r}")
    ws = [lin.weight.detach().t().contiguous().to(torch.float16).to(device) for lin in lins]
    bs = [lin.bias.detach().to(torch.float16).to(device) for lin in lins]
    return ws, bs


def padded_uniform(M, K, Kp, seed=0, device="cpu"):
    """U(0, 1) dense features [M, K] zero-padded to [M, Kp] (DLRM bottom input)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.zeros((M, Kp), dtype=torch.float32)
    x[:, :K] = torch.rand((M, K), generator=g)
    return x.to(torch.float16).to(device)


def padded_normal(M, K, Kp, seed=0, device="cpu"):
    """N(0, 1) features [M, K] zero-padded to [M, Kp] (DLRM top input)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.zeros((M, Kp), dtype=torch.float32)
    x[:, :K] = torch.randn((M, K), generator=g)
    return x.to(torch.float16).to(device)


def positional_encoding(M, octaves, seed=0, device="cpu", unit=False):
    """NeRF positional encoding: [p, sin(2^i p), cos(2^i p) for i < octaves] of
    p ~ U(-1, 1)^3 (or random unit directions), width 3 + 6 octaves."""
    g = torch.Generator().manual_seed(seed)
    p = torch.rand((M, 3), generator=g, dtype=torch.float64) * 2 - 1
    if unit:
        p = p / p.norm(dim=1, keepdim=True).clamp_min(1e-6)
    feats = [p]
    for i in range(octaves):
        feats += [torch.sin((2.0 ** i) * p), torch.cos((2.0 ** i) * p)]
    return torch.cat(feats, dim=1).to(torch.float16).to(device)


def nerf_inputs(M, seed=0, device="cpu", Kx=64, Kd=27):
    """x: encoded positions (63 features, 10 octaves) zero-padded to Kx; d: encoded
    view directions (27 features, 4 octaves) padded to Kd."""
    x = torch.zeros((M, Kx), dtype=torch.float16)
    x[:, :63] = positional_encoding(M, 10, seed=seed)
    d = torch.zeros((M, Kd), dtype=torch.float16)
    d[:, :27] = positional_encoding(M, 4, seed=seed + 1, unit=True)
    return x.to(device), d.to(device)


def nerf_params(Kx=64, Kd=27, Na=1, Nrgb=3, seed=0, device="cpu", zero_pad_rows=63):
    """Parameters w1..w12 / b1..b12 of the NeRF MLP (apps/nerf_full/torch/model.py:5-46,
    hidden 256) in kernel layout with nn.Linear's default (Kaiming-uniform) init.  The
    weight rows of input columns at and past zero_pad_rows (the zero padding of x) are
    set to zero in w1 and in the skip part of w6."""
    shapes = [(Kx, 256)] + [(256, 256)] * 4 + [(256 + Kx, 256), (256, 256), (256, 256), (256, Na), (256, 256),
                                                (256 + Kd, 128), (128, Nrgb)]
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        lins = [torch.nn.Linear(k, n) for k, n in shapes]
    ws = [lin.weight.detach().t().contiguous() for lin in lins]
    bs = [lin.bias.detach() for lin in lins]
    if zero_pad_rows is not None and zero_pad_rows < Kx:
        ws[0][zero_pad_rows:] = 0
        ws[5][256 + zero_pad_rows:] = 0
    h = lambda t: t.to(torch.float16).contiguous().to(device)  # noqa: E731
    return [h(w) for w in ws], [h(b) for b in bs]


def bert_addln_params(H=128, FF=512, seed=0, init="torch", device="cpu", affine_random=False):
    """Parameters of the add + LayerNorm + FFN block of apps/bert_addln_ffn/torch/model.py:3-20
    (y0w0 = Linear(H, H), ln0 = LayerNorm(H), ffn = Linear(H, FF) -> act -> Linear(FF, H),
    ln2 = LayerNorm(H), created in that order) in kernel layout: w0 [H, H], w1 [H, FF],
    w2 [FF, H] (weight.t()), biases, ga0 / be0, ga2 / be2.  init="torch" keeps nn.Linear's
    defaults (the reference app's val.py); "bert" draws weights ~ N(0, 0.02) with zero
    biases.  affine_random draws the LayerNorm affines so that ga0/be0 and ga2/be2 differ."""
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        y0w0 = torch.nn.Linear(H, H)
        ln0 = torch.nn.LayerNorm(H)
        f1 = torch.nn.Linear(H, FF)
        f2 = torch.nn.Linear(FF, H)
        ln2 = torch.nn.LayerNorm(H)
        with torch.no_grad():
            if init == "bert":
                for lin in (y0w0, f1, f2):
                    lin.weight.normal_(0.0, 0.02)
                    lin.bias.zero_()
            elif init != "torch":
                raise ValueError(f"unknown init {init!r}")
            if affine_random:
                for ln in (ln0, ln2):
                    ln.weight.uniform_(0.5, 1.5)
                    ln.bias.uniform_(-0.5, 0.5)

    def h(t):
        return t.detach().to(torch.float16).contiguous().to(device)

    return {"w0": h(y0w0.weight.t()), "b0": h(y0w0.bias), "w1": h(f1.weight.t()), "b1": h(f1.bias),
            "w2": h(f2.weight.t()), "b2": h(f2.bias), "ga0": h(ln0.weight), "be0": h(ln0.bias),
            "ga2": h(ln2.weight), "be2": h(ln2.bias)}


def nerf_a_params(Kx=64, seed=0, device="cpu", zero_pad_rows=None):
    """Parameters w1..w8 / b1..b8 of NerfA (apps/nerf_a/torch/model.py:5-38, hidden 256,
    skip after the fifth layer) in kernel layout with nn.Linear's default init: w1 [Kx, 256],
    w2..w5 [256, 256], w6 [256 + Kx, 256], w7, w8 [256, 256].  zero_pad_rows zeroes the weight
    rows of input columns at and past it (the zero padding of x) in w1 and the skip part of w6."""
    shapes = [(Kx, 256)] + [(256, 256)] * 4 + [(256 + Kx, 256), (256, 256), (256, 256)]
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        lins = [torch.nn.Linear(k, n) for k, n in shapes]
    ws = [lin.weight.detach().t().contiguous() for lin in lins]
    bs = [lin.bias.detach() for lin in lins]
    if zero_pad_rows is not None and zero_pad_rows < Kx:
        ws[0][zero_pad_rows:] = 0
        ws[5][256 + zero_pad_rows:] = 0
    h = lambda t: t.to(torch.float16).contiguous().to(device)  # noqa: E731
    return [h(w) for w in ws], [h(b) for b in bs]
