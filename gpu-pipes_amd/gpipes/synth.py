"""Deterministic synthetic inputs for the MGN MLP and BERT FFN workloads.

Parameters follow torch.nn defaults, which is what the workload definition
asks for: Linear weights Kaiming-uniform(a=sqrt(5)) = U(+-1/sqrt(fan_in)),
biases U(+-1/sqrt(fan_in)), LayerNorm gamma = 1, beta = 0; X ~ N(0, 1).
Weights are returned in the kernel layout [K, N] (nn.Linear.weight.t()),
all fp16, as apps/mgn_fullmlp/pipelined/val.py:15-21 feeds them.
"""
import torch


def mgn_params(K, seed=0, layernorm=True, device="cpu", affine_random=False):
    """Parameters of MgnMlp(K, [128, 128, 128], layernorm) in kernel layout."""
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
        return t.detach().to(torch.float16).contiguous().to(device)

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


def normal_fp16(M, K, seed=0, device="cpu"):
    """X ~ N(0, 1) rounded to fp16, generated on `device` with a seeded generator."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn((M, K), generator=g, device=dev, dtype=torch.float32).to(torch.float16)
