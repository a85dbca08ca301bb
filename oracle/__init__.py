"""CPU oracle for the gpu-pipes fused-MLP path -- TEST INFRASTRUCTURE ONLY.

Thin numpy wrappers over liboracle.so (oracle/oracle.c), the plain-C fp32
restatement of the reference's MLP chain.  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import this package; the product library
(gpu-pipes_amd/) never does.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

ACT_NONE, ACT_RELU, ACT_GELU_TANH, ACT_SIGMOID = 0, 1, 2, 3

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} missing; run python gpu-pipes_amd/build.py")
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, f32, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
        L.oracle_h2f.argtypes = [ctypes.c_uint16]
        L.oracle_h2f.restype = f32
        L.oracle_f2h.argtypes = [f32]
        L.oracle_f2h.restype = ctypes.c_uint16
        L.oracle_h2f_array.argtypes = [i64, vp, vp]
        L.oracle_f2h_array.argtypes = [i64, vp, vp]
        L.oracle_linear.argtypes = [i64, i64, i64, vp, vp, vp, i32, vp]
        L.oracle_layer_norm.argtypes = [i64, i64, vp, vp, vp, f32, vp]
        L.oracle_mgn_mlp.argtypes = [i64, i64] + [vp] * 9 + [f32, vp, vp]
        L.oracle_bert_ffn.argtypes = [i64, i64, i64] + [vp] * 7 + [i32, f32, vp, vp]
        L.oracle_add.argtypes = [i64, vp, vp, vp]
        L.oracle_concat.argtypes = [i64, i64, i64, vp, vp, vp]
        u64 = ctypes.c_uint64
        L.oracle_philox4x32_10.argtypes = [vp, vp, vp]
        L.oracle_log_unit.argtypes = [f32]
        L.oracle_log_unit.restype = f32
        L.oracle_sqrt_small.argtypes = [f32]
        L.oracle_sqrt_small.restype = f32
        L.oracle_sincos_quarter.argtypes = [f32, vp, vp]
        L.oracle_normal_f32.argtypes = [i64, u64, u64, vp]
        L.oracle_normal_16.argtypes = [i64, u64, u64, i32, vp]
        L.oracle_num_threads.restype = i32
        L.oracle_set_num_threads.argtypes = [i32]
        _lib = L
    return _lib


def _f32(a):
    if a is None:
        return None
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def h2f(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().oracle_h2f_array(h.size, _p(h), _p(out))
    return out


def f2h(f):
    f = _f32(f)
    out = np.empty(f.shape, np.uint16)
    lib().oracle_f2h_array(f.size, _p(f), _p(out))
    return out


def philox4x32_10(ctr, key):
    """Philox-4x32-10 of a 4-word counter under a 2-word key (synth.c)."""
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.empty(4, np.uint32)
    lib().oracle_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def log_unit(u):
    return lib().oracle_log_unit(float(u))


def sqrt_small(v):
    return lib().oracle_sqrt_small(float(v))


def sincos_quarter(a):
    s, c = ctypes.c_float(), ctypes.c_float()
    lib().oracle_sincos_quarter(float(a), ctypes.byref(s), ctypes.byref(c))
    return s.value, c.value


def normal(n, seed=0, offset=0, dtype="f32"):
    """Elements offset .. offset + n - 1 of the N(0, 1) stream of `seed`, as gp_fill_normal
    makes them: float32 values ("f32"), or the raw fp16 / bf16 bits ("f16" / "bf16") as uint16."""
    if dtype == "f32":
        out = np.empty(n, np.float32)
        lib().oracle_normal_f32(n, seed, offset, _p(out))
    else:
        out = np.empty(n, np.uint16)
        lib().oracle_normal_16(n, seed, offset, 1 if dtype == "bf16" else 0, _p(out))
    return out


def linear(x, w, b, act=ACT_NONE):
    x, w, b = _f32(x), _f32(w), _f32(b)
    M, K = x.shape
    N = w.shape[1]
    y = np.empty((M, N), np.float32)
    lib().oracle_linear(M, K, N, _p(x), _p(w), _p(b), act, _p(y))
    return y


def layer_norm(x, gamma=None, beta=None, eps=1e-5):
    x = _f32(x)
    M, D = x.shape
    y = np.empty_like(x)
    lib().oracle_layer_norm(M, D, _p(x), _p(_f32(gamma)), _p(_f32(beta)), eps, _p(y))
    return y


def mgn_mlp(x, w1, b1, w2, b2, w3, b3, gamma=None, beta=None, eps=1e-5):
    """MgnMlp forward (common/mlps.py:3-20) in fp32; inputs any float dtype."""
    x = _f32(x)
    M, K = x.shape
    ws = [_f32(a) for a in (w1, b1, w2, b2, w3, b3)]
    g, bt = _f32(gamma), _f32(beta)
    out = np.empty((M, 128), np.float32)
    work = np.empty((2 * M * 128,), np.float32)
    lib().oracle_mgn_mlp(M, K, _p(x), *[_p(a) for a in ws], _p(g), _p(bt), eps, _p(out), _p(work))
    return out


def bert_ffn(x, w1, b1, w2, b2, gamma=None, beta=None, act=ACT_RELU, eps=1e-5):
    """BertFfn forward, LayerNorm(Linear2(act(Linear1(x))) + x), in fp32.

    apps/bert_ffn/torch/model.py:3-14; weights stored [in, out].
    """
    x = _f32(x)
    M, H = x.shape
    FF = np.asarray(w1).shape[1]
    ws = [_f32(a) for a in (w1, b1, w2, b2, gamma, beta)]
    out = np.empty((M, H), np.float32)
    work = np.empty((M * (FF + H),), np.float32)
    lib().oracle_bert_ffn(M, H, FF, _p(x), *[_p(a) for a in ws], act, eps, _p(out), _p(work))
    return out


def mlp(x, ws, bs, acts):
    """DlrmMlp(widths, sigmoid_i) forward in fp32 (common/mlps.py:23-34): every layer
    Linear then its activation (ReLU, or Sigmoid at sigmoid_i); acts gives them per layer."""
    h = _f32(x)
    for w, b, a in zip(ws, bs, acts):
        h = linear(h, w, b, a)
    return h


def nerf(x, d, ws, bs, rgb_act=ACT_NONE):
    """Nerf forward in fp32 (apps/nerf_full/torch/model.py:48-66, hidden 256, skip at
    layer 4, view directions): returns (density [M, Na], rgb [M, Nrgb])."""
    x, d = _f32(x), _f32(d)
    h = x
    for i in range(5):                                 # preskip: 5 x (Linear, ReLU)
        h = linear(h, ws[i], bs[i], ACT_RELU)
    h = concat(h, x)                                   # resid = cat([preskip_out, x])
    for i in range(5, 8):                              # postskip: 3 x (Linear, ReLU)
        h = linear(h, ws[i], bs[i], ACT_RELU)
    alpha = linear(h, ws[8], bs[8])                    # alpha: Linear
    f = linear(h, ws[9], bs[9])                        # bottleneck: Linear
    g = linear(concat(f, d), ws[10], bs[10], ACT_RELU)  # rgb[0], rgb[1]
    rgb = linear(g, ws[11], bs[11], rgb_act)           # rgb[2] (+ the workload's sigmoid)
    return alpha, rgb


def bert_addln_ffn(attn, x, w0, b0, w1, b1, w2, b2, ga0=None, be0=None, ga2=None, be2=None, act=ACT_RELU, eps=1e-5):
    """The add + LayerNorm + FFN block in fp32 (apps/bert_addln_ffn/torch/model.py:3-20):
    h0 = ln0(y0w0(attn) + x);  out = ln2(ffn(h0) + h0), ffn = Linear -> act -> Linear.
    Weights stored [in, out]; None LayerNorm affines mean 1 / 0."""
    h0 = layer_norm(add(linear(attn, w0, b0), x), ga0, be0, eps)
    f = linear(linear(h0, w1, b1, act), w2, b2)
    return layer_norm(add(f, h0), ga2, be2, eps)


def nerf_a(x, ws, bs):
    """NerfA forward in fp32 (apps/nerf_a/torch/model.py:33-38): five Linear + ReLU layers,
    the skip concatenation [h | x], three more Linear + ReLU layers; returns [M, 256]."""
    x = _f32(x)
    h = x
    for i in range(5):
        h = linear(h, ws[i], bs[i], ACT_RELU)
    h = concat(h, x)
    for i in range(5, 8):
        h = linear(h, ws[i], bs[i], ACT_RELU)
    return h


def add(a, b):
    a, b = _f32(a), _f32(b)
    c = np.empty_like(a)
    lib().oracle_add(a.size, _p(a), _p(b), _p(c))
    return c


def concat(a, b):
    a, b = _f32(a), _f32(b)
    M, N0 = a.shape
    N1 = b.shape[1]
    c = np.empty((M, N0 + N1), np.float32)
    lib().oracle_concat(M, N0, N1, _p(a), _p(b), _p(c))
    return c


def num_threads():
    return lib().oracle_num_threads()


def set_num_threads(n):
    lib().oracle_set_num_threads(int(n))


def errors(actual, expected):
    """(max-abs error, relative-L2 error) of actual vs expected (float64 math)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    d = a - e
    max_abs = float(np.max(np.abs(d))) if d.size else 0.0
    den = float(np.linalg.norm(e))
    rel = float(np.linalg.norm(d) / den) if den > 0 else float(np.linalg.norm(d))
    return max_abs, rel


# Parity bar for fp16 I/O against the fp32 oracle (workload definition).
MAX_ABS_TOL = 2e-2
REL_L2_TOL = 5e-3
# bf16 I/O: the same bar scaled by the ratio of the unit roundoffs,
# 2^-8 (bfloat16, 8 significand bits) / 2^-11 (binary16) = 8.
BF16_MAX_ABS_TOL = 8 * MAX_ABS_TOL
BF16_REL_L2_TOL = 8 * REL_L2_TOL
