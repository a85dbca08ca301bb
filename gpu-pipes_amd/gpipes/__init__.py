"""gpipes -- Python mirror of gpu-pipes' operator surface on MI355X (gfx950).

The reference exposes its pipelined MLPs as a PyTorch extension
(``cuda_ext.mgn_fullmlp(x, w1, b1, w2, b2, w3, b3, gamma, beta)`` and the
``*_out`` forms, apps/mgn_fullmlp/pipelined/mgn_fullmlp_pl_ext.cu:24-93,
apps/mgn_linears/pipelined/mgn_linears_pl_ext.cu:24-86).  This module keeps
those names, argument order and layouts (weights [K, N] =
``nn.Linear.weight.t().contiguous()``), and calls the HIP kernels through the
C ABI of ``libgpipes.so`` (include/gpipes.h) on torch's current stream.

Error behaviour: the reference raises RuntimeError for non-CUDA or
non-contiguous tensors (TORCH_CHECK) and asserts on shapes; here every
violation raises RuntimeError, and nothing aborts the process.

There is no CPU fallback: if the library is missing, importing this module
raises.
"""
import ctypes
import os

import torch

__all__ = [
    "lib", "mgn_fullmlp", "mgn_fullmlp_out", "mgn_linears", "mgn_linears_out",
    "mgn_mlp", "mgn_mlp_out", "IMPL_FUSED", "IMPL_PIPELINED", "IMPL_PIPELINED_SPLIT_LN", "GpipesError",
    "linear_out", "linear_layer_norm_out", "layer_norm_out", "add_out", "concat_out", "pipe_ident",
    "pipeline_check", "set_wait_limit", "ACTS", "mgn_edge_gather", "mgn_edge_gather_out", "pipe_route", "ROUTES",
    "gemm_out", "bert_ffn", "bert_ffn_out", "mlp_out", "dlrm_botmlp", "dlrm_botmlp_out", "dlrm_topmlp",
    "dlrm_topmlp_out", "nerf_full", "nerf_full_out", "nerf_full_out_noalloc", "bert_addln_ffn",
    "bert_addln_ffn_out", "nerf_a", "nerf_a_out", "pipe_handoff", "handoff_checksums", "phase_timers",
    "probe_mfma", "fill_normal",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
# GPIPES_PHASE_TIMERS=1 loads the diagnostic build (the same library with the
# fused MGN kernels' phase timers compiled in, see gp_phase_timers_read).
LIB_PATH = os.path.join(_HERE, "libgpipes_phase.so" if os.environ.get("GPIPES_PHASE_TIMERS") == "1"
                        else "libgpipes.so")

GP_OK = 0
IMPL_FUSED = 0
IMPL_PIPELINED = 1
IMPL_PIPELINED_SPLIT_LN = 2
_IMPLS = {"fused": IMPL_FUSED, "pipelined": IMPL_PIPELINED, "pipelined_split_ln": IMPL_PIPELINED_SPLIT_LN}
ACTS = {"none": 0, "relu": 1, "gelu_tanh": 2, "sigmoid": 3}
ROUTES = {"ident": 0, "broadcast": 1, "split": 2, "drain": 3, "handoff": 4, "reload": 5}


class GpipesError(RuntimeError):
    """A C ABI call returned a negative status."""

    def __init__(self, code, msg):
        super().__init__(f"gpipes error {code}: {msg}")
        self.code = code


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `python gpu-pipes_amd/build.py` "
            "(or __graft_entry__.build()) first")
    L = ctypes.CDLL(LIB_PATH)
    vp, i64, f32, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
    L.gp_version.restype = i32
    L.gp_last_error.restype = ctypes.c_char_p
    L.gp_mgn_fullmlp_out.argtypes = [i64] + [vp] * 11
    L.gp_mgn_fullmlp_out.restype = i32
    L.gp_mgn_linears_out.argtypes = [i64] + [vp] * 9
    L.gp_mgn_linears_out.restype = i32
    L.gp_mgn_mlp_out.argtypes = [i64, i64] + [vp] * 9 + [f32, vp, i32, vp]
    L.gp_mgn_mlp_out.restype = i32
    L.gp_mgn_mlp_dtype_out.argtypes = [i64, i64] + [vp] * 9 + [f32, vp, i32, i32, vp]
    L.gp_mgn_mlp_dtype_out.restype = i32
    L.gp_linear_out.argtypes = [i64, i64, vp, vp, vp, vp, i32, vp, vp]
    L.gp_linear_layer_norm_out.argtypes = [i64, i64] + [vp] * 5 + [f32, vp, vp]
    L.gp_layer_norm_out.argtypes = [i64, i64, vp, vp, vp, f32, vp, vp]
    L.gp_add_out.argtypes = [i64, i64, vp, vp, vp, vp]
    L.gp_concat_out.argtypes = [i64, i64, i64, vp, vp, vp, vp]
    L.gp_pipe_ident.argtypes = [i64, vp, vp, i32, vp]
    L.gp_pipe_route.argtypes = [i64, vp, vp, vp, i32, i32, vp]
    L.gp_pipe_route.restype = i32
    L.gp_pipeline_check.argtypes = [vp]
    L.gp_set_wait_limit.argtypes = [i64]
    L.gp_set_wait_limit.restype = i32
    L.gp_phase_timers_read.argtypes = [vp, i64]
    L.gp_phase_timers_read.restype = i32
    L.gp_mgn_edge_gather_out.argtypes = [i64, i64, vp, vp, vp, vp, i32] + [vp] * 8 + [f32, vp, vp]
    L.gp_mgn_edge_gather_out.restype = i32
    L.gp_gemm_out.argtypes = [i64, i64, i64, vp, vp, vp, vp, i32, vp, vp]
    L.gp_gemm_dtype_out.argtypes = [i64, i64, i64, vp, vp, vp, vp, i32, vp, i32, vp]
    L.gp_bert_ffn_out.argtypes = [i64, i64, i64] + [vp] * 7 + [f32, i32, vp, vp]
    L.gp_bert_ffn_dtype_out.argtypes = [i64, i64, i64] + [vp] * 7 + [f32, i32, vp, i32, vp]
    L.gp_bert_ffn_impl_out.argtypes = [i64, i64, i64] + [vp] * 7 + [f32, i32, vp, i32, vp]
    L.gp_probe_mfma.argtypes = [i64, i32, i32, vp, i64, ctypes.POINTER(i64), vp]
    L.gp_fill_normal.argtypes = [vp, i64, ctypes.c_uint64, ctypes.c_uint64, i32, vp]
    L.gp_fill_normal.restype = i32
    L.gp_mlp_out.argtypes = [i64, i32, vp, vp, vp, vp, vp, vp, vp]
    L.gp_mlp_dtype_out.argtypes = [i64, i32, vp, vp, vp, vp, vp, vp, i32, vp]
    L.gp_mlp_dtype_out.restype = i32
    L.gp_dlrm_botmlp_out.argtypes = [i64, i64] + [vp] * 9
    L.gp_dlrm_topmlp_out.argtypes = [i64, i64, i64] + [vp] * 11 + [i32, vp, vp]
    L.gp_nerf_full_out.argtypes = [i64] * 5 + [vp] * 4 + [i32, vp, vp, vp]
    L.gp_nerf_full_out_noalloc.argtypes = [i64] * 5 + [vp] * 4 + [i32, vp, vp, vp]
    L.gp_nerf_full_dtype_out.argtypes = [i64] * 5 + [vp] * 4 + [i32, vp, vp, i32, vp]
    L.gp_nerf_full_dtype_out.restype = i32
    L.gp_bert_addln_ffn_out.argtypes = [i64, i64, i64] + [vp] * 12 + [f32, i32, vp, i32, vp]
    L.gp_bert_addln_ffn_out.restype = i32
    L.gp_bert_addln_ffn_dtype_out.argtypes = [i64, i64, i64] + [vp] * 12 + [f32, i32, vp, i32, i32, vp]
    L.gp_bert_addln_ffn_dtype_out.restype = i32
    L.gp_nerf_a_out.argtypes = [i64, i64, vp, vp, vp, vp, i32, vp]
    L.gp_nerf_a_out.restype = i32
    L.gp_nerf_a_dtype_out.argtypes = [i64, i64, vp, vp, vp, vp, i32, i32, vp]
    L.gp_nerf_a_dtype_out.restype = i32
    L.gp_nerf_full_out_noalloc.restype = i32
    for name in ("gp_mlp_out", "gp_dlrm_botmlp_out", "gp_dlrm_topmlp_out", "gp_nerf_full_out", "gp_gemm_out",
                 "gp_gemm_dtype_out", "gp_bert_ffn_out", "gp_bert_ffn_dtype_out", "gp_linear_out", "gp_linear_layer_norm_out", "gp_layer_norm_out", "gp_add_out",
                 "gp_concat_out", "gp_pipe_ident", "gp_pipeline_check"):
        getattr(L, name).restype = i32
    return L


lib = _load()


def _check(rc):
    if rc != GP_OK:
        raise GpipesError(rc, lib.gp_last_error().decode())


def _stream_ptr(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _check_input(name, t, shape=None, dtype=torch.float16):
    # CHECK_CUDA / CHECK_CONTIGUOUS of mgn_fullmlp_pl_ext.cu:14-16, plus dtype/shape
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if t.dtype != dtype:
        raise RuntimeError(f"{name} must be {str(dtype).replace('torch.', '')} (got {t.dtype})")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise RuntimeError(f"{name} must have shape {tuple(shape)} (got {tuple(t.shape)})")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


_DTYPES = {torch.float16: 0, torch.bfloat16: 1}  # GP_DTYPE_F16, GP_DTYPE_BF16


def mgn_mlp_out(x, w1, b1, w2, b2, w3, b3, gamma, beta, out, eps=1e-5, impl="fused"):
    """MgnMlp(K, [128,128,128], layernorm=gamma is not None) into ``out``.

    K = x.shape[1] in {128, 256, 384}; gamma/beta None -> no LayerNorm.
    Every tensor is float16, or every tensor is bfloat16 (fused impl only:
    gp_mgn_mlp_dtype_out).
    """
    if not isinstance(x, torch.Tensor) or x.dim() != 2:
        raise RuntimeError("x must be a 2-D tensor [M, K]")
    M, K = x.shape
    dt = x.dtype if x.dtype in _DTYPES else torch.float16
    _check_input("x", x, dtype=dt)
    _check_input("w1", w1, (K, 128), dt)
    _check_input("b1", b1, (128,), dt)
    _check_input("w2", w2, (128, 128), dt)
    _check_input("b2", b2, (128,), dt)
    _check_input("w3", w3, (128, 128), dt)
    _check_input("b3", b3, (128,), dt)
    if (gamma is None) != (beta is None):
        raise RuntimeError("gamma and beta must both be given or both be None")
    if gamma is not None:
        _check_input("gamma", gamma, (128,), dt)
        _check_input("beta", beta, (128,), dt)
    _check_input("out", out, (M, 128), dt)
    devs = {t.device for t in (x, w1, b1, w2, b2, w3, b3, out) if t is not None}
    if len(devs) != 1:
        raise RuntimeError("all tensors must be on the same device")
    impl_id = _IMPLS.get(impl, impl)
    with torch.cuda.device(x.device):
        args = (M, K, _ptr(x), _ptr(w1), _ptr(b1), _ptr(w2), _ptr(b2), _ptr(w3), _ptr(b3), _ptr(gamma),
                _ptr(beta), float(eps), _ptr(out), int(impl_id))
        if dt == torch.float16:
            rc = lib.gp_mgn_mlp_out(*args, ctypes.c_void_p(_stream_ptr(x)))
        else:
            rc = lib.gp_mgn_mlp_dtype_out(*args, _DTYPES[dt], ctypes.c_void_p(_stream_ptr(x)))
    _check(rc)
    return out


def mgn_mlp(x, w1, b1, w2, b2, w3, b3, gamma=None, beta=None, eps=1e-5, impl="fused"):
    out = torch.zeros((x.shape[0], 128), dtype=x.dtype, device=x.device)
    return mgn_mlp_out(x, w1, b1, w2, b2, w3, b3, gamma, beta, out, eps=eps, impl=impl)


def mgn_fullmlp_out(x, w1, b1, w2, b2, w3, b3, gamma, beta, out):
    """Edge MLP 384->128->128->128 + LayerNorm(eps=1e-5) into ``out``
    (mgn_fullmlp_pl_ext.cu:24-71)."""
    _check_input("x", x)
    if x.dim() != 2 or x.shape[1] != 384:
        raise RuntimeError("x must be [M, 384]")
    return mgn_mlp_out(x, w1, b1, w2, b2, w3, b3, gamma, beta, out, eps=1e-5)


def mgn_fullmlp(x, w1, b1, w2, b2, w3, b3, gamma, beta):
    """Allocating form: returns a new [M, 128] tensor (mgn_fullmlp_pl_ext.cu:74-88)."""
    out = torch.zeros((x.shape[0], 128), dtype=x.dtype, device=x.device)
    return mgn_fullmlp_out(x, w1, b1, w2, b2, w3, b3, gamma, beta, out)


def mgn_linears_out(x, w1, b1, w2, b2, w3, b3, out):
    """384->128->128->128 without LayerNorm (mgn_linears_pl_ext.cu:24-66)."""
    _check_input("x", x)
    if x.dim() != 2 or x.shape[1] != 384:
        raise RuntimeError("x must be [M, 384]")
    return mgn_mlp_out(x, w1, b1, w2, b2, w3, b3, None, None, out)


def mgn_linears(x, w1, b1, w2, b2, w3, b3):
    out = torch.zeros((x.shape[0], 128), dtype=x.dtype, device=x.device)
    return mgn_linears_out(x, w1, b1, w2, b2, w3, b3, out)


# ---------------------------------------------------------------------------
# Stage-level operations (one library stage over a whole matrix)
# ---------------------------------------------------------------------------

def _opt(name, t, shape, dtype=torch.float16):
    if t is None:
        return None
    _check_input(name, t, shape, dtype)
    return t


def _dtype_of(x):
    """The element type a call runs in: x's, when it is float16 or bfloat16."""
    return x.dtype if isinstance(x, torch.Tensor) and x.dtype in _DTYPES else torch.float16


def _stream(t):
    return ctypes.c_void_p(_stream_ptr(t))


def linear_out(x, w, b=None, acc=None, act="none", out=None):
    """out[M,128] = act(x @ w + b [+ acc]) -- pipe_gemm_bias_relu / pipe_gemm_bias / pipe_gemm."""
    _check_input("x", x)
    M, K = x.shape
    _check_input("w", w, (K, 128))
    _opt("b", b, (128,))
    _opt("acc", acc, (M, 128))
    if out is None:
        out = torch.empty((M, 128), dtype=torch.float16, device=x.device)
    _check_input("out", out, (M, 128))
    with torch.cuda.device(x.device):
        _check(lib.gp_linear_out(M, K, _ptr(x), _ptr(w), _ptr(b), _ptr(acc), ACTS.get(act, act), _ptr(out),
                                 _stream(x)))
    return out


def linear_layer_norm_out(x, w, b, gamma, beta, eps=1e-5, out=None):
    """out = LayerNorm(x @ w + b) * gamma + beta -- pipe_gemm_bias_layer_norm."""
    _check_input("x", x)
    M, K = x.shape
    _check_input("w", w, (K, 128))
    _opt("b", b, (128,))
    _check_input("gamma", gamma, (128,))
    _check_input("beta", beta, (128,))
    if out is None:
        out = torch.empty((M, 128), dtype=torch.float16, device=x.device)
    _check_input("out", out, (M, 128))
    with torch.cuda.device(x.device):
        _check(lib.gp_linear_layer_norm_out(M, K, _ptr(x), _ptr(w), _ptr(b), _ptr(gamma), _ptr(beta), float(eps),
                                            _ptr(out), _stream(x)))
    return out


def layer_norm_out(x, gamma=None, beta=None, eps=1e-5, out=None):
    """LayerNorm over the last dimension (host_layer_norm / pipe_layer_norm)."""
    _check_input("x", x)
    M, D = x.shape
    _opt("gamma", gamma, (D,))
    _opt("beta", beta, (D,))
    if out is None:
        out = torch.empty_like(x)
    _check_input("out", out, (M, D))
    with torch.cuda.device(x.device):
        _check(lib.gp_layer_norm_out(M, D, _ptr(x), _ptr(gamma), _ptr(beta), float(eps), _ptr(out), _stream(x)))
    return out


def add_out(a, b, out=None):
    """c = a + b (host_add2 / pipe_add)."""
    _check_input("a", a)
    M, N = a.shape
    _check_input("b", b, (M, N))
    if out is None:
        out = torch.empty_like(a)
    _check_input("out", out, (M, N))
    with torch.cuda.device(a.device):
        _check(lib.gp_add_out(M, N, _ptr(a), _ptr(b), _ptr(out), _stream(a)))
    return out


def concat_out(a, b, out=None):
    """c = [a | b] row-wise (host_concat2 / pipe_concat)."""
    _check_input("a", a)
    M, N0 = a.shape
    _check_input("b", b)
    if b.shape[0] != M:
        raise RuntimeError("a and b must have the same number of rows")
    N1 = b.shape[1]
    if out is None:
        out = torch.empty((M, N0 + N1), dtype=a.dtype, device=a.device)
    _check_input("out", out, (M, N0 + N1))
    with torch.cuda.device(a.device):
        _check(lib.gp_concat_out(M, N0, N1, _ptr(a), _ptr(b), _ptr(out), _stream(a)))
    return out


def pipe_ident(x, max_pipes=0, out=None):
    """Copy x[M,128] through ring-queue pipelines (the reference's pipeval ident)."""
    _check_input("x", x)
    M, D = x.shape
    if D != 128:
        raise RuntimeError("pipe_ident moves 128-wide rows")
    if out is None:
        out = torch.zeros_like(x)
    _check_input("out", out, (M, D))
    with torch.cuda.device(x.device):
        _check(lib.gp_pipe_ident(M, _ptr(x), _ptr(out), int(max_pipes), _stream(x)))
    return out


def pipe_route(x, route="ident", max_pipes=0):
    """Copy x[M,128] through a queue topology (ident / broadcast / split / drain / reload); returns
    (out, out2) -- out2 is None except for the two-consumer broadcast (the drain's second
    consumer discards its tiles)."""
    _check_input("x", x)
    M, D = x.shape
    if D != 128:
        raise RuntimeError("pipe_route moves 128-wide rows")
    rid = ROUTES.get(route, route)
    out = torch.zeros_like(x)
    out2 = torch.zeros_like(x) if rid == ROUTES["broadcast"] else None
    with torch.cuda.device(x.device):
        _check(lib.gp_pipe_route(M, _ptr(x), _ptr(out), _ptr(out2), int(rid), int(max_pipes), _stream(x)))
    return out, out2


def pipe_handoff(M, max_pipes=0, device=None, out=None):
    """Queue hand-off benchmark (misc_tests/pipeperf/pipeperf.cu:125-163): ceil(M/128)
    generated 128 x 128 fp16 tiles (32 KiB each) pass producer -> two-slot queue ->
    consumer in every pipeline; returns the consumer's per-tile checksums as int32 (uint32
    bit patterns; handoff_checksums gives the expected values)."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    T = (int(M) + 127) // 128
    if out is None:
        out = torch.zeros(max(T, 1), dtype=torch.int32, device=dev)
    if out.dtype != torch.int32 or not out.is_cuda or out.numel() < T or not out.is_contiguous():
        raise RuntimeError("out must be a contiguous int32 CUDA tensor of ceil(M / 128) elements")
    with torch.cuda.device(out.device):
        _check(lib.gp_pipe_route(int(M), None, _ptr(out), None, ROUTES["handoff"], int(max_pipes), _stream(out)))
    return out


def handoff_checksums(M):
    """Expected gp_pipe_route(GP_ROUTE_HANDOFF) checksums (numpy uint32): tile t sums the
    words (t * 0x9E3779B1) ^ (i * 0x85EBCA77), i < 64 * rows, modulo 2^32.  Bit b of the
    sum of a ^ w_i over n words is 2^b times (n - c_b if bit b of a is set, else c_b), c_b
    being how many w_i have bit b set."""
    import numpy as np

    T = (int(M) + 127) // 128
    t = np.arange(T, dtype=np.uint64)
    rows = np.minimum(128, int(M) - 128 * t.astype(np.int64))
    a = (t * np.uint64(0x9E3779B1)) & np.uint64(0xFFFFFFFF)
    bits = np.arange(32, dtype=np.uint64)
    abit = ((a[:, None] >> bits[None, :]) & np.uint64(1)).astype(np.int64)       # [T, 32]
    w = (np.arange(128 * 64, dtype=np.uint64) * np.uint64(0x85EBCA77)) & np.uint64(0xFFFFFFFF)
    wbit = ((w[:, None] >> bits[None, :]) & np.uint64(1)).astype(np.int64)      # [8192, 32]
    cum = np.cumsum(wbit, axis=0)                                               # set bits among w_0..w_i
    n = 64 * rows
    c = cum[n - 1]                                                              # [T, 32]
    ones = np.where(abit == 1, n[:, None] - c, c)
    total = (ones.astype(np.uint64) << bits[None, :]).sum(axis=1)                # < 2^46: no overflow
    return (total & np.uint64(0xFFFFFFFF)).astype(np.uint32)


PHASE_NAMES = {
    "layer1_waves": ["x_wait", "a_barrier", "layer1", "handoff_wait", "handoff_store"],
    "layer23_waves": ["handoff_wait", "layer2", "exchange_free_wait", "exchange_store", "exchange_full_wait",
                      "layer3_issue", "layernorm_store"],
}


_probe_out = {}


def probe_mfma(iters, dtype=torch.float16, device=None, shape=32):
    """Launch the dense-MFMA throughput probe (gp_probe_mfma; shape 32: 32x32x16 MFMAs,
    16: 16x16x32) on the current stream and return the launch's FLOP count; time it with
    events on that stream.  Diagnostics."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    out = _probe_out.get(dev)
    if out is None:
        out = _probe_out[dev] = torch.empty(2 * 1024 * 256, dtype=torch.float32, device=dev)
    flops = ctypes.c_int64(0)
    with torch.cuda.device(dev):
        _check(lib.gp_probe_mfma(int(iters), _DTYPES[dtype], int(shape), _ptr(out), out.numel(),
                                 ctypes.byref(flops), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
    return flops.value


def fill_normal(t, seed=0, offset=0):
    """Fill a contiguous fp16 / bf16 CUDA tensor with elements offset, offset + 1, ... of the
    N(0, 1) stream of `seed` (gp_fill_normal: Philox-4x32-10 + Box-Muller, the same values
    as oracle.normal on the host), on the current stream; returns t."""
    if not t.is_cuda or not t.is_contiguous():
        raise GpipesError("fill_normal needs a contiguous CUDA tensor")
    with torch.cuda.device(t.device):
        _check(lib.gp_fill_normal(_ptr(t), t.numel(), int(seed), int(offset), _DTYPES.get(t.dtype, -1),
                                  ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)))
    return t


def phase_timers():
    """Per-phase shader-clock cycles per tile of the last fused MGN launch, averaged over the
    launch's workgroups (diagnostic build only: GPIPES_PHASE_TIMERS=1); also the loop's
    cycles per tile and the clock they imply (s_memtime ticks / s_memrealtime time), and how
    the workgroups' tile loops end: the loop time of each workgroup (its slowest wave, in µs of
    s_memrealtime) over the launch and averaged per XCD (workgroup b runs on XCD b % 8), with
    each XCD's clock; the weight prologue (kernel entry to loop start) of each workgroup; and
    how far apart the workgroups start and end."""
    import numpy as np

    buf = np.zeros(256 * 8 * 20, dtype=np.uint64)
    torch.cuda.synchronize()
    _check(lib.gp_phase_timers_read(ctypes.c_void_p(buf.ctypes.data), buf.nbytes))
    a = buf.reshape(256, 8, 20).astype(np.float64)
    grid = int(a[0, 0, 11])
    a = a[:grid]
    res = {"grid": grid}
    for kind, waves in (("layer1_waves", slice(0, 4)), ("layer23_waves", slice(4, 8))):
        w = a[:, waves, :]
        tiles = w[..., 10].sum()
        total = w[..., 8].sum()
        res[kind] = {
            "cycles_per_tile": total / tiles,
            "clock_ghz": total / (w[..., 9].sum() * 10.0),
            "phases_per_tile": {nm: w[..., i].sum() / tiles for i, nm in enumerate(PHASE_NAMES[kind])},
        }
    loop_us = a[:, :, 9].max(axis=1) / 100.0  # s_memrealtime runs at 100 MHz
    xcd = np.arange(grid) % 8
    clock = a[:, :, 8].sum(axis=1) / (a[:, :, 9].sum(axis=1) * 10.0)
    res["workgroup_loop_us"] = {"min": float(loop_us.min()), "median": float(np.median(loop_us)),
                                "mean": float(loop_us.mean()), "max": float(loop_us.max())}
    res["xcd_loop_us_mean"] = [float(loop_us[xcd == i].mean()) for i in range(8) if (xcd == i).any()]
    res["xcd_clock_ghz"] = [float(clock[xcd == i].mean()) for i in range(8) if (xcd == i).any()]
    # s_memrealtime at kernel entry, loop start and loop end (one GPU-wide 100 MHz counter)
    entry, start, end = a[:, :, 12].min(axis=1), a[:, :, 13].max(axis=1), a[:, :, 14].max(axis=1)
    pro = (start - entry) / 100.0
    res["prologue_us"] = {"min": float(pro.min()), "median": float(np.median(pro)), "max": float(pro.max())}
    res["entry_spread_us"] = float((entry.max() - entry.min()) / 100.0)
    res["end_spread_us"] = float((end.max() - end.min()) / 100.0)
    res["entry_to_last_end_us"] = float((end.max() - entry.min()) / 100.0)
    # prologue steps (median over workgroups of the slowest wave's time per step, µs):
    # copies of W1 and W2 landed, barrier, their fragments read + barrier, W3 (and the
    # first X tile) landed, W3's fragments read + barriers, then on to the loop
    m = np.concatenate([entry[:, None], a[:, :, 15:20].max(axis=1), start[:, None]], axis=1)
    steps = np.diff(m, axis=1) / 100.0
    names = ("w12_landed", "barrier", "take12", "w3_landed", "take3", "to_loop")
    res["prologue_steps_us"] = {nm: float(np.median(steps[:, i])) for i, nm in enumerate(names)}
    return res


def pipeline_check(device=None):
    """Wait for the current stream; raise GpipesError (code -5) if its last launch that
    reports device-side failures (the MGN MLPs, the gather front end, the pipes) timed out."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    with torch.cuda.device(dev):
        _check(lib.gp_pipeline_check(ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))


def set_wait_limit(polls):
    """Test hook: bound the device-side waits of later launches to ``polls`` polls (0: the
    defaults), so that a launch times out and reports it while its kernels still end."""
    _check(lib.gp_set_wait_limit(int(polls)))


def mgn_edge_gather_out(nf, ef, src, dst, w1, b1, w2, b2, w3, b3, gamma, beta, out, eps=1e-5):
    """Edge update of update_edges (graphmodel/mgn_dp.py:28-32) with the gather fused in:
    out[e] = MgnMlp([nf[src[e]] | ef[e] | nf[dst[e]]]).  src / dst: int32 or int64 [E]."""
    _check_input("nf", nf)
    _check_input("ef", ef)
    if nf.dim() != 2 or nf.shape[1] != 128 or ef.dim() != 2 or ef.shape[1] != 128:
        raise RuntimeError("nf and ef must be [*, 128]")
    E, N = ef.shape[0], nf.shape[0]
    for name, t in (("src", src), ("dst", dst)):
        if not isinstance(t, torch.Tensor) or not t.is_cuda or not t.is_contiguous():
            raise RuntimeError(f"{name} must be a contiguous CUDA tensor")
        if t.dtype not in (torch.int32, torch.int64) or tuple(t.shape) != (E,):
            raise RuntimeError(f"{name} must be int32 or int64 of shape ({E},)")
    if src.dtype != dst.dtype:
        raise RuntimeError("src and dst must have the same dtype")
    _check_input("w1", w1, (384, 128))
    for name, t, shp in (("b1", b1, (128,)), ("w2", w2, (128, 128)), ("b2", b2, (128,)), ("w3", w3, (128, 128)),
                         ("b3", b3, (128,))):
        _check_input(name, t, shp)
    if (gamma is None) != (beta is None):
        raise RuntimeError("gamma and beta must both be given or both be None")
    _opt("gamma", gamma, (128,))
    _opt("beta", beta, (128,))
    _check_input("out", out, (E, 128))
    with torch.cuda.device(ef.device):
        _check(lib.gp_mgn_edge_gather_out(E, N, _ptr(nf), _ptr(ef), _ptr(src), _ptr(dst), src.element_size(),
                                          _ptr(w1), _ptr(b1), _ptr(w2), _ptr(b2), _ptr(w3), _ptr(b3), _ptr(gamma),
                                          _ptr(beta), float(eps), _ptr(out), _stream(ef)))
    return out


def mgn_edge_gather(nf, ef, src, dst, w1, b1, w2, b2, w3, b3, gamma=None, beta=None, eps=1e-5):
    out = torch.empty((ef.shape[0], 128), dtype=torch.float16, device=ef.device)
    return mgn_edge_gather_out(nf, ef, src, dst, w1, b1, w2, b2, w3, b3, gamma, beta, out, eps=eps)


def gemm_out(x, w, b=None, r=None, act="none", out=None):
    """out[M,N] = act(x @ w + b), or x @ w + b + r -- the wide GEMM stage (any N multiple of
    128, K multiple of 64): the N-split PipeGemmBiasRelu / PipeGemmBias blocks of
    apps/bert_ffn/pipelined/bert_ffn_pl.cuh:79-99 and bulksync_gemm.  Every tensor float16,
    or every tensor bfloat16 (gp_gemm_dtype_out)."""
    dt = _dtype_of(x)
    _check_input("x", x, dtype=dt)
    M, K = x.shape
    _check_input("w", w, dtype=dt)
    if w.dim() != 2 or w.shape[0] != K:
        raise RuntimeError(f"w must be [{K}, N]")
    N = w.shape[1]
    _opt("b", b, (N,), dt)
    _opt("r", r, (M, N), dt)
    if out is None:
        out = torch.empty((M, N), dtype=dt, device=x.device)
    _check_input("out", out, (M, N), dt)
    with torch.cuda.device(x.device):
        _check(lib.gp_gemm_dtype_out(M, N, K, _ptr(x), _ptr(w), _ptr(b), _ptr(r), ACTS.get(act, act), _ptr(out),
                                     _DTYPES[dt], _stream(x)))
    return out


def bert_ffn_out(x, w1, b1, w2, b2, ga, be, out, eps=1e-5, act="relu", impl="fused"):
    """LayerNorm(Linear2(act(Linear1(x))) + x) into ``out`` -- bert_ffn_out of
    apps/bert_ffn/pipelined/bert_ffn_pl_ext.cu:24-56 (there H = 128, FF = 512, ReLU,
    eps 1e-5), for H in {128, 256, 512, 1024} and FF a multiple of 128.  Weights
    [in, out] = ``nn.Linear.weight.t().contiguous()``; ga / be may be None (1 / 0).  Every
    tensor float16, or every tensor bfloat16 (gp_bert_ffn_dtype_out).  impl="pipelined"
    runs the reference app's queue-chained layout (gp_bert_ffn_impl_out; H 128, FF 512,
    ReLU or GELU(tanh), float16)."""
    dt = _dtype_of(x)
    _check_input("x", x, dtype=dt)
    if x.dim() != 2:
        raise RuntimeError("x must be 2-D [M, H]")
    M, H = x.shape
    _check_input("w1", w1, dtype=dt)
    if w1.dim() != 2 or w1.shape[0] != H:
        raise RuntimeError(f"w1 must be [{H}, FF]")
    FF = w1.shape[1]
    _opt("b1", b1, (FF,), dt)
    _check_input("w2", w2, (FF, H), dt)
    _opt("b2", b2, (H,), dt)
    _opt("ga", ga, (H,), dt)
    _opt("be", be, (H,), dt)
    _check_input("out", out, (M, H), dt)
    devs = {t.device for t in (x, w1, b1, w2, b2, ga, be, out) if t is not None}
    if len(devs) != 1:
        raise RuntimeError("all tensors must be on the same device")
    impl_id = _IMPLS.get(impl, impl)
    with torch.cuda.device(x.device):
        if impl_id == IMPL_FUSED:
            _check(lib.gp_bert_ffn_dtype_out(M, H, FF, _ptr(x), _ptr(w1), _ptr(b1), _ptr(w2), _ptr(b2), _ptr(ga),
                                             _ptr(be), float(eps), ACTS.get(act, act), _ptr(out), _DTYPES[dt],
                                             _stream(x)))
        else:
            if dt != torch.float16:
                raise RuntimeError("the pipelined layout takes float16 tensors only")
            _check(lib.gp_bert_ffn_impl_out(M, H, FF, _ptr(x), _ptr(w1), _ptr(b1), _ptr(w2), _ptr(b2), _ptr(ga),
                                            _ptr(be), float(eps), ACTS.get(act, act), _ptr(out), impl_id,
                                            _stream(x)))
    return out


def bert_ffn(x, w1, b1, w2, b2, ga, be, eps=1e-5, act="relu", impl="fused"):
    """Allocating form (bert_ffn_pl_ext.cu:59-72)."""
    out = torch.zeros_like(x)
    return bert_ffn_out(x, w1, b1, w2, b2, ga, be, out, eps=eps, act=act, impl=impl)


# ---------------------------------------------------------------------------
# Dense MLP chains: DLRM and NeRF
# ---------------------------------------------------------------------------

def _same_device(*ts):
    devs = {t.device for t in ts if t is not None}
    if len(devs) != 1:
        raise RuntimeError("all tensors must be on the same device")


def mlp_out(x, ws, bs, acts, out=None):
    """DlrmMlp-style chain (common/mlps.py:23-34): layer i = acts[i](h @ ws[i] + bs[i]).
    ws[i] is [in, out] (``weight.t()``); bs[i] may be None; acts are names of ACTS or ids.
    Every tensor float16, or every tensor bfloat16 (gp_mlp_dtype_out)."""
    dt = _dtype_of(x)
    _check_input("x", x, dtype=dt)
    if x.dim() != 2:
        raise RuntimeError("x must be 2-D [M, K]")
    if not (len(ws) == len(bs) == len(acts)) or not ws:
        raise RuntimeError("ws, bs and acts must have the same non-zero length")
    M, K = x.shape
    widths = [K]
    for i, (w, b) in enumerate(zip(ws, bs)):
        _check_input(f"w{i + 1}", w, dtype=dt)
        if w.dim() != 2 or w.shape[0] != widths[-1]:
            raise RuntimeError(f"w{i + 1} must be [{widths[-1]}, N]")
        widths.append(w.shape[1])
        _opt(f"b{i + 1}", b, (w.shape[1],), dt)
    if out is None:
        out = torch.empty((M, widths[-1]), dtype=dt, device=x.device)
    _check_input("out", out, (M, widths[-1]), dt)
    _same_device(x, out, *ws, *bs)
    n = len(ws)
    wa = (ctypes.c_int64 * (n + 1))(*widths)
    wp = (ctypes.c_void_p * n)(*[w.data_ptr() for w in ws])
    bp = (ctypes.c_void_p * n)(*[0 if b is None else b.data_ptr() for b in bs])
    ap = (ctypes.c_int * n)(*[ACTS.get(a, a) for a in acts])
    with torch.cuda.device(x.device):
        _check(lib.gp_mlp_dtype_out(M, n, wa, wp, bp, ap, _ptr(x), _ptr(out), _DTYPES[dt], _stream(x)))
    return out


def dlrm_botmlp_out(x, w1, b1, w2, b2, w3, b3, out):
    """DLRM bottom MLP K0 -> 512 -> 256 -> 128, ReLU each
    (apps/dlrm_botmlp/pipelined/dlrm_botmlp_pl_ext.cu:24-66)."""
    return mlp_out(x, [w1, w2, w3], [b1, b2, b3], ["relu"] * 3, out)


def dlrm_botmlp(x, w1, b1, w2, b2, w3, b3):
    out = torch.zeros((x.shape[0], w3.shape[1]), dtype=x.dtype, device=x.device)
    return dlrm_botmlp_out(x, w1, b1, w2, b2, w3, b3, out)


def dlrm_topmlp_out(x, w1, b1, w2, b2, w3, b3, w4, b4, w5, b5, out, act5="relu"):
    """DLRM top MLP K0 -> 1024 -> 1024 -> 512 -> 256 -> N5, ReLU after the first four layers
    and act5 after the last (apps/dlrm_topmlp/pipelined/dlrm_topmlp_pl_ext.cu:24-71; the
    DLRM click head is N5 = 1 with act5="sigmoid")."""
    return mlp_out(x, [w1, w2, w3, w4, w5], [b1, b2, b3, b4, b5], ["relu"] * 4 + [act5], out)


def dlrm_topmlp(x, w1, b1, w2, b2, w3, b3, w4, b4, w5, b5, act5="relu"):
    out = torch.zeros((x.shape[0], w5.shape[1]), dtype=x.dtype, device=x.device)
    return dlrm_topmlp_out(x, w1, b1, w2, b2, w3, b3, w4, b4, w5, b5, out, act5=act5)


def nerf_full_out(x, d, *wb_and_outs, rgb_act="none"):
    """NeRF MLP (apps/nerf_full/pipelined/nerf_full_pl_ext.cu:24-97): arguments
    x, d, w1, b1, ..., w12, b12, out_r, out_rgb; see gp_nerf_full_out for the shapes.
    Every tensor float16, or every tensor bfloat16 (gp_nerf_full_dtype_out)."""
    if len(wb_and_outs) != 26:
        raise RuntimeError("expected w1, b1, ..., w12, b12, out_r, out_rgb")
    ws, bs = list(wb_and_outs[0:24:2]), list(wb_and_outs[1:24:2])
    out_r, out_rgb = wb_and_outs[24], wb_and_outs[25]
    dt = _dtype_of(x)
    _check_input("x", x, dtype=dt)
    _check_input("d", d, dtype=dt)
    if x.dim() != 2 or d.dim() != 2 or d.shape[0] != x.shape[0]:
        raise RuntimeError("x and d must be 2-D with the same number of rows")
    M, Kx = x.shape
    Kd = d.shape[1]
    Na, Nrgb = ws[8].shape[1], ws[11].shape[1]
    shapes = [(Kx, 256)] + [(256, 256)] * 4 + [(256 + Kx, 256), (256, 256), (256, 256), (256, Na), (256, 256),
                                                (256 + Kd, 128), (128, Nrgb)]
    for i, (w, b, shp) in enumerate(zip(ws, bs, shapes)):
        _check_input(f"w{i + 1}", w, shp, dt)
        _opt(f"b{i + 1}", b, (shp[1],), dt)
    _check_input("out_r", out_r, (M, Na), dt)
    _check_input("out_rgb", out_rgb, (M, Nrgb), dt)
    _same_device(x, d, out_r, out_rgb, *ws, *bs)
    wp = (ctypes.c_void_p * 12)(*[w.data_ptr() for w in ws])
    bp = (ctypes.c_void_p * 12)(*[0 if b is None else b.data_ptr() for b in bs])
    with torch.cuda.device(x.device):
        _check(lib.gp_nerf_full_dtype_out(M, Kx, Kd, Na, Nrgb, _ptr(x), _ptr(d), wp, bp, ACTS.get(rgb_act, rgb_act),
                                          _ptr(out_r), _ptr(out_rgb), _DTYPES[dt], _stream(x)))
    return out_r, out_rgb


def bert_addln_ffn_out(attn_out, x, w0, b0, w1, b1, w2, b2, ga0, be0, ga2, be2, out, eps=1e-5, act="relu",
                       impl="fused"):
    """ln2(ffn(h0) + h0) with h0 = ln0(attn_out @ w0 + b0 + x), into ``out`` -- bert_addln_ffn_out of
    apps/bert_addln_ffn/pipelined/bert_addln_ffn_pl_ext.cu:17-58 (H 128, FF 512, ReLU, eps 1e-5
    there), for H in {128, 256, 512, 1024} and FF a multiple of 128.  Weights [in, out] =
    ``weight.t().contiguous()``; biases and LayerNorm affines may be None.  impl "fused" (one
    GEMM launch per layer with fused epilogues) or "pipelined" (the reference's queue-chained
    layout, H 128 / FF 512 only).  Every tensor float16, or every tensor bfloat16 (fused impl
    only: gp_bert_addln_ffn_dtype_out)."""
    dt = _dtype_of(attn_out)
    _check_input("attn_out", attn_out, dtype=dt)
    if attn_out.dim() != 2:
        raise RuntimeError("attn_out must be 2-D [M, H]")
    M, H = attn_out.shape
    _check_input("x", x, (M, H), dt)
    _check_input("w0", w0, (H, H), dt)
    _check_input("w1", w1, dtype=dt)
    if w1.dim() != 2 or w1.shape[0] != H:
        raise RuntimeError(f"w1 must be [{H}, FF]")
    FF = w1.shape[1]
    _check_input("w2", w2, (FF, H), dt)
    for name, t, n in (("b0", b0, H), ("b1", b1, FF), ("b2", b2, H), ("ga0", ga0, H), ("be0", be0, H),
                       ("ga2", ga2, H), ("be2", be2, H)):
        _opt(name, t, (n,), dt)
    _check_input("out", out, (M, H), dt)
    _same_device(attn_out, x, w0, b0, w1, b1, w2, b2, ga0, be0, ga2, be2, out)
    impl_id = _IMPLS.get(impl, impl)
    with torch.cuda.device(x.device):
        _check(lib.gp_bert_addln_ffn_dtype_out(M, H, FF, _ptr(attn_out), _ptr(x), _ptr(w0), _ptr(b0), _ptr(w1),
                                               _ptr(b1), _ptr(w2), _ptr(b2), _ptr(ga0), _ptr(be0), _ptr(ga2),
                                               _ptr(be2), float(eps), ACTS.get(act, act), _ptr(out), int(impl_id),
                                               _DTYPES[dt], _stream(x)))
    return out


def bert_addln_ffn(attn_out, x, w0, b0, w1, b1, w2, b2, ga0, be0, ga2, be2, eps=1e-5, act="relu", impl="fused"):
    """Allocating form (bert_addln_ffn_pl_ext.cu:61-76, which passes be0 for be2 -- not
    reproduced: ga2 / be2 are used as given)."""
    out = torch.zeros_like(x)
    return bert_addln_ffn_out(attn_out, x, w0, b0, w1, b1, w2, b2, ga0, be0, ga2, be2, out, eps=eps, act=act,
                              impl=impl)


def nerf_a_out(x, *wb_and_out, impl="fused"):
    """NerfA (apps/nerf_a/torch/model.py:5-38) into ``out``: arguments x, w1, b1, ..., w8, b8, out,
    the order of nerf_a_out (apps/nerf_a/pipelined/nerf_a_pl_ext.cu:24-76).  w1 [Kx, 256],
    w6 [256 + Kx, 256], the others [256, 256]; biases may be None; out [M, 256].  impl "fused"
    (the NeRF kernel's first eight layers for Kx <= 64, else one GEMM launch per layer) or
    "pipelined" (the reference's queue-chained layout, Kx a
    multiple of 8 up to 128).  Every tensor float16, or every tensor bfloat16 (fused impl only:
    gp_nerf_a_dtype_out)."""
    if len(wb_and_out) != 17:
        raise RuntimeError("expected w1, b1, ..., w8, b8, out")
    ws, bs, out = list(wb_and_out[0:16:2]), list(wb_and_out[1:16:2]), wb_and_out[16]
    dt = _dtype_of(x)
    _check_input("x", x, dtype=dt)
    if x.dim() != 2:
        raise RuntimeError("x must be 2-D [M, Kx]")
    M, Kx = x.shape
    shapes = [(Kx, 256)] + [(256, 256)] * 4 + [(256 + Kx, 256), (256, 256), (256, 256)]
    for i, (w, b, shp) in enumerate(zip(ws, bs, shapes)):
        _check_input(f"w{i + 1}", w, shp, dt)
        _opt(f"b{i + 1}", b, (256,), dt)
    _check_input("out", out, (M, 256), dt)
    _same_device(x, out, *ws, *bs)
    wp = (ctypes.c_void_p * 8)(*[w.data_ptr() for w in ws])
    bp = (ctypes.c_void_p * 8)(*[0 if b is None else b.data_ptr() for b in bs])
    impl_id = _IMPLS.get(impl, impl)
    with torch.cuda.device(x.device):
        _check(lib.gp_nerf_a_dtype_out(M, Kx, _ptr(x), wp, bp, _ptr(out), int(impl_id), _DTYPES[dt], _stream(x)))
    return out


def nerf_a(x, *wb, impl="fused"):
    """Allocating form: returns a new [M, 256] tensor (nerf_a_pl_ext.cu:79-110)."""
    if len(wb) != 16:
        raise RuntimeError("expected w1, b1, ..., w8, b8")
    out = torch.zeros((x.shape[0], 256), dtype=x.dtype, device=x.device)
    return nerf_a_out(x, *wb, out, impl=impl)


def nerf_full_out_noalloc(x, d, *wb_and_outs, rgb_act="none"):
    """nerf_full_out through the allocation-free entry point (gp_nerf_full_out_noalloc): the
    fused kernel's shapes only (Kx <= 64, Kd <= 32, Na <= 64, Nrgb <= 64), x and d 16-byte
    aligned; its scratch is a static per-GPU array shared by every call on the GPU: eager
    calls are chained by the library (each waits for the previous call's kernels, whatever
    its stream), graph replays are not and race if they overlap."""
    if len(wb_and_outs) != 26:
        raise RuntimeError("expected w1, b1, ..., w12, b12, out_r, out_rgb")
    ws, bs = list(wb_and_outs[0:24:2]), list(wb_and_outs[1:24:2])
    out_r, out_rgb = wb_and_outs[24], wb_and_outs[25]
    for name, t in (("x", x), ("d", d), ("out_r", out_r), ("out_rgb", out_rgb)):
        _check_input(name, t)
    M, Kx = x.shape
    _same_device(x, d, out_r, out_rgb, *ws, *bs)
    wp = (ctypes.c_void_p * 12)(*[w.data_ptr() for w in ws])
    bp = (ctypes.c_void_p * 12)(*[0 if b is None else b.data_ptr() for b in bs])
    with torch.cuda.device(x.device):
        _check(lib.gp_nerf_full_out_noalloc(M, Kx, d.shape[1], out_r.shape[1], out_rgb.shape[1], _ptr(x), _ptr(d), wp,
                                            bp, ACTS.get(rgb_act, rgb_act), _ptr(out_r), _ptr(out_rgb), _stream(x)))
    return out_r, out_rgb


def nerf_full(x, d, *wb, rgb_act="none"):
    """Allocating form: returns (out_r, out_rgb) (nerf_full_pl_ext.cu:99-126)."""
    if len(wb) != 24:
        raise RuntimeError("expected w1, b1, ..., w12, b12")
    out_r = torch.zeros((x.shape[0], wb[16].shape[1]), dtype=x.dtype, device=x.device)
    out_rgb = torch.zeros((x.shape[0], wb[22].shape[1]), dtype=x.dtype, device=x.device)
    return nerf_full_out(x, d, *wb, out_r, out_rgb, rgb_act=rgb_act)
