"""C ABI checks that need no GPU: the library loads, exports every symbol that
include/gpipes.h declares, and rejects bad arguments before touching a device."""
import ctypes
import os
import re

import pytest
import torch

from conftest import ROOT

import gpipes

HEADERS = [os.path.join(ROOT, "include", "gpipes.h")]


def declared_symbols():
    syms = set()
    for h in HEADERS:
        txt = open(h).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        syms |= set(re.findall(r"\b(gp_[a-z0-9_]+)\s*\(", txt))
    return sorted(syms)


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("gp_mgn_fullmlp_out", "gp_mgn_linears_out", "gp_mgn_mlp_out", "gp_last_error", "gp_version"):
        assert s in syms


@pytest.mark.parametrize("sym", declared_symbols())
def test_library_exports(sym):
    assert hasattr(gpipes.lib, sym), f"{sym} declared in include/ but not exported"


def test_version():
    assert gpipes.lib.gp_version() >= 0x000100


def _call(M=16, K=384, x=16, w=16, b=16, g=16, bt=16, eps=1e-5, out=16, impl=0):
    """Call gp_mgn_mlp_out with fake (never dereferenced) pointers."""
    vp = ctypes.c_void_p
    P = lambda v: vp(v) if v else None  # noqa: E731
    return gpipes.lib.gp_mgn_mlp_out(M, K, P(x), P(w), P(b), P(w), P(b), P(w), P(b), P(g), P(bt),
                                     eps, P(out), impl, None)


@pytest.mark.parametrize("kw,code", [
    (dict(K=100), -2), (dict(K=512), -2), (dict(M=-1), -1), (dict(w=0), -1), (dict(b=0), -1),
    (dict(g=0), -1), (dict(x=0), -1), (dict(out=0), -1), (dict(x=24), -3), (dict(out=8), -3),
    (dict(w=40), -3), (dict(impl=7), -1), (dict(eps=-1.0), -1), (dict(eps=float("nan")), -1),
])
def test_argument_errors(kw, code):
    rc = _call(**kw)
    assert rc == code
    assert gpipes.lib.gp_last_error().decode() != ""


def test_empty_batch_is_a_noop():
    assert _call(M=0, x=0, out=0) == 0
    assert gpipes.lib.gp_last_error().decode() == ""


def _call_dtype(dtype, impl=0, M=16, K=384):
    vp = ctypes.c_void_p
    return gpipes.lib.gp_mgn_mlp_dtype_out(M, K, vp(16), vp(16), vp(16), vp(16), vp(16), vp(16), vp(16), vp(16),
                                           vp(16), 1e-5, vp(16), impl, dtype, None)


@pytest.mark.parametrize("dtype,impl,code", [(2, 0, -1), (-1, 0, -1), (1, 1, -1), (1, 2, -1)])
def test_dtype_errors(dtype, impl, code):
    """Unknown dtypes, and bf16 on a queue-chained impl, fail before any device call."""
    assert _call_dtype(dtype, impl) == code
    assert gpipes.lib.gp_last_error().decode() != ""


def test_dtype_entry_validates_like_the_fp16_call():
    assert _call_dtype(1, K=100) == -2
    assert _call_dtype(0, M=-1) == -1
    assert _call_dtype(1, M=0) == 0


def test_wide_dtype_entry_points_reject_before_any_device_call():
    """gp_gemm_dtype_out, gp_bert_ffn_dtype_out, gp_bert_addln_ffn_dtype_out,
    gp_nerf_full_dtype_out and gp_nerf_a_dtype_out: unknown dtypes, bf16 on the queue-chained bert_addln layout, and the fp16
    calls' own shape checks all fail before touching a device."""
    vp = ctypes.c_void_p
    L = gpipes.lib
    assert L.gp_gemm_dtype_out(16, 256, 64, vp(16), vp(16), None, None, 0, vp(16), 2, None) == -1
    assert L.gp_gemm_dtype_out(16, 200, 64, vp(16), vp(16), None, None, 0, vp(16), 1, None) == -2
    assert L.gp_gemm_dtype_out(0, 256, 64, None, vp(16), None, None, 0, None, 1, None) == 0
    args = [vp(16)] * 7
    assert L.gp_bert_ffn_dtype_out(16, 1024, 4096, *args, 1e-12, 2, vp(16), 5, None) == -1
    assert L.gp_bert_ffn_dtype_out(16, 768, 4096, *args, 1e-12, 2, vp(16), 1, None) == -2
    args12 = [vp(16)] * 12
    assert L.gp_bert_addln_ffn_dtype_out(16, 128, 512, *args12, 1e-5, 1, vp(16), 1, 1, None) == -1  # bf16 + pipelined
    assert L.gp_bert_addln_ffn_dtype_out(16, 128, 512, *args12, 1e-5, 1, vp(16), 0, 3, None) == -1
    w = (vp * 12)(*([16] * 12))
    b = (vp * 12)()
    assert L.gp_nerf_full_dtype_out(16, 64, 27, 1, 3, vp(16), vp(16), w, b, 3, vp(16), vp(16), 7, None) == -1
    assert L.gp_nerf_full_dtype_out(16, 0, 27, 1, 3, vp(16), vp(16), w, b, 3, vp(16), vp(16), 1, None) == -2
    assert L.gp_last_error().decode() != ""
    assert L.gp_nerf_full_dtype_out(0, 64, 27, 1, 3, None, None, w, b, 3, None, None, 1, None) == 0
    w8 = (vp * 8)(*([16] * 8))
    b8 = (vp * 8)()
    assert L.gp_nerf_a_dtype_out(16, 64, vp(16), w8, b8, vp(16), 0, 9, None) == -1
    assert L.gp_nerf_a_dtype_out(16, 64, vp(16), w8, b8, vp(16), 1, 1, None) == -1  # bf16 + pipelined
    assert L.gp_nerf_a_dtype_out(0, 64, None, w8, b8, None, 0, 1, None) == 0


def test_fullmlp_requires_affine():
    vp = ctypes.c_void_p
    rc = gpipes.lib.gp_mgn_fullmlp_out(16, vp(16), vp(16), vp(16), vp(16), vp(16), vp(16), vp(16), None,
                                       None, vp(16), None)
    assert rc == -1


def test_python_mirror_rejects_cpu_and_bad_tensors():
    x = torch.zeros(4, 384, dtype=torch.float16)
    w1 = torch.zeros(384, 128, dtype=torch.float16)
    w = torch.zeros(128, 128, dtype=torch.float16)
    b = torch.zeros(128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="CUDA"):
        gpipes.mgn_fullmlp(x, w1, b, w, b, w, b, b, b)
    with pytest.raises(RuntimeError):
        gpipes.mgn_linears(torch.zeros(4, 256, dtype=torch.float16), w1, b, w, b, w, b)


def test_cpp_wrappers_throw_with_message(tmp_path):
    """include/gpipes.hpp: the reference-named C++ wrappers turn a negative
    status into gpipes::Error carrying the library's message (no GPU needed:
    the arguments are rejected before any device call)."""
    import subprocess
    src = tmp_path / "t.cpp"
    src.write_text(r'''
#include <cstdio>
#include "gpipes.hpp"
int main() {
  try {
    gpipes::mgn_fullmlp_out(16, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr);
  } catch (const gpipes::Error& e) {
    std::printf("%d|%s\n", e.code(), e.what());
    return 0;
  }
  return 1;
}
''')
    exe = tmp_path / "t"
    libdir = os.path.dirname(gpipes.LIB_PATH)
    subprocess.run(["g++", "-std=c++17", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe),
                    "-L", libdir, "-lgpipes", f"-Wl,-rpath,{libdir}"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    code, msg = r.stdout.strip().split("|", 1)
    assert int(code) < 0 and "gpipes error" in msg


def _ffn(M=16, H=1024, FF=4096, x=16, w1=16, b1=16, w2=16, b2=16, g=16, bt=16, eps=1e-12, act=2, out=16):
    """Call gp_bert_ffn_out with fake (never dereferenced) pointers."""
    vp = ctypes.c_void_p
    P = lambda v: vp(v) if v else None  # noqa: E731
    return gpipes.lib.gp_bert_ffn_out(M, H, FF, P(x), P(w1), P(b1), P(w2), P(b2), P(g), P(bt), eps, act, P(out),
                                      None)


@pytest.mark.parametrize("kw,code", [
    (dict(H=768), -2), (dict(H=64), -2), (dict(FF=100), -2), (dict(FF=32768), -2), (dict(FF=0), -2),
    (dict(M=-1), -1), (dict(w1=0), -1), (dict(w2=0), -1), (dict(x=0), -1), (dict(out=0), -1),
    (dict(act=9), -1), (dict(eps=-1.0), -1), (dict(eps=float("nan")), -1),
    (dict(x=24), -3), (dict(out=8), -3), (dict(w1=40), -3), (dict(b2=8), -3), (dict(g=8), -3),
])
def test_bert_ffn_argument_errors(kw, code):
    assert _ffn(**kw) == code
    assert gpipes.lib.gp_last_error().decode() != ""


def test_bert_ffn_empty_batch_is_a_noop():
    assert _ffn(M=0, x=0, out=0) == 0
    assert gpipes.lib.gp_last_error().decode() == ""


def _ffn_impl(M=16, H=128, FF=512, x=16, w1=16, b1=16, w2=16, b2=16, g=16, bt=16, eps=1e-5, act=1, out=16, impl=1):
    """Call gp_bert_ffn_impl_out with fake (never dereferenced) pointers."""
    vp = ctypes.c_void_p
    P = lambda v: vp(v) if v else None  # noqa: E731
    return gpipes.lib.gp_bert_ffn_impl_out(M, H, FF, P(x), P(w1), P(b1), P(w2), P(b2), P(g), P(bt), eps, act,
                                           P(out), impl, None)


@pytest.mark.parametrize("kw,code", [
    (dict(impl=5), -1), (dict(impl=-1), -1), (dict(H=256), -2), (dict(FF=1024), -2), (dict(M=-1), -1),
    (dict(act=3), -1), (dict(act=0), -1), (dict(eps=-1.0), -1), (dict(w1=0), -1), (dict(x=0), -1),
    (dict(x=24), -3), (dict(out=8), -3), (dict(w2=40), -3), (dict(g=8), -3),
    (dict(impl=0, H=768), -2),  # impl 0 is gp_bert_ffn_out's own validation
])
def test_bert_ffn_impl_argument_errors(kw, code):
    """gp_bert_ffn_impl_out: the queue-chained layout is the app's shape (H 128,
    FF 512) with ReLU or GELU(tanh); bad arguments fail before any device call."""
    assert _ffn_impl(**kw) == code
    assert gpipes.lib.gp_last_error().decode() != ""


def test_bert_ffn_impl_empty_batch_is_a_noop():
    assert _ffn_impl(M=0, x=0, out=0) == 0
    assert _ffn_impl(M=0, x=0, out=0, impl=0) == 0


@pytest.mark.parametrize("M,N,K,x,w,r,act,out,code", [
    (16, 100, 128, 16, 16, 0, 0, 16, -2), (16, 128, 96, 16, 16, 0, 0, 16, -2), (16, 32768, 128, 16, 16, 0, 0, 16, -2),
    (-1, 128, 128, 16, 16, 0, 0, 16, -1), (16, 128, 128, 16, 0, 0, 0, 16, -1), (16, 128, 128, 16, 16, 16, 1, 16, -1),
    (16, 128, 128, 8, 16, 0, 0, 16, -3), (16, 128, 128, 16, 16, 8, 0, 16, -3), (16, 128, 128, 16, 16, 0, 7, 16, -1),
    (0, 128, 128, 0, 16, 0, 0, 0, 0),
])
def test_gemm_argument_errors(M, N, K, x, w, r, act, out, code):
    vp = ctypes.c_void_p
    P = lambda v: vp(v) if v else None  # noqa: E731
    assert gpipes.lib.gp_gemm_out(M, N, K, P(x), P(w), None, P(r), act, P(out), None) == code


def test_mlp_chain_argument_errors():
    vp = ctypes.c_void_p
    L = gpipes.lib
    widths = (ctypes.c_int64 * 3)(16, 512, 128)
    w = (ctypes.c_void_p * 2)(16, 16)
    b = (ctypes.c_void_p * 2)(0, 0)
    acts = (ctypes.c_int * 2)(1, 1)
    bad_w = (ctypes.c_int64 * 3)(16, 0, 128)
    assert L.gp_mlp_out(16, 2, bad_w, w, b, acts, vp(16), vp(16), None) == -2
    assert L.gp_mlp_out(16, 0, widths, w, b, acts, vp(16), vp(16), None) == -1
    nullw = (ctypes.c_void_p * 2)(16, 0)
    assert L.gp_mlp_out(16, 2, widths, nullw, b, acts, vp(16), vp(16), None) == -1
    bad_act = (ctypes.c_int * 2)(1, 9)
    assert L.gp_mlp_out(16, 2, widths, w, b, bad_act, vp(16), vp(16), None) == -1
    assert L.gp_mlp_out(-1, 2, widths, w, b, acts, vp(16), vp(16), None) == -1
    assert L.gp_mlp_out(0, 2, widths, w, b, acts, None, None, None) == 0


def test_nerf_argument_errors():
    vp = ctypes.c_void_p
    L = gpipes.lib
    w = (ctypes.c_void_p * 12)(*([16] * 12))
    b = (ctypes.c_void_p * 12)(*([0] * 12))
    assert L.gp_nerf_full_out(16, 0, 27, 1, 3, vp(16), vp(16), w, b, 3, vp(16), vp(16), None) == -2
    assert L.gp_nerf_full_out(16, 64, 27, 1, 3, vp(16), None, w, b, 3, vp(16), vp(16), None) == -1
    w11 = (ctypes.c_void_p * 12)(*([16] * 11 + [0]))
    assert L.gp_nerf_full_out(16, 64, 27, 1, 3, vp(16), vp(16), w11, b, 3, vp(16), vp(16), None) == -1
    assert L.gp_nerf_full_out(16, 64, 27, 1, 3, vp(16), vp(16), w, b, 7, vp(16), vp(16), None) == -1
    assert L.gp_nerf_full_out(0, 64, 27, 1, 3, None, None, w, b, 3, None, None, None) == 0


def _handoff_brute(M):
    import numpy as np
    out = []
    for t in range((M + 127) // 128):
        rows, a = min(128, M - 128 * t), (t * 0x9E3779B1) & 0xFFFFFFFF
        out.append(sum(a ^ ((i * 0x85EBCA77) & 0xFFFFFFFF) for i in range(64 * rows)) & 0xFFFFFFFF)
    return np.array(out, dtype=np.uint32)


@pytest.mark.parametrize("M", [1, 2, 127, 128, 129, 255, 1000])
def test_handoff_checksums_closed_form(M):
    """The per-bit counting form of the hand-off checksums equals the plain sum."""
    import numpy as np
    assert np.array_equal(gpipes.handoff_checksums(M), _handoff_brute(M))


def test_handoff_route_argument_errors():
    vp = ctypes.c_void_p
    L = gpipes.lib
    assert L.gp_pipe_route(256, vp(16), vp(16), None, 4, 0, None) == -1   # takes no input
    assert L.gp_pipe_route(256, None, None, None, 4, 0, None) == -1       # no checksum buffer
    assert L.gp_pipe_route(256, None, vp(18), None, 4, 0, None) == -3     # misaligned
    assert L.gp_pipe_route(256, None, vp(16), None, 9, 0, None) == -1     # unknown route
    assert L.gp_pipe_route(0, None, None, None, 4, 0, None) == 0          # empty: no-op


@pytest.mark.parametrize("iters,dtype,shape,out,flops,code", [
    (0, 0, 32, 16, True, -1), (16, 5, 32, 16, True, -1), (16, 0, 32, 0, True, -1), (16, 0, 32, 16, False, -1),
    (16, 0, 8, 16, True, -1),
])
def test_probe_argument_errors(iters, dtype, shape, out, flops, code):
    """gp_probe_mfma rejects bad arguments before any device call."""
    f = ctypes.c_int64(0)
    rc = gpipes.lib.gp_probe_mfma(iters, dtype, shape, ctypes.c_void_p(out) if out else None, 1 << 20,
                                  ctypes.byref(f) if flops else None, None)
    assert rc == code
    assert gpipes.lib.gp_last_error().decode() != ""


@pytest.mark.parametrize("dst,n,dtype,code", [
    (16, -1, 0, -1), (16, 8, 7, -1), (0, 8, 0, -1), (17, 8, 1, -3), (0, 0, 0, 0), (16, 0, 1, 0),
])
def test_fill_normal_argument_errors(dst, n, dtype, code):
    """gp_fill_normal rejects bad arguments before any device call (and n = 0 is a no-op)."""
    rc = gpipes.lib.gp_fill_normal(ctypes.c_void_p(dst) if dst else None, n, 0, 0, dtype, None)
    assert rc == code
    if code:
        assert gpipes.lib.gp_last_error().decode() != ""
