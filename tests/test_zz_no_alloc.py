"""The allocation-free NeRF entry point, gp_nerf_full_out_noalloc, called
through the C ABI: its outputs must be bit-identical to gp_nerf_full_out's on
the same inputs (the same kernels run; only the scratch differs), on two calls
in a row, the second with a smaller batch, so that the shared static scratch
is reused with what the first call left in it.  Calls on two streams are
chained by the library, so they do not race on that scratch.  Shapes it
cannot run are rejected before any launch."""
import ctypes

import numpy as np
import pytest
import torch

import gpipes
import oracle
from gpipes.synth import nerf_inputs, nerf_params

pytestmark = pytest.mark.gpu

L = gpipes.lib
vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
L.gp_nerf_full_out_noalloc.argtypes = [i64] * 5 + [vp] * 4 + [i32, vp, vp, vp]
L.gp_nerf_full_out_noalloc.restype = i32
ACT_SIGMOID = 3


def call_noalloc(x, d, ws, bs, out_r, out_rgb, rgb_act=ACT_SIGMOID):
    M, Kx = x.shape
    Kd, Na, Nrgb = d.shape[1], out_r.shape[1], out_rgb.shape[1]
    wp = (ctypes.c_void_p * 12)(*[w.data_ptr() for w in ws])
    bp = (ctypes.c_void_p * 12)(*[b.data_ptr() for b in bs])
    stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
    return L.gp_nerf_full_out_noalloc(M, Kx, Kd, Na, Nrgb, vp(x.data_ptr()), vp(d.data_ptr()), wp, bp, rgb_act,
                                      vp(out_r.data_ptr()), vp(out_rgb.data_ptr()), stream)


def call_default(x, d, ws, bs):
    wb = [t for pair in zip(ws, bs) for t in pair]
    return gpipes.nerf_full(x, d, *wb, rgb_act="sigmoid")


def bits(t):
    return t.view(torch.int16).cpu().numpy()


def test_noalloc_matches_default_two_calls(cuda):
    # The second call has a smaller batch and other weights: the static scratch
    # then holds the first call's packed weights when the packing kernel runs.
    for M, seed in ((70000, 0), (3001, 7)):
        print(f"[noalloc] M={M} seed={seed}", flush=True)
        ws, bs = nerf_params(64, 27, 1, 3, seed=seed, device=cuda)
        x, d = nerf_inputs(M, seed=seed, device=cuda)
        ref_r, ref_rgb = call_default(x, d, ws, bs)
        out_r = torch.full((M, 1), 0x7E00, dtype=torch.int16, device=cuda).view(torch.float16)
        out_rgb = torch.full((M, 3), 0x7E00, dtype=torch.int16, device=cuda).view(torch.float16)
        rc = call_noalloc(x, d, ws, bs, out_r, out_rgb)
        assert rc == 0, L.gp_last_error().decode()
        torch.cuda.synchronize()
        assert np.array_equal(bits(out_r), bits(ref_r)), f"density differs at M={M}"
        assert np.array_equal(bits(out_rgb), bits(ref_rgb)), f"colour differs at M={M}"
        # and against the oracle on a row sample, to the parity bar
        rows = np.linspace(0, M - 1, 600).astype(np.int64)
        f = lambda t: t.detach().float().cpu().numpy()  # noqa: E731
        wa, wr = oracle.nerf(f(x)[rows], f(d)[rows], [f(w) for w in ws], [f(b) for b in bs], oracle.ACT_SIGMOID)
        for got, want in ((f(out_r)[rows], wa), (f(out_rgb)[rows], wr)):
            max_abs, rel = oracle.errors(got, want)
            assert max_abs <= oracle.MAX_ABS_TOL and rel <= oracle.REL_L2_TOL, (M, max_abs, rel)


def test_noalloc_rejects_what_it_cannot_run(cuda):
    M = 256
    ws, bs = nerf_params(64, 27, 1, 3, seed=1, device=cuda)
    x, d = nerf_inputs(M, seed=1, device=cuda)
    out_r = torch.empty((M, 1), dtype=torch.float16, device=cuda)
    out_rgb = torch.empty((M, 3), dtype=torch.float16, device=cuda)
    # a density head wider than the fused kernel's: GP_ERR_SHAPE, nothing launched
    ws_wide, bs_wide = nerf_params(64, 27, 65, 3, seed=1, device=cuda)
    out_wide = torch.empty((M, 65), dtype=torch.float16, device=cuda)
    assert call_noalloc(x, d, ws_wide, bs_wide, out_wide, out_rgb) == -2
    assert "fused" in L.gp_last_error().decode()
    # an x that is not 16-byte aligned (a column slice): GP_ERR_ALIGN
    xw = torch.zeros((M, 65), dtype=torch.float16, device=cuda)
    xs = xw[:, 1:]
    assert call_noalloc(xs, d, ws, bs, out_r, out_rgb) == -3
    # M = 0 is a no-op
    z = torch.empty((0, 64), dtype=torch.float16, device=cuda)
    assert call_noalloc(z, d[:0], ws, bs, out_r[:0], out_rgb[:0]) == 0


def test_noalloc_calls_on_two_streams_are_chained(cuda):
    """Calls on two streams, issued back to back without a host wait, share the
    static scratch; the library chains them (each call's stream waits for the
    previous call's kernels), so each output is bit-identical to the default
    entry point's on its own inputs and weights."""
    M = 120000
    cases = []
    for seed in (11, 12):
        ws, bs = nerf_params(64, 27, 1, 3, seed=seed, device=cuda)
        x, d = nerf_inputs(M, seed=seed, device=cuda)
        ref_r, ref_rgb = call_default(x, d, ws, bs)
        out_r = torch.empty((M, 1), dtype=torch.float16, device=cuda)
        out_rgb = torch.empty((M, 3), dtype=torch.float16, device=cuda)
        cases.append((x, d, ws, bs, ref_r, ref_rgb, out_r, out_rgb))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(cuda), torch.cuda.Stream(cuda)]
    for rnd in range(3):
        print(f"[noalloc two streams] round {rnd}", flush=True)
        for _, _, _, _, _, _, out_r, out_rgb in cases:
            out_r.fill_(float("nan"))
            out_rgb.fill_(float("nan"))
        torch.cuda.synchronize()
        order = (0, 1) if rnd % 2 == 0 else (1, 0)
        for i in order:
            x, d, ws, bs, _, _, out_r, out_rgb = cases[i]
            with torch.cuda.stream(streams[i]):
                assert call_noalloc(x, d, ws, bs, out_r, out_rgb) == 0, L.gp_last_error().decode()
        torch.cuda.synchronize()
        for i, (_, _, _, _, ref_r, ref_rgb, out_r, out_rgb) in enumerate(cases):
            assert np.array_equal(bits(out_r), bits(ref_r)), f"density of call {i} differs (round {rnd})"
            assert np.array_equal(bits(out_rgb), bits(ref_rgb)), f"colour of call {i} differs (round {rnd})"
