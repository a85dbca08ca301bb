"""The C++ surface (include/gpipes.hpp, the reference's operator names with
throwing error handling) exercised by the stand-alone driver
gpu-pipes_amd/apps/mgn_mlp_cc, the counterpart of the reference's *_pl_cc.cu
mains: its output for the golden fixtures must meet the parity bar, and a
misaligned input must make the wrapper throw gpipes::Error(GP_ERR_ALIGN)."""
import os
import subprocess

import numpy as np
import pytest

import oracle
from conftest import ROOT, load_golden

pytestmark = pytest.mark.gpu

EXE = os.path.join(ROOT, "gpu-pipes_amd", "apps", "mgn_mlp_cc")
KEYS = ("x", "w1", "b1", "w2", "b2", "w3", "b3", "gamma", "beta")


@pytest.mark.parametrize("name,impl", [("mgn_edge_ln.npz", 0), ("mgn_edge_linears.npz", 0), ("mgn_node_ln.npz", 0),
                                       ("mgn_edge_ln_affine.npz", 1), ("mgn_edge_ln_affine.npz", 2)])
def test_cc_driver_matches_fixture(tmp_path, name, impl):
    z = load_golden(name)
    M, K = z["x"].shape
    ln = "gamma" in z
    for k in KEYS:
        if k in z:
            np.ascontiguousarray(z[k].astype(np.float16)).tofile(tmp_path / k)
    (tmp_path / "shape").write_text(f"{M} {K} {int(ln)} {impl}\n")
    print(f"[cc] {name} impl={impl}", flush=True)
    r = subprocess.run([EXE, "check", str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "misaligned x: error code -3" in r.stdout
    if impl == 0 and K == 384:
        assert ("mgn_fullmlp_out" if ln else "mgn_linears_out") in r.stdout
    got = np.fromfile(tmp_path / "out", dtype=np.float16).reshape(M, 128).astype(np.float32)
    max_abs, rel = oracle.errors(got, z["expected"])
    assert max_abs <= oracle.MAX_ABS_TOL and rel <= oracle.REL_L2_TOL, (max_abs, rel)
