"""The dense-MFMA throughput probe (gp_probe_mfma, diagnostics): it reports
the FLOP count of its launch -- two workgroups per CU, four waves each, eight
32x32x16 MFMAs (or sixteen 16x16x32) per wave and round -- and its outputs are
finite and the same on every run (the operands are fixed functions of the
lane)."""
import pytest
import torch

import gpipes

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [32, 16])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_probe_flops_and_outputs(cuda, dtype, shape):
    ncu = torch.cuda.get_device_properties(cuda).multi_processor_count
    iters = 16
    flops = gpipes.probe_mfma(iters, dtype, cuda, shape=shape)
    assert flops == 2 * ncu * 4 * iters * 8 * 2 * 32 * 32 * 16
    torch.cuda.synchronize()
    out = gpipes._probe_out[cuda][: 2 * ncu * 256].clone()
    assert torch.isfinite(out).all()
    gpipes.probe_mfma(iters, dtype, cuda, shape=shape)
    torch.cuda.synchronize()
    assert torch.equal(out, gpipes._probe_out[cuda][: 2 * ncu * 256])
