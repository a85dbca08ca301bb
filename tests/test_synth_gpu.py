"""gp_fill_normal on the device against the host restatement (oracle.normal):
the same seed and element indices give the same fp16 / bf16 bits, for ragged
counts, offsets that do not start a Philox group and a destination that is
not 8-byte aligned, whatever the grid shape."""
import numpy as np
import pytest
import torch

import gpipes
import oracle

pytestmark = pytest.mark.gpu

DT = {"f16": torch.float16, "bf16": torch.bfloat16}


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("n,offset,seed", [(1, 0, 0), (7, 3, 1), (5_000_003, 0, 0), (3_000_001, 6, 0x1234567890),
                                           (1 << 20, 1 << 40, 5)])
def test_fill_normal_matches_oracle(cuda, dtype, n, offset, seed):
    print(f"[fill_normal] {dtype} n={n} offset={offset} seed={seed}", flush=True)
    t = torch.empty(n, dtype=DT[dtype], device=cuda)
    gpipes.fill_normal(t, seed=seed, offset=offset)
    got = t.view(torch.int16).cpu().numpy().view(np.uint16)
    want = oracle.normal(n, seed=seed, offset=offset, dtype=dtype)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (bad[:8], got[bad[:8]], want[bad[:8]])


def test_fill_normal_unaligned_slice(cuda):
    """Filling buf[3:] with the stream from element 3 gives buf's own elements 3.. ."""
    n = 100_003
    whole = gpipes.fill_normal(torch.empty(n, dtype=torch.float16, device=cuda), seed=9)
    buf = torch.zeros(n, dtype=torch.float16, device=cuda)
    gpipes.fill_normal(buf[3:], seed=9, offset=3)
    torch.cuda.synchronize()
    assert torch.equal(buf[3:].view(torch.int16), whole[3:].view(torch.int16))
    assert torch.equal(buf[:3], torch.zeros(3, dtype=torch.float16, device=cuda))


def test_fill_normal_rejects_other_dtypes(cuda):
    with pytest.raises(gpipes.GpipesError):
        gpipes.fill_normal(torch.empty(8, dtype=torch.float32, device=cuda))
