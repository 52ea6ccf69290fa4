"""The HIP operators on the committed golden fixtures (tests/golden/*.npz).

Each fixture holds its inputs, the rotated queries and the float64 brute-force
output (tests/golden/make_golden.py).  The paged and varlen operators must
reproduce the rotation bit for bit (through the standalone rope operators) and
the output under the tolerance rule of test_gpu_parity.close; the paged
fixtures also go through the C ABI directly.
"""
import glob
import os

import numpy as np
import pytest
import torch

from test_gpu_parity import close

pytestmark = pytest.mark.gpu

DT = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}
FILES = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def load(fn, dev):
    z = np.load(fn, allow_pickle=False)
    dt = DT[str(z["dtype"])]
    t = {k: torch.from_numpy(np.ascontiguousarray(z[k])).to(dev) for k in z.files
         if k not in ("kind", "dtype", "scale")}
    for k in ("queries", "k_cache", "v_cache", "rotated"):
        t[k] = t[k].to(dt)
    return str(z["kind"]), dt, float(z["scale"]), t


def test_fixtures_present():
    assert len(FILES) >= 5


@pytest.mark.parametrize("fn", FILES, ids=[os.path.basename(f)[:-4] for f in FILES])
def test_golden(gpu, fn):
    import dvattention_amd as dv
    kind, dt, scale, t = load(fn, gpu)
    if kind == "paged":
        rq = dv.dvattn_rope(t["queries"], t["cosines"], t["sines"])
        out = dv.dvattn_paged_sdpa(t["queries"], t["locations"], t["cosines"], t["sines"], t["fragment_lengths"],
                                   t["k_cache"], t["v_cache"], t["block_tables"], scale)
        from dvattention_amd import capi
        out2 = torch.empty_like(out)
        capi.paged_sdpa(out2, scale, t["locations"], t["queries"], t["cosines"], t["sines"],
                        t["fragment_lengths"], t["k_cache"], t["v_cache"], t["block_tables"])
        torch.cuda.synchronize()
        assert torch.equal(out, out2), "C ABI and torch operator differ"
    else:
        rq = dv.dvattn_varlen_rope(t["queries"], t["cosines"], t["sines"])
        out = dv.dvattn_varlen_paged_sdpa(t["queries"], t["locations"], t["cosines"], t["sines"],
                                          t["fragment_lengths"], t["k_cache"], t["v_cache"], t["block_tables"],
                                          t["cu_seqlens_q"], t["cu_seqlens_q"], scale)
    assert torch.equal(rq.cpu(), t["rotated"].cpu())
    close(out, t["expected"].cpu(), dt, os.path.basename(fn))
