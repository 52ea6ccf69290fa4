"""The five benchmark configurations at full size (dvattention_amd.workloads,
the inputs bench.py times): the HIP output of sampled rows against the CPU
oracle run on just those rows (their queries, locations, cos/sin and the pages
their block tables name, remapped into a compact cache), and a second call
bit-identical to the first.  Tolerance rule of test_gpu_parity.close.
"""
import numpy as np
import pytest
import torch

from oracle import dvattn_oracle as O
from test_gpu_parity import close

pytestmark = pytest.mark.gpu


def compact_pages(t, rows, dev):
    """Block tables of ``rows`` remapped onto a compact CPU copy of the pages they name."""
    bt = t["block_tables"][rows].cpu()
    pages, inv = torch.unique(bt, return_inverse=True)
    idx = pages.to(dev)
    return (t["k_cache"][idx].cpu(), t["v_cache"][idx].cpu(), inv.reshape(bt.shape).to(torch.int32))


def paged_rows(wl, rows, dev):
    t = wl.t
    r = torch.tensor(rows)
    kc, vc, bt = compact_pages(t, r.to(dev), dev)
    return dict(locations=t["locations"][:, r.to(dev)].cpu(), queries=t["queries"][r.to(dev)].cpu(),
                cosines=t["cosines"][:, r.to(dev)].cpu(), sines=t["sines"][:, r.to(dev)].cpu(),
                fragment_lengths=t["fragment_lengths"].cpu(), k_cache=kc, v_cache=vc, block_tables=bt)


def varlen_rows(wl, rows, dev):
    # one query token per sequence (token t belongs to sequence t)
    t = wl.t
    r = torch.tensor(rows).to(dev)
    kc, vc, bt = compact_pages(t, r, dev)
    n = len(rows)
    return dict(locations=t["locations"][:, r].cpu(), queries=t["queries"][r].cpu(),
                cosines=t["cosines"][:, r].cpu(), sines=t["sines"][:, r].cpu(),
                fragment_lengths=t["fragment_lengths"].cpu(), k_cache=kc, v_cache=vc, block_tables=bt,
                cu_seqlens_q=torch.arange(n + 1, dtype=torch.int32),
                cu_seqlens_k=torch.zeros(n + 1, dtype=torch.int32))


@pytest.mark.parametrize("cfg,rows", [(1, None), (2, [0, 13, 31]), (3, [0, 5, 40, 63]), (4, [2]), (5, [0, 11])])
def test_config_rows_vs_oracle(gpu, cfg, rows):
    from dvattention_amd import workloads as WL
    wl = WL.config(cfg, device=gpu, seed=4321)
    out = WL.run(wl)
    torch.cuda.synchronize()
    again = WL.run(wl)
    torch.cuda.synchronize()
    assert torch.equal(out, again), "repeat call differs"
    t = wl.t
    if wl.op == "fused":
        ref, _ = O.fused(wl.scale, t["locations"].cpu(), t["queries"].cpu(), t["fragment_lengths"].cpu(),
                         [k.cpu() for k in t["keys"]], [v.cpu() for v in t["values"]], t["cosines"].cpu(),
                         t["sines"].cpu())
        close(out, ref, wl.dtype, f"config {cfg}")
    elif wl.op == "paged":
        ref = O.paged_sdpa(wl.scale, **paged_rows(wl, rows, gpu))
        close(out[torch.tensor(rows).to(gpu)], ref, wl.dtype, f"config {cfg} rows {rows}")
    else:
        ref = O.varlen_paged_sdpa(wl.scale, **varlen_rows(wl, rows, gpu))
        close(out[torch.tensor(rows).to(gpu)], ref, wl.dtype, f"config {cfg} rows {rows}")
