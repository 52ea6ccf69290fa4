"""dvattention_amd.attention.dvattn_sdpa_pt (the PyTorch debugging helper of
the reference API, attention.py:36-65) against the CPU oracle, on the CPU.

The oracle's contiguous attention (oracle.contig_sdpa) additionally bounds
visible keys by fragment_lengths and returns zeros for a query with no visible
key; with fragment_lengths equal to the tensor lengths the two agree on every
query that sees a key, and the helper gives NaN on the others (as the
reference's helper does).
"""
import numpy as np
import pytest
import torch

from oracle import dvattn_oracle as O


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("F,W,S,Hkv,lens,batch", [
    (1, 1, 1, 1, [64], [1]),
    (3, 2, 2, 2, [10, 0, 33], [2, 1, 0]),     # batch 1 broadcast, a 3-D fragment, an empty view
    (2, 3, 4, 1, [40, 17], [3, 3]),
])
def test_sdpa_pt_vs_oracle(dtype, F, W, S, Hkv, lens, batch):
    from dvattention_amd.attention import dvattn_sdpa_pt
    g = torch.Generator().manual_seed(F * 31 + W)
    rng = np.random.default_rng(S)
    keys, vals = [], []
    for L, B in zip(lens, batch):
        shp = (Hkv, L, 128) if B == 0 else (B, Hkv, L, 128)
        keys.append(torch.randn(shp, generator=g).to(dtype))
        vals.append(torch.randn(shp, generator=g).to(dtype))
    loc = torch.from_numpy(rng.integers(-2, max(lens) + 2, size=(F, W, S)).astype(np.int32))
    rq = torch.randn(F, W, 16 * Hkv, S, 128, generator=g).to(dtype)
    fl = torch.tensor(lens, dtype=torch.int32)
    ref = O.contig_sdpa(0.08, loc, rq, fl, keys, vals)
    out, qk, att = dvattn_sdpa_pt(rq, loc, keys, vals, 0.08, return_intermediate_results=True)
    total = sum(lens)
    assert out.dtype == torch.float32 and out.shape == (W, 16 * Hkv, S, 128)
    assert qk.shape == att.shape == (W, 16 * Hkv, S, total)
    seen = torch.zeros(W, S, dtype=torch.bool)
    for f in range(F):
        seen |= (loc[f] >= 0) & (lens[f] > 0)
    rows = seen[:, None, :].expand(W, 16 * Hkv, S)
    assert torch.allclose(out[rows], ref[rows], atol=2e-5, rtol=1e-5)
    assert torch.isnan(out[~rows]).all()
    # masked scores are -inf, the weights of a seeing query sum to one
    assert torch.allclose(att[rows].sum(-1), torch.ones(int(rows.sum())), atol=1e-5)
    low = dvattn_sdpa_pt(rq, loc, keys, vals, 0.08)
    assert low.dtype == dtype
    assert torch.equal(low[rows], out[rows].to(dtype))


def test_sdpa_pt_scores_are_unscaled_masked_dot_products():
    from dvattention_amd.attention import dvattn_sdpa_pt
    g = torch.Generator().manual_seed(3)
    k = torch.randn(1, 1, 5, 128, generator=g)
    v = torch.randn(1, 1, 5, 128, generator=g)
    q = torch.randn(1, 1, 16, 1, 128, generator=g)
    loc = torch.tensor([[[2]]], dtype=torch.int32)
    _, qk, _ = dvattn_sdpa_pt(q, loc, [k], [v], 0.5, True)
    want = q[0, 0, :, 0] @ k[0, 0].T                         # [16, 5]
    assert torch.allclose(qk[0, :, 0, :3], want[:, :3], atol=1e-5)
    assert torch.isinf(qk[0, :, 0, 3:]).all()
