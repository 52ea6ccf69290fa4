"""Seeded random sweep of the attention operators against the CPU oracle:
paged, varlen and contiguous (dvattn_sdpa) with random view counts, lengths
(including empty views), locations (including negative and past-the-end),
block sizes, KV heads, query tokens per sequence (S = 1 takes the decode
kernels, S >= 2 the multi-query kernel for 16-bit types) and dtypes.  Each case
is small enough for the oracle to finish in well under a second.
"""
import numpy as np
import pytest
import torch

from oracle import dvattn_oracle as O
from test_gpu_parity import close, hf_cs, rand_paged, rand_varlen, run_paged, run_varlen

pytestmark = pytest.mark.gpu

DT = [torch.float32, torch.float16, torch.bfloat16]
CASES = 40


@pytest.fixture(scope="module")
def dv(gpu):
    import dvattention_amd
    return dvattention_amd


def draw(seed):
    rng = np.random.default_rng(1000 + seed)
    F = int(rng.choice([1, 1, 2, 3, 4, 6]))
    lens = [int(x) for x in rng.choice([0, 1, 7, 31, 32, 33, 100, 257, 600, 2100], size=F)]
    if max(lens) == 0:
        lens[0] = 50
    return rng, F, lens, DT[int(rng.integers(0, 3))], int(rng.choice([1, 2, 3]))


@pytest.mark.parametrize("seed", range(CASES))
def test_random_paged(dv, gpu, seed):
    rng, F, lens, dtype, Hkv = draw(seed)
    W = int(rng.integers(1, 4))
    S = int(rng.choice([1, 1, 2, 5, 16, 17]))
    bs = int(rng.choice([1, 3, 8, 16, 64]))
    R = int(rng.choice([0, 16, 64, 128]))
    d = rand_paged(F, W, S, Hkv, bs, lens, R, dtype, seed=seed)
    out = run_paged(dv, d, 0.09, gpu)
    close(out, O.paged_sdpa(0.09, **d), dtype, f"paged seed {seed}: F={F} W={W} S={S} Hkv={Hkv} bs={bs} "
                                               f"lens={lens} R={R} {dtype}")


@pytest.mark.parametrize("seed", range(CASES))
def test_random_varlen(dv, gpu, seed):
    rng, F, lens, dtype, Hkv = draw(seed)
    W = int(rng.integers(1, 5))
    counts = rng.integers(0, 3, size=W)
    cu = [0] + np.cumsum(counts).tolist()
    T = max(int(cu[-1]), 1)
    if cu[-1] == 0:
        cu[-1] = 1
    bs = int(rng.choice([1, 4, 16]))
    R = int(rng.choice([16, 64, 128]))
    d = rand_varlen(F, W, T, cu, Hkv, bs, lens, R, dtype, seed=seed)
    out = run_varlen(dv, d, 0.09, gpu)
    close(out, O.varlen_paged_sdpa(0.09, **d), dtype, f"varlen seed {seed}: F={F} W={W} cu={cu} Hkv={Hkv} "
                                                       f"bs={bs} lens={lens} R={R} {dtype}")


@pytest.mark.parametrize("seed", range(CASES))
def test_random_contiguous(dv, gpu, seed):
    rng, F, lens, dtype, Hkv = draw(seed)
    W = int(rng.integers(1, 4))
    S = int(rng.choice([1, 2, 16]))
    g = torch.Generator().manual_seed(seed)
    keys, vals = [], []
    for L in lens:
        shared = bool(rng.integers(0, 2))
        shp = (Hkv, L, 128) if shared else (W, Hkv, L, 128)
        keys.append(torch.randn(shp, generator=g).to(dtype))
        vals.append(torch.randn(shp, generator=g).to(dtype))
    loc = torch.from_numpy(rng.integers(-2, max(lens) + 3, size=(F, W, S)).astype(np.int32))
    fl = torch.tensor(lens, dtype=torch.int32)
    q = torch.randn(W, 16 * Hkv, S, 128, generator=g).to(dtype)
    c, s = hf_cs(rng.integers(0, 9000, size=(F, W, S)), 64)
    rq = O.rope_q(q, c, s)
    ref = O.contig_sdpa(0.09, loc, rq, fl, keys, vals)
    out = dv.dvattn_sdpa(rq.to(gpu), loc.to(gpu), [k.to(gpu) for k in keys], [v.to(gpu) for v in vals], 0.09,
                         fl.to(gpu))
    close(out, ref, dtype, f"contiguous seed {seed}: F={F} W={W} S={S} Hkv={Hkv} lens={lens} {dtype}")


@pytest.mark.parametrize("seed", range(CASES))
def test_random_kv_append(dv, gpu, seed):
    """K/V append bit-exact against the oracle: random shapes, block sizes,
    positions (negative, past the table, on invalid pages), page tables with
    invalid entries, rotary widths, cos/sin dtypes and key layouts."""
    rng = np.random.default_rng(5000 + seed)
    dtype = DT[int(rng.integers(0, 3))]
    W, S = int(rng.integers(1, 5)), int(rng.integers(1, 9))
    Hkv = int(rng.choice([1, 2, 8]))
    bs = int(rng.choice([1, 4, 16, 64]))
    maxB = int(rng.integers(1, 6))
    R = int(rng.choice([0, 16, 32, 64, 128]))
    g = torch.Generator().manual_seed(seed)
    P = W * maxB + 2
    bt = torch.from_numpy(rng.permutation(P)[: W * maxB].astype(np.int32).reshape(W, maxB))
    bad = rng.random((W, maxB)) < 0.15
    bt[torch.from_numpy(bad)] = torch.from_numpy(rng.choice([-1, P, P + 9], size=int(bad.sum())).astype(np.int32))
    pos = torch.from_numpy(rng.integers(-2, maxB * bs + 2, size=(W, S)).astype(np.int32))
    for w in range(W):   # one write per cache row: distinct in-table positions
        seen = set()
        for s_ in range(S):
            p_ = int(pos[w, s_])
            if 0 <= p_ < maxB * bs:
                if p_ in seen:
                    pos[w, s_] = -1
                seen.add(p_)
    if rng.integers(0, 2):   # k_proj(...).view(B, L, H, D).transpose(1, 2)
        keys = torch.randn(W, S, Hkv, 128, generator=g).to(dtype).transpose(1, 2)
        vals = torch.randn(W, S, Hkv, 128, generator=g).to(dtype).transpose(1, 2)
    else:
        keys = torch.randn(W, Hkv, S, 128, generator=g).to(dtype)
        vals = torch.randn(W, Hkv, S, 128, generator=g).to(dtype)
    kc = torch.randn(P, bs, Hkv, 128, generator=g).to(dtype)
    vc = torch.randn(P, bs, Hkv, 128, generator=g).to(dtype)
    c, s = hf_cs(rng.integers(0, 200000, size=(W, S)), R) if R else (torch.zeros(W, S, 0), torch.zeros(W, S, 0))
    if R and dtype != torch.float32 and rng.integers(0, 2):
        c, s = c.to(dtype), s.to(dtype)
    k_ref, v_ref = O.kv_append(kc, vc, bt, pos, keys, vals, c, s)
    kg, vg = kc.to(gpu), vc.to(gpu)
    keys_g = keys.to(gpu) if keys.is_contiguous() else keys.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
    vals_g = vals.to(gpu) if vals.is_contiguous() else vals.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
    dv.dvattn_paged_kv_append(keys_g, vals_g, pos.to(gpu), c.to(gpu), s.to(gpu), kg, vg, bt.to(gpu))
    torch.cuda.synchronize()
    what = f"seed {seed}: W={W} S={S} Hkv={Hkv} bs={bs} maxB={maxB} R={R} {dtype} cos {c.dtype}"
    assert torch.equal(kg.cpu(), k_ref), "K cache differs, " + what
    assert torch.equal(vg.cpu(), v_ref), "V cache differs, " + what
