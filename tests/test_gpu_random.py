"""Seeded random sweep of the attention operators against the CPU oracle:
paged, varlen and contiguous (dvattn_sdpa) with random view counts, lengths
(including empty views), locations (including negative and past-the-end),
block sizes, KV heads, query tokens per sequence (S = 1 takes the decode
kernels, S >= 2 the multi-query kernel for 16-bit types; varlen calls with two
or more packed tokens per sequence on average take the multi-query kernel too,
in groups of up to 16 tokens of one sequence, including runs of 16 and 17 and
malformed cu_seqlens_q tables) and dtypes.  Each case is small enough for the
oracle to finish in well under a second.

DVATTN_RANDOM_CASES (default 200) and DVATTN_RANDOM_SEED0 (default 0) widen or
move the sweep; the default run is the one the suite commits to.
"""
import os

import numpy as np
import pytest
import torch

from oracle import dvattn_oracle as O
from test_gpu_parity import close, hf_cs, rand_paged, rand_varlen, run_paged, run_varlen

pytestmark = pytest.mark.gpu

DT = [torch.float32, torch.float16, torch.bfloat16]
CASES = int(os.environ.get("DVATTN_RANDOM_CASES", "200"))
SEED0 = int(os.environ.get("DVATTN_RANDOM_SEED0", "0"))


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


@pytest.mark.parametrize("seed", range(SEED0, SEED0 + CASES))
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


@pytest.mark.parametrize("seed", range(SEED0, SEED0 + CASES))
def test_random_varlen(dv, gpu, seed):
    rng, F, lens, dtype, Hkv = draw(seed)
    W = int(rng.integers(1, 5))
    counts = rng.choice([0, 1, 1, 2, 2, 5, 16, 17], size=W)
    cu = [0] + np.cumsum(counts).tolist()
    T = max(int(cu[-1]), 1)
    if cu[-1] == 0:
        cu[-1] = 1
    if rng.random() < 0.2:  # a malformed table (tokens map by the first i with t < cu[i + 1])
        cu[int(rng.integers(1, W + 1))] = int(rng.integers(-2, T + 6))
    bs = int(rng.choice([1, 4, 16]))
    R = int(rng.choice([16, 64, 128]))
    d = rand_varlen(F, W, T, cu, Hkv, bs, lens, R, dtype, seed=seed)
    out = run_varlen(dv, d, 0.09, gpu)
    close(out, O.varlen_paged_sdpa(0.09, **d), dtype, f"varlen seed {seed}: F={F} W={W} cu={cu} Hkv={Hkv} "
                                                       f"bs={bs} lens={lens} R={R} {dtype}")


@pytest.mark.parametrize("seed", range(SEED0, SEED0 + CASES))
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


@pytest.mark.parametrize("seed", range(SEED0, SEED0 + CASES))
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


@pytest.mark.parametrize("seed", range(SEED0, SEED0 + CASES // 2))
def test_random_view_metadata(dv, gpu, seed):
    """View locations bit-exact and cos/sin within the trigonometric tolerance of
    test_gpu_cache: random segment counts, lengths, per-sequence orders (with
    missing, repeated and padding entries), token counts, rotary widths, scaling
    and rounding."""
    from test_gpu_cache import TRIG_TOL
    rng = np.random.default_rng(7000 + seed)
    F, W, S = int(rng.integers(1, 7)), int(rng.integers(1, 6)), int(rng.integers(1, 5))
    R = int(rng.choice([16, 64, 128]))
    lens = [int(x) for x in rng.integers(0, 70000, size=F)]
    order = np.stack([rng.permutation(F) for _ in range(W)]).astype(np.int32)
    for w in range(W):
        if F > 1 and rng.random() < 0.3:
            order[w, int(rng.integers(0, F))] = int(rng.choice([-1, order[w, 0]]))
    scaling = float(rng.choice([1.0, 0.9, 1.3]))
    round_to = [None, torch.bfloat16, torch.float16][int(rng.integers(0, 3))]
    base = float(rng.choice([1e4, 5e5]))
    inv_freq = (1.0 / (base ** (torch.arange(0, R, 2, dtype=torch.float) / R))).float()
    loc_r, cos_r, sin_r = O.view_metadata(lens, order.tolist(), S, inv_freq, scaling, round_to)
    loc, cos, sin = dv.dvattn_view_metadata(torch.tensor(lens, dtype=torch.int32, device=gpu),
                                            torch.from_numpy(order).to(gpu), S, inv_freq.to(gpu), scaling, round_to)
    what = f"seed {seed}: F={F} W={W} S={S} R={R} lens={lens} scaling={scaling} round_to={round_to}"
    assert torch.equal(loc.cpu(), loc_r), "locations differ, " + what
    dc, ds = (cos.cpu() - cos_r).abs(), (sin.cpu() - sin_r).abs()
    if round_to is None:
        assert dc.max().item() <= TRIG_TOL * scaling and ds.max().item() <= TRIG_TOL * scaling, what
    else:   # one step of the 16-bit type where the fp32 values straddle a rounding boundary
        step = 2 ** -8 if round_to == torch.bfloat16 else 2 ** -11
        assert dc.max().item() <= step * scaling * 2 and ds.max().item() <= step * scaling * 2, what
