"""Pins for the CPU oracle (oracle/dvattn_oracle.py).  CPU only.

Each check is independent of the oracle's own formulas: the reference's
compiled rope_cpu (oracle/_ref), transformers' Qwen2 rotary helpers, torch's
scaled_dot_product_attention, a float64 brute force written from the
reference kernels' index arithmetic (oracle/bruteforce.c), closed-form special
cases and the dynamic-view identity.
"""
import math

import numpy as np
import pytest
import torch

from oracle import checkers
from oracle import dvattn_oracle as O

RNG = np.random.default_rng(0)


def hf_cs(pos, R, base=1e4):
    pos = np.asarray(pos, dtype=np.float64)
    inv = 1.0 / (base ** (np.arange(0, R, 2, dtype=np.float64) / R))
    fr = pos[..., None] * inv
    emb = np.concatenate([fr, fr], -1)
    return torch.from_numpy(np.cos(emb).astype(np.float32)), torch.from_numpy(np.sin(emb).astype(np.float32))


# ---------------------------------------------------------------- rotation --

@pytest.mark.skipif(not checkers.ref_rope_available(), reason="reference tree was not present at build time")
@pytest.mark.parametrize("R", [128, 64, 32, 0])
def test_rope_matches_reference_rope_cpu(R):
    F, W, Hq, S, E = 3, 2, 4, 3, 128
    q = torch.randn(W, Hq, S, E)
    c, s = hf_cs(RNG.integers(0, 70000, size=(F, W, S)), R) if R else (torch.zeros(F, W, S, 0),) * 2
    ours = O.rope_q(q, c, s)
    ref = checkers.ref_rope_cpu(q.numpy(), c.numpy(), s.numpy())
    assert np.array_equal(ours.numpy(), ref), "oracle rotation differs from the reference's rope_cpu"


@pytest.mark.parametrize("R", [128, 64, 32])
def test_rope_matches_transformers_qwen2(R):
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb
    F, W, Hq, S, E = 2, 2, 4, 2, 128
    q = torch.randn(W, Hq, S, E)
    c, s = hf_cs(RNG.integers(0, 70000, size=(F, W, S)), R)
    ours = O.rope_q(q, c, s)
    for f in range(F):
        qr, _ = apply_rotary_pos_emb(q[..., :R], q[..., :R], c[f], s[f], unsqueeze_dim=1)
        ref = torch.cat([qr, q[..., R:]], -1)
        assert torch.equal(ours[f], ref)


def test_rope_reads_only_first_half_of_cos_sin():
    # rope.cuh:24-46 reads cos/sin[0:R/2] for both halves; the second half is ignored
    W, Hq, S, E, R = 1, 2, 1, 128, 64
    q = torch.randn(W, Hq, S, E)
    c, s = hf_cs([[[777]]], R)
    c2, s2 = c.clone(), s.clone()
    c2[..., R // 2:] = 123.0
    s2[..., R // 2:] = -7.0
    assert torch.equal(O.rope_q(q, c, s), O.rope_q(q, c2, s2))


def test_rope_closed_forms():
    W, Hq, S, E, R = 2, 3, 2, 128, 64
    q = torch.randn(W, Hq, S, E)
    c0, s0 = hf_cs(np.zeros((1, W, S)), R)
    assert torch.equal(O.rope_q(q, c0, s0)[0], q)                      # angle 0 -> identity
    c, s = hf_cs(RNG.integers(1, 5000, size=(1, W, S)), R)
    r = O.rope_q(q, c, s)[0]
    assert torch.equal(r[..., R:], q[..., R:])                          # pass-through dims
    h = R // 2
    n0 = q[..., :h] ** 2 + q[..., h:R] ** 2
    n1 = r[..., :h] ** 2 + r[..., h:R] ** 2
    assert torch.allclose(n0, n1, rtol=1e-5, atol=1e-5)                 # pairwise norms kept
    # a quarter turn on dimension pair 0 (theta_0 = pos): x0 -> -x_h, x_h -> x0
    qq = torch.randn(1, 1, 1, E)
    cq = torch.zeros(1, 1, 1, R)
    sq = torch.zeros(1, 1, 1, R)
    cq[..., 0] = 0.0
    sq[..., 0] = 1.0
    cq[..., 1:] = 1.0
    out = O.rope_q(qq, cq, sq)[0, 0, 0, 0]
    assert out[0] == -qq[0, 0, 0, h] and out[h] == qq[0, 0, 0, 0]


def test_relative_rotation_identity():
    # rot(q, a) . rot(k, b) == rot(q, a - b) . k  -- the DVAttn equivalence
    E, R = 128, 128
    q = torch.randn(1, 1, 1, E, dtype=torch.float64)
    k = torch.randn(1, 1, 1, E, dtype=torch.float64)
    a, b = 9123, 4321

    def rot(x, p):
        inv = 1.0 / (1e4 ** (np.arange(0, R, 2, dtype=np.float64) / R))
        ang = torch.from_numpy(p * inv)[None, None, None]
        return O._rotate(x, torch.cos(ang), torch.sin(ang), R)

    lhs = (rot(q, a) * rot(k, b)).sum()
    rhs = (rot(q, a - b) * k).sum()
    assert abs(float(lhs - rhs)) < 1e-9 * float((q.abs() * k.abs()).sum())


def test_rope_varlen_equals_full_width_variant():
    # half-width [F,T,R/2] cos/sin == full-width [F,W=T,S=1,R] with duplicated halves
    F, T, H, E, R = 3, 5, 4, 128, 64
    q = torch.randn(T, H, E).to(torch.bfloat16)
    c, s = hf_cs(RNG.integers(0, 65536, size=(F, T)), R)           # [F,T,R]
    v = O.rope_q_varlen(q, c[..., : R // 2].contiguous(), s[..., : R // 2].contiguous())
    full = O.rope_q(q[:, :, None, :], c[:, :, None, :], s[:, :, None, :])   # [F,T,H,1,E]
    assert v.dtype == torch.bfloat16
    assert torch.equal(v, full[:, :, :, 0])


# --------------------------------------------------------------- attention --

def _rand_paged(F, W, S, Hkv, bs, lens, R=64, dtype=torch.float32, seed=0, extra_pages=3):
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    Hq, E = 16 * Hkv, 128
    lens = np.asarray(lens)                                   # [F] fragment lengths
    tot = int(lens.sum())
    maxB = (tot + bs - 1) // bs + 1
    P = W * maxB + extra_pages
    perm = rng.permutation(P).astype(np.int32)
    bt = perm[: W * maxB].reshape(W, maxB).copy()
    loc = rng.integers(-2, lens.max() + 3, size=(F, W, S)).astype(np.int32)
    q = torch.randn(W, Hq, S, E, generator=g).to(dtype)
    kc = torch.randn(P, bs, Hkv, E, generator=g).to(dtype)
    vc = torch.randn(P, bs, Hkv, E, generator=g).to(dtype)
    c, s = hf_cs(rng.integers(0, 50000, size=(F, W, S)), R)
    return dict(locations=torch.from_numpy(loc), queries=q, cosines=c, sines=s,
                fragment_lengths=torch.from_numpy(lens.astype(np.int32)), k_cache=kc, v_cache=vc,
                block_tables=torch.from_numpy(bt))


@pytest.mark.parametrize("F,W,S,Hkv,bs,lens", [
    (1, 2, 1, 1, 16, [40]),
    (2, 3, 2, 2, 4, [13, 9]),
    (3, 2, 3, 1, 5, [7, 0, 11]),
])
def test_paged_oracle_vs_bruteforce(F, W, S, Hkv, bs, lens):
    d = _rand_paged(F, W, S, Hkv, bs, lens, seed=F * 10 + S)
    scale = 128 ** -0.5
    ours = O.paged_sdpa(scale, **d)
    rq = O.rope_q(d["queries"], d["cosines"], d["sines"])
    bf = checkers.bruteforce_paged(scale, d["locations"], rq, d["fragment_lengths"], d["k_cache"], d["v_cache"],
                                   d["block_tables"])
    assert np.abs(ours.numpy() - bf).max() < 2e-5


def test_paged_oracle_matches_torch_sdpa():
    # gathered contiguous K/V through torch's scaled_dot_product_attention
    W, S, Hkv, bs, L = 2, 1, 2, 16, 70
    d = _rand_paged(1, W, S, Hkv, bs, [L], seed=5)
    d["locations"][:] = torch.tensor([[[55], [69]]], dtype=torch.int32)
    scale = 0.07
    ours = O.paged_sdpa(scale, **d)
    rq = O.rope_q(d["queries"], d["cosines"], d["sines"])[0].float()        # [W,Hq,S,E]
    for w in range(W):
        n = int(d["locations"][0, w, 0]) + 1
        pos = np.arange(n)
        pages = d["block_tables"][w].numpy()[pos // bs]
        k = d["k_cache"][pages, pos % bs].permute(1, 0, 2).float()           # [Hkv,n,E]
        v = d["v_cache"][pages, pos % bs].permute(1, 0, 2).float()
        k = k.repeat_interleave(16, 0)
        v = v.repeat_interleave(16, 0)
        ref = torch.nn.functional.scaled_dot_product_attention(rq[w][:, :, :], k, v, scale=scale)
        assert torch.allclose(ours[w], ref, atol=2e-6, rtol=1e-5)


def test_varlen_oracle_vs_bruteforce():
    rng = np.random.default_rng(3)
    F, W, Hkv, bs = 3, 4, 1, 8
    T = 7
    cu_q = np.array([0, 2, 2, 5, 7], dtype=np.int32)        # one empty sequence
    lens = np.array([10, 5, 9])
    maxB = (lens.sum() + bs - 1) // bs + 1
    P = W * maxB
    bt = rng.permutation(P).astype(np.int32).reshape(W, maxB)
    loc = rng.integers(-3, 12, size=(F, T)).astype(np.int32)
    q = torch.randn(T, 16 * Hkv, 128)
    kc = torch.randn(P, bs, Hkv, 128)
    vc = torch.randn(P, bs, Hkv, 128)
    c, s = hf_cs(rng.integers(0, 60000, size=(F, T)), 32)
    c, s = c[..., :16].contiguous(), s[..., :16].contiguous()
    args = dict(locations=torch.from_numpy(loc), queries=q, cosines=c, sines=s,
                fragment_lengths=torch.from_numpy(lens.astype(np.int32)), k_cache=kc, v_cache=vc,
                block_tables=torch.from_numpy(bt), cu_seqlens_q=torch.from_numpy(cu_q),
                cu_seqlens_k=torch.zeros(W + 1, dtype=torch.int32))
    ours = O.varlen_paged_sdpa(0.1, **args)
    rq = O.rope_q_varlen(q, c, s)
    bf = checkers.bruteforce_varlen(0.1, loc, rq, lens, kc, vc, bt, cu_q)
    assert np.abs(ours.numpy() - bf).max() < 2e-5


def test_varlen_token_to_sequence_rule():
    # first i with t < cu[i+1]; 0 when none (varlen_paged_kernel_v21.cuh:40-47)
    cu = np.array([0, 3, 3, 8])
    assert O.varlen_token_to_seq(cu, 10).tolist() == [0, 0, 0, 2, 2, 2, 2, 2, 0, 0]
    cu = np.array([2, 4, 1, 6])                               # malformed: non-monotone
    assert O.varlen_token_to_seq(cu, 7).tolist() == [0, 0, 0, 0, 2, 2, 0]


def test_contig_oracle_vs_bruteforce_and_broadcast():
    g = torch.Generator().manual_seed(7)
    F, W, Hkv, S = 2, 3, 1, 2
    Ls = [9, 17]
    rq = torch.randn(F, W, 16 * Hkv, S, 128, generator=g)
    keys = [torch.randn(W, Hkv, Ls[0], 128, generator=g), torch.randn(1, Hkv, Ls[1], 128, generator=g)]
    vals = [torch.randn(W, Hkv, Ls[0], 128, generator=g), torch.randn(1, Hkv, Ls[1], 128, generator=g)]
    loc = torch.tensor(np.random.default_rng(1).integers(-1, 20, size=(F, W, S)), dtype=torch.int32)
    fl = torch.tensor([9, 12], dtype=torch.int32)
    ours = O.contig_sdpa(0.09, loc, rq, fl, keys, vals)
    bf = checkers.bruteforce_contig(0.09, loc, rq, fl, keys, vals)
    assert np.abs(ours.numpy() - bf).max() < 2e-5
    # 3-D fragment == batch-1 fragment
    ours3 = O.contig_sdpa(0.09, loc, rq, fl, [keys[0], keys[1][0]], [vals[0], vals[1][0]])
    assert torch.equal(ours, ours3)


def test_contig_matches_reference_pt_helper_semantics():
    # attention.py:36-65 with fragment_lengths == tensor lengths and no empty rows
    g = torch.Generator().manual_seed(11)
    F, W, Hkv, S = 2, 2, 2, 1
    rq = torch.randn(F, W, 16 * Hkv, S, 128, generator=g)
    keys = [torch.randn(W, Hkv, L, 128, generator=g) for L in (6, 10)]
    vals = [torch.randn(W, Hkv, L, 128, generator=g) for L in (6, 10)]
    loc = torch.tensor([[[3], [5]], [[9], [0]]], dtype=torch.int32)
    fl = torch.tensor([6, 10], dtype=torch.int32)
    ours = O.contig_sdpa(0.1, loc, rq, fl, keys, vals)
    # restated reference helper (independent arrangement: repeat_interleave GQA)
    qk, vs = [], []
    for f in range(F):
        k = keys[f].repeat_interleave(16, -3)
        v = vals[f].repeat_interleave(16, -3)
        kp = torch.arange(k.size(-2))[None, None, None, :]
        qp = loc[f][:, None, :, None]
        a = rq[f] @ k.transpose(-1, -2)
        a.masked_fill_(kp > qp, float("-inf"))
        qk.append(a)
        vs.append(v)
    ref = torch.softmax(0.1 * torch.cat(qk, -1), -1) @ torch.cat(vs, -2)
    assert torch.allclose(ours, ref, atol=1e-6, rtol=1e-5)


def test_single_visible_key_is_exact():
    # one visible key -> output is exactly that value row (page/row addressing pin)
    W, S, Hkv, bs = 2, 1, 2, 4
    d = _rand_paged(2, W, S, Hkv, bs, [6, 5], seed=9)
    d["locations"][0] = -1          # view 0 hidden
    d["locations"][1] = 0           # only key 0 of view 1
    out = O.paged_sdpa(0.3, **d)
    for w in range(W):
        p = 6                       # view 1 starts after fragment_lengths[0] = 6 tokens
        page = int(d["block_tables"][w, p // bs])
        for h in range(16 * Hkv):
            assert torch.equal(out[w, h, 0], d["v_cache"][page, p % bs, h // 16].float())


def test_uniform_weights_give_mean():
    # q = 0 -> uniform softmax -> mean of the visible value rows (exact for small ints)
    W, S, Hkv, bs, L = 1, 1, 1, 8, 16
    d = _rand_paged(1, W, S, Hkv, bs, [L], seed=4)
    d["queries"].zero_()
    d["locations"][:] = L - 1
    vals = torch.randint(-8, 9, d["v_cache"].shape).float()
    d["v_cache"] = vals
    out = O.paged_sdpa(1.0, **d)
    pos = np.arange(L)
    rows = vals[d["block_tables"][0].numpy()[pos // bs], pos % bs, 0]
    assert torch.equal(out[0, 0, 0], rows.mean(0))


def test_empty_rows_are_zero():
    d = _rand_paged(2, 2, 2, 1, 4, [5, 3], seed=2)
    d["locations"][:, 1, :] = -5
    out = O.paged_sdpa(0.2, **d)
    assert torch.count_nonzero(out[1]) == 0
    assert torch.count_nonzero(out[0]) > 0


def test_page_permutation_invariance():
    # physical placement must not matter: identity vs permuted pages, bit-exact
    W, S, Hkv, bs, L = 2, 1, 1, 4, 13
    d = _rand_paged(1, W, S, Hkv, bs, [L], seed=12, extra_pages=0)
    out = O.paged_sdpa(0.1, **d)
    P = d["k_cache"].shape[0]
    perm = torch.from_numpy(np.random.default_rng(5).permutation(P))
    inv = torch.argsort(perm)
    d2 = dict(d)
    d2["k_cache"] = d["k_cache"][perm]
    d2["v_cache"] = d["v_cache"][perm]
    d2["block_tables"] = inv[d["block_tables"].long()].to(torch.int32)
    assert torch.equal(out, O.paged_sdpa(0.1, **d2))


def test_dynamic_view_identity():
    """Views with view-local key rotation + relative query rotation ==
    ordinary causal attention at absolute positions (README.md:5-9)."""
    g = torch.Generator().manual_seed(21)
    Hkv, E, R, base = 1, 128, 128, 1e4
    Ls = [11, 7, 9]                       # three segments of one sequence
    Ltot = sum(Ls)
    qpos = Ltot + 4                       # query position after the whole cache
    q = torch.randn(1, 16 * Hkv, 1, E, generator=g, dtype=torch.float64)
    k_raw = torch.randn(Hkv, Ltot, E, generator=g, dtype=torch.float64)
    v = torch.randn(Hkv, Ltot, E, generator=g, dtype=torch.float64)

    def rot(x, pos):
        inv = 1.0 / (base ** (np.arange(0, R, 2, dtype=np.float64) / R))
        ang = torch.from_numpy(np.asarray(pos, dtype=np.float64)[..., None] * inv)
        return O._rotate(x, torch.cos(ang), torch.sin(ang), R)

    # absolute: keys rotated at absolute positions, query at qpos
    ka = rot(k_raw, np.arange(Ltot)[None, :])
    qa = rot(q, np.array([[[qpos]]]))
    sc = (qa[0].reshape(16 * Hkv, E) @ ka[0].T) * 0.05
    ref = torch.softmax(sc, -1) @ v[0]
    # views: keys rotated at view-local positions, query rotated by (qpos - view start)
    starts = np.concatenate([[0], np.cumsum(Ls)[:-1]])
    keys, vals, rqs = [], [], []
    for f, (st, L) in enumerate(zip(starts, Ls)):
        keys.append(rot(k_raw[:, st:st + L], np.arange(L)[None, :]))
        vals.append(v[:, st:st + L])
        rqs.append(rot(q, np.array([[[qpos - st]]]))[0])
    rq = torch.stack(rqs)                                   # [F, Hq, 1, E]
    loc = torch.tensor([[L - 1] for L in Ls])               # all keys visible
    out = O.sdpa_views(rq, loc, keys, vals, Ls, 0.05)
    assert torch.allclose(out[:, 0].double(), ref, atol=2e-6)   # oracle computes in fp32


# ------------------------------------------------------------ golden files --

def test_golden_fixtures():
    import glob
    import os
    files = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))
    assert files, "tests/golden/*.npz missing (run tests/golden/make_golden.py)"
    for fn in files:
        z = np.load(fn, allow_pickle=False)
        kind = str(z["kind"])
        dt = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}[str(z["dtype"])]
        scale = float(z["scale"])
        if kind == "paged":
            out = O.paged_sdpa(scale, torch.from_numpy(z["locations"]), torch.from_numpy(z["queries"]).to(dt),
                               torch.from_numpy(z["cosines"]), torch.from_numpy(z["sines"]),
                               torch.from_numpy(z["fragment_lengths"]), torch.from_numpy(z["k_cache"]).to(dt),
                               torch.from_numpy(z["v_cache"]).to(dt), torch.from_numpy(z["block_tables"]))
        elif kind == "varlen":
            out = O.varlen_paged_sdpa(scale, torch.from_numpy(z["locations"]), torch.from_numpy(z["queries"]).to(dt),
                                      torch.from_numpy(z["cosines"]), torch.from_numpy(z["sines"]),
                                      torch.from_numpy(z["fragment_lengths"]), torch.from_numpy(z["k_cache"]).to(dt),
                                      torch.from_numpy(z["v_cache"]).to(dt), torch.from_numpy(z["block_tables"]),
                                      torch.from_numpy(z["cu_seqlens_q"]), torch.from_numpy(z["cu_seqlens_q"]))
        else:
            raise AssertionError(kind)
        assert np.abs(out.numpy() - z["expected"]).max() < 2e-5, fn
        rq_name = "rotated"
        if rq_name in z:
            rq = (O.rope_q if kind == "paged" else O.rope_q_varlen)(
                torch.from_numpy(z["queries"]).to(dt), torch.from_numpy(z["cosines"]), torch.from_numpy(z["sines"]))
            assert np.array_equal(rq.float().numpy(), z[rq_name]), fn


# ------------------------------------------------- K-side append, view metadata --

def _rand(shape, dt):
    return torch.randn(shape).to(dt)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("cos_dt", ["f32", "model"])
@pytest.mark.parametrize("R", [128, 64])
def test_key_rotation_matches_transformers_qwen2(dt, cos_dt, R):
    """attention.py:82-88 (oracle apply_rotary) against transformers' Qwen2
    apply_rotary_pos_emb on the rotated block, bit for bit, in the dtypes
    PyTorch promotes to (model dtype cos/sin: every op rounded to it)."""
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb
    W, H, S, E = 2, 3, 5, 128
    k = _rand((W, H, S, E), dt)
    c, s = hf_cs(RNG.integers(0, 200000, size=(W, S)), R)
    if cos_dt == "model":
        c, s = c.to(dt), s.to(dt)
    ours = O.apply_rotary(k, c[:, None], s[:, None])
    _, kr = apply_rotary_pos_emb(k[..., :R], k[..., :R], c, s, unsqueeze_dim=1)
    assert torch.equal(ours[..., :R], kr.to(dt))
    assert torch.equal(ours[..., R:], k[..., R:])
    assert ours.dtype == dt


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_key_rotation_closed_forms(dt):
    x = _rand((4, 128), dt)
    R = 96
    one, zero = torch.ones(R), torch.zeros(R)
    assert torch.equal(O.apply_rotary(x, one, zero), x)                       # angle 0
    q = O.apply_rotary(x, zero, one)                                          # quarter turn
    assert torch.equal(q[:, :48], -x[:, 48:96]) and torch.equal(q[:, 48:96], x[:, :48])
    assert torch.equal(q[:, 96:], x[:, 96:])
    assert torch.equal(O.apply_rotary(x, torch.zeros(0), torch.zeros(0)), x)  # R = 0
    # float64 rotation of each (e, e + R/2) pair by its angle
    th = torch.from_numpy(RNG.uniform(-7, 7, size=R // 2))
    c = torch.cat([th.cos(), th.cos()]).float()
    s = torch.cat([th.sin(), th.sin()]).float()
    y = O.apply_rotary(x.float(), c, s).double()
    xd = x.double()
    a, b = xd[:, :R // 2], xd[:, R // 2:R]
    want = torch.cat([a * th.cos() - b * th.sin(), b * th.cos() + a * th.sin(), xd[:, R:]], 1)
    assert torch.allclose(y, want, atol=1e-5, rtol=1e-5)


def test_kv_append_oracle_places_tokens_by_page_table():
    """Logical position p of sequence w lands in page bt[w, p // bs], row p % bs;
    pages come from a known permutation, so the expected cache is built
    independently; masked and out-of-table tokens leave the sentinel."""
    W, Hkv, S, E, bs, maxB = 3, 2, 4, 16, 4, 3
    P = W * maxB + 2
    perm = torch.from_numpy(RNG.permutation(P)[: W * maxB].astype(np.int32)).reshape(W, maxB)
    pos = torch.tensor([[0, 5, 11, -1], [3, 4, 7, 12], [1, 2, 9, 10]], dtype=torch.int32)  # 12: past the table
    keys = torch.arange(W * Hkv * S * E, dtype=torch.float32).reshape(W, Hkv, S, E)
    vals = -keys
    kc = torch.full((P, bs, Hkv, E), 7.0)
    vc = torch.full((P, bs, Hkv, E), 7.0)
    one = torch.ones(1, 1, 0)
    k2, v2 = O.kv_append(kc, vc, perm, pos, keys, vals, one, one)
    want_k = kc.clone()
    want_v = vc.clone()
    for w in range(W):
        for s in range(S):
            p = int(pos[w, s])
            if p < 0 or p >= maxB * bs:
                continue
            page = int(perm[w][p // bs])
            want_k[page, p % bs] = keys[w, :, s]
            want_v[page, p % bs] = vals[w, :, s]
    assert torch.equal(k2, want_k) and torch.equal(v2, want_v)
    assert int((k2 != 7.0).any(-1).any(-1).sum()) == 10  # ten tokens written


def test_kv_append_merge_is_rotation_additive():
    """merge_caches re-rotates keys already rotated at position a by the target
    length b (attention.py:245-251): the result is the rotation at a + b
    (fp32, to rounding)."""
    E, R = 128, 128
    k = torch.randn(3, E)
    a, b = 1234, 40000
    ca, sa = hf_cs([a], R)
    cb, sb = hf_cs([b], R)
    cab, sab = hf_cs([a + b], R)
    twice = O.apply_rotary(O.apply_rotary(k, ca[0], sa[0]), cb[0], sb[0])
    once = O.apply_rotary(k, cab[0], sab[0])
    assert torch.allclose(twice, once, atol=2e-5)


def test_view_metadata_hand_computed_locations():
    # lengths [5, 3, 4]; sequence 0 orders its segments 0,1,2 and sequence 1 2,0,1
    loc, cos, sin = O.view_metadata([5, 3, 4], [[0, 1, 2], [2, 0, 1]], 2, torch.tensor([1.0, 0.25]))
    want = torch.tensor([[[10, 11], [6, 7]], [[5, 6], [1, 2]], [[2, 3], [10, 11]]], dtype=torch.int32)
    assert torch.equal(loc, want)
    assert torch.equal(cos[..., :2], cos[..., 2:])
    assert cos[0, 0, 0, 0].item() == np.float32(np.cos(np.float32(10.0)))
    # a segment missing from a sequence's order: location -1, identity rotation
    loc, cos, sin = O.view_metadata([4, 4], [[0, 1], [1, 1]], 1, torch.tensor([0.5]))
    assert loc[0, 1, 0].item() == -1 and cos[0, 1, 0, 0].item() == 1.0 and sin[0, 1, 0, 0].item() == 0.0
    assert loc[1, 1, 0].item() == 7  # first place of a repeated segment wins (the backward walk assigns it last)


@pytest.mark.parametrize("round_to", [None, torch.bfloat16])
def test_view_metadata_cos_sin_match_transformers_rotary(round_to):
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding
    cfg = Qwen2Config(hidden_size=256, num_attention_heads=2, num_key_value_heads=1, head_dim=128,
                      rope_theta=500000.0, max_position_embeddings=1 << 20)
    rot = Qwen2RotaryEmbedding(cfg)
    lens = [70000, 33, 900]
    order = [[0, 1, 2], [1, 2, 0], [2, 0, 1], [0, 2, 1]]
    S = 3
    loc, cos, sin = O.view_metadata(lens, order, S, rot.inv_freq, 1.0, round_to)
    x = torch.zeros(1, dtype=round_to or torch.float32)
    c_ref, s_ref = rot(x, loc.reshape(-1, S).long())
    assert torch.equal(cos, c_ref.float().reshape(cos.shape))
    assert torch.equal(sin, s_ref.float().reshape(sin.shape))
