"""GPU parity of the cache-side kernels (marked ``gpu``): the K-side append
(key rotation + page writes, also merge_caches' re-rotation) and the on-device
view metadata, against the CPU oracle.

The append is integer/byte work plus a rotation PyTorch evaluates with fixed
roundings, so whole caches are compared bit for bit (untouched rows keep their
sentinel values).  View locations are bit-exact; cos/sin are within 1e-6 of the
oracle (the GPU's cosf/sinf against PyTorch's CPU cos/sin of the same fp32
angle).
"""
import numpy as np
import pytest
import torch

from oracle import dvattn_oracle as O

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
TRIG_TOL = 1e-6


def hf_cs(pos, R, base=1e4):
    pos = np.asarray(pos, dtype=np.float64)
    inv = 1.0 / (base ** (np.arange(0, R, 2, dtype=np.float64) / R))
    fr = pos[..., None] * inv
    emb = np.concatenate([fr, fr], -1)
    return torch.from_numpy(np.cos(emb).astype(np.float32)), torch.from_numpy(np.sin(emb).astype(np.float32))


@pytest.fixture(scope="module")
def dv(gpu):
    import dvattention_amd
    return dvattention_amd


def append_case(dtype, R, layout, seed, W=3, Hkv=4, S=5, E=128, bs=16, maxB=4, cos_model=False):
    """Caches filled with sentinels, a page table with an invalid entry per
    sequence, positions with a masked token and one past the table."""
    g = torch.Generator().manual_seed(seed)
    P = W * maxB + 3
    perm = torch.randperm(P, generator=g)[: W * maxB].to(torch.int32).reshape(W, maxB)
    perm[0, 3] = -1
    perm[1, 3] = P + 5
    pos = torch.empty(W, S, dtype=torch.int32)
    for w in range(W):
        pos[w] = torch.randperm(maxB * bs, generator=g)[:S].to(torch.int32)
    pos[0, 1] = -1
    pos[2, 0] = maxB * bs + 3
    pos[0, 2] = 3 * bs + 2  # on the invalid page of sequence 0
    pos[1, 2] = 3 * bs + 7  # page id past num_blocks
    if layout == "hf_view":   # k_proj(...).view(B, L, H, D).transpose(1, 2)
        keys = torch.randn(W, S, Hkv, E, generator=g).to(dtype).transpose(1, 2)
        vals = torch.randn(W, S, Hkv, E, generator=g).to(dtype).transpose(1, 2)
    else:
        keys = torch.randn(W, Hkv, S, E, generator=g).to(dtype)
        vals = torch.randn(W, Hkv, S, E, generator=g).to(dtype)
    kc = torch.randn(P, bs, Hkv, E, generator=g).to(dtype)
    vc = torch.randn(P, bs, Hkv, E, generator=g).to(dtype)
    if R:
        c, s = hf_cs(np.random.default_rng(seed).integers(0, 200000, size=(W, S)), R)
    else:
        c, s = torch.zeros(W, S, 0), torch.zeros(W, S, 0)
    if cos_model:
        c, s = c.to(dtype), s.to(dtype)
    return kc, vc, perm, pos, keys, vals, c, s


def run_append(dv, gpu, kc, vc, bt, pos, keys, vals, c, s):
    kg, vg = kc.to(gpu), vc.to(gpu)
    keys_g = keys.to(gpu) if keys.is_contiguous() else keys.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
    vals_g = vals.to(gpu) if vals.is_contiguous() else vals.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
    dv.dvattn_paged_kv_append(keys_g, vals_g, pos.to(gpu), c.to(gpu), s.to(gpu), kg, vg, bt.to(gpu))
    torch.cuda.synchronize()
    return kg.cpu(), vg.cpu()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("cos_model", [False, True])
@pytest.mark.parametrize("R", [128, 64, 0])
@pytest.mark.parametrize("layout", ["contig", "hf_view"])
def test_kv_append_bit_exact(dv, gpu, dtype, cos_model, R, layout):
    if cos_model and dtype == torch.float32:
        pytest.skip("model-dtype cos/sin are float32 here")
    case = append_case(dtype, R, layout, seed=R + 7 * int(cos_model) + (layout == "hf_view"), cos_model=cos_model)
    kc, vc, bt, pos, keys, vals, c, s = case
    if layout == "hf_view":
        assert not keys.is_contiguous() and keys.stride(3) == 1
    k_ref, v_ref = O.kv_append(kc, vc, bt, pos, keys, vals, c, s)
    k_gpu, v_gpu = run_append(dv, gpu, *case)
    assert torch.equal(k_gpu, k_ref), "K cache differs"
    assert torch.equal(v_gpu, v_ref), "V cache differs"
    assert not torch.equal(k_ref, kc)  # something was written


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("E,R,offset", [(128, 8, 0), (100, 20, 0), (128, 128, 1), (64, 24, 0)])
def test_kv_append_element_path(dv, gpu, dtype, E, R, offset):
    """Shapes or alignments the 16-byte path cannot take (R/2 or E not a
    multiple of a run, keys at an odd element offset) use the per-element path."""
    kc, vc, bt, pos, keys, vals, c, s = append_case(dtype, R, "contig", seed=E + R + offset, E=E)
    if offset:
        big = torch.randn(keys.shape[:-1] + (E + offset,)).to(dtype)
        big[..., offset:] = keys
        keys = big[..., offset:]
        assert keys.stride(3) == 1 and keys.storage_offset() == offset
    k_ref, v_ref = O.kv_append(kc, vc, bt, pos, keys, vals, c, s)
    kg, vg = kc.to(gpu), vc.to(gpu)
    keys_g = keys.to(gpu) if not offset else big.to(gpu)[..., offset:]
    dv.dvattn_paged_kv_append(keys_g, vals.to(gpu), pos.to(gpu), c.to(gpu), s.to(gpu), kg, vg, bt.to(gpu))
    assert torch.equal(kg.cpu(), k_ref) and torch.equal(vg.cpu(), v_ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_merge_caches_paged(dv, gpu, dtype):
    """merge_caches (attention.py:245-251): source keys re-rotated by the target
    length, one cos/sin row for every token, written at the target's next
    positions."""
    Hkv, L, E, bs, R = 2, 37, 128, 16, 128
    tgt_len = 50
    maxB = (tgt_len + L + bs - 1) // bs
    P = maxB + 4
    g = torch.Generator().manual_seed(3)
    bt = torch.randperm(P, generator=g)[:maxB].to(torch.int32).reshape(1, maxB)
    src_k = torch.randn(1, Hkv, L, E, generator=g).to(dtype)
    src_v = torch.randn(1, Hkv, L, E, generator=g).to(dtype)
    kc = torch.randn(P, bs, Hkv, E, generator=g).to(dtype)
    vc = torch.randn(P, bs, Hkv, E, generator=g).to(dtype)
    c, s = hf_cs([tgt_len], R)
    c, s = c[0].to(dtype), s[0].to(dtype)  # the model's rotary output dtype
    pos = (tgt_len + torch.arange(L, dtype=torch.int32)).reshape(1, L)
    k_ref, v_ref = O.kv_append(kc, vc, bt, pos, src_k, src_v, c.reshape(1, 1, R), s.reshape(1, 1, R))
    kg, vg = kc.to(gpu), vc.to(gpu)
    dv.merge_caches_paged(src_k.to(gpu), src_v.to(gpu), c.to(gpu), s.to(gpu), kg, vg, bt.to(gpu), pos.to(gpu))
    assert torch.equal(kg.cpu(), k_ref) and torch.equal(vg.cpu(), v_ref)


def test_kv_append_into_contiguous_cache(dv, gpu):
    """A contiguous [B,Hkv,L,E] cache (the dvattn_sdpa layout) written through
    its [B,L,Hkv,E] view: one page per sequence, block_size L."""
    dtype = torch.bfloat16
    B, Hkv, L, E, S, R = 3, 2, 40, 128, 4, 64
    cache_k = torch.randn(B, Hkv, L, E).to(dtype)
    cache_v = torch.randn(B, Hkv, L, E).to(dtype)
    keys = torch.randn(B, Hkv, S, E).to(dtype)
    vals = torch.randn(B, Hkv, S, E).to(dtype)
    pos = torch.tensor([[30, 31, 32, 33], [0, 1, 2, 3], [36, 37, 38, 39]], dtype=torch.int32)
    bt = torch.arange(B, dtype=torch.int32).reshape(B, 1)
    c, s = hf_cs(np.arange(B * S).reshape(B, S) + 100, R)
    k_ref, v_ref = O.kv_append(cache_k.permute(0, 2, 1, 3), cache_v.permute(0, 2, 1, 3), bt, pos, keys, vals, c, s)
    kg, vg = cache_k.to(gpu), cache_v.to(gpu)
    dv.dvattn_paged_kv_append(keys.to(gpu), vals.to(gpu), pos.to(gpu), c.to(gpu), s.to(gpu),
                              kg.permute(0, 2, 1, 3), vg.permute(0, 2, 1, 3), bt.to(gpu))
    assert torch.equal(kg.permute(0, 2, 1, 3).cpu(), k_ref) and torch.equal(vg.permute(0, 2, 1, 3).cpu(), v_ref)


def test_decode_step_append_then_attend(dv, gpu):
    """One decode step: append the new token's K/V at position L_w, then attend
    with locations L_w (the newest key visible) -- the GPU result matches the
    oracle run on the oracle's appended cache."""
    dtype = torch.bfloat16
    W, Hkv, E, bs, R = 4, 2, 128, 16, 128
    lens = [33, 70, 5, 128]
    maxB = 10
    P = W * maxB
    g = torch.Generator().manual_seed(11)
    bt = torch.randperm(P, generator=g).to(torch.int32).reshape(W, maxB)
    kc = (torch.randn(P, bs, Hkv, E, generator=g) * 0.5).to(dtype)
    vc = torch.randn(P, bs, Hkv, E, generator=g).to(dtype)
    keys = torch.randn(W, Hkv, 1, E, generator=g).to(dtype)
    vals = torch.randn(W, Hkv, 1, E, generator=g).to(dtype)
    pos = torch.tensor(lens, dtype=torch.int32).reshape(W, 1)
    kcos, ksin = hf_cs(np.array(lens).reshape(W, 1), R)
    k_ref, v_ref = O.kv_append(kc, vc, bt, pos, keys, vals, kcos, ksin)
    kg, vg = kc.to(gpu), vc.to(gpu)
    dv.dvattn_paged_kv_append(keys.to(gpu), vals.to(gpu), pos.to(gpu), kcos.to(gpu), ksin.to(gpu), kg, vg,
                              bt.to(gpu))
    assert torch.equal(kg.cpu(), k_ref) and torch.equal(vg.cpu(), v_ref)
    q = torch.randn(W, 16 * Hkv, 1, E, generator=g).to(dtype)
    loc = torch.tensor(lens, dtype=torch.int32).reshape(1, W, 1)
    qc, qs = hf_cs(np.array(lens).reshape(1, W, 1), R)
    fl = torch.tensor([max(lens) + 1], dtype=torch.int32)
    ref = O.paged_sdpa(E ** -0.5, loc, q, qc, qs, fl, k_ref, v_ref, bt)
    out = dv.dvattn_paged_sdpa(q.to(gpu), loc.to(gpu), qc.to(gpu), qs.to(gpu), fl.to(gpu), kg, vg, bt.to(gpu),
                               E ** -0.5)
    err = (out.float().cpu() - ref.float()).abs().max().item()
    assert err <= 2e-2, err


@pytest.mark.parametrize("scaling,round_to", [(1.0, None), (1.25, None), (1.0, torch.bfloat16)])
def test_view_metadata(dv, gpu, scaling, round_to):
    F, W, S, R = 4, 6, 3, 128
    rng = np.random.default_rng(5)
    lens = [131000, 17, 2048, 900]
    order = np.stack([rng.permutation(F) for _ in range(W)]).astype(np.int32)
    order[5] = [1, 1, 3, 2]  # view 0 missing, view 1 twice
    inv_freq = (1.0 / (500000.0 ** (torch.arange(0, R, 2, dtype=torch.float) / R))).float()
    loc_r, cos_r, sin_r = O.view_metadata(lens, order.tolist(), S, inv_freq, scaling, round_to)
    loc, cos, sin = dv.dvattn_view_metadata(torch.tensor(lens, dtype=torch.int32, device=gpu),
                                            torch.from_numpy(order).to(gpu), S, inv_freq.to(gpu), scaling, round_to)
    assert torch.equal(loc.cpu(), loc_r)
    dc = (cos.cpu() - cos_r).abs()
    ds = (sin.cpu() - sin_r).abs()
    if round_to is None:
        assert dc.max().item() <= TRIG_TOL * scaling and ds.max().item() <= TRIG_TOL * scaling
    else:
        # one bf16 step where the fp32 values straddle a rounding boundary
        assert dc.max().item() <= 2 ** -8 and ds.max().item() <= 2 ** -8
        assert (dc > 0).float().mean().item() < 1e-2


def test_capi_entry_points_match_ops(dv, gpu):
    from dvattention_amd import capi
    kc, vc, bt, pos, keys, vals, c, s = append_case(torch.bfloat16, 128, "hf_view", seed=21)
    ka, va = run_append(dv, gpu, kc, vc, bt, pos, keys, vals, c, s)
    kg, vg = kc.to(gpu), vc.to(gpu)
    keys_g = keys.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
    vals_g = vals.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
    capi.kv_append(kg, vg, bt.to(gpu), pos.to(gpu), keys_g, vals_g, c.to(gpu), s.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(kg.cpu(), ka) and torch.equal(vg.cpu(), va)
    F, W, S, R = 2, 3, 2, 64
    fl = torch.tensor([40, 9], dtype=torch.int32, device=gpu)
    order = torch.tensor([[0, 1], [1, 0], [0, 1]], dtype=torch.int32, device=gpu)
    inv = torch.rand(R // 2, device=gpu)
    l1, c1, s1 = dv.dvattn_view_metadata(fl, order, S, inv)
    l2 = torch.empty_like(l1)
    c2 = torch.empty_like(c1)
    s2 = torch.empty_like(s1)
    capi.view_metadata(l2, c2, s2, fl, order, inv)
    torch.cuda.synchronize()
    assert torch.equal(l1, l2) and torch.equal(c1, c2) and torch.equal(s1, s2)


def test_kv_append_rejects_bad_arguments(dv, gpu):
    kc, vc, bt, pos, keys, vals, c, s = [t.to(gpu) for t in append_case(torch.bfloat16, 64, "contig", seed=1)]
    with pytest.raises(RuntimeError, match="cosines must be float32"):
        dv.dvattn_paged_kv_append(keys, vals, pos, c.half(), s.half(), kc, vc, bt)
    with pytest.raises(RuntimeError, match="keys must have dtype"):
        dv.dvattn_paged_kv_append(keys.float(), vals, pos, c, s, kc, vc, bt)
    with pytest.raises(RuntimeError, match="even"):
        dv.dvattn_paged_kv_append(keys, vals, pos, c[..., :63], s[..., :63], kc, vc, bt)


def test_kv_append_and_metadata_replay_in_a_graph(dv, gpu):
    """Both ops allocate nothing and set no memory with memset nodes, so a
    decode step can capture them; every replay (with eager work between
    replays) equals the eager result."""
    kc, vc, bt, pos, keys, vals, c, s = [t.to(gpu) for t in append_case(torch.bfloat16, 128, "contig", seed=9)]
    k0, v0 = kc.clone(), vc.clone()
    dv.dvattn_paged_kv_append(keys, vals, pos, c, s, kc, vc, bt)
    k_eager, v_eager = kc.clone(), vc.clone()
    fl = torch.tensor([300, 20, 7], dtype=torch.int32, device=gpu)
    order = torch.tensor([[0, 1, 2], [2, 1, 0]], dtype=torch.int32, device=gpu)
    inv = torch.rand(64, device=gpu)
    l_e, c_e, s_e = dv.dvattn_view_metadata(fl, order, 2, inv)
    loc, cos, sin = torch.empty_like(l_e), torch.empty_like(c_e), torch.empty_like(s_e)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        dv.dvattn_paged_kv_append(keys, vals, pos, c, s, kc, vc, bt)
        torch.ops.libdvatt.dvattn_view_metadata(loc, cos, sin, fl, order, inv, 1.0, None)
    for _ in range(3):
        kc.copy_(k0)
        vc.copy_(v0)
        loc.zero_()
        cos.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(kc, k_eager) and torch.equal(vc, v_eager)
        assert torch.equal(loc, l_e) and torch.equal(cos, c_e) and torch.equal(sin, s_e)
