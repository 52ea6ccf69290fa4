"""Model integration (dvattention_amd.hf: DVAttnCache / AttentionModule /
model_surgery, python/dvattn/attention.py:100-343) on a random-init Qwen2 of
transformers 5 (no checkpoint is available offline).

Exact reductions pin the integration: with one view the dynamic-view decode is
ordinary causal attention, and workers that see only a shared prompt plus their
own tokens each decode like a single sequence -- both must match transformers'
own eager attention on the concatenated tokens.  Workers that see each other's
segments have no such reduction; there the HIP run is compared with the same
module code driven by the CPU oracle.

CPU tests drive the module code with the oracle ops (host logic of the
integration); GPU tests use the HIP operators.
"""
import copy

import pytest
import torch

from oracle import dvattn_oracle as O

transformers = pytest.importorskip("transformers")


class OracleOps:
    """The three device operations of a decode step, computed by the CPU oracle."""

    @staticmethod
    def kv_append(keys, values, positions, cos, sin, k_pages, v_pages, block_tables):
        k2, v2 = O.kv_append(k_pages.cpu(), v_pages.cpu(), block_tables.cpu(), positions.cpu(), keys.cpu(),
                             values.cpu(), cos.cpu(), sin.cpu())
        k_pages.copy_(k2)
        v_pages.copy_(v2)

    @staticmethod
    def view_metadata(fragment_lengths, order, S, inv_freq, attention_scaling, round_to):
        dev = fragment_lengths.device
        loc, c, s = O.view_metadata(fragment_lengths.tolist(), order.tolist(), S, inv_freq.cpu(), attention_scaling,
                                    round_to)
        return loc.to(dev), c.to(dev), s.to(dev)

    @staticmethod
    def fused(queries, locations, keys, values, scale, fragment_lengths, cosines, sines, rotated_queries, out):
        o, rq = O.fused(scale, locations.cpu(), queries.cpu(), fragment_lengths.cpu(), [k.cpu() for k in keys],
                        [v.cpu() for v in values], cosines.cpu(), sines.cpu())
        rotated_queries.copy_(rq)
        out.copy_(o.to(out.dtype))
        return out


def tiny_qwen2(dtype, device, seed=0):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    cfg = Qwen2Config(vocab_size=320, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=16, num_key_value_heads=1, head_dim=128, max_position_embeddings=8192,
                      rope_theta=10000.0)
    cfg._attn_implementation = "eager"
    torch.manual_seed(seed)
    m = Qwen2ForCausalLM(cfg).eval()
    with torch.no_grad():  # sharper attention than the default 0.02 init
        for layer in m.model.layers:
            layer.self_attn.q_proj.weight.mul_(6.0)
            layer.self_attn.k_proj.weight.mul_(6.0)
    return m.to(device=device, dtype=dtype)


def surgery_copy(model, device=None, dtype=None, attn="sdpa"):
    """A copy of ``model`` with DVAttn attention; ``attn`` is the configured
    attention implementation ("eager" selects the module's PyTorch path, any
    other the ``ops.fused`` path)."""
    from dvattention_amd import hf
    m = copy.deepcopy(model)
    if device is not None:
        m = m.to(device=device, dtype=dtype)
    m.config._attn_implementation = attn
    hf.model_surgery(m)
    assert m.model.layers[0].self_attn.config._attn_implementation == attn
    return m


def ref_logits(model, tokens):
    """transformers' own forward (eager attention, no cache) on one sequence."""
    with torch.no_grad():
        return model(input_ids=tokens[None]).logits[0].float()


def run_steps(model, cache, steps):
    """Feed ``steps`` = list of [W, S] token tensors; returns the logits of each."""
    outs = []
    with torch.no_grad():
        for ids in steps:
            out = model(**cache.get_input_kwargs(ids))
            outs.append(out.logits.float())
    return outs


def single_worker(model, ops, dtype, device, P=11, steps=3, seed=1):
    from dvattention_amd import hf
    g = torch.Generator().manual_seed(seed)
    toks = torch.randint(0, 320, (P + steps,), generator=g).to(device)
    pool = hf.SegmentPool(model.config, 1, 64, dtype, device)
    cache = hf.DVAttnCache([[pool[0]]], model, ops=ops)
    feeds = [toks[:P][None]] + [toks[P + i:P + i + 1][None] for i in range(steps - 1)]
    return toks, run_steps(model, cache, feeds)


def independent_workers(model, ops, dtype, device, P=9, steps=3, seed=2):
    """A shared prompt segment, then two workers that each see [prompt, own]."""
    from dvattention_amd import hf
    g = torch.Generator().manual_seed(seed)
    prompt = torch.randint(0, 320, (P,), generator=g).to(device)
    own = torch.randint(0, 320, (2, steps), generator=g).to(device)
    pool = hf.SegmentPool(model.config, 3, 64, dtype, device)
    pre = hf.DVAttnCache([[pool[0]]], model, ops=ops)
    run_steps(model, pre, [prompt[None]])
    cache = hf.DVAttnCache([[pool[0], pool[1]], [pool[0], pool[2]]], model, ops=ops)
    outs = run_steps(model, cache, [own[:, i:i + 1] for i in range(steps)])
    return prompt, own, outs


# ------------------------------------------------------------------ CPU --

def test_single_worker_matches_transformers_cpu():
    model = tiny_qwen2(torch.float32, "cpu")
    ours = surgery_copy(model)
    toks, outs = single_worker(ours, OracleOps, torch.float32, "cpu")
    P = 11
    ref = ref_logits(model, toks[:P + 2])
    assert torch.allclose(outs[0][0], ref[:P], atol=1e-4, rtol=1e-4)
    for i, o in enumerate(outs[1:]):
        assert torch.allclose(o[0, -1], ref[P + i], atol=1e-4, rtol=1e-4)


def test_independent_workers_match_transformers_cpu():
    model = tiny_qwen2(torch.float32, "cpu")
    ours = surgery_copy(model)
    prompt, own, outs = independent_workers(ours, OracleOps, torch.float32, "cpu")
    for w in range(2):
        ref = ref_logits(model, torch.cat([prompt, own[w]]))
        for i, o in enumerate(outs):
            assert torch.allclose(o[w, -1], ref[len(prompt) + i], atol=1e-4, rtol=1e-4), (w, i)


def test_cache_positions_and_views_cpu():
    """Left padding: masked tokens are not written and do not advance the
    worker's segment; locations follow each worker's own segment order."""
    from dvattention_amd import hf
    model = surgery_copy(tiny_qwen2(torch.float32, "cpu"))
    pool = hf.SegmentPool(model.config, 3, 32, torch.float32, "cpu")
    cache = hf.DVAttnCache([[pool[0], pool[2], pool[1]], [pool[0], pool[1], pool[2]]], model, ops=OracleOps)
    ids = torch.tensor([[5, 6, 7], [8, 9, 10]])
    mask = torch.tensor([[0, 1, 1], [1, 1, 1]])
    with torch.no_grad():
        model(**cache.get_input_kwargs(ids, mask))
    assert [pool[1].get_seq_length(l) for l in range(2)] == [2, 2]
    assert [pool[2].get_seq_length(l) for l in range(2)] == [3, 3]
    assert pool[0].get_seq_length() == 0
    # views ordered as worker 0's structure: [seg0, seg2, seg1]; worker 0 sees 0,2,1 and
    # worker 1 sees 0,1,2 (suffix sums of lengths 0 / 3 / 2, minus S=3, plus s)
    want = torch.tensor([[[2, 3, 4], [2, 3, 4]], [[2, 3, 4], [0, 1, 2]], [[-1, 0, 1], [2, 3, 4]]], dtype=torch.int32)
    assert torch.equal(cache.locations, want)
    assert torch.all(pool.k[0][1, :, 2:] == 0)  # nothing past the two real tokens


def test_eager_module_matches_transformers_cpu():
    """_attn_implementation == "eager": the module's PyTorch attention
    (dvattn_sdpa_pt over per-view rotated queries) on the oracle cache ops
    decodes like transformers' own attention."""
    model = tiny_qwen2(torch.float32, "cpu")
    ours = surgery_copy(model, attn="eager")
    prompt, own, outs = independent_workers(ours, OracleOps, torch.float32, "cpu")
    for w in range(2):
        ref = ref_logits(model, torch.cat([prompt, own[w]]))
        for i, o in enumerate(outs):
            assert torch.allclose(o[w, -1], ref[len(prompt) + i], atol=1e-4, rtol=1e-4), (w, i)


def test_workers_sharing_a_write_segment_append_in_turn_cpu():
    """Two workers whose new tokens go to one segment: worker 0's rows first,
    then worker 1's (attention.py:141-152 appends the workers in turn); no row
    is overwritten and none is left unwritten."""
    from dvattention_amd import hf
    model = surgery_copy(tiny_qwen2(torch.float32, "cpu"))
    pool = hf.SegmentPool(model.config, 2, 32, torch.float32, "cpu")
    run_steps(model, hf.DVAttnCache([[pool[0]]], model, ops=OracleOps), [torch.tensor([[1, 2, 3]])])
    shared = hf.DVAttnCache([[pool[0], pool[1]], [pool[0], pool[1]]], model, write_to=[pool[1], pool[1]],
                            ops=OracleOps)
    ids = torch.tensor([[4, 5], [6, 7]])
    kw = shared.get_input_kwargs(ids)
    captured = []
    orig = OracleOps.kv_append

    def spy(keys, values, positions, cos, sin, k_pages, v_pages, block_tables):
        captured.append((keys.clone(), values.clone(), positions.clone()))
        orig(keys, values, positions, cos, sin, k_pages, v_pages, block_tables)

    shared.ops = type("SpyOps", (OracleOps,), {"kv_append": staticmethod(spy)})
    with torch.no_grad():
        model(**kw)
    assert [pool[1].get_seq_length(l) for l in range(2)] == [4, 4]
    keys, values, positions = captured[0]                   # layer 0
    assert torch.equal(positions, torch.tensor([[0, 1], [2, 3]], dtype=torch.int32))
    v_seg = pool.v[0][1]                                    # [Hkv, capacity, E]
    assert torch.equal(v_seg[:, 0:2], values[0])
    assert torch.equal(v_seg[:, 2:4], values[1])
    assert torch.all(v_seg[:, 4:] == 0)


def test_segments_from_transformers_caches_cpu():
    """A prompt prefilled by transformers itself (its DynamicCache) copied into a
    pool segment, then decoded through the DVAttn module: the logits follow
    transformers' forward on the whole sequence."""
    from dvattention_amd import hf
    model = tiny_qwen2(torch.float32, "cpu")
    ours = surgery_copy(model)
    g = torch.Generator().manual_seed(8)
    toks = torch.randint(0, 320, (12,), generator=g)
    with torch.no_grad():
        pre = model(input_ids=toks[None, :9], use_cache=True).past_key_values
    pool = hf.SegmentPool(ours.config, 1, 64, torch.float32, "cpu")
    segs = hf.segments_from_caches([pre], pool)
    assert [segs[0].get_seq_length(l) for l in range(2)] == [9, 9]
    outs = run_steps(ours, hf.DVAttnCache([segs], ours, ops=OracleOps), [toks[9 + i:10 + i][None] for i in range(3)])
    ref = ref_logits(model, toks)
    for i, o in enumerate(outs):
        assert torch.allclose(o[0, -1], ref[9 + i], atol=1e-4, rtol=1e-4), i


def reference_caller(model, ops, prompt, own, nxt, capacity=None, stock=None):
    """The reference's call shape (attention.py:109-118, 208-251) on transformers
    caches: a prompt cache filled through a one-worker DVAttnCache on an empty
    DynamicCache (or by the unmodified model ``stock``, transformers itself),
    two workers with empty DynamicCaches that each see [prompt, own],
    ``merge_caches(prompt_cache, worker0_cache, decoder)``, then one more token
    on the merged cache.  Returns the logits of every step and the caches."""
    from transformers import DynamicCache

    from dvattention_amd import hf
    if stock is not None:
        with torch.no_grad():
            pre = stock(input_ids=prompt[None], use_cache=True).past_key_values
    else:
        pre = DynamicCache()
        run_steps(model, hf.DVAttnCache([[pre]], model, ops=ops), [prompt[None]])
    w0, w1 = DynamicCache(), DynamicCache()
    cache = hf.DVAttnCache([[pre, w0], [pre, w1]], model, ops=ops, capacity=capacity)
    outs = run_steps(model, cache, [own[:, i:i + 1] for i in range(own.shape[1])])
    hf.merge_caches(pre, w0, model.model, ops=ops)
    solo = hf.DVAttnCache([[pre, DynamicCache()]], model, ops=ops)
    outs += run_steps(model, solo, [nxt[None, None]])
    return outs, pre, w0, w1


def test_reference_signature_with_transformers_caches_cpu():
    """DVAttnCache / merge_caches driven with transformers DynamicCaches in the
    reference's call shape: each worker decodes like transformers on [prompt,
    own], the caller's caches show the appended tokens (their own keys rotated
    at worker-local positions), and after the merge the prompt cache holds the
    worker's keys re-rotated to absolute positions -- transformers' own cache of
    the concatenated sequence -- and decodes the next token like it."""
    model = tiny_qwen2(torch.float32, "cpu")
    ours = surgery_copy(model)
    g = torch.Generator().manual_seed(12)
    P, n = 9, 3
    prompt = torch.randint(0, 320, (P,), generator=g)
    own = torch.randint(0, 320, (2, n), generator=g)
    nxt = torch.randint(0, 320, (), generator=g)
    # capacity 12: the pool doubles while the workers decode; stock: the prompt
    # cache comes from transformers' own forward
    for capacity, stock in ((None, None), (12, None), (None, model)):
        outs, pre, w0, w1 = reference_caller(ours, OracleOps, prompt, own, nxt, capacity, stock)
        for w in range(2):
            ref = ref_logits(model, torch.cat([prompt, own[w]]))
            for i in range(n):
                assert torch.allclose(outs[i][w, -1], ref[P + i], atol=1e-4, rtol=1e-4), (capacity, stock, w, i)
        assert w0.get_seq_length() == n and w1.get_seq_length() == n and pre.get_seq_length() == P + n
        with torch.no_grad():
            full = model(input_ids=torch.cat([prompt, own[0]])[None], use_cache=True).past_key_values
        for layer in range(2):
            assert torch.allclose(pre.layers[layer].keys, full.layers[layer].keys, atol=1e-5, rtol=1e-5)
            assert torch.allclose(pre.layers[layer].values, full.layers[layer].values, atol=1e-6)
        ref = ref_logits(model, torch.cat([prompt, own[0], nxt[None]]))
        assert torch.allclose(outs[-1][0, -1], ref[-1], atol=1e-4, rtol=1e-4), capacity


def test_merge_caches_plain_transformers_caches_cpu():
    """merge_caches on two caches no DVAttnCache holds: the reference's own
    steps (keys rotated by the target's length, then target.update).  The
    appended keys must be those transformers computes for the source tokens at
    positions shifted by the target's length (rotary attention depends on
    relative positions only, so the source's hidden states are unchanged), its
    values the source's own, and the target's tokens untouched."""
    from dvattention_amd import hf
    model = tiny_qwen2(torch.float32, "cpu")
    g = torch.Generator().manual_seed(13)
    a = torch.randint(0, 320, (7,), generator=g)
    b = torch.randint(0, 320, (4,), generator=g)
    with torch.no_grad():
        ca = model(input_ids=a[None], use_cache=True).past_key_values
        cb = model(input_ids=b[None], use_cache=True).past_key_values
        shifted = model(input_ids=b[None], position_ids=torch.arange(7, 11)[None], use_cache=True).past_key_values
    before = [(ca.layers[l].keys.clone(), ca.layers[l].values.clone()) for l in range(2)]
    hf.merge_caches(ca, cb, model.model)
    assert ca.get_seq_length() == 11
    for layer in range(2):
        k, v = ca.layers[layer].keys, ca.layers[layer].values
        assert torch.equal(k[:, :, :7], before[layer][0]) and torch.equal(v[:, :, :7], before[layer][1])
        assert torch.allclose(k[:, :, 7:], shifted.layers[layer].keys, atol=1e-4, rtol=1e-4), layer
        assert torch.equal(v[:, :, 7:], cb.layers[layer].values)


def test_reference_import_path_cpu():
    """``import dvattn.attention`` (the reference's module path) registers the
    operators and exposes the reference's names over this build."""
    import dvattn.attention as A
    import dvattention_amd
    from dvattention_amd import hf
    assert hasattr(torch.ops.libdvatt, "dvattn_paged_sdpa")
    for name in ("dvattn_fused", "dvattn_sdpa", "dvattn_sdpa_pt", "dvattn_rope", "rotate_half",
                 "apply_rotary_pos_emb"):
        assert getattr(A, name) is getattr(dvattention_amd, name)
    for name in ("CacheStructure", "DVAttnCache", "merge_caches", "AttentionModule", "model_surgery"):
        assert getattr(A, name) is getattr(hf, name)


# ------------------------------------------------------------------ GPU --

@pytest.mark.gpu
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 5e-4), (torch.bfloat16, 6e-2)])
def test_single_worker_matches_transformers_gpu(gpu, dtype, tol):
    from dvattention_amd import hf
    model = tiny_qwen2(dtype, gpu)
    ours = surgery_copy(model)
    toks, outs = single_worker(ours, hf.HipOps, dtype, gpu)
    P = 11
    ref = ref_logits(model, toks[:P + 2])
    err = (outs[0][0] - ref[:P]).abs().max().item()
    for i, o in enumerate(outs[1:]):
        err = max(err, (o[0, -1] - ref[P + i]).abs().max().item())
    assert err <= tol, err


@pytest.mark.gpu
def test_independent_workers_match_transformers_gpu(gpu):
    from dvattention_amd import hf
    model = tiny_qwen2(torch.bfloat16, gpu)
    ours = surgery_copy(model)
    prompt, own, outs = independent_workers(ours, hf.HipOps, torch.bfloat16, gpu)
    for w in range(2):
        ref = ref_logits(model, torch.cat([prompt, own[w]]))
        for i, o in enumerate(outs):
            err = (o[w, -1] - ref[len(prompt) + i]).abs().max().item()
            assert err <= 6e-2, (w, i, err)


@pytest.mark.gpu
def test_cross_visible_workers_and_merge_match_oracle_gpu(gpu):
    """Two workers that see each other's segments ([prompt, other, own]), then
    merge_caches of worker 1 into worker 0: the HIP run against the same module
    code on the CPU oracle, fp32."""
    from dvattention_amd import hf
    base = tiny_qwen2(torch.float32, "cpu", seed=3)
    m_gpu = surgery_copy(base, gpu, torch.float32)
    m_cpu = surgery_copy(base)
    g = torch.Generator().manual_seed(4)
    prompt = torch.randint(0, 320, (7,), generator=g)
    own = torch.randint(0, 320, (2, 4), generator=g)
    results = []
    for model, ops, dev in ((m_gpu, hf.HipOps, gpu), (m_cpu, OracleOps, "cpu")):
        pool = hf.SegmentPool(model.config, 3, 64, torch.float32, dev)
        run_steps(model, hf.DVAttnCache([[pool[0]]], model, ops=ops), [prompt[None].to(dev)])
        cache = hf.DVAttnCache([[pool[0], pool[2], pool[1]], [pool[0], pool[1], pool[2]]], model, ops=ops)
        outs = run_steps(model, cache, [own[:, i:i + 1].to(dev) for i in range(3)])
        hf.merge_caches(pool[1], pool[2], model, ops=ops)
        solo = hf.DVAttnCache([[pool[0], pool[1]]], model, ops=ops)
        outs += run_steps(model, solo, [own[:1, 3:4].to(dev)])
        results.append(([o.cpu() for o in outs], [pool.k[0].cpu(), pool.v[1].cpu()]))
    (a, ca), (b, cb) = results
    for x, y in zip(a, b):
        assert torch.allclose(x, y, atol=5e-4, rtol=1e-4), (x - y).abs().max().item()
    for x, y in zip(ca, cb):
        assert torch.allclose(x, y, atol=1e-5, rtol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 5e-4), (torch.bfloat16, 6e-2)])
def test_eager_and_hip_modules_agree_gpu(gpu, dtype, tol):
    """The module's PyTorch attention ("eager") and the HIP dvattn_fused path,
    both on the GPU with the HIP cache operations, on cross-visible workers."""
    from dvattention_amd import hf
    base = tiny_qwen2(dtype, gpu, seed=5)
    g = torch.Generator().manual_seed(6)
    prompt = torch.randint(0, 320, (9,), generator=g).to(gpu)
    own = torch.randint(0, 320, (2, 3), generator=g).to(gpu)
    results = []
    for attn in ("eager", "sdpa"):
        model = surgery_copy(base, attn=attn)
        pool = hf.SegmentPool(model.config, 3, 64, dtype, gpu)
        run_steps(model, hf.DVAttnCache([[pool[0]]], model, ops=hf.HipOps), [prompt[None]])
        cache = hf.DVAttnCache([[pool[0], pool[2], pool[1]], [pool[0], pool[1], pool[2]]], model, ops=hf.HipOps)
        results.append(run_steps(model, cache, [own[:, i:i + 1] for i in range(3)]))
    for x, y in zip(*results):
        err = (x - y).abs().max().item()
        assert err <= tol, err


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 5e-4), (torch.bfloat16, 6e-2)])
def test_reference_signature_with_transformers_caches_gpu(gpu, dtype, tol):
    """The reference's call shape on transformers DynamicCaches with the HIP
    operators: workers against transformers on [prompt, own], then the merged
    prompt cache against transformers' cache of the concatenated sequence and
    the next token's logits."""
    from dvattention_amd import hf
    model = tiny_qwen2(dtype, gpu)
    ours = surgery_copy(model)
    g = torch.Generator().manual_seed(12)
    P, n = 9, 3
    prompt = torch.randint(0, 320, (P,), generator=g).to(gpu)
    own = torch.randint(0, 320, (2, n), generator=g).to(gpu)
    nxt = torch.randint(0, 320, (), generator=g).to(gpu)
    outs, pre, w0, w1 = reference_caller(ours, hf.HipOps, prompt, own, nxt, capacity=12)
    for w in range(2):
        ref = ref_logits(model, torch.cat([prompt, own[w]]))
        for i in range(n):
            err = (outs[i][w, -1] - ref[P + i]).abs().max().item()
            assert err <= tol, (w, i, err)
    assert w0.get_seq_length() == n and pre.get_seq_length() == P + n
    with torch.no_grad():
        full = model(input_ids=torch.cat([prompt, own[0]])[None], use_cache=True).past_key_values
    ktol = 1e-5 if dtype == torch.float32 else 3e-2
    for layer in range(2):
        err = (pre.layers[layer].keys.float() - full.layers[layer].keys.float()).abs().max().item()
        assert err <= ktol * max(1.0, full.layers[layer].keys.abs().max().item()), (layer, err)
    ref = ref_logits(model, torch.cat([prompt, own[0], nxt[None]]))
    assert (outs[-1][0, -1] - ref[-1]).abs().max().item() <= tol


@pytest.mark.gpu
def test_reference_import_path_gpu(gpu):
    """``from dvattn.attention import dvattn_fused`` runs the HIP operator
    (configuration 1's shape) and matches the oracle."""
    from dvattn.attention import dvattn_fused
    g = torch.Generator().manual_seed(9)
    q = torch.randn(1, 16, 1, 128, generator=g)
    k = torch.randn(1, 1, 512, 128, generator=g)
    v = torch.randn(1, 1, 512, 128, generator=g)
    loc = torch.tensor([[[512]]], dtype=torch.int32)
    fl = torch.tensor([512], dtype=torch.int32)
    ang = 512 * (1e4 ** (-torch.arange(0, 64, 2, dtype=torch.float64) / 64))
    c = torch.cat([ang, ang]).cos().float().reshape(1, 1, 1, 64)
    s = torch.cat([ang, ang]).sin().float().reshape(1, 1, 1, 64)
    rq = torch.empty(1, 1, 16, 1, 128, device=gpu)
    out = torch.empty(1, 16, 1, 128, device=gpu)
    dvattn_fused(q.to(gpu), loc.to(gpu), [k.to(gpu)], [v.to(gpu)], 128 ** -0.5, fl.to(gpu), c.to(gpu), s.to(gpu),
                 rotated_queries=rq, out=out)
    ref, rq_ref = O.fused(128 ** -0.5, loc, q, fl, [k], [v], c, s)
    assert torch.equal(rq.cpu(), rq_ref)
    assert (out.cpu() - ref).abs().max().item() <= 1e-5
