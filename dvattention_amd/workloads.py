"""Synthetic, seeded inputs for the five benchmark configurations of the
paged / varlen / contiguous DVAttn operators, plus their algorithmic byte and
flop counts (what a roofline measurement divides by).

Conventions follow the reference's in-tree caller (python/dvattn/attention.py:
158-192): HF-style cos/sin (``cat(freqs, freqs)``, angles in float64, stored
fp32), views laid out back to back in each sequence's logical token stream
(view f starts at ``sum_{g<f} fragment_lengths[g]``), ``locations`` = last
visible key of each view.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

DTYPES = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}
ESIZE = {torch.float32: 4, torch.float16: 2, torch.bfloat16: 2}


def hf_cos_sin(positions, rotary_dim: int, base: float):
    """cos/sin of ``positions`` (int array, any shape) -> fp32 ``[..., rotary_dim]``
    with the HF convention ``emb = cat(freqs, freqs)``."""
    pos = np.asarray(positions, dtype=np.float64)
    inv = 1.0 / (base ** (np.arange(0, rotary_dim, 2, dtype=np.float64) / rotary_dim))
    freqs = pos[..., None] * inv
    emb = np.concatenate([freqs, freqs], axis=-1)
    return torch.from_numpy(np.cos(emb).astype(np.float32)), torch.from_numpy(np.sin(emb).astype(np.float32))


def _randn(shape, dtype, device, gen, scale=1.0):
    t = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    if scale != 1.0:
        t.mul_(scale)
    return t.to(dtype)


@dataclass
class Workload:
    name: str
    op: str                      # "paged" | "varlen" | "fused" | "sdpa"
    dtype: torch.dtype
    scale: float
    t: dict = field(default_factory=dict)   # tensors (on the workload's device)
    alg_bytes: int = 0
    flops: int = 0
    meta: dict = field(default_factory=dict)

    def out_like(self) -> torch.Tensor:
        return torch.empty(self.meta["out_shape"], dtype=self.dtype, device=self.t["queries"].device)


# ---------------------------------------------------------------------------
def paged_workload(name, *, W, Hkv, S, lengths, R, base, bs, dtype, device, seed, k_scale=1.0,
                   slack_pages=0, causal_chunk=False) -> Workload:
    """One view per sequence.  ``lengths[w]`` tokens live in the cache of
    sequence w; with ``causal_chunk`` the S queries are the last S tokens
    (locations = L - S + s), else every query sees all L tokens."""
    gen = torch.Generator(device=device).manual_seed(seed)
    Hq = 16 * Hkv
    E = 128
    lengths = np.asarray(lengths, dtype=np.int64)
    npages = (lengths + bs - 1) // bs
    P = int(npages.sum()) + slack_pages
    rng = np.random.default_rng(seed)
    perm = rng.permutation(P).astype(np.int32)
    maxB = int(npages.max())
    bt = np.zeros((W, maxB), dtype=np.int32)
    o = 0
    for w in range(W):
        bt[w, :npages[w]] = perm[o:o + npages[w]]
        o += npages[w]
    if causal_chunk:
        loc = lengths[:, None] - S + np.arange(S)[None, :]
    else:
        loc = np.repeat((lengths - 1)[:, None], S, axis=1)
    loc = loc[None].astype(np.int32)                         # [1,W,S]
    cos, sin = hf_cos_sin(loc, R, base)                     # [1,W,S,R]
    fl = np.array([int(lengths.max())], dtype=np.int32)
    t = {
        "queries": _randn((W, Hq, S, E), dtype, device, gen),
        "k_cache": _randn((P, bs, Hkv, E), dtype, device, gen, k_scale),
        "v_cache": _randn((P, bs, Hkv, E), dtype, device, gen),
        "locations": torch.from_numpy(loc).to(device),
        "cosines": cos.to(device),
        "sines": sin.to(device),
        "fragment_lengths": torch.from_numpy(fl).to(device),
        "block_tables": torch.from_numpy(bt).to(device),
    }
    es = ESIZE[dtype]
    vis = np.minimum(lengths, loc[0].max(axis=1) + 1)       # union over the S queries
    kv = int(vis.sum()) * Hkv * 2 * E * es
    qo = 2 * W * S * Hq * E * es
    cs = 2 * 1 * W * S * R * 4
    idx = W * S * 4 + int(((vis + bs - 1) // bs).sum()) * 4 + 4
    per_q_vis = np.minimum(lengths[:, None], loc[0] + 1)    # [W,S]
    flops = int(per_q_vis.sum()) * Hq * 4 * E
    return Workload(name, "paged", dtype, E ** -0.5, t, kv + qo + cs + idx, flops,
                    {"out_shape": (W, Hq, S, E), "W": W, "S": S, "Hkv": Hkv, "bs": bs, "R": R,
                     "lengths": lengths.tolist(), "kv_bytes": kv, "P": P})


def varlen_workload(name, *, W, Hkv, R, base, bs, dtype, device, seed, median=2048, sigma=1.0,
                    lo=64, hi=32768, nviews=(2, 3, 4), F=4, max_offset=65535) -> Workload:
    """One query token per sequence (T = W), each sequence's cache cut into
    2-4 views; a view's query rotation uses a random relative offset."""
    gen = torch.Generator(device=device).manual_seed(seed)
    rng = np.random.default_rng(seed)
    Hq = 16 * Hkv
    E = 128
    L = np.clip(np.round(rng.lognormal(math.log(median), sigma, size=W)), lo, hi).astype(np.int64)
    nv = rng.choice(np.asarray(nviews), size=W)
    lens = np.zeros((W, F), dtype=np.int64)
    for w in range(W):
        n = int(min(nv[w], L[w]))
        cuts = np.sort(rng.choice(np.arange(1, L[w]), size=n - 1, replace=False)) if n > 1 else np.array([], int)
        edges = np.concatenate([[0], cuts, [L[w]]])
        lens[w, :n] = np.diff(edges)
        nv[w] = n
    fl = lens.max(axis=0).astype(np.int32)                  # [F]
    off = np.concatenate([[0], np.cumsum(fl)[:-1]]).astype(np.int64)
    maxB = int((int(fl.sum()) + bs - 1) // bs)
    # back only the touched logical pages, permuted over the pool
    touched = []
    for w in range(W):
        pages = set()
        for f in range(int(nv[w])):
            if lens[w, f] > 0:
                pages.update(range(int(off[f] // bs), int((off[f] + lens[w, f] - 1) // bs) + 1))
        touched.append(sorted(pages))
    P = sum(len(p) for p in touched)
    perm = rng.permutation(P).astype(np.int32)
    bt = np.zeros((W, maxB), dtype=np.int32)
    o = 0
    for w in range(W):
        for lp in touched[w]:
            bt[w, lp] = perm[o]
            o += 1
    loc = np.ascontiguousarray(np.where(np.arange(F)[None, :] < nv[:, None], lens - 1, -1).T.astype(np.int32))  # [F,T]
    rel = rng.integers(0, max_offset + 1, size=(F, W))
    cos, sin = hf_cos_sin(rel, R, base)                     # [F,T,R]
    cos, sin = cos[..., : R // 2].contiguous(), sin[..., : R // 2].contiguous()
    cu_q = np.arange(W + 1, dtype=np.int32)
    cu_k = np.concatenate([[0], np.cumsum(L)]).astype(np.int32)
    t = {
        "queries": _randn((W, Hq, E), dtype, device, gen),
        "k_cache": _randn((P, bs, Hkv, E), dtype, device, gen),
        "v_cache": _randn((P, bs, Hkv, E), dtype, device, gen),
        "locations": torch.from_numpy(loc).to(device),
        "cosines": cos.to(device),
        "sines": sin.to(device),
        "fragment_lengths": torch.from_numpy(fl).to(device),
        "block_tables": torch.from_numpy(bt).to(device),
        "cu_seqlens_q": torch.from_numpy(cu_q).to(device),
        "cu_seqlens_k": torch.from_numpy(cu_k).to(device),
    }
    es = ESIZE[dtype]
    vis = int(np.where(loc.T >= 0, np.minimum(lens, loc.T + 1), 0).sum())
    kv = vis * Hkv * 2 * E * es
    qo = 2 * W * Hq * E * es
    cs = 2 * F * W * (R // 2) * 4
    idx = F * W * 4 + sum(len(p) for p in touched) * 4 + F * 4 + (W + 1) * 4
    flops = vis * Hq * 4 * E
    return Workload(name, "varlen", dtype, E ** -0.5, t, kv + qo + cs + idx, flops,
                    {"out_shape": (W, Hq, E), "W": W, "Hkv": Hkv, "bs": bs, "R": R, "lengths": L.tolist(),
                     "views": nv.tolist(), "kv_bytes": kv, "sigma": sigma, "P": P})


def fused_workload(name, *, W, Hkv, L, R, base, dtype, device, seed, position=None) -> Workload:
    """``dvattn_fused`` on one contiguous view of L tokens per sequence; the
    query sits at ``position`` (default L) and sees all L keys."""
    gen = torch.Generator(device=device).manual_seed(seed)
    Hq = 16 * Hkv
    E = 128
    pos = L if position is None else position
    loc = np.full((1, W, 1), pos, dtype=np.int32)
    cos, sin = hf_cos_sin(loc, R, base)                     # [1,W,1,R]
    t = {
        "queries": _randn((W, Hq, 1, E), dtype, device, gen),
        "keys": [_randn((W, Hkv, L, E), dtype, device, gen)],
        "values": [_randn((W, Hkv, L, E), dtype, device, gen)],
        "locations": torch.from_numpy(loc).to(device),
        "cosines": cos.to(device),
        "sines": sin.to(device),
        "fragment_lengths": torch.tensor([L], dtype=torch.int32, device=device),
    }
    es = ESIZE[dtype]
    vis = min(L, pos + 1)
    kv = W * vis * Hkv * 2 * E * es
    qo = W * Hq * E * es * 3          # q read, rq written and read back
    out = W * Hq * E * es
    cs = 2 * W * R * 4
    flops = W * vis * Hq * 4 * E
    return Workload(name, "fused", dtype, E ** -0.5, t, kv + qo + out + cs + 8, flops,
                    {"out_shape": (W, Hq, 1, E), "rq_shape": (1, W, Hq, 1, E), "kv_bytes": kv})


# ---------------------------------------------------------------------------
# The five configurations of the benchmark (seeded).
def config(i: int, device="cuda", seed=1234) -> Workload:
    if i == 1:
        return fused_workload("cfg1_fused_fp32_L512", W=1, Hkv=1, L=512, R=64, base=1e4, dtype=torch.float32,
                              device=device, seed=seed)
    if i == 2:
        rng = np.random.default_rng(seed)
        lengths = rng.integers(1024, 8192, size=32, endpoint=True)
        return paged_workload("cfg2_paged_bf16_b32_L1k-8k", W=32, Hkv=8, S=1, lengths=lengths, R=128, base=1e4,
                              bs=16, dtype=torch.bfloat16, device=device, seed=seed)
    if i == 3:
        return varlen_workload("cfg3_varlen_fp16_b64_views2-4", W=64, Hkv=4, R=64, base=1e4, bs=16,
                               dtype=torch.float16, device=device, seed=seed)
    if i == 4:
        return paged_workload("cfg4_paged_bf16_b4_L128k", W=4, Hkv=8, S=1, lengths=[131072] * 4, R=128,
                              base=5e5, bs=64, dtype=torch.bfloat16, device=device, seed=seed, k_scale=0.5)
    if i == 5:
        return paged_workload("cfg5_chunk_bf16_b16_S16_L8208", W=16, Hkv=8, S=16, lengths=[8192 + 16] * 16, R=32,
                              base=1e4, bs=16, dtype=torch.bfloat16, device=device, seed=seed, causal_chunk=True)
    raise ValueError(f"no config {i}")


def as_varlen(wl: Workload) -> Workload:
    """The same problem through ``dvattn_varlen_paged_sdpa``: a paged workload's
    S query tokens per sequence packed as T = W*S tokens (cu_seqlens_q =
    S * arange(W + 1)), locations ``[F,T]``, half-width cos/sin ``[F,T,R/2]``
    (the first R/2 entries of each full-width row), queries ``[T,Hq,E]``.  The
    output ``[T,Hq,E]`` is the paged output with its S axis moved next to W."""
    assert wl.op == "paged"
    t = wl.t
    W, S, R = wl.meta["W"], wl.meta["S"], wl.meta["R"]
    F = t["locations"].shape[0]
    T = W * S
    Hq = t["queries"].shape[1]
    dev = t["queries"].device
    vt = {
        "queries": t["queries"].permute(0, 2, 1, 3).reshape(T, Hq, -1).contiguous(),
        "locations": t["locations"].reshape(F, T).contiguous(),
        "cosines": t["cosines"].reshape(F, T, R)[..., : R // 2].contiguous(),
        "sines": t["sines"].reshape(F, T, R)[..., : R // 2].contiguous(),
        "fragment_lengths": t["fragment_lengths"],
        "k_cache": t["k_cache"],
        "v_cache": t["v_cache"],
        "block_tables": t["block_tables"],
        "cu_seqlens_q": (S * torch.arange(W + 1, dtype=torch.int32)).to(dev),
        "cu_seqlens_k": torch.zeros(W + 1, dtype=torch.int32, device=dev),
    }
    cs = 2 * F * T * (R // 2) * 4
    alg = wl.alg_bytes - 2 * F * T * R * 4 + cs + (W + 1) * 4
    meta = dict(wl.meta, out_shape=(T, Hq, t["queries"].shape[-1]), T=T, paged_name=wl.name)
    return Workload(wl.name.replace("cfg5_chunk", "cfg5v_varlen_chunk"), "varlen", wl.dtype, wl.scale, vt, alg,
                    wl.flops, meta)


def workload(key, device="cuda", seed=1234) -> Workload:
    """A configuration by key: 1-5, "5v" (configuration 5 through the varlen op),
    "5f" (configuration 5's shape in fp32: the fp32 multi-query kernel), or "2u"
    (configuration 2 with every sequence at 8192 keys: the north star's "batch
    32 x 8k context" taken literally)."""
    if str(key) == "5v":
        return as_varlen(config(5, device=device, seed=seed))
    if str(key) == "5f":
        return paged_workload("cfg5f_chunk_fp32_b16_S16_L8208", W=16, Hkv=8, S=16, lengths=[8192 + 16] * 16, R=32,
                              base=1e4, bs=16, dtype=torch.float32, device=device, seed=seed, causal_chunk=True)
    if str(key) == "2u":
        return paged_workload("cfg2u_paged_bf16_b32_L8k", W=32, Hkv=8, S=1, lengths=[8192] * 32, R=128, base=1e4,
                              bs=16, dtype=torch.bfloat16, device=device, seed=seed)
    return config(int(key), device=device, seed=seed)


def run(wl: Workload, out: torch.Tensor | None = None, rq: torch.Tensor | None = None):
    """Run a workload through the torch operator API of dvattention_amd."""
    from . import attention as A
    t = wl.t
    if out is None:
        out = wl.out_like()
    if wl.op == "paged":
        A.dvattn_paged_sdpa(t["queries"], t["locations"], t["cosines"], t["sines"], t["fragment_lengths"],
                            t["k_cache"], t["v_cache"], t["block_tables"], wl.scale, out=out)
    elif wl.op == "varlen":
        A.dvattn_varlen_paged_sdpa(t["queries"], t["locations"], t["cosines"], t["sines"], t["fragment_lengths"],
                                   t["k_cache"], t["v_cache"], t["block_tables"], t["cu_seqlens_q"],
                                   t["cu_seqlens_k"], wl.scale, out=out)
    elif wl.op == "fused":
        if rq is None:
            rq = torch.empty(wl.meta["rq_shape"], dtype=wl.dtype, device=out.device)
        A.dvattn_fused(t["queries"], t["locations"], t["keys"], t["values"], wl.scale, t["fragment_lengths"],
                       t["cosines"], t["sines"], rotated_queries=rq, out=out)
    else:
        raise ValueError(wl.op)
    return out
