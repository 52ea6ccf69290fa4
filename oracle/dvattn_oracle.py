"""CPU oracle for the DVAttn hot path -- TEST INFRASTRUCTURE ONLY.

This module restates, on the CPU in float32 (torch CPU tensors), what the
reference operators compute.  It is the checker for the HIP implementation in
``dvattention_amd``; it is never the thing that is measured or shipped.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.

Every function cites the reference lines (paths relative to the reference
repository root) whose behaviour it restates:

* ``rope_q``          -- src/rope.cuh:2-52 (full-width cos/sin, only entries
                         ``[0, R/2)`` are read), src/binding.cu:41-77.
* ``rope_q_varlen``   -- src/rope.cuh:67-100 (half-width cos/sin),
                         src/binding.cu:205-247.
* ``sdpa_views``      -- python/dvattn/attention.py:36-65 (``dvattn_sdpa_pt``)
                         with the kernels' extra bound ``l < fragment_lengths[f]``
                         (src/kernels/kernel_v21.cuh:85-87) and their all-zero
                         output for a row with no visible key
                         (src/kernels/paged_kernel_v21.cuh:318-345).
* ``paged_sdpa``      -- src/binding.cu:151-203 + paged_kernel_v21.cuh:80-120,198
                         (page-table gather, concatenated view layout).
* ``varlen_paged_sdpa`` -- src/binding.cu:249-296 +
                         varlen_paged_kernel_v21.cuh:40-47,75-104.
* ``contig_sdpa``     -- src/binding.cu:79-149 + kernel_v21.cuh:84-114
                         (per-view contiguous fragments ``[B, Hkv, L, E]``).
* ``fused``           -- src/binding.cu:356-372 (rope, then contiguous sdpa).
* ``apply_rotary``    -- python/dvattn/attention.py:75-88 (``rotate_half`` /
                         ``apply_rotary_pos_emb``, the key-side rotation) as
                         PyTorch evaluates it in the input dtypes.
* ``kv_append``       -- attention.py:304 (key rotation) + 141-152 (append to the
                         sequence's own cache) + 245-251 (merge_caches), on a
                         paged cache.
* ``view_metadata``   -- attention.py:158-186 (per-view locations from the
                         segment orders, then the transformers rotary embedding).

Pins (see tests/test_oracle.py): the rotation is checked against the
reference's own ``rope_cpu`` (src/q_rope.h:3-35, compiled into ``oracle/_ref``
when the reference tree is present) and against transformers' Qwen2
``apply_rotary_pos_emb``; attention against torch's
``scaled_dot_product_attention`` and a float64 brute force (``oracle/bruteforce.c``);
view/offset semantics against the dynamic-view identity (relative query
rotation == absolute-position causal attention); page-table and varlen indexing
against exact special cases (single visible key, uniform weights, id-coded V).
The key-side rotation is checked against transformers' Qwen2
``apply_rotary_pos_emb`` (bit for bit) and closed forms (identity, quarter
turn, float64 rotation); the append against pages built from a known
permutation; the view metadata against hand-computed locations and
transformers' ``Qwen2RotaryEmbedding``.
"""
from __future__ import annotations

import numpy as np
import torch

__all__ = [
    "rope_q",
    "rope_q_varlen",
    "sdpa_views",
    "paged_sdpa",
    "varlen_paged_sdpa",
    "contig_sdpa",
    "fused",
    "varlen_token_to_seq",
    "apply_rotary",
    "kv_append",
    "view_metadata",
]


def _rotate(x: torch.Tensor, c: torch.Tensor, s: torch.Tensor, rotary: int) -> torch.Tensor:
    """Rotate the first ``rotary`` dims of ``x`` (fp32) with half-width c/s.

    rope.cuh:24-51: for e < R/2, out = x[e]*c[e] - x[e+R/2]*s[e];
    for R/2 <= e < R, out = x[e]*c[e-R/2] + x[e-R/2]*s[e-R/2]; e >= R copies.
    Each product and the sum are separately rounded fp32 operations.
    """
    half = rotary // 2
    x1 = x[..., :half]
    x2 = x[..., half:rotary]
    first = x1 * c - x2 * s
    second = x2 * c + x1 * s
    rest = x[..., rotary:]
    rest = rest.expand(first.shape[:-1] + rest.shape[-1:])
    return torch.cat((first, second, rest), dim=-1)


def rope_q(queries: torch.Tensor, cosines: torch.Tensor, sines: torch.Tensor) -> torch.Tensor:
    """Query rotation per view: ``[W,Hq,S,E]`` -> ``[F,W,Hq,S,E]`` (rope.cuh:2-52).

    ``cosines``/``sines`` are fp32 ``[F,W,S,R]`` (full width, R = size(3),
    binding.cu:52); only entries ``[0, R/2)`` are read (rope.cuh:24-46).  Math is
    fp32, the result is rounded to ``queries.dtype`` (rope.cuh:43-50 store).
    """
    F, W, S, R = cosines.shape
    half = R // 2
    x = queries.to(torch.float32)[None]                      # [1,W,Hq,S,E]
    c = cosines[..., :half].to(torch.float32)[:, :, None]    # [F,W,1,S,R/2]
    s = sines[..., :half].to(torch.float32)[:, :, None]
    return _rotate(x, c, s, R).to(queries.dtype)


def rope_q_varlen(queries: torch.Tensor, cosines: torch.Tensor, sines: torch.Tensor) -> torch.Tensor:
    """Varlen query rotation: ``[T,H,E]`` -> ``[F,T,H,E]`` (rope.cuh:67-100).

    ``cosines``/``sines`` are fp32 half width ``[F,T,R/2]`` and R = 2*size(2)
    (binding.cu:217); entry ``e mod R/2`` is used (rope.cuh:84-87).
    """
    F, T, half = cosines.shape
    x = queries.to(torch.float32)[None]                      # [1,T,H,E]
    c = cosines.to(torch.float32)[:, :, None]                # [F,T,1,R/2]
    s = sines.to(torch.float32)[:, :, None]
    return _rotate(x, c, s, 2 * half).to(queries.dtype)


def _gqa_rows(q_f: torch.Tensor, Hkv: int) -> torch.Tensor:
    """``[Hq, S, E]`` -> ``[Hkv, G*S, E]``: head h uses kv head h // G."""
    Hq, S, E = q_f.shape
    return q_f.reshape(Hkv, (Hq // Hkv) * S, E)


def sdpa_views(rq: torch.Tensor, loc: torch.Tensor, keys: list, vals: list,
               frag_len: list, scale: float) -> torch.Tensor:
    """Attention of one sequence's rotated queries over F views.

    rq: ``[F, Hq, S, E]`` (already rotated, any float dtype); loc: ``[F, S]`` int;
    keys/vals[f]: ``[Hkv, L_f, E|Ev]``; frag_len[f]: python int.  Key ``l`` of view
    ``f`` is visible to query ``s`` iff ``l <= loc[f, s]`` and ``l < frag_len[f]``
    (paged_kernel_v21.cuh:83-85, attention.py:48-52).  Returns fp32 ``[Hq,S,Ev]``.
    """
    F, Hq, S, E = rq.shape
    if F == 0:
        raise ValueError("at least one view is required")
    Hkv = keys[0].shape[0]
    G = Hq // Hkv
    Ev = vals[0].shape[-1]
    scores, values = [], []
    for f in range(F):
        lim = min(keys[f].shape[1], max(0, int(frag_len[f])))
        k = keys[f][:, :lim].to(torch.float32)                   # [Hkv, L, E]
        v = vals[f][:, :lim].to(torch.float32)
        q = _gqa_rows(rq[f].to(torch.float32), Hkv)              # [Hkv, G*S, E]
        kp = torch.arange(lim)[None, :]                          # attention.py:48,50
        qp = loc[f].to(torch.int64)[:, None]                     # attention.py:49,51
        mask = (kp > qp)[None].expand(G, S, lim).reshape(G * S, lim)  # attention.py:52
        att = q @ k.transpose(-1, -2)                            # attention.py:53
        att = att.masked_fill(mask[None], float("-inf"))         # attention.py:54
        scores.append(att)
        values.append(v)
    qk = torch.cat(scores, dim=-1)                               # attention.py:58
    v = torch.cat(values, dim=-2)                                # attention.py:59
    if qk.shape[-1] == 0:
        return torch.zeros(Hq, S, Ev)
    empty = torch.isinf(qk).all(dim=-1, keepdim=True)
    att = torch.softmax(scale * qk, dim=-1)                      # attention.py:60
    att = torch.where(empty, torch.zeros_like(att), att)        # paged:318-345 (zeros)
    out = att @ v                                                # attention.py:61
    return out.reshape(Hq, S, Ev)


def _gather_pages(cache: torch.Tensor, bt_row: np.ndarray, start: int, count: int) -> torch.Tensor:
    """Rows ``start .. start+count-1`` of one sequence's logical token stream.

    Logical position p lives in page ``bt_row[p // bs]``, row ``p % bs`` of a
    ``[num_blocks, bs, Hkv, E]`` cache (binding.cu:194-195, paged:101-115).
    Returns ``[Hkv, count, E]``.
    """
    bs = cache.shape[1]
    pos = np.arange(start, start + count, dtype=np.int64)
    lp = pos // bs
    if count and lp.max() >= bt_row.shape[0]:
        raise ValueError("logical page beyond block_tables row")
    pages = torch.from_numpy(bt_row[lp].astype(np.int64))
    rows = torch.from_numpy(pos % bs)
    if count and (pages.min() < 0 or pages.max() >= cache.shape[0]):
        raise ValueError("block_tables entry outside the page pool")
    return cache[pages, rows].permute(1, 0, 2)


def paged_sdpa(scale: float, locations: torch.Tensor, queries: torch.Tensor,
               cosines: torch.Tensor, sines: torch.Tensor, fragment_lengths: torch.Tensor,
               k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor) -> torch.Tensor:
    """``dvattn_paged_sdpa`` (binding.cu:151-203, paged_kernel_v21.cuh:17-374).

    Shapes: locations ``[F,W,S]`` i32, queries ``[W,Hq,S,E]``, cos/sin
    ``[F,W,S,R]`` f32, fragment_lengths ``[F]`` i32, k/v_cache
    ``[P,bs,Hkv,E|Ev]``, block_tables ``[W,maxB]`` i32.  View f of sequence w
    occupies logical positions ``off_f + l`` with ``off_f = sum_{g<f} L_g``
    (paged:80,102,198).  Returns fp32 ``[W,Hq,S,Ev]``.
    """
    F, W, S = locations.shape
    Hq = queries.shape[1]
    Ev = v_cache.shape[-1]
    rq = rope_q(queries, cosines, sines)                     # [F,W,Hq,S,E] rounded to T
    fl = [int(x) for x in fragment_lengths.tolist()]
    loc = locations.to(torch.int64)
    bt = block_tables.numpy()
    out = torch.zeros(W, Hq, S, Ev)
    for w in range(W):
        off = 0
        keys, vals, lens = [], [], []
        for f in range(F):
            vis = max(0, min(fl[f], int(loc[f, w].max()) + 1)) if S else 0
            keys.append(_gather_pages(k_cache, bt[w], off, vis))
            vals.append(_gather_pages(v_cache, bt[w], off, vis))
            lens.append(vis)
            off += fl[f]
        out[w] = sdpa_views(rq[:, w], loc[:, w], keys, vals, lens, scale)
    return out


def varlen_token_to_seq(cu_seqlens_q: np.ndarray, T: int) -> np.ndarray:
    """Sequence of each packed token (varlen_paged_kernel_v21.cuh:40-47):
    the first i with ``t < cu_seqlens_q[i+1]``; 0 when there is none."""
    W = cu_seqlens_q.shape[0] - 1
    out = np.zeros(T, dtype=np.int64)
    for t in range(T):
        for i in range(W):
            if t < cu_seqlens_q[i + 1]:
                out[t] = i
                break
    return out


def varlen_paged_sdpa(scale: float, locations: torch.Tensor, queries: torch.Tensor,
                      cosines: torch.Tensor, sines: torch.Tensor, fragment_lengths: torch.Tensor,
                      k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
                      cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor) -> torch.Tensor:
    """``dvattn_varlen_paged_sdpa`` (binding.cu:249-296, varlen kernel :17-371).

    locations ``[F,T]``, queries ``[T,Hq,E]``, half-width cos/sin ``[F,T,R/2]``.
    A view with ``locations[f,t] < 0`` is skipped (its length still advances the
    logical offset, varlen:76-80).  ``cu_seqlens_k`` is accepted and unused, as in
    the reference (binding.cu:279,290).  Returns fp32 ``[T,Hq,Ev]``.
    """
    F, T = locations.shape
    Hq = queries.shape[1]
    Ev = v_cache.shape[-1]
    rq = rope_q_varlen(queries, cosines, sines)              # [F,T,Hq,E]
    fl = [int(x) for x in fragment_lengths.tolist()]
    loc = locations.to(torch.int64)
    bt = block_tables.numpy()
    seq = varlen_token_to_seq(cu_seqlens_q.numpy().astype(np.int64), T)
    out = torch.zeros(T, Hq, Ev)
    for t in range(T):
        w = int(seq[t])
        off = 0
        keys, vals, lens = [], [], []
        for f in range(F):
            lf = int(loc[f, t])
            vis = 0 if lf < 0 else max(0, min(fl[f], lf + 1))
            keys.append(_gather_pages(k_cache, bt[w], off, vis))
            vals.append(_gather_pages(v_cache, bt[w], off, vis))
            lens.append(vis)
            off += fl[f]
        res = sdpa_views(rq[:, t, :, None, :], loc[:, t, None], keys, vals, lens, scale)
        out[t] = res[:, 0]
    return out


def contig_sdpa(scale: float, locations: torch.Tensor, rq: torch.Tensor,
                fragment_lengths: torch.Tensor, key_fragments: list, value_fragments: list) -> torch.Tensor:
    """``dvattn_sdpa`` on already-rotated queries (binding.cu:79-149).

    rq ``[F,W,Hq,S,E]``, locations ``[F,W,S]``, key/value fragments
    ``[B,Hkv,L_f,E]`` or ``[Hkv,L_f,E]``; a batch of 1 (or no batch dim) is
    shared by all sequences, as the PyTorch reference broadcasts it
    (attention.py:45,53).  Returns fp32 ``[W,Hq,S,Ev]``.
    """
    F, W, Hq, S, E = rq.shape
    fl = [int(x) for x in fragment_lengths.tolist()]
    Ev = value_fragments[0].shape[-1]
    out = torch.zeros(W, Hq, S, Ev)
    loc = locations.to(torch.int64)
    for w in range(W):
        keys, vals = [], []
        for f in range(F):
            k, v = key_fragments[f], value_fragments[f]
            if k.dim() == 4:
                k = k[w] if k.shape[0] > 1 else k[0]
                v = v[w] if v.shape[0] > 1 else v[0]
            keys.append(k)
            vals.append(v)
        out[w] = sdpa_views(rq[:, w], loc[:, w], keys, vals, fl, scale)
    return out


def fused(scale: float, locations: torch.Tensor, queries: torch.Tensor, fragment_lengths: torch.Tensor,
          key_fragments: list, value_fragments: list, cosines: torch.Tensor, sines: torch.Tensor):
    """``dvattn_fused`` (binding.cu:356-372): returns (fp32 out, rotated queries)."""
    rq = rope_q(queries, cosines, sines)
    return contig_sdpa(scale, locations, rq, fragment_lengths, key_fragments, value_fragments), rq


def apply_rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Partial RoPE of the last dim as attention.py:82-88 computes it: dims
    ``< R = cos.shape[-1]`` become ``x*cos + rotate_half(x)*sin`` (rotate_half =
    ``cat(-x2, x1)``, attention.py:75-79), the rest pass through; every operation
    in PyTorch's dtype promotion of (x, cos), the result cast back to x's dtype.
    cos/sin broadcast against ``x[..., :R]``."""
    R = cos.shape[-1]
    x_rot, x_pass = x[..., :R], x[..., R:]
    h = R // 2
    rh = torch.cat((-x_rot[..., h:], x_rot[..., :h]), dim=-1)
    emb = (x_rot * cos) + (rh * sin)
    return torch.cat((emb, x_pass.to(emb.dtype)), dim=-1).to(x.dtype)


def kv_append(k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor, positions: torch.Tensor,
              keys: torch.Tensor, values: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """Write rotated keys and values of new tokens into a paged cache; returns
    updated copies (CPU).

    keys/values ``[W,Hkv,S,E]``; positions ``[W,S]``: logical position ``p`` of
    token (w, s) in sequence w's token stream, stored at page
    ``block_tables[w, p // bs]``, row ``p % bs`` of ``[P,bs,Hkv,E]`` caches (the
    layout of the paged operators, binding.cu:194-196; paged_kernel_v21.cuh:102-120);
    ``p < 0`` (a masked token, attention.py:141-147 copies only unmasked ones), a
    logical page past the table row or a page outside ``[0, P)`` is not written.
    cos/sin ``[W|1, S|1, R]``: the rotation of attention.py:304 at that token.
    """
    k = k_cache.clone()
    v = v_cache.clone()
    W, Hkv, S, E = keys.shape
    P, bs = k.shape[0], k.shape[1]
    maxB = block_tables.shape[1]
    R = cos.shape[-1]
    cb = cos.expand(W, S, R)
    sb = sin.expand(W, S, R)
    for w in range(W):
        for s in range(S):
            p = int(positions[w, s])
            if p < 0:
                continue
            lp, row = divmod(p, bs)
            if lp >= maxB:
                continue
            page = int(block_tables[w, lp])
            if page < 0 or page >= P:
                continue
            k[page, row] = apply_rotary(keys[w, :, s, :], cb[w, s], sb[w, s])
            v[page, row] = values[w, :, s, :]
    return k, v


def view_metadata(fragment_lengths, order, S: int, inv_freq: torch.Tensor, attention_scaling: float = 1.0,
                  round_to=None):
    """Per-view locations and cos/sin of a decode step (attention.py:158-186).

    For each sequence w the reference walks its segment list backwards,
    accumulating lengths (which already include the S new tokens), and gives the
    segment at which it stands the locations ``arange(pos - S, pos)``
    (attention.py:167-176).  cos/sin are transformers' default rotary embedding at
    those positions: ``angle = float(position) * inv_freq`` (a K=1 fp32 matmul),
    ``emb = cat(angle, angle)``, ``cos(emb) * scaling`` (and sin), returned in the
    model dtype and converted to float32 (attention.py:181-184; ``round_to`` is
    that model dtype).  A view absent from a sequence's order has no location in
    the reference (it fails); here it gets -1 and the identity rotation.  Order
    entries outside ``[0, F)`` are padding and skipped.
    """
    fl = [int(x) for x in fragment_lengths]
    F = len(fl)
    W = len(order)
    loc = torch.full((F, W, S), -1, dtype=torch.int32)
    present = torch.zeros((F, W), dtype=torch.bool)
    for w in range(W):
        pos = 0
        for g in reversed([int(x) for x in order[w]]):
            if not 0 <= g < F:
                continue  # padding of a sequence that lists fewer views
            pos += fl[g]
            loc[g, w] = torch.arange(pos - S, pos, dtype=torch.int32)
            present[g, w] = True
    R = 2 * inv_freq.numel()
    ang = loc.reshape(F * W, S).float()[:, :, None] * inv_freq.float()[None, None, :]
    emb = torch.cat((ang, ang), dim=-1)
    cos = emb.cos() * attention_scaling
    sin = emb.sin() * attention_scaling
    if round_to is not None:
        cos = cos.to(round_to).float()
        sin = sin.to(round_to).float()
    cos = cos.reshape(F, W, S, R)
    sin = sin.reshape(F, W, S, R)
    miss = ~present
    cos[miss] = 1.0
    sin[miss] = 0.0
    return loc, cos, sin
