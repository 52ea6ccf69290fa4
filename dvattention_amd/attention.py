"""Python operator API, mirroring python/dvattn/attention.py:17-88 of the reference.

Every ``dvattn_*`` wrapper calls ``torch.ops.libdvatt.<op>`` (registered by
``_libdvatt.so`` over the HIP kernels); there is no eager fallback.  The
function names, argument order and defaults are the reference's; the paged /
varlen operators, which the reference exposes only through ``torch.ops``, get
thin wrappers as well.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch


def dvattn_fused(queries: torch.Tensor, locations: torch.Tensor, keys: list, values: list,
                 scale: float, fragment_lengths, cosines: torch.Tensor, sines: torch.Tensor, *,
                 rotated_queries, out):
    """Rope + attention over contiguous views (attention.py:17-21).

    queries ``[W,Hq,S,E]``, cosines/sines ``[F,W,S,R]`` fp32; writes the rotated
    queries ``[F,W,Hq,S,E]`` into ``rotated_queries`` and the result into ``out``.
    """
    torch.ops.libdvatt.dvattn_fused(out, rotated_queries, scale, locations, queries.contiguous(),
                                    fragment_lengths, keys, values, cosines, sines)
    return out


def dvattn_sdpa(queries: torch.Tensor, locations: torch.Tensor, keys: list, values: list,
                scale: float, fragment_lengths=None, out=None) -> torch.Tensor:
    """Attention of already-rotated queries ``[F,W,Hq,S,E]`` over contiguous views
    (attention.py:24-33)."""
    if out is None:
        out = torch.empty((queries.size(1), queries.size(2), queries.size(3), values[0].size(-1)),
                          dtype=queries.dtype, device=queries.device)
    if fragment_lengths is None:
        fragment_lengths = torch.tensor([k.size(-2) for k in keys], dtype=torch.int32, device=queries.device)
    keys = [k.contiguous() for k in keys]
    values = [v.contiguous() for v in values]
    torch.ops.libdvatt.dvattn_sdpa(out, scale, locations, queries.contiguous(), fragment_lengths, keys, values)
    return out


def dvattn_rope(queries: torch.Tensor, cosines: torch.Tensor, sines: torch.Tensor, out=None):
    """Rotate ``[W,Hq,S,E]`` queries once per view -> ``[F,W,Hq,S,E]`` (attention.py:68-72)."""
    if out is None:
        out = torch.empty((cosines.size(0), queries.size(0), queries.size(1), queries.size(2), queries.size(3)),
                          dtype=queries.dtype, device=queries.device)
    torch.ops.libdvatt.dvattn_rope(out, queries, cosines, sines)
    return out


def dvattn_varlen_rope(queries: torch.Tensor, cosines: torch.Tensor, sines: torch.Tensor, out=None):
    """Rotate packed ``[T,H,E]`` queries with half-width cos/sin ``[F,T,R/2]`` -> ``[F,T,H,E]``
    (op ``dvattn_varlen_rope``, binding.cu:205-247)."""
    if out is None:
        out = torch.empty((cosines.size(0),) + tuple(queries.shape), dtype=queries.dtype, device=queries.device)
    torch.ops.libdvatt.dvattn_varlen_rope(out, queries, cosines, sines)
    return out


def dvattn_paged_sdpa(queries: torch.Tensor, locations: torch.Tensor, cosines: torch.Tensor, sines: torch.Tensor,
                      fragment_lengths: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                      block_tables: torch.Tensor, scale: float, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Paged multi-view decode attention with fused query rotation (op
    ``dvattn_paged_sdpa``, binding.cu:151-203).  queries ``[W,Hq,S,E]`` ->
    out ``[W,Hq,S,Ev]``."""
    if out is None:
        out = torch.empty(tuple(queries.shape[:3]) + (v_cache.size(-1),), dtype=queries.dtype,
                          device=queries.device)
    torch.ops.libdvatt.dvattn_paged_sdpa(out, scale, locations, queries, cosines, sines, fragment_lengths,
                                         k_cache, v_cache, block_tables)
    return out


def dvattn_varlen_paged_sdpa(queries: torch.Tensor, locations: torch.Tensor, cosines: torch.Tensor,
                             sines: torch.Tensor, fragment_lengths: torch.Tensor, k_cache: torch.Tensor,
                             v_cache: torch.Tensor, block_tables: torch.Tensor, cu_seqlens_q: torch.Tensor,
                             cu_seqlens_k: torch.Tensor, scale: float,
                             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Varlen (packed tokens) paged multi-view attention (op
    ``dvattn_varlen_paged_sdpa``, binding.cu:249-296).  queries ``[T,Hq,E]`` ->
    out ``[T,Hq,Ev]``."""
    if out is None:
        out = torch.empty(tuple(queries.shape[:2]) + (v_cache.size(-1),), dtype=queries.dtype,
                          device=queries.device)
    torch.ops.libdvatt.dvattn_varlen_paged_sdpa(out, scale, locations, queries, cosines, sines, fragment_lengths,
                                                k_cache, v_cache, block_tables, cu_seqlens_q, cu_seqlens_k)
    return out


def dvattn_paged_kv_append(keys: torch.Tensor, values: torch.Tensor, positions: torch.Tensor,
                           cosines: torch.Tensor, sines: torch.Tensor, k_cache: torch.Tensor,
                           v_cache: torch.Tensor, block_tables: torch.Tensor):
    """The K side of a decode step on a paged cache: rotate the new keys with the
    model's (cos, sin) and write keys and values into their pages (the reference
    rotates ``key_states`` at attention.py:304 and appends them to the sequence's
    own cache at attention.py:141-152).

    keys/values ``[W,Hkv,S,E]`` (strided views such as k_proj's output
    transposed are fine), positions ``[W,S]`` int32 logical positions in each
    sequence's token stream (negative: masked, not written), cosines/sines
    ``[W,S,R]`` / ``[S,R]`` / ``[R]`` in float32 or the model dtype, read in full
    (``apply_rotary_pos_emb``, attention.py:82-88, evaluated with PyTorch's
    rounding).  Caches ``[num_blocks, block_size, Hkv, E]`` are updated in place.
    """
    W, _, S, _ = keys.shape
    R = cosines.size(-1)
    cos = cosines.reshape((1,) * (3 - cosines.dim()) + tuple(cosines.shape)) if cosines.dim() < 3 else cosines
    sin = sines.reshape((1,) * (3 - sines.dim()) + tuple(sines.shape)) if sines.dim() < 3 else sines
    cos = cos.expand(W, S, R)
    sin = sin.expand(W, S, R)
    torch.ops.libdvatt.dvattn_paged_kv_append(k_cache, v_cache, block_tables, positions, keys, values, cos, sin)
    return k_cache, v_cache


def merge_caches_paged(source_keys: torch.Tensor, source_values: torch.Tensor, offset_cos: torch.Tensor,
                       offset_sin: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       block_tables: torch.Tensor, positions: torch.Tensor):
    """``merge_caches`` (attention.py:245-251) into a paged target: the source
    keys ``[1,Hkv,L,E]`` are re-rotated by the target's length (one cos/sin row,
    ``offset_cos``/``offset_sin`` ``[R]``: the rotary embedding at that length)
    and written with the source values at ``positions`` ``[1,L]`` (the target's
    next L logical positions)."""
    return dvattn_paged_kv_append(source_keys, source_values, positions, offset_cos.reshape(-1),
                                  offset_sin.reshape(-1), k_cache, v_cache, block_tables)


def dvattn_view_metadata(fragment_lengths: torch.Tensor, order: torch.Tensor, num_new_tokens: int,
                         inv_freq: torch.Tensor, attention_scaling: float = 1.0,
                         round_to: Optional[torch.dtype] = None):
    """Per-view locations and query cos/sin for a decode step, on the device
    (attention.py:158-186).

    fragment_lengths ``[F]`` int32: segment lengths including the new tokens;
    order ``[W,F]`` int32: sequence w's segments in its own order (view indices,
    its own segment last); inv_freq ``[R/2]`` float32: the model's rotary inverse
    frequencies (``model.rotary_emb.inv_freq``).  Returns ``(locations [F,W,S]
    int32, cosines [F,W,S,R], sines [F,W,S,R])`` float32, ready for
    ``dvattn_paged_sdpa`` / ``dvattn_fused``.  ``round_to`` rounds cos/sin through
    the model dtype, as the reference's rotary call does.
    """
    F = fragment_lengths.numel()
    W = order.size(0)
    R = 2 * inv_freq.numel()
    dev = fragment_lengths.device
    loc = torch.empty((F, W, num_new_tokens), dtype=torch.int32, device=dev)
    cos = torch.empty((F, W, num_new_tokens, R), dtype=torch.float32, device=dev)
    sin = torch.empty_like(cos)
    torch.ops.libdvatt.dvattn_view_metadata(loc, cos, sin, fragment_lengths, order, inv_freq,
                                            float(attention_scaling), round_to)
    return loc, cos, sin


def dvattn_sdpa_pt(queries: torch.Tensor, locations: torch.Tensor, keys: list, values: list,
                   scale: float, return_intermediate_results: bool = False):
    """Pure-PyTorch attention over already-rotated queries and contiguous views,
    for testing and debugging; the reference's helper of the same name and
    contract (attention.py:36-65).  No operator of this package calls it.

    queries ``[F,W,Hq,S,E]`` (rotated per view), locations ``[F,W,S]``,
    keys[f] / values[f] ``[B,Hkv,L_f,E|Ev]`` or ``[Hkv,L_f,E|Ev]`` (B = 1
    broadcasts over the W sequences).  Key ``l`` of view ``f`` is visible to
    query ``(w, s)`` iff ``l <= locations[f, w, s]``; one fp32 softmax of
    ``scale * q.k`` runs over the keys of all views.  Returns the output in
    ``queries.dtype``; with ``return_intermediate_results``, the fp32 output
    ``[W,Hq,S,Ev]``, the masked unscaled scores and the softmax weights
    ``[W,Hq,S,sum_f L_f]``.  A query that sees no key gets NaN here (the HIP
    operators write zeros, as the reference's kernels do).

    GQA without replicating K/V: the 16 query heads of a KV head are viewed as
    16*S query rows of that head.  The views' scores fill one preallocated
    key axis, and visibility is one comparison of every key's in-view position
    against the query's location in that key's view.
    """
    F, W, Hq, S, E = queries.shape
    Hkv = keys[0].shape[-3]
    G = Hq // Hkv
    Ev = values[0].shape[-1]
    dev = queries.device
    lens = [int(k.shape[-2]) for k in keys]
    total = sum(lens)
    view_of = torch.repeat_interleave(torch.arange(F, device=dev), torch.tensor(lens, device=dev))
    pos_in_view = torch.cat([torch.arange(n, device=dev) for n in lens]) if total else \
        torch.zeros(0, dtype=torch.long, device=dev)

    scores = torch.empty((W, Hkv, G * S, total), dtype=torch.float32, device=dev)
    v_all = torch.empty((W, Hkv, total, Ev), dtype=torch.float32, device=dev)
    start = 0
    for f, n in enumerate(lens):
        q_rows = queries[f].to(torch.float32).reshape(W, Hkv, G * S, E)
        scores[..., start:start + n] = q_rows @ keys[f].to(torch.float32).transpose(-1, -2)
        v_all[:, :, start:start + n] = values[f].to(torch.float32)
        start += n
    scores = scores.view(W, Hq, S, total)
    hidden = pos_in_view > locations.to(device=dev, dtype=torch.long)[view_of].permute(1, 2, 0)  # [W,S,total]
    scores.masked_fill_(hidden[:, None], float("-inf"))
    weights = torch.softmax(scores * scale, dim=-1)
    result = (weights.view(W, Hkv, G * S, total) @ v_all).view(W, Hq, S, Ev)
    if return_intermediate_results:
        return result, scores, weights
    return result.to(queries.dtype)


def rotate_half(x):
    """Rotates half the hidden dims of the input (attention.py:75-79)."""
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def apply_rotary_pos_emb(x, cos, sin, unsqueeze_dim=1):
    """Partial RoPE on the first ``cos.shape[-1]`` dims (attention.py:82-88)."""
    cos = cos.unsqueeze(unsqueeze_dim)
    sin = sin.unsqueeze(unsqueeze_dim)
    rotary_dim = cos.shape[-1]
    x_rot, x_pass = x[..., :rotary_dim], x[..., rotary_dim:]
    x_rot_emb = (x_rot * cos) + (rotate_half(x_rot) * sin)
    return torch.cat((x_rot_emb, x_pass), dim=-1).to(x.dtype)


__all__ = [
    "dvattn_fused", "dvattn_sdpa", "dvattn_rope", "dvattn_varlen_rope", "dvattn_paged_sdpa",
    "dvattn_varlen_paged_sdpa", "dvattn_sdpa_pt", "rotate_half", "apply_rotary_pos_emb",
    "dvattn_paged_kv_append", "merge_caches_paged", "dvattn_view_metadata",
]
