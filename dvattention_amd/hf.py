"""Transformers integration of the DVAttn decode path: ``DVAttnCache``,
``AttentionModule`` and ``model_surgery`` of the reference
(python/dvattn/attention.py:100-343), for transformers 5, over this package's
HIP operators.

What changes against the reference, and why:

* Segments (the reference's per-worker HF caches, attention.py:109-119) live in
  one preallocated pool per layer, ``[num_segments, Hkv, capacity, E]`` for K and
  for V, instead of tensors that ``torch.cat`` regrows every step.  A segment is
  a slice of the pool; the attention op reads it in place (its
  ``fragment_lengths`` bound the visible keys, so the unused capacity is never
  read).
* The K side of a step is one ``dvattn_paged_kv_append`` launch for all workers:
  key rotation (attention.py:304) fused with the write into each worker's
  segment (attention.py:141-152), the pool seen as ``[segments, capacity, Hkv,
  E]`` pages of ``capacity`` tokens.
* Locations and query cos/sin (attention.py:158-186) come from one
  ``dvattn_view_metadata`` launch per step; the host only uploads the segment
  lengths and orders.
* The attention is ``dvattn_fused`` as in the reference's non-eager path
  (attention.py:319-331).
* ``DVAttnCache`` and ``merge_caches`` also take transformers ``Cache`` objects,
  as the reference's do (attention.py:109-118, 245-251).  Their contents are
  copied once into a pool the cache creates (it grows when a segment fills),
  and each caller cache is rebound to views of its segment.  Its layers then
  show every appended token, and its ``get_seq_length`` stays correct without
  a second copy.  A later ``DVAttnCache`` or ``merge_caches`` call on the same
  cache objects finds their segments again.

The three device operations are reached through an ``ops`` object (default:
this package's HIP operators), so the module code can also be driven by a
checker implementation in tests.
"""
from __future__ import annotations

import weakref
from dataclasses import dataclass
from typing import Any, Dict, List, Optional

import torch
from torch import nn

from . import attention as _A


class HipOps:
    """The device operations of a decode step (this package's HIP operators)."""

    @staticmethod
    def kv_append(keys, values, positions, cos, sin, k_pages, v_pages, block_tables):
        _A.dvattn_paged_kv_append(keys, values, positions, cos, sin, k_pages, v_pages, block_tables)

    @staticmethod
    def view_metadata(fragment_lengths, order, S, inv_freq, attention_scaling, round_to):
        return _A.dvattn_view_metadata(fragment_lengths, order, S, inv_freq, attention_scaling, round_to)

    @staticmethod
    def fused(queries, locations, keys, values, scale, fragment_lengths, cosines, sines, rotated_queries, out):
        return _A.dvattn_fused(queries, locations, keys, values, scale, fragment_lengths, cosines, sines,
                               rotated_queries=rotated_queries, out=out)


@dataclass
class CacheStructure:
    """What the attention of one layer needs (attention.py:100-106)."""
    keys: list       # per view: [1, Hkv, capacity, E]
    values: list
    frags: torch.Tensor  # fragment_lengths [F] int32
    cos: torch.Tensor    # [F, W, S, R] float32
    sin: torch.Tensor
    loc: torch.Tensor    # [F, W, S] int32


class SegmentPool:
    """Preallocated K/V storage for ``num_segments`` segments of every layer."""

    def __init__(self, config, num_segments: int, capacity: int, dtype: torch.dtype, device):
        self.num_layers = config.num_hidden_layers
        self.Hkv = config.num_key_value_heads
        self.E = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads
        self.capacity = capacity
        shape = (num_segments, self.Hkv, capacity, self.E)
        self.k = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(self.num_layers)]
        self.v = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(self.num_layers)]
        self.segments = [Segment(self, i) for i in range(num_segments)]
        self.growable = False   # pools made for caller caches grow when a segment fills
        self.mirrors = []       # (weak reference to a caller cache, its segment)

    def __getitem__(self, i: int) -> "Segment":
        return self.segments[i]

    def resize(self, num_segments: Optional[int] = None, capacity: Optional[int] = None) -> None:
        """Reallocate with more segments and/or a larger capacity, keeping every
        segment's tokens; the caller caches bound to this pool are rebound."""
        n0 = len(self.segments)
        n = max(n0, num_segments or n0)
        cap = max(self.capacity, capacity or self.capacity)
        if n == n0 and cap == self.capacity:
            return
        for layer in range(self.num_layers):
            for name in ("k", "v"):
                old = getattr(self, name)[layer]
                new = torch.zeros((n, self.Hkv, cap, self.E), dtype=old.dtype, device=old.device)
                new[:n0, :, :self.capacity].copy_(old)
                getattr(self, name)[layer] = new
        self.capacity = cap
        self.segments += [Segment(self, i) for i in range(n0, n)]
        for layer in range(self.num_layers):
            self.sync_mirrors(layer)

    def sync_mirrors(self, layer: int, only=None) -> None:
        """Rebind the caller caches of this pool (those of segments ``only``) to
        views of their segments' filled part of ``layer``."""
        live = []
        for ref, seg in self.mirrors:
            cache = ref()
            if cache is None:
                continue
            live.append((ref, seg))
            if only is None or any(seg is o for o in only):
                L = seg.get_seq_length(layer)
                _set_cache_layer(cache, layer, self.k[layer][seg.index:seg.index + 1, :, :L],
                                 self.v[layer][seg.index:seg.index + 1, :, :L])
        self.mirrors = live


class Segment:
    """One segment (a contiguous run of tokens shared by the workers that see
    it); stands in for the reference's per-segment HF cache."""

    def __init__(self, pool: SegmentPool, index: int):
        self.pool = pool
        self.index = index
        self.lengths = [0] * pool.num_layers

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        return self.lengths[layer_idx or 0]

    def keys(self, layer_idx: int) -> torch.Tensor:
        return self.pool.k[layer_idx][self.index:self.index + 1]

    def values(self, layer_idx: int) -> torch.Tensor:
        return self.pool.v[layer_idx][self.index:self.index + 1]


def _cache_layer(cache, layer: int):
    """(keys, values) ``[1, Hkv, L, E]`` of one layer of a transformers cache
    (``layers[i].keys`` in transformers 5, ``key_cache[i]`` before), or
    (None, None) for a layer the cache has not filled yet."""
    if hasattr(cache, "layers"):
        if layer >= len(cache.layers) or not getattr(cache.layers[layer], "is_initialized", True):
            return None, None
        return cache.layers[layer].keys, cache.layers[layer].values
    if layer >= len(cache.key_cache):
        return None, None
    return cache.key_cache[layer], cache.value_cache[layer]


def _set_cache_layer(cache, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
    """Make ``k``/``v`` the contents of one layer of a transformers cache."""
    if hasattr(cache, "layers"):
        while len(cache.layers) <= layer:
            make = getattr(cache, "layer_class_to_replicate", None)
            if make is None:
                from transformers.cache_utils import DynamicLayer as make
            cache.layers.append(make())
        lay = cache.layers[layer]
        lay.keys, lay.values = k, v
        lay.dtype, lay.device = k.dtype, k.device
        lay.is_initialized = True
    else:
        while len(cache.key_cache) <= layer:
            cache.key_cache.append(k[:, :, :0])
            cache.value_cache.append(v[:, :, :0])
        cache.key_cache[layer], cache.value_cache[layer] = k, v


# caller cache -> its segment, for caches a DVAttnCache has taken into a pool
_POOLED = weakref.WeakKeyDictionary()


def _segment_of(x) -> Optional["Segment"]:
    if isinstance(x, Segment):
        return x
    try:
        return _POOLED.get(x)
    except TypeError:
        return None


def _rotary(model):
    """The rotary embedding of ``model``: a causal-LM wrapper (``model.model``)
    or the decoder itself, as the reference's merge_caches is given."""
    rot = getattr(model, "rotary_emb", None)
    return rot if rot is not None else model.model.rotary_emb


def _config(model):
    inner = model.model if hasattr(model, "model") and hasattr(model.model, "layers") else model
    return inner.config


def pool_caches(caches, model, capacity: Optional[int] = None) -> List["Segment"]:
    """The segments of transformers caches ``caches``.  Caches already in a
    pool keep their segments; the others are copied into that pool (new
    segments), or into a new one.  Afterwards every cache's layers are views of
    its segment.  The pool holds ``capacity`` tokens per segment (default:
    the longest cache plus 1024, rounded up to a power of two) and doubles when
    an append or merge would overflow it."""
    pools = {id(_segment_of(c).pool): _segment_of(c).pool for c in caches if _segment_of(c) is not None}
    if len(pools) > 1:
        raise ValueError("DVAttnCache: the caches belong to different pools (different DVAttnCache structures "
                         "that were never merged)")
    fresh = []
    for c in caches:
        if _segment_of(c) is None and not any(c is f for f in fresh):
            fresh.append(c)
    cfg = _config(model)
    n_layers = cfg.num_hidden_layers
    lengths = [max((_cache_layer(c, l)[0].shape[2] for l in range(n_layers) if _cache_layer(c, l)[0] is not None),
                   default=0) for c in fresh]
    if pools:
        pool = next(iter(pools.values()))
        first = len(pool.segments)
        pool.resize(num_segments=first + len(fresh), capacity=max(lengths, default=0))
    else:
        ref = next((_cache_layer(c, 0)[0] for c in fresh if _cache_layer(c, 0)[0] is not None), None)
        if ref is None:
            ref = next(model.parameters())
        need = max(lengths, default=0) + 1024
        cap = capacity if capacity is not None else 1 << (need - 1).bit_length()
        pool = SegmentPool(cfg, len(fresh), max(cap, max(lengths, default=0)), ref.dtype, ref.device)
        pool.growable = True
        first = 0
    segs = segments_from_caches(fresh, pool, first)
    for c, seg in zip(fresh, segs):
        _POOLED[c] = seg
        pool.mirrors.append((weakref.ref(c), seg))
    for layer in range(pool.num_layers):
        pool.sync_mirrors(layer, only=segs)
    return [_segment_of(c) for c in caches]


def segments_from_caches(caches, pool: SegmentPool, first: int = 0) -> List[Segment]:
    """Copy caller-owned transformers caches into pool segments ``first``,
    ``first + 1``, ...: the reference's ``DVAttnCache`` takes such caches, one
    per segment (attention.py:109-119); here each becomes a segment of ``pool``
    holding the same (already rotated) keys and values, in the cache's own
    position numbering (the segment's token 0 at position 0).  Returns the
    segments, for a ``DVAttnCache`` structure."""
    out = []
    for j, cache in enumerate(caches):
        seg = pool[first + j]
        for layer in range(pool.num_layers):
            k, v = _cache_layer(cache, layer)
            if k is None or k.numel() == 0:
                seg.lengths[layer] = 0
                continue
            if k.dim() != 4 or k.shape[0] != 1:
                raise ValueError(f"cache {j} layer {layer}: expected keys [1, Hkv, L, E], got {tuple(k.shape)}")
            L = k.shape[2]
            if L > pool.capacity:
                raise RuntimeError(f"cache {j} holds {L} tokens, more than the pool's {pool.capacity}")
            pool.k[layer][seg.index, :, :L].copy_(k[0])
            pool.v[layer][seg.index, :, :L].copy_(v[0])
            seg.lengths[layer] = L
        out.append(seg)
    return out


class DVAttnCache:
    """Multi-worker dynamic-view cache (attention.py:109-239).

    ``cache_structure[w]`` lists the segments worker w attends to, in its own
    order (its own segment, where its new tokens go, last by default:
    ``write_to``).  The entries are segments of one ``SegmentPool``, or -- the
    reference's signature -- transformers ``Cache`` objects (``DynamicCache``),
    which are taken into a pool (``pool_caches``) and kept showing their
    segments' tokens.  Unlike the reference, a worker may leave out segments
    other workers list; it does not see them.
    """

    def __init__(self, cache_structure: List[List[Any]], model, write_to: Optional[List[Any]] = None,
                 ops=HipOps, capacity: Optional[int] = None):
        self.model = model.model
        if not all(isinstance(x, Segment) for cl in cache_structure for x in cl) or \
                (write_to and not all(isinstance(x, Segment) for x in write_to)):
            flat = [x for cl in cache_structure for x in cl] + list(write_to or [])
            segs = pool_caches(flat, model, capacity)
            it = iter(segs)
            cache_structure = [[next(it) for _ in cl] for cl in cache_structure]
            write_to = [next(it) for _ in write_to] if write_to else None
        self.cache_structure = cache_structure
        self.write_to = write_to if write_to else [cl[-1] for cl in cache_structure]
        self.pool = cache_structure[0][0].pool
        self.ops = ops
        self.cosines = None
        self.sines = None
        self.locations = None
        self.segments: List[Segment] = []
        self.frags = None
        self.queries_buffer = None
        self.att_buffer = None
        self._positions = None
        self._wt_table = None

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        return self.cache_structure[0][-1].get_seq_length(layer_idx)

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: Optional[Dict[str, Any]] = None) -> CacheStructure:
        """Rotate and append the new keys/values of every worker into its
        ``write_to`` segment, then (layer 0) rebuild the view metadata.

        key_states: ``[W, Hkv, S, E]`` *before* rotation (the reference rotates
        at attention.py:304 and appends at :141-152; here both are one launch);
        cache_kwargs: ``cos``/``sin`` (the model's position embeddings ``[W, S,
        R]``) and an optional left-padding ``mask`` ``[W, S]``.
        """
        W, _, S, _ = key_states.shape
        assert W == len(self.cache_structure)
        dev = key_states.device
        mask = cache_kwargs.get("mask") if cache_kwargs else None
        if layer_idx == 0:
            # positions of the new tokens in each worker's segment (left padding -> -1),
            # shared by all layers of this step
            n_new = mask.sum(dim=1).tolist() if mask is not None else [S] * W
            pos = torch.full((W, S), -1, dtype=torch.int32)
            # workers that write to the same segment append one after another,
            # in worker order (the reference updates their caches in turn,
            # attention.py:141-152)
            next_pos = {}
            for w in range(W):
                n = int(n_new[w])
                seg = self.write_to[w]
                base = next_pos.get(id(seg), seg.get_seq_length(0))
                if base + n > self.pool.capacity:
                    if not self.pool.growable:
                        raise RuntimeError(f"segment {seg.index} is full ({base} + {n} > "
                                           f"{self.pool.capacity} tokens)")
                    self.pool.resize(capacity=1 << (base + n - 1).bit_length())
                pos[w, S - n:] = torch.arange(base, base + n, dtype=torch.int32)
                next_pos[id(seg)] = base + n
            self._n_new = [int(n) for n in n_new]
            self._positions = pos.to(dev, non_blocking=True)
            self._wt_table = torch.tensor([[seg.index] for seg in self.write_to], dtype=torch.int32).to(dev)
        cos, sin = cache_kwargs["cos"], cache_kwargs["sin"]
        pages_k = self.pool.k[layer_idx].permute(0, 2, 1, 3)  # [segments, capacity, Hkv, E]
        pages_v = self.pool.v[layer_idx].permute(0, 2, 1, 3)
        self.ops.kv_append(key_states, value_states, self._positions, cos, sin, pages_k, pages_v, self._wt_table)
        for w in range(W):
            self.write_to[w].lengths[layer_idx] += self._n_new[w]
        if self.pool.mirrors:
            self.pool.sync_mirrors(layer_idx, only=self.write_to)

        if layer_idx == 0:
            # views in the order of worker 0's structure (attention.py:158-166), then
            # any segment only other workers list; each worker's location for a view
            # sums the lengths from that view to the end of its own order
            # (attention.py:167-176).  A worker whose structure omits a view does
            # not see it (location -1); the reference requires every worker to list
            # every segment
            segments = []
            index = {}
            for cl in self.cache_structure:
                for seg in cl:
                    if id(seg) not in index:
                        index[id(seg)] = len(segments)
                        segments.append(seg)
            F = len(segments)
            rows = [[-1] * (F - len(cl)) + [index[id(seg)] for seg in cl] for cl in self.cache_structure]
            order = torch.tensor(rows, dtype=torch.int32).to(dev)
            frags = torch.tensor([seg.get_seq_length(0) for seg in segments], dtype=torch.int32).to(dev)
            # inv_freq as the rotary embedding uses it (a model cast to a 16-bit dtype
            # rounds the buffer; transformers converts it back to float32)
            rot = self.model.rotary_emb
            round_to = key_states.dtype if key_states.dtype != torch.float32 else None
            self.locations, self.cosines, self.sines = self.ops.view_metadata(
                frags, order, S, rot.inv_freq.float(), float(rot.attention_scaling), round_to)
            self.segments = segments
            self.frags = frags
        return CacheStructure(keys=[seg.keys(layer_idx) for seg in self.segments],
                              values=[seg.values(layer_idx) for seg in self.segments],
                              cos=self.cosines, sin=self.sines, loc=self.locations, frags=self.frags)

    def get_queries_buffer(self, queries: torch.Tensor, layer_idx: int) -> torch.Tensor:
        if layer_idx == 0:  # attention.py:194-199
            self.queries_buffer = torch.empty((self.cosines.size(0),) + tuple(queries.shape), dtype=queries.dtype,
                                              device=queries.device)
        return self.queries_buffer

    def get_att_buffer(self, r_queries: torch.Tensor, layer_idx: int) -> torch.Tensor:
        if layer_idx == 0:  # attention.py:201-206
            self.att_buffer = torch.empty(tuple(r_queries.shape[1:4]) + (self.pool.E,), dtype=r_queries.dtype,
                                          device=r_queries.device)
        return self.att_buffer

    def get_input_kwargs(self, input_ids: torch.Tensor, attention_mask: Optional[torch.Tensor] = None):
        """Model inputs of one step (attention.py:208-236): per-worker position ids
        continue each worker's own segment; the mask is handed to the layers as
        is (transformers skips its own mask construction for a prepared dict)."""
        nw = len(self.cache_structure)
        assert input_ids.shape[0] == nw, (input_ids.shape, nw)
        if attention_mask is not None:
            new_tokens = attention_mask.sum(dim=1).tolist()
        else:
            new_tokens = [input_ids.shape[1]] * nw
        pos_ids = []
        for w in range(nw):
            e = self.write_to[w].get_seq_length() + int(new_tokens[w])
            pos_ids.append(torch.arange(e - input_ids.shape[1], e, dtype=torch.int64, device=input_ids.device))
        return {
            "input_ids": input_ids,
            "attention_mask": {"full_attention": attention_mask},
            "past_key_values": self,
            "use_cache": True,
            "position_ids": torch.stack(pos_ids, dim=0),
        }


def merge_caches(target, source, model, ops=HipOps) -> None:
    """Append ``source`` to ``target`` with its keys re-rotated by the target's
    length (attention.py:245-251).  ``target`` and ``source`` are segments or
    transformers caches; ``model`` the causal LM or its decoder (the reference
    passes the decoder).  A target in a pool (a segment, or a cache a
    DVAttnCache took in) gets one append per layer with a single cos/sin row,
    the pool growing if it must; a plain target cache gets the reference's own
    steps: the source's keys rotated in PyTorch, then ``target.update``."""
    rot = _rotary(model)
    t_seg, s_seg = _segment_of(target), _segment_of(source)
    n_layers = _config(model).num_hidden_layers

    def source_layer(layer):
        if s_seg is not None:
            L = s_seg.get_seq_length(layer)
            return s_seg.keys(layer)[:, :, :L], s_seg.values(layer)[:, :, :L]
        return _cache_layer(source, layer)

    if t_seg is None:
        k0, _ = source_layer(0)
        Ls = 0 if k0 is None else k0.shape[2]
        if Ls == 0:
            return
        lt = target.get_seq_length()
        cos, sin = rot(k0, torch.full((1, Ls), lt, dtype=torch.int64, device=k0.device))
        for layer in range(n_layers):
            k, v = source_layer(layer)
            target.update(_A.apply_rotary_pos_emb(k, cos, sin), v, layer)
        return
    pool = t_seg.pool
    dev = pool.k[0].device
    for layer in range(pool.num_layers):
        k, v = source_layer(layer)
        L = 0 if k is None else k.shape[2]
        if L == 0:
            continue
        t0 = t_seg.get_seq_length(layer)
        if t0 + L > pool.capacity:
            if not pool.growable:
                raise RuntimeError("merge_caches: target segment is full")
            pool.resize(capacity=1 << (t0 + L - 1).bit_length())
            if s_seg is not None and s_seg.pool is pool:
                k, v = source_layer(layer)
        cos, sin = rot(pool.k[layer], torch.full((1, 1), t0, dtype=torch.int64, device=dev))
        pos = (t0 + torch.arange(L, dtype=torch.int32, device=dev)).reshape(1, L)
        table = torch.tensor([[t_seg.index]], dtype=torch.int32, device=dev)
        ops.kv_append(k.to(device=dev, dtype=pool.k[layer].dtype), v.to(device=dev, dtype=pool.v[layer].dtype), pos,
                      cos.reshape(1, 1, -1), sin.reshape(1, 1, -1), pool.k[layer].permute(0, 2, 1, 3),
                      pool.v[layer].permute(0, 2, 1, 3), table)
        t_seg.lengths[layer] += L
        if pool.mirrors:
            pool.sync_mirrors(layer, only=[t_seg])


class AttentionModule(nn.Module):
    """Drop-in self-attention of a transformers decoder layer (attention.py:254-331).

    A model configured with ``_attn_implementation == "eager"`` runs the
    attention in PyTorch (``dvattn_sdpa_pt``, as the reference does at
    attention.py:309-312); any other setting runs the HIP ``dvattn_fused``."""

    def __init__(self, config, layer_idx: int):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.head_dim = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads
        self.num_key_value_groups = config.num_attention_heads // config.num_key_value_heads
        self.scaling = self.head_dim ** -0.5
        self.attention_dropout = config.attention_dropout
        self.is_causal = True
        self.q_proj = nn.Linear(config.hidden_size, config.num_attention_heads * self.head_dim, bias=True)
        self.k_proj = nn.Linear(config.hidden_size, config.num_key_value_heads * self.head_dim, bias=True)
        self.v_proj = nn.Linear(config.hidden_size, config.num_key_value_heads * self.head_dim, bias=True)
        self.o_proj = nn.Linear(config.num_attention_heads * self.head_dim, config.hidden_size, bias=False)

    def forward(self, hidden_states: torch.Tensor, position_embeddings=None, attention_mask=None,
                past_key_values: Optional[DVAttnCache] = None, past_key_value: Optional[DVAttnCache] = None,
                position_ids: Optional[torch.Tensor] = None, **kwargs):
        cache_obj = past_key_values if past_key_values is not None else past_key_value
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, self.head_dim)
        if input_shape[0] != 1:
            assert position_ids is not None, "When processing multiple workers, `position_ids` are mandatory"
        query_states = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        key_states = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        value_states = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        cos, sin = position_embeddings
        # the key rotation (attention.py:304) happens inside the cache append
        cache = cache_obj.update(key_states, value_states, self.layer_idx,
                                 {"cos": cos, "sin": sin, "mask": attention_mask})
        if self.config._attn_implementation == "eager":
            # PyTorch path of the attention (attention.py:309-312): the query
            # rotated for every view, then one softmax over all views' keys
            # (each view cut to its filled length; later keys are masked anyway)
            F = cache.cos.size(0)
            rq = _A.apply_rotary_pos_emb(query_states[None].expand(F, -1, -1, -1, -1), cache.cos, cache.sin,
                                         unsqueeze_dim=2)
            keys = [k[:, :, :seg.get_seq_length(self.layer_idx)] for k, seg in zip(cache.keys, cache_obj.segments)]
            vals = [v[:, :, :seg.get_seq_length(self.layer_idx)] for v, seg in zip(cache.values, cache_obj.segments)]
            out = _A.dvattn_sdpa_pt(rq, cache.loc, keys, vals, self.scaling)
        else:
            rq = cache_obj.get_queries_buffer(query_states, self.layer_idx)
            out = cache_obj.get_att_buffer(rq, self.layer_idx)
            cache_obj.ops.fused(query_states, cache.loc, cache.keys, cache.values, self.scaling, cache.frags,
                                cache.cos, cache.sin, rq, out)
        attn_output = out.transpose(1, 2).reshape(*input_shape, -1).contiguous()
        return self.o_proj(attn_output), None


def model_surgery(model) -> None:
    """Swap every decoder layer's self-attention for ``AttentionModule``, keeping
    its projection weights (attention.py:334-343).  Masks are handed through by
    ``DVAttnCache.get_input_kwargs``."""
    for layer in model.model.layers:
        old = layer.self_attn
        new = AttentionModule(model.model.config, old.layer_idx)
        new.q_proj, new.k_proj, new.v_proj, new.o_proj = old.q_proj, old.k_proj, old.v_proj, old.o_proj
        layer.self_attn = new


__all__ = ["CacheStructure", "SegmentPool", "Segment", "DVAttnCache", "merge_caches", "AttentionModule",
           "model_surgery", "HipOps", "segments_from_caches", "pool_caches"]
