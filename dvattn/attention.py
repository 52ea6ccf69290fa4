"""``dvattn.attention``: the reference's module path (python/dvattn/attention.py)
over this build.

Importing it loads the operator library, as the reference's module does at
import (attention.py:10-14) -- here ``dvattention_amd/_libdvatt.so`` (the
``libdvatt`` namespace with the reference's six schemas) over the HIP kernels
of ``libdvattn_amd.so``.  Unlike the reference there is no fallback: a missing
library raises ``ImportError``.  The names are the reference's:

* operators and helpers -- ``dvattn_fused``, ``dvattn_sdpa``, ``dvattn_sdpa_pt``,
  ``dvattn_rope``, ``rotate_half``, ``apply_rotary_pos_emb`` (attention.py:17-88),
  plus the paged / varlen wrappers of this build;
* model integration -- ``CacheStructure``, ``DVAttnCache``, ``merge_caches``,
  ``AttentionModule``, ``model_surgery`` (attention.py:100-343).  As in the
  reference, ``DVAttnCache(cache_structure, model, write_to)`` and
  ``merge_caches(target, source, model)`` take transformers ``Cache`` objects;
  they also take ``SegmentPool`` segments, the storage the caches are moved
  into.
"""
from dvattention_amd.attention import (  # noqa: F401  (importing dvattention_amd registers the ops)
    apply_rotary_pos_emb,
    dvattn_fused,
    dvattn_paged_kv_append,
    dvattn_paged_sdpa,
    dvattn_rope,
    dvattn_sdpa,
    dvattn_sdpa_pt,
    dvattn_varlen_paged_sdpa,
    dvattn_varlen_rope,
    dvattn_view_metadata,
    merge_caches_paged,
    rotate_half,
)
from dvattention_amd.hf import (  # noqa: F401
    AttentionModule,
    CacheStructure,
    DVAttnCache,
    Segment,
    SegmentPool,
    merge_caches,
    model_surgery,
    segments_from_caches,
)

__all__ = [
    "apply_rotary_pos_emb", "dvattn_fused", "dvattn_paged_kv_append", "dvattn_paged_sdpa", "dvattn_rope",
    "dvattn_sdpa", "dvattn_sdpa_pt", "dvattn_varlen_paged_sdpa", "dvattn_varlen_rope", "dvattn_view_metadata",
    "merge_caches_paged", "rotate_half", "AttentionModule", "CacheStructure", "DVAttnCache", "Segment",
    "SegmentPool", "merge_caches", "model_surgery", "segments_from_caches",
]
