"""dvattention_amd -- MI355X (gfx950) native DVAttn.

Drop-in for the reference's ``dvattn`` operator API (python/dvattn/attention.py
and the ``torch.ops.libdvatt`` operators of src/binding.cu): the same operator
names, schemas, tensor layouts and page-table / ``cu_seqlens`` conventions,
implemented by hand-written HIP kernels for gfx950 behind a C ABI
(``include/dvattn_amd.h``, ``libdvattn_amd.so``).

Importing the package registers ``torch.ops.libdvatt.*`` from the in-tree
``_libdvatt.so``.  There is no fallback: if the native libraries are missing the
import fails (build them with ``python dvattention_amd/_build.py``, which runs
without importing the package).
"""
from __future__ import annotations

import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
TORCH_OPS_LIBRARY = os.path.join(_HERE, "_libdvatt.so")
CAPI_LIBRARY = os.path.join(_HERE, "libdvattn_amd.so")


def _load_ops() -> None:
    if not os.path.exists(TORCH_OPS_LIBRARY) or not os.path.exists(CAPI_LIBRARY):
        raise ImportError(
            "dvattention_amd: native libraries are not built "
            f"({TORCH_OPS_LIBRARY}, {CAPI_LIBRARY}); run `python dvattention_amd/_build.py`")
    if not hasattr(torch.ops.libdvatt, "dvattn_paged_sdpa"):
        torch.ops.load_library(TORCH_OPS_LIBRARY)


_load_ops()

from .attention import (  # noqa: E402
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

__all__ = [
    "apply_rotary_pos_emb",
    "dvattn_fused",
    "dvattn_paged_kv_append",
    "dvattn_paged_sdpa",
    "dvattn_rope",
    "dvattn_sdpa",
    "dvattn_sdpa_pt",
    "dvattn_varlen_paged_sdpa",
    "dvattn_varlen_rope",
    "dvattn_view_metadata",
    "merge_caches_paged",
    "rotate_half",
    "TORCH_OPS_LIBRARY",
    "CAPI_LIBRARY",
]
