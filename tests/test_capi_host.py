"""Host-side tests of the native boundary (CPU only, no kernel launches).

* libdvattn_amd.so loads and exports every function include/dvattn_amd.h declares.
* Argument validation of the C ABI rejects bad calls before touching the GPU.
* torch.ops.libdvatt carries the reference's six schemas (src/binding.cu:410-420)
  with the needs_fixed_stride_order tag, and has no CPU kernels (no fallback).
"""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dvattn_amd.h")

REFERENCE_SCHEMAS = {
    "dvattn_sdpa": "dvattn_sdpa(Tensor(a!) output, float scale, Tensor locations, Tensor queries, "
                   "Tensor fragment_lengths, Tensor[] key_fragments, Tensor[] value_fragments) -> ()",
    "dvattn_paged_sdpa": "dvattn_paged_sdpa(Tensor(a!) output, float scale, Tensor locations, Tensor queries, "
                         "Tensor cosines, Tensor sines, Tensor fragment_lengths, Tensor k_cache, Tensor v_cache, "
                         "Tensor block_tables) -> ()",
    "dvattn_rope": "dvattn_rope(Tensor(a!) output, Tensor queries, Tensor cosines, Tensor sines) -> ()",
    "dvattn_fused": "dvattn_fused(Tensor(a!) output, Tensor(b!) rq, float scale, Tensor locations, Tensor queries, "
                    "Tensor fragment_lengths, Tensor[] key_fragments, Tensor[] value_fragments, Tensor cosines, "
                    "Tensor sines) -> ()",
    "dvattn_varlen_rope": "dvattn_varlen_rope(Tensor(a!) output, Tensor queries, Tensor cosines, Tensor sines) -> ()",
    "dvattn_varlen_paged_sdpa": "dvattn_varlen_paged_sdpa(Tensor(a!) output, float scale, Tensor locations, "
                                "Tensor queries, Tensor cosines, Tensor sines, Tensor fragment_lengths, "
                                "Tensor k_cache, Tensor v_cache, Tensor block_tables, Tensor cu_seqlens_q, "
                                "Tensor cu_seqlens_k) -> ()",
}


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"DVATTN_API\s+[\w\s\*]*?\b(dvattn_\w+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    from dvattention_amd import capi
    assert header_functions() == sorted(capi.EXPORTED)


def test_library_exports_every_declared_symbol():
    from dvattention_amd import capi
    lib = capi.lib()
    for name in header_functions():
        assert hasattr(lib, name), f"{name} declared in include/dvattn_amd.h but not exported"
    assert lib.dvattn_abi_version() == 1


def _shape(**kw):
    from dvattention_amd import capi
    base = dict(F=1, W=1, Hq=16, Hkv=1, E=128, Ev=128, S=1, block_size=16, max_blocks_per_seq=4,
                total_q_tokens=1, num_blocks=4, rotary_dim=64)
    base.update(kw)
    return capi.Shape(**base)


def _paged(shape, dtype=2, out=1, ws_bytes=1 << 30):
    from dvattention_amd import capi
    L = capi.lib()
    p = ctypes.c_void_p(0x1000)
    return L.dvattn_paged_sdpa(dtype, p if out else None, 0.1, p, p, p, p, p, p, p, p, ctypes.byref(shape), p,
                               ws_bytes, None)


@pytest.mark.parametrize("kw,status,needle", [
    (dict(Hq=32), 2, "GQA 16"),
    (dict(E=64), 2, "E == Ev == 128"),
    (dict(Ev=64), 2, "E == Ev == 128"),
    (dict(rotary_dim=63), 2, "rotary_dim"),
    (dict(rotary_dim=130), 2, "rotary_dim"),
    (dict(block_size=0), 1, "block_size"),
    (dict(F=-1), 1, "negative"),
    # cache rows (block, slot, KV head) are indexed in 32 bits by the kernels
    (dict(num_blocks=1 << 28, block_size=16, Hkv=1, Hq=16), 2, "2^32 rows"),
])
def test_paged_rejects_unsupported_shapes(kw, status, needle):
    from dvattention_amd import capi
    st = _paged(_shape(**kw))
    assert st == status
    assert needle in capi.lib().dvattn_last_error().decode()


def test_paged_rejects_bad_dtype_and_null_output_and_small_workspace():
    from dvattention_amd import capi
    L = capi.lib()
    assert _paged(_shape(), dtype=7) == 2
    assert "dtype" in L.dvattn_last_error().decode()
    assert _paged(_shape(), out=0) == 1
    assert _paged(_shape(), ws_bytes=16) == 3
    assert "workspace" in L.dvattn_last_error().decode()


def test_empty_problems_succeed_without_launch():
    # W*S == 0 -> nothing to do (paged_kernel_v21.cuh:385-386)
    assert _paged(_shape(W=0)) == 0
    assert _paged(_shape(S=0)) == 0


def test_rope_validation():
    from dvattention_amd import capi
    L = capi.lib()
    p = ctypes.c_void_p(0x1000)
    s = _shape(rotary_dim=7)
    assert L.dvattn_rope(2, p, p, p, p, ctypes.byref(s), None) == 2
    s = _shape(F=0)
    assert L.dvattn_rope(2, p, p, p, p, ctypes.byref(s), None) == 0      # empty -> no-op (rope.cuh:58-60)


def test_contig_rejects_bad_fragment_batch():
    from dvattention_amd import capi
    L = capi.lib()
    p = ctypes.c_void_p(0x1000)
    s = _shape(W=3, F=1)
    kp = (ctypes.c_void_p * 1)(0x2000)
    toks = (ctypes.c_int * 1)(8)
    batch = (ctypes.c_int * 1)(2)              # neither 1 nor W
    st = L.dvattn_sdpa(2, p, 0.1, p, p, p, kp, kp, toks, batch, ctypes.byref(s), p, 1 << 30, None)
    assert st == 1 and "batch" in L.dvattn_last_error().decode()


PAGED_ARGS = ["out", "locations", "queries", "cosines", "sines", "fragment_lengths", "k_cache", "v_cache",
              "block_tables", "cu_seqlens_q", "workspace"]


def _fake_ptrs(names, bad=None, offset=0):
    """Distinct fake device addresses (never dereferenced: every call below is
    refused on the host), the one named `bad` moved by `offset` bytes."""
    return {n: ctypes.c_void_p(0x10000 * (i + 1) + (offset if n == bad else 0)) for i, n in enumerate(names)}


def _paged_call(L, a, s, ws_bytes=1 << 30):
    return L.dvattn_paged_sdpa(2, a["out"], 0.1, a["locations"], a["queries"], a["cosines"], a["sines"],
                               a["fragment_lengths"], a["k_cache"], a["v_cache"], a["block_tables"],
                               ctypes.byref(s), a["workspace"], ws_bytes, None)


def _varlen_call(L, a, s, ws_bytes=1 << 30):
    return L.dvattn_varlen_paged_sdpa(2, a["out"], 0.1, a["locations"], a["queries"], a["cosines"], a["sines"],
                                      a["fragment_lengths"], a["k_cache"], a["v_cache"], a["block_tables"],
                                      a["cu_seqlens_q"], None, ctypes.byref(s), a["workspace"], ws_bytes, None)


# 16-byte vectors / DMAs on the tensors, 4-byte words on the int32 / fp32 arrays
@pytest.mark.parametrize("name,offset,align", [
    ("out", 8, 16), ("queries", 2, 16), ("k_cache", 4, 16), ("v_cache", 8, 16), ("workspace", 8, 16),
    ("locations", 2, 4), ("fragment_lengths", 1, 4), ("cosines", 2, 4), ("sines", 1, 4), ("block_tables", 2, 4),
])
def test_paged_and_varlen_refuse_misaligned_pointers(name, offset, align):
    from dvattention_amd import capi
    L = capi.lib()
    s = _shape()
    a = _fake_ptrs(PAGED_ARGS, name, offset)
    for call in (_paged_call, _varlen_call):
        assert call(L, a, s) == 1
        assert L.dvattn_last_error().decode().startswith(f"{name} must be {align}-byte aligned")
    a = _fake_ptrs(PAGED_ARGS, "cu_seqlens_q", 2)
    assert _varlen_call(L, a, s) == 1 and "cu_seqlens_q must be 4-byte" in L.dvattn_last_error().decode()
    # aligned pointers pass these checks and stop at the (too small) workspace, before any launch
    a = _fake_ptrs(PAGED_ARGS)
    assert _paged_call(L, a, s, ws_bytes=16) == 3 and _varlen_call(L, a, s, ws_bytes=16) == 3


def test_contig_fused_and_rope_refuse_misaligned_pointers():
    from dvattention_amd import capi
    L = capi.lib()
    s = _shape(W=2, F=1)
    names = ["out", "rq", "locations", "queries", "fragment_lengths", "cosines", "sines", "workspace", "k", "v"]
    toks = (ctypes.c_int * 1)(8)
    batch = (ctypes.c_int * 1)(2)

    def sdpa(a):
        kp, vp = (ctypes.c_void_p * 1)(a["k"].value), (ctypes.c_void_p * 1)(a["v"].value)
        return L.dvattn_sdpa(2, a["out"], 0.1, a["locations"], a["rq"], a["fragment_lengths"], kp, vp, toks, batch,
                             ctypes.byref(s), a["workspace"], 1 << 30, None)

    def fused(a):
        kp, vp = (ctypes.c_void_p * 1)(a["k"].value), (ctypes.c_void_p * 1)(a["v"].value)
        return L.dvattn_fused(2, a["out"], a["rq"], 0.1, a["locations"], a["queries"], a["fragment_lengths"], kp, vp,
                              toks, batch, a["cosines"], a["sines"], ctypes.byref(s), a["workspace"], 1 << 30, None)

    for name, offset, align in [("out", 8, 16), ("rq", 4, 16), ("workspace", 8, 16), ("locations", 2, 4),
                                ("fragment_lengths", 1, 4)]:
        for call in (sdpa, fused):
            assert call(_fake_ptrs(names, name, offset)) == 1
            assert L.dvattn_last_error().decode().startswith(f"{name.replace('rq', 'rotated_queries')} must be "
                                                             f"{align}-byte aligned"), (name, call)
    for name in ("k", "v"):
        assert sdpa(_fake_ptrs(names, name, 8)) == 1 and "16-byte aligned" in L.dvattn_last_error().decode()
    # fused: element alignment for the rotation, 16 bytes for the single launch's query reads
    assert fused(_fake_ptrs(names, "queries", 1)) == 1
    assert L.dvattn_last_error().decode().startswith("queries must be 2-byte aligned")
    assert fused(_fake_ptrs(names, "queries", 2)) == 1
    assert L.dvattn_last_error().decode().startswith("queries must be 16-byte aligned")
    assert fused(_fake_ptrs(names, "cosines", 2)) == 1 and "cosines must be 4-byte" in L.dvattn_last_error().decode()
    # standalone rope: natural alignment of the storage type (fp32 4, bf16 2) and of fp32 cos/sin
    a = _fake_ptrs(names, "out", 2)
    assert L.dvattn_rope(0, a["out"], a["queries"], a["cosines"], a["sines"], ctypes.byref(s), None) == 1
    assert L.dvattn_last_error().decode().startswith("out must be 4-byte aligned")
    a = _fake_ptrs(names, "queries", 1)
    assert L.dvattn_varlen_rope(2, a["out"], a["queries"], a["cosines"], a["sines"], ctypes.byref(s), None) == 1
    assert L.dvattn_last_error().decode().startswith("queries must be 2-byte aligned")


def test_kv_append_refuses_misaligned_pointers():
    from dvattention_amd import capi
    L = capi.lib()
    s = _kv_shape()
    lay = capi.KvLayout()
    names = ["k_cache", "v_cache", "block_tables", "positions", "keys", "values", "cosines", "sines"]
    for name, offset, rope_dt, align in [("keys", 1, 0, 2), ("v_cache", 1, 0, 2), ("positions", 2, 0, 4),
                                         ("block_tables", 1, 0, 4), ("cosines", 2, 0, 4), ("sines", 1, 2, 2)]:
        a = _fake_ptrs(names, name, offset)
        st = L.dvattn_paged_kv_append(2, rope_dt, *[a[n] for n in names], ctypes.byref(s), ctypes.byref(lay), None)
        assert st == 1 and L.dvattn_last_error().decode().startswith(f"{name} must be {align}-byte aligned")


def test_workspace_query_is_bounded():
    from dvattention_amd import capi
    L = capi.lib()
    s = _shape(W=32, Hkv=8, Hq=128)
    n = L.dvattn_paged_sdpa_workspace_size(2, ctypes.byref(s), 0)
    assert 0 < n < 64 << 20


def test_torch_ops_schemas_match_reference():
    import dvattention_amd  # noqa: F401  (registers torch.ops.libdvatt)
    for name, schema in REFERENCE_SCHEMAS.items():
        op = getattr(torch.ops.libdvatt, name).default
        assert str(op._schema) == "libdvatt::" + schema
        assert torch.Tag.needs_fixed_stride_order in op.tags


def test_no_cpu_fallback():
    import dvattention_amd
    q = torch.zeros(1, 16, 1, 128)
    c = torch.zeros(1, 1, 1, 64)
    with pytest.raises(Exception):
        dvattention_amd.dvattn_rope(q, c, c)


def test_python_api_mirrors_reference_names():
    import inspect
    import dvattention_amd.attention as A
    sig = inspect.signature(A.dvattn_fused)
    assert list(sig.parameters)[:8] == ["queries", "locations", "keys", "values", "scale", "fragment_lengths",
                                        "cosines", "sines"]
    assert sig.parameters["rotated_queries"].kind is inspect.Parameter.KEYWORD_ONLY
    assert list(inspect.signature(A.dvattn_sdpa).parameters) == ["queries", "locations", "keys", "values", "scale",
                                                                 "fragment_lengths", "out"]
    assert list(inspect.signature(A.dvattn_rope).parameters) == ["queries", "cosines", "sines", "out"]
    x = torch.randn(2, 3, 4, 8)
    c = torch.randn(2, 4, 6)
    s = torch.randn(2, 4, 6)
    y = A.apply_rotary_pos_emb(x, c, s)
    assert torch.equal(y[..., 6:], x[..., 6:])


def _kv_shape(**kw):
    from dvattention_amd import capi
    d = dict(F=0, W=2, Hq=0, Hkv=8, E=128, Ev=128, S=4, block_size=16, max_blocks_per_seq=4, total_q_tokens=0,
             num_blocks=8, rotary_dim=128)
    d.update(kw)
    return capi.Shape(**d)


@pytest.mark.parametrize("kw,rope_dt,status,needle", [
    (dict(W=1 << 16, S=4096), 0, 2, "2^31"),     # 32-bit element indexing
    (dict(), 1, 2, "cos/sin dtype"),             # f16 cos/sin for a bf16 cache
    (dict(rotary_dim=7), 0, 2, "rotary_dim"),
    (dict(rotary_dim=256), 0, 2, "rotary_dim"),  # R > E
    (dict(block_size=0), 0, 1, "block_size"),
    (dict(S=-1), 0, 1, "negative"),
])
def test_kv_append_validation(kw, rope_dt, status, needle):
    from dvattention_amd import capi
    L = capi.lib()
    p = ctypes.c_void_p(0x1000)
    s = _kv_shape(**kw)
    lay = capi.KvLayout()
    st = L.dvattn_paged_kv_append(2, rope_dt, p, p, p, p, p, p, p, p, ctypes.byref(s), ctypes.byref(lay), None)
    assert st == status and needle in L.dvattn_last_error().decode()


def test_kv_append_and_metadata_null_and_empty():
    from dvattention_amd import capi
    L = capi.lib()
    p = ctypes.c_void_p(0x1000)
    lay = capi.KvLayout()
    s = _kv_shape()
    assert L.dvattn_paged_kv_append(2, 0, p, None, p, p, p, p, p, p, ctypes.byref(s), ctypes.byref(lay), None) == 1
    s = _kv_shape(W=0)
    assert L.dvattn_paged_kv_append(2, 0, None, None, None, None, None, None, None, None, ctypes.byref(s),
                                    ctypes.byref(lay), None) == 0
    # view metadata: odd rotary dim, unknown rounding dtype, null pointers, empty
    assert L.dvattn_view_metadata(p, p, p, p, p, p, 1.0, -1, 2, 3, 1, 63, None) == 2
    assert L.dvattn_view_metadata(p, p, p, p, p, p, 1.0, 7, 2, 3, 1, 64, None) == 2
    assert L.dvattn_view_metadata(p, None, p, p, p, p, 1.0, -1, 2, 3, 1, 64, None) == 1
    assert L.dvattn_view_metadata(p, p, p, p, p, p, 1.0, -1, -1, 3, 1, 64, None) == 1
    assert L.dvattn_view_metadata(None, None, None, None, None, None, 1.0, -1, 0, 3, 1, 64, None) == 0


def test_options_set_get_and_refuse():
    """dvattn_set_option / dvattn_get_option (host only, no GPU call)."""
    from dvattention_amd import capi
    before = capi.get_option("small_path")
    assert before in capi.SMALL_PATH.values()
    try:
        for v in capi.SMALL_PATH.values():
            capi.set_option("small_path", v)
            assert capi.get_option("small_path") == v
        with pytest.raises(capi.DvattnError):
            capi.set_option("small_path", 9)
        with pytest.raises(capi.DvattnError):
            capi.set_option("no_such_option", 1)
        assert capi.get_option("no_such_option") == -1
    finally:
        capi.set_option("small_path", before)
