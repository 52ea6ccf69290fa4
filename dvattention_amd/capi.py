"""ctypes binding of the C ABI in include/dvattn_amd.h (libdvattn_amd.so).

This is the binding a non-torch caller would use; it is also how the GPU parity
tests reach the kernels without going through the torch operator layer.  The
functions take torch tensors for convenience but pass only raw device pointers,
int sizes, a workspace pointer and the current HIP stream across the boundary.
``import torch`` happens first so the library binds to the HIP runtime torch
already loaded.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(_HERE, "libdvattn_amd.so")

DVATTN_F32, DVATTN_F16, DVATTN_BF16 = 0, 1, 2
STATUS = {0: "DVATTN_OK", 1: "DVATTN_ERR_INVALID", 2: "DVATTN_ERR_UNSUPPORTED", 3: "DVATTN_ERR_WORKSPACE",
          4: "DVATTN_ERR_HIP"}

# Every function include/dvattn_amd.h declares.
EXPORTED = [
    "dvattn_last_error", "dvattn_abi_version", "dvattn_set_option", "dvattn_get_option",
    "dvattn_paged_sdpa_workspace_size", "dvattn_paged_sdpa", "dvattn_paged_sdpa_noalloc",
    "dvattn_varlen_paged_sdpa_workspace_size", "dvattn_varlen_paged_sdpa",
    "dvattn_sdpa_workspace_size", "dvattn_sdpa", "dvattn_fused",
    "dvattn_rope", "dvattn_varlen_rope",
    "dvattn_paged_kv_append", "dvattn_view_metadata",
]


class Shape(ctypes.Structure):
    """dvattn_shape (mirrors Shape, src/common.h:5-20)."""
    _fields_ = [(n, ctypes.c_int) for n in (
        "F", "W", "Hq", "Hkv", "E", "Ev", "S", "block_size", "max_blocks_per_seq",
        "total_q_tokens", "num_blocks", "rotary_dim")]


class KvLayout(ctypes.Structure):
    """dvattn_kv_layout: element strides of keys/values (w, h, s), cos/sin (w, s)
    and the caches (page, row, head)."""
    _fields_ = [("key_strides", ctypes.c_longlong * 3), ("value_strides", ctypes.c_longlong * 3),
                ("rope_strides", ctypes.c_longlong * 2), ("k_cache_strides", ctypes.c_longlong * 3),
                ("v_cache_strides", ctypes.c_longlong * 3)]


class DvattnError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status


_VP = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_SP = ctypes.POINTER(Shape)

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            raise ImportError(f"{LIBRARY} is not built; run `python dvattention_amd/_build.py`")
        L = ctypes.CDLL(LIBRARY)
        L.dvattn_last_error.restype = ctypes.c_char_p
        L.dvattn_last_error.argtypes = []
        L.dvattn_abi_version.restype = _I
        L.dvattn_abi_version.argtypes = []
        for n in ("dvattn_paged_sdpa_workspace_size", "dvattn_varlen_paged_sdpa_workspace_size",
                  "dvattn_sdpa_workspace_size"):
            getattr(L, n).restype = _SZ
            getattr(L, n).argtypes = [_I, _SP, _I]
        L.dvattn_paged_sdpa.restype = _I
        L.dvattn_paged_sdpa.argtypes = [_I, _VP, _F, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _SP, _VP, _SZ, _VP]
        L.dvattn_paged_sdpa_noalloc.restype = _I
        L.dvattn_paged_sdpa_noalloc.argtypes = [_I, _VP, _F, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _SP, _VP]
        L.dvattn_varlen_paged_sdpa.restype = _I
        L.dvattn_varlen_paged_sdpa.argtypes = [_I, _VP, _F, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _SP,
                                               _VP, _SZ, _VP]
        L.dvattn_sdpa.restype = _I
        L.dvattn_sdpa.argtypes = [_I, _VP, _F, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _SP, _VP, _SZ, _VP]
        L.dvattn_fused.restype = _I
        L.dvattn_fused.argtypes = [_I, _VP, _VP, _F, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _SP, _VP, _SZ,
                                   _VP]
        L.dvattn_rope.restype = _I
        L.dvattn_rope.argtypes = [_I, _VP, _VP, _VP, _VP, _SP, _VP]
        L.dvattn_varlen_rope.restype = _I
        L.dvattn_varlen_rope.argtypes = [_I, _VP, _VP, _VP, _VP, _SP, _VP]
        L.dvattn_paged_kv_append.restype = _I
        L.dvattn_paged_kv_append.argtypes = [_I, _I, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _SP,
                                             ctypes.POINTER(KvLayout), _VP]
        L.dvattn_view_metadata.restype = _I
        L.dvattn_view_metadata.argtypes = [_VP, _VP, _VP, _VP, _VP, _VP, _F, _I, _I, _I, _I, _I, _VP]
        L.dvattn_set_option.restype = _I
        L.dvattn_set_option.argtypes = [ctypes.c_char_p, _I]
        L.dvattn_get_option.restype = _I
        L.dvattn_get_option.argtypes = [ctypes.c_char_p]
        _lib = L
    return _lib


# dvattn_set_option values of "small_path"
SMALL_PATH = {"off": 0, "auto": 1, "require": 2, "force": 3}


def set_option(name: str, value: int) -> None:
    """Process-wide switch of the library (include/dvattn_amd.h: dvattn_set_option)."""
    _check(lib().dvattn_set_option(name.encode(), int(value)))


def get_option(name: str) -> int:
    return lib().dvattn_get_option(name.encode())


def dtype_code(dt: torch.dtype) -> int:
    return {torch.float32: DVATTN_F32, torch.float16: DVATTN_F16, torch.bfloat16: DVATTN_BF16}[dt]


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _check(st: int) -> None:
    if st != 0:
        raise DvattnError(st, lib().dvattn_last_error().decode())


def _workspace(nbytes: int, like: torch.Tensor) -> torch.Tensor:
    return torch.empty(max(1, nbytes), dtype=torch.uint8, device=like.device)


def paged_shape(queries, locations, cosines, k_cache, v_cache, block_tables) -> Shape:
    W, Hq, S, E = queries.shape
    return Shape(F=locations.shape[0], W=W, Hq=Hq, Hkv=k_cache.shape[2], E=E, Ev=v_cache.shape[3], S=S,
                 block_size=k_cache.shape[1], max_blocks_per_seq=block_tables.shape[1], total_q_tokens=0,
                 num_blocks=k_cache.shape[0], rotary_dim=cosines.shape[3])


def paged_sdpa(out, scale, locations, queries, cosines, sines, fragment_lengths, k_cache, v_cache, block_tables,
               shape: Shape | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    L = lib()
    s = shape or paged_shape(queries, locations, cosines, k_cache, v_cache, block_tables)
    dt = dtype_code(out.dtype)
    need = L.dvattn_paged_sdpa_workspace_size(dt, ctypes.byref(s), out.device.index or 0)
    ws = workspace if workspace is not None and workspace.numel() >= need else _workspace(need, out)
    _check(L.dvattn_paged_sdpa(dt, _ptr(out), scale, _ptr(locations), _ptr(queries), _ptr(cosines), _ptr(sines),
                               _ptr(fragment_lengths), _ptr(k_cache), _ptr(v_cache), _ptr(block_tables),
                               ctypes.byref(s), _ptr(ws), ws.numel(), _stream(out)))
    return out


def paged_sdpa_noalloc(out, scale, locations, queries, cosines, sines, fragment_lengths, k_cache, v_cache,
                       block_tables, shape: Shape | None = None) -> torch.Tensor:
    """dvattn_paged_sdpa_noalloc: dvattn_paged_sdpa on the library's static
    per-GPU scratch (no workspace argument, nothing allocated)."""
    L = lib()
    s = shape or paged_shape(queries, locations, cosines, k_cache, v_cache, block_tables)
    _check(L.dvattn_paged_sdpa_noalloc(dtype_code(out.dtype), _ptr(out), scale, _ptr(locations), _ptr(queries),
                                       _ptr(cosines), _ptr(sines), _ptr(fragment_lengths), _ptr(k_cache),
                                       _ptr(v_cache), _ptr(block_tables), ctypes.byref(s), _stream(out)))
    return out


NOALLOC_SCRATCH_BYTES = 64 << 20   # DVATTN_NOALLOC_SCRATCH_BYTES


def varlen_paged_sdpa(out, scale, locations, queries, cosines, sines, fragment_lengths, k_cache, v_cache,
                      block_tables, cu_seqlens_q, cu_seqlens_k, workspace: torch.Tensor | None = None):
    L = lib()
    T, Hq, E = queries.shape
    s = Shape(F=locations.shape[0], W=cu_seqlens_q.shape[0] - 1, Hq=Hq, Hkv=k_cache.shape[2], E=E,
              Ev=v_cache.shape[3], S=1, block_size=k_cache.shape[1], max_blocks_per_seq=block_tables.shape[1],
              total_q_tokens=T, num_blocks=k_cache.shape[0], rotary_dim=2 * cosines.shape[2])
    dt = dtype_code(out.dtype)
    need = L.dvattn_varlen_paged_sdpa_workspace_size(dt, ctypes.byref(s), out.device.index or 0)
    ws = workspace if workspace is not None and workspace.numel() >= need else _workspace(need, out)
    _check(L.dvattn_varlen_paged_sdpa(dt, _ptr(out), scale, _ptr(locations), _ptr(queries), _ptr(cosines),
                                      _ptr(sines), _ptr(fragment_lengths), _ptr(k_cache), _ptr(v_cache),
                                      _ptr(block_tables), _ptr(cu_seqlens_q), _ptr(cu_seqlens_k), ctypes.byref(s),
                                      _ptr(ws), ws.numel(), _stream(out)))
    return out


def _frag_arrays(keys, values):
    F = len(keys)
    kp = (ctypes.c_void_p * max(F, 1))(*[k.data_ptr() for k in keys])
    vp = (ctypes.c_void_p * max(F, 1))(*[v.data_ptr() for v in values])
    toks = (ctypes.c_int * max(F, 1))(*[k.shape[-2] for k in keys])
    batch = (ctypes.c_int * max(F, 1))(*[(k.shape[0] if k.dim() == 4 else 1) for k in keys])
    return kp, vp, toks, batch


def contig_shape(rq, keys, values, cos=None) -> Shape:
    F, W, Hq, S, E = rq.shape
    k0 = keys[0]
    Hkv = k0.shape[1] if k0.dim() == 4 else k0.shape[0]
    return Shape(F=F, W=W, Hq=Hq, Hkv=Hkv, E=E, Ev=values[0].shape[-1], S=S, block_size=0, max_blocks_per_seq=0,
                 total_q_tokens=0, num_blocks=0, rotary_dim=0 if cos is None else cos.shape[3])


def sdpa(out, scale, locations, rq, fragment_lengths, keys, values, workspace=None):
    L = lib()
    s = contig_shape(rq, keys, values)
    dt = dtype_code(out.dtype)
    need = L.dvattn_sdpa_workspace_size(dt, ctypes.byref(s), out.device.index or 0)
    ws = workspace if workspace is not None and workspace.numel() >= need else _workspace(need, out)
    kp, vp, toks, batch = _frag_arrays(keys, values)
    _check(L.dvattn_sdpa(dt, _ptr(out), scale, _ptr(locations), _ptr(rq), _ptr(fragment_lengths), kp, vp, toks,
                         batch, ctypes.byref(s), _ptr(ws), ws.numel(), _stream(out)))
    return out


def fused(out, rq, scale, locations, queries, fragment_lengths, keys, values, cosines, sines, workspace=None):
    L = lib()
    s = contig_shape(rq, keys, values, cosines)
    dt = dtype_code(out.dtype)
    need = L.dvattn_sdpa_workspace_size(dt, ctypes.byref(s), out.device.index or 0)
    ws = workspace if workspace is not None and workspace.numel() >= need else _workspace(need, out)
    kp, vp, toks, batch = _frag_arrays(keys, values)
    _check(L.dvattn_fused(dt, _ptr(out), _ptr(rq), scale, _ptr(locations), _ptr(queries), _ptr(fragment_lengths),
                          kp, vp, toks, batch, _ptr(cosines), _ptr(sines), ctypes.byref(s), _ptr(ws), ws.numel(),
                          _stream(out)))
    return out, rq


def rope(out, queries, cosines, sines):
    F, W, Hq, S, E = out.shape
    s = Shape(F=F, W=W, Hq=Hq, Hkv=0, E=E, Ev=0, S=S, block_size=0, max_blocks_per_seq=0, total_q_tokens=0,
              num_blocks=0, rotary_dim=cosines.shape[3])
    _check(lib().dvattn_rope(dtype_code(out.dtype), _ptr(out), _ptr(queries), _ptr(cosines), _ptr(sines),
                             ctypes.byref(s), _stream(out)))
    return out


def varlen_rope(out, queries, cosines, sines):
    F, T, H, E = out.shape
    s = Shape(F=F, W=0, Hq=H, Hkv=0, E=E, Ev=0, S=1, block_size=0, max_blocks_per_seq=0, total_q_tokens=T,
              num_blocks=0, rotary_dim=2 * cosines.shape[2])
    _check(lib().dvattn_varlen_rope(dtype_code(out.dtype), _ptr(out), _ptr(queries), _ptr(cosines), _ptr(sines),
                                    ctypes.byref(s), _stream(out)))
    return out


def kv_append(k_cache, v_cache, block_tables, positions, keys, values, cosines, sines):
    """dvattn_paged_kv_append: keys/values [W,Hkv,S,E] (any strides, last dim
    contiguous), cos/sin [W|1, S|1, R], caches [P,bs,Hkv,E] (strided views allowed)."""
    W, Hkv, S, E = keys.shape
    s = Shape(F=0, W=W, Hq=0, Hkv=Hkv, E=E, Ev=values.shape[3], S=S, block_size=k_cache.shape[1],
              max_blocks_per_seq=block_tables.shape[1], total_q_tokens=0, num_blocks=k_cache.shape[0],
              rotary_dim=cosines.shape[2])
    lay = KvLayout()
    for i in range(3):
        lay.key_strides[i] = keys.stride(i)
        lay.value_strides[i] = values.stride(i)
        lay.k_cache_strides[i] = k_cache.stride(i)
        lay.v_cache_strides[i] = v_cache.stride(i)
    lay.rope_strides[0] = 0 if cosines.shape[0] == 1 else cosines.stride(0)
    lay.rope_strides[1] = 0 if cosines.shape[1] == 1 else cosines.stride(1)
    dt = dtype_code(k_cache.dtype)
    rdt = DVATTN_F32 if cosines.dtype == torch.float32 else dtype_code(cosines.dtype)
    _check(lib().dvattn_paged_kv_append(dt, rdt, _ptr(k_cache), _ptr(v_cache), _ptr(block_tables), _ptr(positions),
                                        _ptr(keys), _ptr(values), _ptr(cosines), _ptr(sines), ctypes.byref(s),
                                        ctypes.byref(lay), _stream(k_cache)))
    return k_cache, v_cache


def view_metadata(locations, cosines, sines, fragment_lengths, order, inv_freq, attention_scaling=1.0,
                  round_to=None):
    """dvattn_view_metadata: locations [F,W,S] i32, cos/sin [F,W,S,R] f32."""
    F, W, S = locations.shape
    rd = -1 if round_to in (None, torch.float32) else dtype_code(round_to)
    _check(lib().dvattn_view_metadata(_ptr(locations), _ptr(cosines), _ptr(sines), _ptr(fragment_lengths),
                                      _ptr(order), _ptr(inv_freq), attention_scaling, rd, F, W, S,
                                      cosines.shape[3], _stream(locations)))
    return locations, cosines, sines
