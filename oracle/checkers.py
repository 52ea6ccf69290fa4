"""ctypes front-ends for the compiled checkers -- TEST INFRASTRUCTURE ONLY.

* ``bruteforce_*``: float64 loops of ``oracle/bruteforce.c`` (built by
  ``oracle/Makefile`` into ``oracle/libbruteforce.so``).
* ``ref_rope_cpu``: the reference's own ``rope_cpu`` (src/q_rope.h:3-35),
  compiled from the reference tree into ``oracle/_ref/libqrope_ref.so``;
  ``None`` where that tree was not present at build time.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_BF = None
_REF = None


def _bf():
    global _BF
    if _BF is None:
        path = os.path.join(_HERE, "libbruteforce.so")
        if not os.path.exists(path):
            raise RuntimeError("oracle/libbruteforce.so is not built (run `make -C oracle`)")
        _BF = ctypes.CDLL(path)
    return _BF


def ref_rope_available() -> bool:
    return os.path.exists(os.path.join(_HERE, "_ref", "libqrope_ref.so"))


def _ref():
    global _REF
    if _REF is None:
        _REF = ctypes.CDLL(os.path.join(_HERE, "_ref", "libqrope_ref.so"))
    return _REF


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def ref_rope_cpu(queries, cosines, sines) -> np.ndarray:
    """Reference ``rope_cpu<float>``: q ``[W,Hq,S,E]``, cos/sin ``[F,W,S,R]`` -> ``[F,W,Hq,S,E]``."""
    q = _f32(queries)
    c = _f32(cosines)
    s = _f32(sines)
    W, Hq, S, E = q.shape
    F, _, _, R = c.shape
    out = np.zeros((F, W, Hq, S, E), dtype=np.float32)
    _ref().ref_rope_cpu_f32(_p(out), _p(q), _p(c), _p(s), F, W, Hq, S, E, R)
    return out


def bruteforce_paged(scale, loc, rq, fl, kc, vc, bt) -> np.ndarray:
    loc, fl, bt = _i32(loc), _i32(fl), _i32(bt)
    rq, kc, vc = _f32(rq), _f32(kc), _f32(vc)
    F, W, Hq, S, E = rq.shape
    P, bs, Hkv, _ = kc.shape
    Ev = vc.shape[-1]
    out = np.zeros((W, Hq, S, Ev), dtype=np.float64)
    rc = _bf().bf_paged(_p(out), ctypes.c_double(scale), _p(loc), _p(rq), _p(fl), _p(kc), _p(vc), _p(bt),
                        F, W, Hq, S, E, Ev, P, bs, Hkv, bt.shape[1])
    if rc != 0:
        raise ValueError("bruteforce_paged: index outside block_tables or page pool")
    return out


def bruteforce_varlen(scale, loc, rq, fl, kc, vc, bt, cu_q) -> np.ndarray:
    loc, fl, bt, cu_q = _i32(loc), _i32(fl), _i32(bt), _i32(cu_q)
    rq, kc, vc = _f32(rq), _f32(kc), _f32(vc)
    F, T, Hq, E = rq.shape
    P, bs, Hkv, _ = kc.shape
    Ev = vc.shape[-1]
    out = np.zeros((T, Hq, Ev), dtype=np.float64)
    rc = _bf().bf_varlen(_p(out), ctypes.c_double(scale), _p(loc), _p(rq), _p(fl), _p(kc), _p(vc), _p(bt),
                         _p(cu_q), F, T, cu_q.shape[0] - 1, Hq, E, Ev, P, bs, Hkv, bt.shape[1])
    if rc != 0:
        raise ValueError("bruteforce_varlen: index outside block_tables or page pool")
    return out


def bruteforce_contig(scale, loc, rq, fl, key_fragments, value_fragments) -> np.ndarray:
    """Fragments: list of arrays ``[B,Hkv,L,E]`` (B == 1 shared, or B == W) or ``[Hkv,L,E]``."""
    loc, fl, rq = _i32(loc), _i32(fl), _f32(rq)
    F, W, Hq, S, E = rq.shape
    ks, vs, koff, voff, Ls, bstr = [], [], [], [], [], []
    kpos = vpos = 0
    for k, v in zip(key_fragments, value_fragments):
        k, v = _f32(k), _f32(v)
        if k.ndim == 3:
            k, v = k[None], v[None]
        Hkv = k.shape[1]
        koff.append(kpos)
        voff.append(vpos)
        kpos += k.size
        vpos += v.size
        ks.append(k.ravel())
        vs.append(v.ravel())
        Ls.append(k.shape[2])
        bstr.append(1 if k.shape[0] > 1 else 0)
    Ev = value_fragments[0].shape[-1]
    kf, vf = np.concatenate(ks), np.concatenate(vs)
    koff = np.asarray(koff, dtype=np.int64)
    voff = np.asarray(voff, dtype=np.int64)
    Ls, bstr = _i32(Ls), _i32(bstr)
    out = np.zeros((W, Hq, S, Ev), dtype=np.float64)
    _bf().bf_contig(_p(out), ctypes.c_double(scale), _p(loc), _p(rq), _p(fl), _p(kf), _p(vf), _p(koff), _p(voff),
                    _p(Ls), _p(bstr), F, W, Hq, S, E, Ev, Hkv)
    return out
