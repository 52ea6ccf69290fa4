"""Writes the small golden fixtures in tests/golden/*.npz.

Expected outputs come from the float64 brute force of oracle/bruteforce.c (loops
over the reference kernels' index arithmetic), applied to queries rotated by
the oracle's rotation (itself pinned against the reference's rope_cpu and
transformers' rotary helpers in tests/test_oracle.py).  Inputs are stored as
float32 arrays (bf16/fp16 values are exact in float32) with their storage dtype.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import checkers  # noqa: E402
from oracle import dvattn_oracle as O  # noqa: E402

DT = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


def cs(pos, R, base=1e4):
    pos = np.asarray(pos, dtype=np.float64)
    inv = 1.0 / (base ** (np.arange(0, R, 2, dtype=np.float64) / R))
    fr = pos[..., None] * inv
    emb = np.concatenate([fr, fr], -1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def paged_case(name, dtype, F, W, S, Hkv, bs, lens, R, seed, loc_mode="random"):
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    dt = DT[dtype]
    Hq, E = 16 * Hkv, 128
    lens = np.asarray(lens, dtype=np.int32)
    maxB = int((lens.sum() + bs - 1) // bs) + 1
    P = W * maxB + 2
    bt = rng.permutation(P)[: W * maxB].astype(np.int32).reshape(W, maxB)
    if loc_mode == "causal":
        loc = (lens[:, None, None] - S + np.arange(S)[None, None, :]).repeat(W, 1).astype(np.int32)
    else:
        loc = rng.integers(-2, int(lens.max()) + 2, size=(F, W, S)).astype(np.int32)
    q = torch.randn(W, Hq, S, E, generator=g).to(dt)
    kc = torch.randn(P, bs, Hkv, E, generator=g).to(dt)
    vc = torch.randn(P, bs, Hkv, E, generator=g).to(dt)
    c, s = cs(rng.integers(0, 70000, size=(F, W, S)), R)
    rq = O.rope_q(q, torch.from_numpy(c), torch.from_numpy(s))
    scale = 128 ** -0.5
    exp = checkers.bruteforce_paged(scale, loc, rq.float().numpy(), lens, kc.float().numpy(), vc.float().numpy(), bt)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), kind="paged", dtype=dtype, scale=scale,
                        locations=loc, queries=q.float().numpy(), cosines=c, sines=s, fragment_lengths=lens,
                        k_cache=kc.float().numpy(), v_cache=vc.float().numpy(), block_tables=bt,
                        rotated=rq.float().numpy(), expected=exp.astype(np.float32))


def varlen_case(name, dtype, F, W, T, cu_q, Hkv, bs, lens, R, seed):
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    dt = DT[dtype]
    Hq, E = 16 * Hkv, 128
    lens = np.asarray(lens, dtype=np.int32)
    maxB = int((lens.sum() + bs - 1) // bs) + 1
    P = W * maxB
    bt = rng.permutation(P).astype(np.int32).reshape(W, maxB)
    loc = rng.integers(-3, int(lens.max()) + 2, size=(F, T)).astype(np.int32)
    q = torch.randn(T, Hq, E, generator=g).to(dt)
    kc = torch.randn(P, bs, Hkv, E, generator=g).to(dt)
    vc = torch.randn(P, bs, Hkv, E, generator=g).to(dt)
    c, s = cs(rng.integers(0, 65536, size=(F, T)), R)
    c, s = np.ascontiguousarray(c[..., : R // 2]), np.ascontiguousarray(s[..., : R // 2])
    rq = O.rope_q_varlen(q, torch.from_numpy(c), torch.from_numpy(s))
    scale = 128 ** -0.5
    cu_q = np.asarray(cu_q, dtype=np.int32)
    exp = checkers.bruteforce_varlen(scale, loc, rq.float().numpy(), lens, kc.float().numpy(), vc.float().numpy(),
                                     bt, cu_q)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), kind="varlen", dtype=dtype, scale=scale,
                        locations=loc, queries=q.float().numpy(), cosines=c, sines=s, fragment_lengths=lens,
                        k_cache=kc.float().numpy(), v_cache=vc.float().numpy(), block_tables=bt,
                        cu_seqlens_q=cu_q, rotated=rq.float().numpy(), expected=exp.astype(np.float32))


def main():
    paged_case("paged_fp32_f1_s1", "fp32", F=1, W=2, S=1, Hkv=1, bs=16, lens=[45], R=64, seed=1)
    paged_case("paged_bf16_f3_s2_bs5", "bf16", F=3, W=2, S=2, Hkv=2, bs=5, lens=[9, 0, 14], R=32, seed=2)
    paged_case("paged_fp16_causal_s4", "fp16", F=1, W=2, S=4, Hkv=1, bs=8, lens=[37], R=128, seed=3,
               loc_mode="causal")
    varlen_case("varlen_fp16_f3", "fp16", F=3, W=3, T=5, cu_q=[0, 1, 3, 5], Hkv=1, bs=4, lens=[7, 3, 12], R=64,
                seed=4)
    varlen_case("varlen_bf16_malformed_cu", "bf16", F=2, W=3, T=6, cu_q=[0, 4, 2, 5], Hkv=1, bs=16,
                lens=[20, 6], R=0, seed=5)


if __name__ == "__main__":
    main()
