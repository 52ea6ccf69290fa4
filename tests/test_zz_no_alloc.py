"""dvattn_paged_sdpa_noalloc (static per-GPU scratch, nothing allocated) against
dvattn_paged_sdpa with a caller workspace, through the C ABI: two calls in a
row, the second with a smaller input, bit-identical to the workspace entry
point and within the parity tolerance of the oracle; the decode (S = 1) and
the multi-query (S >= 2) kernels; a shape whose scratch need exceeds the
static array rejected before anything runs; and, for the callers the entry
point is for, repeated calls that leave the device's free memory unchanged
and a captured graph whose replays (with eager calls on the same scratch
between them) equal the eager result.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import dvattn_oracle as O
from test_gpu_parity import close, rand_paged, to

pytestmark = pytest.mark.gpu


def both(d, scale, gpu):
    from dvattention_amd import capi
    g = to(d, gpu)
    W, Hq, S, E = g["queries"].shape
    a = torch.full((W, Hq, S, E), float("nan"), dtype=g["queries"].dtype, device=gpu)
    b = torch.full_like(a, float("nan"))
    args = (scale, g["locations"], g["queries"], g["cosines"], g["sines"], g["fragment_lengths"], g["k_cache"],
            g["v_cache"], g["block_tables"])
    capi.paged_sdpa_noalloc(a, *args)
    capi.paged_sdpa(b, *args)
    torch.cuda.synchronize()
    return a, b


@pytest.mark.parametrize("first,second", [
    # (F, W, S, Hkv, bs, lens, R, dtype): decode kernel, then a smaller call
    ((2, 6, 1, 8, 16, [900, 1400], 128, torch.bfloat16), (1, 2, 1, 2, 16, [100], 64, torch.bfloat16)),
    # multi-query kernel, then a smaller decode call of another dtype
    ((1, 4, 16, 8, 16, [2100], 32, torch.bfloat16), (2, 3, 1, 1, 8, [60, 33], 64, torch.float16)),
    # fp32 decode, then a smaller multi-query call
    ((1, 3, 1, 4, 16, [700], 64, torch.float32), (1, 2, 4, 1, 16, [150], 32, torch.float16)),
])
def test_noalloc_matches_workspace_entry(gpu, first, second):
    for i, (F, W, S, Hkv, bs, lens, R, dt) in enumerate((first, second)):
        print(f"noalloc call {i}: F={F} W={W} S={S} Hkv={Hkv} bs={bs} lens={lens} R={R} {dt}", flush=True)
        d = rand_paged(F, W, S, Hkv, bs, lens, R, dt, seed=100 + i)
        a, b = both(d, 0.09, gpu)
        assert torch.equal(a, b), f"call {i}: no-alloc output differs from the workspace entry point"
        close(a, O.paged_sdpa(0.09, **d), dt, f"noalloc call {i}")


def test_noalloc_rejects_oversize(gpu):
    from dvattention_amd import capi
    d = to(rand_paged(1, 2, 1, 8, 16, [64], 128, torch.bfloat16, seed=7), gpu)
    out = torch.zeros(2, 128, 1, 128, dtype=torch.bfloat16, device=gpu)
    # a shape claiming 4096 sequences: its workspace exceeds the static scratch,
    # so the call returns before it reads any pointer
    s = capi.paged_shape(d["queries"], d["locations"], d["cosines"], d["k_cache"], d["v_cache"], d["block_tables"])
    s.W = 4096
    need = capi.lib().dvattn_paged_sdpa_workspace_size(capi.DVATTN_BF16, ctypes.byref(s), 0)
    assert need > capi.NOALLOC_SCRATCH_BYTES
    with pytest.raises(capi.DvattnError) as ei:
        capi.paged_sdpa_noalloc(out, 0.1, d["locations"], d["queries"], d["cosines"], d["sines"],
                                d["fragment_lengths"], d["k_cache"], d["v_cache"], d["block_tables"], shape=s)
    assert ei.value.status == 3 and "scratch" in str(ei.value)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0


@pytest.mark.parametrize("S", [1, 16])
def test_noalloc_allocates_nothing_and_replays(gpu, S):
    from dvattention_amd import capi
    print(f"noalloc graph: S={S}", flush=True)
    d = rand_paged(2, 6, S, 8, 16, [900, 1400], 128, torch.bfloat16, seed=31)
    e = to(rand_paged(1, 3, 1, 4, 16, [500], 64, torch.bfloat16, seed=32), gpu)
    g = to(d, gpu)
    out = torch.empty(6, 128, S, 128, dtype=torch.bfloat16, device=gpu)
    other = torch.empty(3, 64, 1, 128, dtype=torch.bfloat16, device=gpu)
    args = (0.09, g["locations"], g["queries"], g["cosines"], g["sines"], g["fragment_lengths"], g["k_cache"],
            g["v_cache"], g["block_tables"])
    eargs = (0.07, e["locations"], e["queries"], e["cosines"], e["sines"], e["fragment_lengths"], e["k_cache"],
             e["v_cache"], e["block_tables"])
    capi.paged_sdpa_noalloc(out, *args)
    torch.cuda.synchronize()
    eager = out.clone()
    close(eager, O.paged_sdpa(0.09, **d), torch.bfloat16, "noalloc eager")
    # nothing allocated: the device's free memory is the same after more calls
    free0 = torch.cuda.mem_get_info(gpu)[0]
    for _ in range(3):
        capi.paged_sdpa_noalloc(out, *args)
        capi.paged_sdpa_noalloc(other, *eargs)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(gpu)[0] == free0
    # captured, then replayed with eager calls on the shared scratch between
    stream = torch.cuda.Stream(gpu)
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        capi.paged_sdpa_noalloc(out, *args)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        capi.paged_sdpa_noalloc(out, *args)
    eref = None
    for i in range(4):
        capi.paged_sdpa_noalloc(other, *eargs)
        torch.cuda.synchronize()
        if eref is None:
            eref = other.clone()
        assert torch.equal(other, eref), f"eager call {i} between replays"
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
    del graph
