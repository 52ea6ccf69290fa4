"""The single-launch path for short contiguous views (dv_small.hip: rotation,
attention and chunk merge in one kernel; dvattn_sdpa / dvattn_fused in fp32,
fp16 and bf16).

Every call here runs with the library option small_path = require
(dvattn_set_option), which makes a call the single launch cannot take fail
instead of falling back, so each case is known to exercise it.  Outputs are checked against the CPU oracle (tolerances 1e-5
fp32, 1e-3 fp16, 2e-2 bf16, as in test_gpu_parity) and against the general
path (small_path = off) on the same inputs; rotated queries bit-exactly
against the oracle's rotation (fp32 math rounded to the storage type).
A call whose rows have more than one chunk (one long view, or several
views) takes the single launch only up to 160 (fp32) or 96 (16-bit)
workgroups (rows x KV heads x chunks): past that the call must be refused
under require; only a single-chunk call (one view of at most 64 keys) has no
such limit.  The chunk merge
is exercised from one chunk (direct output) to the 64-chunk maximum, with
empty views, views past every location, batch-1 views, fragment lengths
below the tensor length and several query tokens per sequence.  The arrival
counters live in the caller's workspace: calls on a workspace full of
arbitrary bytes, and replays of a captured graph (the same counter tag on
every replay), must give the eager result.
"""
import numpy as np
import pytest
import torch

from oracle import dvattn_oracle as O
from test_gpu_parity import close, dv, hf_cs  # noqa: F401 (dv: fixture)

pytestmark = pytest.mark.gpu


@pytest.fixture
def require_small():
    from dvattention_amd import capi
    capi.set_option("small_path", capi.SMALL_PATH["require"])
    yield
    capi.set_option("small_path", capi.SMALL_PATH["auto"])


DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def max_merged(dtype):
    """Most workgroups of a single launch whose rows have several chunks."""
    return 160 if dtype == torch.float32 else 96


def make_case(F, W, S, Hkv, Ls, batch, fls=None, seed=0, loc_range=None, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    keys, vals = [], []
    for L, B in zip(Ls, batch):
        shp = (Hkv, L, 128) if B == 0 else (B, Hkv, L, 128)
        keys.append(torch.randn(shp, generator=g).to(dtype))
        vals.append(torch.randn(shp, generator=g).to(dtype))
    lo, hi = loc_range if loc_range else (-2, max(Ls) + 2)
    loc = torch.from_numpy(rng.integers(lo, hi, size=(F, W, S)).astype(np.int32))
    fl = torch.tensor(fls if fls is not None else Ls, dtype=torch.int32)
    q = torch.randn(W, 16 * Hkv, S, 128, generator=g).to(dtype)
    c, s = hf_cs(rng.integers(0, 9000, size=(F, W, S)), 64)
    return dict(keys=keys, vals=vals, loc=loc, fl=fl, q=q, c=c, s=s)


def run_fused(dv, d, gpu, scale=0.1):
    F, (W, Hq, S, _) = d["loc"].shape[0], d["q"].shape
    dt = d["q"].dtype
    rq = torch.empty(F, W, Hq, S, 128, dtype=dt, device=gpu)
    out = torch.empty(W, Hq, S, 128, dtype=dt, device=gpu)
    dv.dvattn_fused(d["q"].to(gpu), d["loc"].to(gpu), [k.to(gpu) for k in d["keys"]],
                    [v.to(gpu) for v in d["vals"]], scale, d["fl"].to(gpu), d["c"].to(gpu), d["s"].to(gpu),
                    rotated_queries=rq, out=out)
    return out, rq


CASES = [
    # F, W, S, Hkv, Ls, batch, fragment_lengths
    (1, 1, 1, 1, [512], [1], None),                    # the benchmark's configuration 1 (8 chunks)
    (1, 1, 1, 1, [64], [1], None),                     # one chunk: written straight to the output
    (1, 2, 1, 1, [1], [2], None),                      # one key
    (3, 2, 2, 2, [16, 0, 90], [0, 2, 2], None),        # an empty view, a 3-D (batch-1) fragment
    (16, 2, 1, 1, [5 + 3 * i for i in range(16)], [2] * 16, None),   # 16 views: the most in kernel arguments
    (1, 1, 1, 1, [4096], [1], None),                   # 64 chunks: the most per row
    (1, 2, 1, 4, [1000], [2], None),                   # 16 chunks x 8 rows: 128 workgroups (16-bit: refused)
    (1, 32, 1, 8, [64], [32], None),                   # one chunk per row, 256 rows: no merge, no limit
    (2, 2, 4, 1, [700, 33], [2, 1], None),             # four query tokens per sequence
    (2, 2, 3, 2, [300, 150], [2, 0], None),            # three query tokens per sequence, 8 chunks
    (3, 2, 3, 2, [300, 90, 64], [2, 2, 2], [211, 90, 1]),   # fragment_lengths below the tensor lengths
]


def chunks_of(Ls):
    return sum(max(1, -(-L // 64)) for L in Ls)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("F,W,S,Hkv,Ls,batch,fls", CASES)
def test_small_vs_oracle_and_general_path(dv, gpu, require_small, dtype, F, W, S, Hkv, Ls, batch,
                                          fls):
    d = make_case(F, W, S, Hkv, Ls, batch, fls, seed=F * 7 + W + S, dtype=dtype)
    chunks = chunks_of(Ls)
    if chunks > 1 and W * S * Hkv * chunks > max_merged(dtype):
        with pytest.raises(RuntimeError):  # the general path's case: refused under require
            run_fused(dv, d, gpu)
        return
    rq_ref = O.rope_q(d["q"], d["c"], d["s"])
    ref = O.contig_sdpa(0.1, d["loc"], rq_ref, d["fl"], d["keys"], d["vals"])
    out, rq = run_fused(dv, d, gpu)
    assert torch.equal(rq.cpu(), rq_ref)
    close(out, ref, dtype, "single launch, dvattn_fused")
    gk = [k.to(gpu) for k in d["keys"]]
    gv = [v.to(gpu) for v in d["vals"]]
    pre = dv.dvattn_sdpa(rq_ref.to(gpu), d["loc"].to(gpu), gk, gv, 0.1, d["fl"].to(gpu))
    assert torch.equal(pre, out)  # same chunks, same merge order
    from dvattention_amd import capi
    capi.set_option("small_path", capi.SMALL_PATH["off"])
    gen, rq2 = run_fused(dv, d, gpu)
    assert torch.equal(rq2, rq)
    close(gen, ref, dtype, "general path")
    if dtype == torch.float32:
        assert (gen - out).abs().max().item() <= 1e-5


@pytest.mark.parametrize("dtype", DTYPES)
def test_small_locations_hide_everything(dv, gpu, require_small, dtype):
    # every location negative: no visible key anywhere, zeros out
    d = make_case(2, 2, 1, 1, [200, 40], [2, 2], seed=5, loc_range=(-5, 0), dtype=dtype)
    out, _ = run_fused(dv, d, gpu)
    assert torch.equal(out.cpu(), torch.zeros_like(out.cpu()))


@pytest.mark.parametrize("shape", [
    (1, 1, 1, 1, [4097], [1]),    # 65 chunks, one more than a row takes
    (1, 4, 1, 8, [512], [4]),     # 32 rows x 8 chunks: 256 workgroups
])
def test_small_refuses_what_it_cannot_take(dv, gpu, require_small, shape):
    d = make_case(*shape, seed=2)
    with pytest.raises(RuntimeError):
        run_fused(dv, d, gpu)


@pytest.mark.parametrize("dtype", DTYPES)
def test_small_on_a_dirty_workspace(gpu, require_small, dtype):
    # the arrival counters sit in the workspace: bytes left there (all ones,
    # random words) must not change the result
    from dvattention_amd import capi
    d = make_case(2, 2, 1, 2, [700, 130], [2, 1], seed=11, dtype=dtype)
    args = lambda out, rq, ws: capi.fused(out, rq, 0.1, d["loc"].to(gpu), d["q"].to(gpu), d["fl"].to(gpu),
                                          [k.to(gpu) for k in d["keys"]], [v.to(gpu) for v in d["vals"]],
                                          d["c"].to(gpu), d["s"].to(gpu), workspace=ws)
    shape = (2, 32, 1, 128)
    ref_out, ref_rq = torch.empty(shape, dtype=dtype, device=gpu), torch.empty(2, 2, 32, 1, 128, dtype=dtype,
                                                                               device=gpu)
    args(ref_out, ref_rq, None)
    torch.cuda.synchronize()
    nbytes = 64 << 20
    for fill in ("ones", "random"):
        ws = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
        if fill == "ones":
            ws.fill_(255)
        else:
            ws.copy_(torch.randint(0, 256, (nbytes,), dtype=torch.uint8))
        for _ in range(3):  # the same workspace again: counters reset by the last arrival
            out = torch.empty(shape, dtype=dtype, device=gpu)
            rq = torch.empty(2, 2, 32, 1, 128, dtype=dtype, device=gpu)
            args(out, rq, ws)
            torch.cuda.synchronize()
            assert torch.equal(out, ref_out), fill
            assert torch.equal(rq, ref_rq)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_small_graph_replays(dv, gpu, require_small, dtype):
    # a captured call replays with the same counter tag: each replay must start
    # from counters the previous one left at zero
    d = make_case(1, 2, 1, 1, [512], [2], seed=3, dtype=dtype)
    e = make_case(1, 2, 1, 1, [512], [2], seed=4, dtype=dtype)
    q, loc, fl, c, s = (d[k].to(gpu) for k in ("q", "loc", "fl", "c", "s"))
    gk, gv = [k.to(gpu) for k in d["keys"]], [v.to(gpu) for v in d["vals"]]
    rq = torch.empty(1, 2, 16, 1, 128, dtype=dtype, device=gpu)
    out = torch.empty(2, 16, 1, 128, dtype=dtype, device=gpu)

    def call():
        dv.dvattn_fused(q, loc, gk, gv, 0.1, fl, c, s, rotated_queries=rq, out=out)

    call()
    torch.cuda.synchronize()
    eager = out.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        call()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    run_fused(dv, e, gpu)  # eager work between capture and replays
    for i in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        run_fused(dv, e, gpu)
        torch.cuda.synchronize()
    del graph


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_many_views_graph_replays(dv, gpu, dtype):
    # more views than kernel arguments hold (20 > 16) take the general path,
    # whose view table is written on the device by a launch that carries the
    # descriptors: a captured call must replay correctly after the host-side
    # arrays of the capturing call are gone
    F = 20
    d = make_case(F, 2, 1, 1, [5 + 7 * i for i in range(F)], [2] * F, seed=21, dtype=dtype)
    e = make_case(F, 2, 1, 1, [9 + 3 * i for i in range(F)], [2] * F, seed=22, dtype=dtype)
    q, loc, fl, c, s = (d[k].to(gpu) for k in ("q", "loc", "fl", "c", "s"))
    gk, gv = [k.to(gpu) for k in d["keys"]], [v.to(gpu) for v in d["vals"]]
    rq = torch.empty(F, 2, 16, 1, 128, dtype=dtype, device=gpu)
    out = torch.empty(2, 16, 1, 128, dtype=dtype, device=gpu)

    def call():
        dv.dvattn_fused(q, loc, gk, gv, 0.1, fl, c, s, rotated_queries=rq, out=out)

    call()
    torch.cuda.synchronize()
    eager = out.clone()
    ref = O.fused(0.1, d["loc"], d["q"], d["fl"], d["keys"], d["vals"], d["c"], d["s"])[0]
    close(eager, ref, dtype, "20 views eager")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        call()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for i in range(4):
        run_fused(dv, e, gpu)  # eager calls of another 20-view shape between replays
        torch.cuda.synchronize()
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
    del graph
