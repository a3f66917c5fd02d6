"""The allocation-free tiled entry point (pa_tiled_fwd_noalloc) against pa_tiled_fwd.

pa_tiled_fwd_noalloc runs the same three tiled kernels with the score workspace taken from the
library's static device array instead of a caller-allocated buffer, so its output must equal
pa_tiled_fwd's bit for bit. Two calls in a row, the second on a smaller input (the array keeps
the first call's scores; every score the second call reads it writes first), both through the
C ABI, and under HIP graph capture. Sizes past the array's limit are rejected before any launch
(tested without a device in test_api.py).
"""
from __future__ import annotations

import pytest
import torch

import cuda_attn
from cuda_attn import _native
from cuda_attn.workloads import make_qkv

pytestmark = pytest.mark.gpu

SCRATCH_SCORES = 16 << 20
CODE = {torch.float32: _native.DTYPE_F32, torch.float16: _native.DTYPE_F16}


def noalloc(q, k, v, causal):
    b, h, n, d = q.shape
    o = torch.empty_like(q)
    rc = _native.lib().pa_tiled_fwd_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), CODE[q.dtype],
                                            b * h, n, d, int(causal), torch.cuda.current_stream().cuda_stream)
    _native.check(rc, "tiled_forward_noalloc")
    return o


def workspace(q, k, v, causal):
    """pa_tiled_fwd through the C ABI with a torch-allocated score workspace."""
    b, h, n, d = q.shape
    o = torch.empty_like(q)
    s = torch.empty((b * h, n, n), dtype=torch.float32, device=q.device)
    rc = _native.lib().pa_tiled_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), s.data_ptr(),
                                    CODE[q.dtype], b * h, n, d, int(causal), torch.cuda.current_stream().cuda_stream)
    _native.check(rc, "tiled_forward")
    return o


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("causal", [False, True])
def test_noalloc_matches_workspace_entry_point(dtype, causal):
    # the first call fills most of the array; the second is smaller and reuses it
    for seed, shape in ((1, (2, 8, 1000, 64)), (2, (1, 3, 333, 80))):
        print(f"[noalloc] {shape} {dtype} causal={causal}", flush=True)
        q, k, v = make_qkv(*shape, dtype, seed=seed, device="cuda")
        got = noalloc(q, k, v, causal)
        want = workspace(q, k, v, causal)
        torch.cuda.synchronize()
        assert torch.equal(got, want), shape
        assert torch.equal(want, cuda_attn.tiled(q, k, v, causal))


def test_noalloc_accepts_the_limit():
    """A call of exactly the array's size runs and matches. (Sizes past the limit are rejected
    before any HIP call; that is tested in the CPU suite, test_api.py, where no device exists, so
    a broken size check there fails its assertion and can never launch a kernel.)"""
    q, k, v = make_qkv(1, 1, 4096, 64, torch.float16, seed=3, device="cuda")   # 4096^2 = the limit
    assert 4096 * 4096 == SCRATCH_SCORES
    assert torch.equal(noalloc(q, k, v, False), workspace(q, k, v, False))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("causal", [False, True])
def test_noalloc_under_graph_capture(dtype, causal):
    """One pa_tiled_fwd_noalloc call captured in a HIP graph (after a warm-up call outside the
    capture, which looks up the array's device address), replayed on new inputs copied into the
    captured buffers, with eager work and synchronisation between replays; every replay equals
    the eager pa_tiled_fwd bit for bit."""
    shape = (1, 3, 333, 64)
    b, h, n, d = shape
    q, k, v = make_qkv(*shape, dtype, seed=5, device="cuda")
    o = torch.empty_like(q)
    lib = _native.lib()

    def call(stream):
        rc = lib.pa_tiled_fwd_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), CODE[dtype], b * h, n,
                                      d, int(causal), stream)
        _native.check(rc, "tiled_forward_noalloc")

    call(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(torch.cuda.current_stream().cuda_stream)
    for seed in (6, 7, 8):
        print(f"[noalloc graph] {shape} {dtype} causal={causal} replay seed {seed}", flush=True)
        nq, nk, nv = make_qkv(*shape, dtype, seed=seed, device="cuda")
        q.copy_(nq)
        k.copy_(nk)
        v.copy_(nv)
        graph.replay()
        torch.cuda.synchronize()
        want = workspace(nq, nk, nv, causal)
        torch.cuda.synchronize()
        assert torch.equal(o, want), seed
