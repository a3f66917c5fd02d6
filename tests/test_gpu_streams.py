"""Stream contract of the drop-in package (reference: launches go to the caller's current stream,
asynchronously, `attn_*.cu`; here `cuda_attn` passes `torch.cuda.current_stream()` to the C ABI).

* Launches on several side streams at once give the same bits as on the default stream (no
  shared mutable state in the library).
* A launch consumes inputs produced on the same side stream just before it, with no extra sync.
* The fused entry points can be captured in a HIP graph; every replay (with new inputs copied in
  eagerly between replays) matches the eager result bit for bit.
* Eight host threads calling the library at once, each on its own stream, get the same bits and
  their own error messages.
All streams keep the default priority.
"""
from __future__ import annotations

import pytest
import torch

import cuda_attn
from cuda_attn.workloads import make_qkv

pytestmark = pytest.mark.gpu

# (entry, shape, dtype, causal, kwargs); the first GRAPH_CASES also run under graph capture (the
# unfused entries allocate their score workspace per call). The causal fused_tc cases take the
# causal persistent launch: per-XCD lists (B*H a multiple of 8), and one list over the device
# (B*H = 4).
CASES = [
    ("fused_tc", (2, 8, 512, 128), torch.bfloat16, False, {}),
    ("fused_tc", (2, 8, 1000, 64), torch.float16, False, {}),
    ("fused_tc", (2, 8, 1024, 128), torch.bfloat16, True, {}),
    ("fused_tc", (2, 8, 512, 64), torch.float16, True, {}),
    ("fused_tc", (1, 4, 2048, 128), torch.bfloat16, True, {}),
    ("fused_tuned", (1, 8, 512, 64), torch.float16, False, {"br": 128, "bc": 64, "double_buffer": True}),
    ("fused", (1, 8, 256, 64), torch.float32, False, {}),
    ("tiled", (1, 4, 256, 64), torch.float32, False, {}),
    ("tiled", (1, 4, 512, 64), torch.float16, True, {}),
]
GRAPH_CASES = 7


def case_id(c):
    return f"{c[0]}-{str(c[2])[6:]}-{c[1][1] * c[1][0]}x{c[1][2]}x{c[1][3]}" + ("-causal" if c[3] else "")


@pytest.mark.parametrize("name, shape, dtype, causal, kw", CASES, ids=[case_id(c) for c in CASES])
def test_side_streams_match_default_stream(name, shape, dtype, causal, kw):
    print(f"[streams] {name} {shape} {dtype} causal={causal}", flush=True)
    fn = getattr(cuda_attn, name)
    inputs = [make_qkv(*shape, dtype, seed=60 + i, device="cuda") for i in range(3)]
    want = [fn(q, k, v, causal, **kw) for q, k, v in inputs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in inputs]
    got = [None] * len(inputs)
    for _ in range(3):
        for i, ((q, k, v), s) in enumerate(zip(inputs, streams)):
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                got[i] = fn(q, k, v, causal, **kw)
        for s in streams:
            torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        for g, w in zip(got, want):
            assert torch.equal(g, w)


def test_launch_uses_the_current_stream():
    """Inputs written on a side stream right before the call are the ones the kernel reads."""
    q, k, v = make_qkv(2, 8, 1024, 128, torch.bfloat16, seed=71, device="cuda")
    want = cuda_attn.fused_tc(q, k, v)
    s = torch.cuda.Stream()
    for trial in range(5):
        q2 = torch.empty_like(q)
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            torch.cuda._sleep(2_000_000)          # keep the side stream busy before the copy
            q2.copy_(q)
            out = cuda_attn.fused_tc(q2, k, v)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"trial {trial}"


@pytest.mark.parametrize("name, shape, dtype, causal, kw", CASES[:GRAPH_CASES], ids=[case_id(c) for c in CASES[:GRAPH_CASES]])
def test_graph_capture_replays_match_eager(name, shape, dtype, causal, kw):
    print(f"[graph] {name} {shape} {dtype} causal={causal}", flush=True)
    fn = getattr(cuda_attn, name)
    q, k, v = (t.clone() for t in make_qkv(*shape, dtype, seed=80, device="cuda"))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):                    # warm-up outside the graph, as torch requires
        fn(q, k, v, causal, **kw)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn(q, k, v, causal, **kw)
    for replay in range(4):
        nq, nk, nv = make_qkv(*shape, dtype, seed=90 + replay, device="cuda")
        q.copy_(nq)
        k.copy_(nk)
        v.copy_(nv)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = fn(nq, nk, nv, causal, **kw)       # eager, between replays
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {replay}"


def test_host_threads_call_concurrently():
    """Eight host threads, each on its own stream, call fused_tc concurrently (ctypes releases the
    GIL in the library call) on shapes that exercise the launch caches: causal shapes whose walk is
    counted and cached, non-causal persistent and key-split shapes; between calls each thread makes
    a rejected call and reads back its own error message (per-thread). Every output equals the same
    call made alone on the default stream."""
    import threading

    from cuda_attn import _native
    shapes = [((2, 8, 1024, 128), torch.bfloat16, True), ((1, 12, 2048, 128), torch.bfloat16, True),
              ((2, 8, 512, 64), torch.float16, True), ((2, 8, 1000, 64), torch.float16, False),
              ((1, 42, 128, 64), torch.float16, False), ((2, 16, 768, 128), torch.bfloat16, False)]
    inputs = [(make_qkv(*shp, dt, seed=80 + i, device="cuda"), causal) for i, (shp, dt, causal) in enumerate(shapes)]
    want = [cuda_attn.fused_tc(q, k, v, causal) for (q, k, v), causal in inputs]
    torch.cuda.synchronize()
    failures = []

    def worker(t):
        stream = torch.cuda.Stream()
        p = 256
        try:
            for r in range(6):
                for j in range(len(inputs)):
                    i = (j + t + r) % len(inputs)
                    (q, k, v), causal = inputs[i]
                    with torch.cuda.stream(stream):
                        out = cuda_attn.fused_tc(q, k, v, causal)
                    stream.synchronize()
                    if not torch.equal(out, want[i]):
                        failures.append(f"thread {t}: case {i} differs")
                    d = 96 + 16 * (t % 2)   # 96 and 112: uncompiled head dims, rejected before any launch
                    rc = _native.lib().pa_fused_tc_fwd(p, p, p, p, _native.DTYPE_F16, _native.DTYPE_F16, 1, 64, d, 0, None)
                    msg = _native.last_error()
                    if rc != _native.ERR_UNSUPPORTED or f"(got {d})" not in msg:
                        failures.append(f"thread {t}: rc {rc}, message {msg!r}")
        except Exception as e:   # noqa: BLE001 - reported below
            failures.append(f"thread {t}: {e!r}")

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(8)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not failures, failures[:5]
