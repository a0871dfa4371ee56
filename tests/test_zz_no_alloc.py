"""The allocation-free head + candidates entry point
(fp8lin_linear_candidates_static) against fp8lin_linear_candidates, the same
operation with a caller workspace: bit-identical candidates on consecutive
calls (the second one smaller, so stale scratch contents from the first call
must not leak into it) and under HIP graph capture, all through the C ABI."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def with_workspace(F, x, codes, scales, offset):
    L = F.lib()
    m, k = x.shape
    n = codes.size(0)
    need = L.fp8lin_linear_candidates_workspace_bytes(m, n, k)
    ws = torch.empty(need, dtype=torch.uint8, device=x.device)
    out = torch.empty((m, 2), dtype=torch.float64, device=x.device)
    rc = L.fp8lin_linear_candidates(_p(x), _p(codes), _p(scales), scales.size(1), m, n, k, offset, _p(out),
                                    _p(ws), need, _stream())
    assert rc == 0, L.fp8lin_last_error()
    return out


def static(F, x, codes, scales, offset, out=None):
    L = F.lib()
    m, k = x.shape
    n = codes.size(0)
    if out is None:
        out = torch.empty((m, 2), dtype=torch.float64, device=x.device)
    rc = L.fp8lin_linear_candidates_static(_p(x), _p(codes), _p(scales), scales.size(1), m, n, k, offset,
                                           _p(out), _stream())
    assert rc == 0, L.fp8lin_last_error()
    return out


def test_static_candidates_match_workspace_form(fp8lin, gpu, oracle):
    F = fp8lin
    cases = [  # (M, N, K, offset): the decode head shard, an MTP row block, then smaller calls
        (1, 75968, 5120, 75968),
        (4, 75968, 5120, 0),
        (24, 31040, 4096, 0),   # 17..32 rows: the row-range kernel's two-tile candidate form
        (16, 31040, 4096, 11),  # 9..16 rows: its one-tile candidate form
        (1, 10000, 2048, 123),
        (8, 4100, 512, 7),
        (2, 257, 256, 0),
    ]
    for i, (m, n, k, offset) in enumerate(cases):
        codes, scales = F.gen_weights(n, k, seed=0, tag=30 + i, device=gpu)
        x = F.gen_activations(m, k, seed=0, tag=40 + i, device=gpu)
        got = static(F, x, codes, scales, offset)
        want = with_workspace(F, x, codes, scales, offset)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (m, n, k, offset)
        logits = F.fp8_linear(x, codes, scales, True)
        ref = oracle.vocab_candidates(logits.view(torch.int16).cpu().numpy().view(np.uint16), offset)
        assert np.array_equal(got.cpu().numpy(), ref), (m, n, k, offset)


def test_static_candidates_graph_replay(fp8lin, gpu):
    """Captured with no allocation inside the call; each replay sees the new
    activations and matches the workspace form."""
    F = fp8lin
    m, n, k = 2, 30000, 1024
    codes, scales = F.gen_weights(n, k, seed=0, tag=50, device=gpu)
    x = F.gen_activations(m, k, seed=0, tag=51, device=gpu)
    out = torch.empty((m, 2), dtype=torch.float64, device=gpu)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        static(F, x, codes, scales, 5, out)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            static(F, x, codes, scales, 5, out)
    for i in range(3):
        x.copy_(F.gen_activations(m, k, seed=1, tag=52 + i, device=gpu))
        # an eager call of another shape in between reuses the same scratch
        small = F.gen_activations(1, k, seed=2, tag=60 + i, device=gpu)
        static(F, small, codes[:1000], scales[:1000], 0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = with_workspace(F, x, codes, scales, 5)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"


FIRST_USE_UNDER_CAPTURE = r"""
import ctypes, sys
sys.path[:0] = [{root!r}, {pkg!r}]
import torch
import fp8lin                 # loading the library prepares the current device
L = fp8lin.lib()
dev = torch.device("cuda:0")
torch.cuda.set_device(dev)
m, n, k = 2, 20000, 1024
g = torch.Generator(device="cpu").manual_seed(5)
codes = torch.randint(0, 126, (n, k), generator=g, dtype=torch.uint8).to(dev)
scales = (torch.rand(n, k // 128, generator=g) * 0.01 + 0.001).to(dev)
x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(dev)
out = torch.zeros((m, 2), dtype=torch.float64, device=dev)
P = lambda t: ctypes.c_void_p(t.data_ptr())
stream = torch.cuda.Stream()
graph = torch.cuda.CUDAGraph()
torch.cuda.synchronize()
with torch.cuda.stream(stream):
    # the first fp8lin call of this process is inside the capture
    with torch.cuda.graph(graph, stream=stream):
        rc = L.fp8lin_linear_candidates_static(P(x), P(codes), P(scales), k // 128, m, n, k, 0, P(out),
                                               ctypes.c_void_p(stream.cuda_stream))
assert rc == 0, L.fp8lin_last_error()
for i in range(3):
    x.copy_(torch.randn(m, k, generator=g).to(torch.bfloat16))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    want = fp8lin.linear_candidates(x, codes, scales, 0)
    torch.cuda.synchronize()
    assert torch.equal(out, want), ("replay", i)
print("first use under capture: ok", flush=True)
"""


def test_static_candidates_first_call_under_capture(fp8lin, gpu):
    """In a fresh process whose first library call is captured into a graph:
    the device preparation that loading the library runs keeps the one-time
    runtime queries out of the capture, and the replays match the workspace
    form."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    script = FIRST_USE_UNDER_CAPTURE.format(root=root, pkg=os.path.join(root, "a100-vision-infer_amd"))
    r = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "first use under capture: ok" in r.stdout
