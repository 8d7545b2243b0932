"""The allocation-free entry intent_q4k_projection_noalloc against intent_q4k_projection
(caller-provided record buffer), through the C ABI: identical outputs, on two calls in
a row, the second smaller, covering the path that reads the records back (G > 64) and
the fused one (G <= 64). Also the limit check."""
import numpy as np
import pytest
import torch

from intent_amd import _native, errors, inputs

pytestmark = pytest.mark.gpu


def _reference(w, x, N, G):
    rec = torch.empty(G * 292, dtype=torch.uint8, device="cuda")
    y = torch.empty(N, dtype=torch.float32, device="cuda")
    _native.call("intent_q4k_projection", w.data_ptr(), N, G, G * 144, x.data_ptr(), 256, rec.data_ptr(),
                 y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    return y


def _noalloc(w, x, N, G):
    y = torch.full((N,), float("nan"), dtype=torch.float32, device="cuda")
    _native.call("intent_q4k_projection_noalloc", w.data_ptr(), N, G, G * 144, x.data_ptr(), 256, y.data_ptr(),
                 torch.cuda.current_stream().cuda_stream)
    return y


@pytest.mark.parametrize("first,second", [((1000, 32768), (333, 20480)), ((64, 262144), (4096, 4096)),
                                          ((1000, 8192), (333, 2048))])
def test_noalloc_matches_workspace_entry(gpu, first, second):
    for seed, (N, K) in enumerate((first, second)):
        d = inputs.kquant_projection(seed + 7, N=N, K=K)
        w = torch.from_numpy(d["w"]).cuda()
        x = torch.from_numpy(d["x"]).cuda()
        G = K // 256
        got = _noalloc(w, x, N, G)
        ref = _reference(w, x, N, G)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), ref.view(torch.int32)), (N, K)


def test_noalloc_rejects_oversize(gpu):
    status = _native.library().intent_q4k_projection_noalloc(0x1000, 4, 1025, 1025 * 144, 0x1000, 256, 0x1000,
                                                             torch.cuda.current_stream().cuda_stream)
    assert status == errors.INTENT_ERR_UNSUPPORTED
    assert "allocation-free limit" in _native.last_error()


@pytest.mark.parametrize("N,K", [(1000, 8192), (333, 32768)])
def test_noalloc_under_graph_capture(gpu, N, K):
    """The use the entry exists for: after one eager call on the device it is
    captured in a HIP graph (nothing allocated inside the capture) and replayed,
    with eager work and synchronisations between replays; every replay equals
    the workspace entry."""
    d = inputs.kquant_projection(11, N=N, K=K)
    w = torch.from_numpy(d["w"]).cuda()
    x = torch.from_numpy(d["x"]).cuda()
    G = K // 256
    ref = _reference(w, x, N, G)
    y = torch.full((N,), float("nan"), dtype=torch.float32, device="cuda")
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        _native.call("intent_q4k_projection_noalloc", w.data_ptr(), N, G, G * 144, x.data_ptr(), 256, y.data_ptr(),
                     stream.cuda_stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        _native.call("intent_q4k_projection_noalloc", w.data_ptr(), N, G, G * 144, x.data_ptr(), 256, y.data_ptr(),
                     stream.cuda_stream)
    for rep in range(3):
        y.fill_(float("nan"))
        _reference(w, x, N // 2, G)  # eager work on the same entry family between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), ref.view(torch.int32)), rep
