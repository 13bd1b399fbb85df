"""The library under HIP graph capture: a linear captured once and replayed
must give the eager call's bits on every replay.  The allocation-free linear
(phi_hip_q8_linear_noalloc) exists for such callers; the K-tiled linear with
caller scratch is captured too.  Nothing in the library records a memset or
allocates, so each replay only re-runs the captured kernels: the test replays
three times, with other eager work and a synchronisation between replays, and
clears the output before each one."""
import pytest
import torch

import phi_qlinear as Q
from phi_qlinear import synth

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.view(torch.int16)


@pytest.mark.parametrize("M,K,N", [(4352, 3072, 12288), (300, 3072, 1000)])
def test_noalloc_linear_replays_in_a_graph(dev, M, K, N):
    x = synth.activations(M, K, seed=M, device=dev)
    W = synth.int8_weight(N, K, seed=1, device=dev)
    sW = synth.weight_scale(0.002, device=dev)
    b = synth.bias(N, seed=2, device=dev)
    want = Q.q8_linear(x, W, sW, b)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    Q.q8_linear_noalloc(x, W, sW, b, C=y)  # eager first call: the scratch's address is looked up here
    torch.cuda.synchronize()
    assert torch.equal(_bits(y), _bits(want))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        Q.q8_linear_noalloc(x, W, sW, b, C=y)
    x2 = synth.activations(M, K, seed=M + 1, device=dev)
    for _ in range(3):
        y.zero_()
        other = Q.q8_linear(x2, W, sW, b)  # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(_bits(y), _bits(want))
        assert not torch.equal(_bits(other), _bits(want))


def test_k_tiled_linear_replays_in_a_graph(dev):
    M, K, N = 4352, 3072, 12288
    x = synth.activations(M, K, seed=3, device=dev)
    W = synth.int8_weight(N, K, seed=4, device=dev)
    Wk = Q.pack_k_tiled(W)
    sW = synth.weight_scale(0.002, device=dev)
    b = synth.bias(N, seed=5, device=dev)
    want = Q.q8_linear(x, W, sW, b)
    q8 = torch.empty((M * K,), dtype=torch.int8, device=dev)
    s8 = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    Q.q8_linear_kt(x, Wk, N, sW, b, q8=q8, s8=s8, C=y)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        Q.q8_linear_kt(x, Wk, N, sW, b, q8=q8, s8=s8, C=y)
    for _ in range(3):
        y.zero_()
        s8.zero_()
        Q.quant_rotate(synth.activations(64, K, seed=9, device=dev))  # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(_bits(y), _bits(want))
