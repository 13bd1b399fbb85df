"""The allocation-free W8A8 linear (phi_hip_q8_linear_noalloc): its q8/s8
scratch is the library's static device array.  Through the C ABI, its output
must equal phi_hip_q8_linear's (caller scratch) bit for bit, on two calls in a
row, the second smaller than the first (the array keeps the first call's
contents), and a call past the array's size must be refused before any launch."""
import ctypes

import numpy as np
import pytest
import torch

import phi_qlinear as Q
from phi_qlinear import synth


def u16(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.gpu
def test_noalloc_matches_caller_scratch(dev, orc):
    cases = [(300, 3072, 1000, torch.bfloat16, True), (64, 1024, 512, torch.float32, False)]
    for i, (M, K, N, xdt, with_bias) in enumerate(cases):
        x = synth.activations(M, K, seed=40 + i, dtype=xdt).to(dev)
        W = synth.int8_weight(N, K, seed=50 + i).to(dev)
        sW = (torch.rand(N) * 0.01 + 0.001).to(dev) if i else synth.weight_scale(0.002, device=dev)
        b = synth.bias(N, seed=60 + i, device=dev) if with_bias else None
        y0 = Q.q8_linear_noalloc(x, W, sW, b)
        q8 = torch.empty((M, K), dtype=torch.int8, device=dev)
        s8 = torch.empty((M,), dtype=torch.float32, device=dev)
        y1 = Q.q8_linear(x, W, sW, b, q8=q8, s8=s8)
        torch.cuda.synchronize()
        assert torch.equal(y0.view(torch.int16), y1.view(torch.int16)), f"call {i}: outputs differ"
        xin = u16(x) if xdt == torch.bfloat16 else x.cpu().numpy()
        yo, qo, so, _ = orc.q8_linear(xin, W.cpu().numpy(), sW.cpu().numpy(), None if b is None else u16(b))
        assert np.array_equal(u16(y0), yo), f"call {i}: differs from the oracle"


@pytest.mark.gpu
def test_noalloc_refuses_past_the_array(dev):
    lib = Q.load()
    cap = lib.phi_hip_noalloc_scratch_bytes()
    K = 4096
    M = cap // K + 1  # q8 alone is past the array
    fake = ctypes.c_void_p(0x10000)
    rc = lib.phi_hip_q8_linear_noalloc(None, fake, Q.BF16, K, M, K, fake, K, fake, 1, None, Q.F32, 64, fake,
                                       Q.BF16, 64, 0)
    assert rc == 4 and "static scratch" in Q.last_error()
