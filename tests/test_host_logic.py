"""Host-side logic: synthetic operand generators and the bench contract."""
import os
import subprocess
import sys

import numpy as np
import torch

from phi_qlinear import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_activation_distribution_and_outliers():
    x = synth.activations(64, 3072, seed=0).float()
    col_amax = x.abs().amax(0)
    n_out = int((col_amax > 10).sum())
    assert n_out == 3  # 0.1 % of 3072 channels, scaled x20
    body = x[:, col_amax <= 10]
    assert abs(body.mean().item()) < 0.02 and abs(body.std().item() - 1) < 0.02
    assert torch.equal(synth.activations(64, 3072, seed=0), synth.activations(64, 3072, seed=0))


def test_weight_and_bias_generators():
    w = synth.int8_weight(256, 512, seed=1)
    assert w.dtype == torch.int8 and int(w.min()) >= -127 and int(w.max()) == 127
    b = synth.bias(4096, seed=2).float()
    assert abs(b.std().item() - 0.02) < 0.002
    assert synth.weight_scale().item() == np.float32(0.002)


def test_w4a8_parameterisation_reproduces_zero_point_form():
    """w = (code - zp) * s_g is reproduced by grid(level * s_rel) * s_ch + corr
    up to the int8-grid step (half a step of s_ch) plus fp16 rounding of s_rel."""
    import oracle as O

    N, K, g = 32, 512, 128
    codes, s_rel, sch, corr = synth.w4a8_weight(N, K, g, seed=4)
    # rebuild the generator's own draws to get s_g and zp back
    gen = torch.Generator().manual_seed(4)
    c = torch.randint(0, 16, (N, K), generator=gen, dtype=torch.int32)
    s_g = (torch.rand((N, K // g), generator=gen) * 0.009 + 0.001).to(torch.float16).float()
    zp = torch.randint(6, 10, (N, K // g), generator=gen, dtype=torch.int32)
    want = (c - torch.repeat_interleave(zp, g, 1)).float() * torch.repeat_interleave(s_g, g, 1)
    _, _, v = O.w4a8_expand(codes.numpy(), s_rel.view(torch.int16).numpy().view(np.uint16), O.F16,
                            sch.numpy(), k=K, group=g, correction=corr.numpy(), return_values=True)
    err = np.abs(v - want.numpy())
    assert err.max() <= 0.5 * sch.max().item() + 8 * 2 ** -11 * s_g.max().item() + 1e-6
    assert (s_rel.float() * sch[:, None] - s_g).abs().max() < 2e-3 * s_g.max()


def test_bench_refuses_more_than_one_gpu():
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=60)
    assert out.returncode == 2 and "one GPU" in out.stderr


def test_tile_order_division_by_multiplier():
    """The persistent GEMMs divide tile indices by loop-invariant d with the
    multiplier m = (2^32 - 1) / d + 1 (mod 2^32): q = hi32(n * m), minus one
    where q * d > n (persist_common.hpp, udiv_inv; d = 1 takes q = n).  The
    claim is exactness for every n < 2^32; checked here by brute force over
    every divisor up to 2^13 and spread-out larger ones, at the n where an
    error would first show (multiples of d and their neighbours) and across
    the range."""
    rng = np.random.default_rng(7)
    ds = list(range(1, 1 << 13)) + [int(v) for v in rng.integers(1 << 13, 1 << 31, 200)] + [(1 << 31) - 1, 1 << 31, (1 << 32) - 1]
    for d in ds:
        d = np.uint64(d)
        m = (np.uint64(0xFFFFFFFF) // d + np.uint64(1)) & np.uint64(0xFFFFFFFF)
        k = rng.integers(0, (1 << 32) // int(d) + 1, 64, dtype=np.uint64)
        n = np.concatenate([k * d, k * d + d - np.uint64(1), k * d - np.uint64(1),
                            rng.integers(0, 1 << 32, 64, dtype=np.uint64),
                            np.array([0, 1, (1 << 32) - 1], dtype=np.uint64)])
        n = n[n < np.uint64(1 << 32)]
        q = n if d == 1 else (n * m) >> np.uint64(32)
        q = np.where(q * d > n, q - np.uint64(1), q)
        assert np.array_equal(q, n // d), int(d)


def test_prologue_scale_divisions_equal_ieee_division():
    """The prologue's fast scale divisions (phi-agent_amd/csrc/qt_scale.hpp):
    rmax / qmax from the rounded 1/qmax with one fma correction, and 1 / scale
    by two Newton steps from an estimate, equal IEEE division for every
    significand and every integer qmax in [1, 127] (tests/cpp/scale_exact.c,
    checked against C's own division).  The GPU side, with v_rcp_f32 as the
    estimate, is test_gpu_quant_rotate.py::test_scale_divisions_on_device."""
    cdir = os.path.join(ROOT, "tests", "cpp")
    subprocess.run(["make", "-C", cdir, "scale_exact"], check=True, capture_output=True)
    out = subprocess.run([os.path.join(cdir, "scale_exact")], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "div_qmax_mismatches 0 rcp_mismatches 0 all_ones_mismatches 0" in out.stdout
