"""The committed golden fixtures (tests/golden/, written by gen_golden.py after
cross-checking against the reference's own CPU path) reproduced by the oracle
on the CPU and by the HIP path on the GPU."""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def u16(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def test_oracle_reproduces_quant_fixture():
    f = load("quant_small.npz")
    q, s = O.quantize_rows(f["x"])
    assert np.array_equal(q, f["q_rot"]) and np.array_equal(s, f["s_rot"])
    q, s = O.quantize_rows(f["x"], rotate=False)
    assert np.array_equal(q, f["q_plain"]) and np.array_equal(s, f["s_plain"])
    q, s = O.quantize_rows(f["x"], rotate=False, round_mode=O.ROUND_HALF_EVEN)
    assert np.array_equal(q, f["q_even"]) and np.array_equal(s, f["s_even"])
    # the tie row: half away from zero, and 0.5 - 2^-25 rounds to 0
    assert list(f["q_plain"][7, :8]) == [1, -1, 2, -3, 127, -127, 127, 0]


def test_oracle_reproduces_linear_fixture():
    f = load("linear_small.npz")
    y, q, s, acc = O.q8_linear(f["x_bf16"], f["w"], f["sw"], f["bias_bf16"])
    for name, v in (("y_bf16", y), ("q", q), ("s", s), ("acc", acc)):
        assert np.array_equal(v, f[name]), name


def test_oracle_reproduces_w4a8_fixture():
    f = load("w4a8_small.npz")
    q, s = O.w4a8_expand(f["codes"], f["s_rel"], O.F32, f["s_channel"], k=256, group=128,
                         correction=f["correction"])
    assert np.array_equal(q, f["q"]) and np.array_equal(s, f["s"])


def test_synth_inputs_still_match_config0_fixture():
    from phi_qlinear import synth

    meta = json.load(open(os.path.join(GOLD, "config0_digest.json")))
    assert digest(u16(synth.activations(256, 3072, seed=0))) == meta["inputs"]["x_bf16"]
    assert digest(synth.int8_weight(3072, 3072, seed=1).numpy()) == meta["inputs"]["w"]
    assert digest(u16(synth.bias(3072, seed=2))) == meta["inputs"]["bias_bf16"]


@pytest.mark.slow
def test_oracle_reproduces_config0_digests():
    from phi_qlinear import synth

    meta = json.load(open(os.path.join(GOLD, "config0_digest.json")))
    x = u16(synth.activations(256, 3072, seed=0))
    W = synth.int8_weight(3072, 3072, seed=1).numpy()
    b = u16(synth.bias(3072, seed=2))
    y, q, s, acc = O.q8_linear(x, W, np.array([0.002], np.float32), b)
    got = {"q": digest(q), "s": digest(s), "acc": digest(acc), "y_bf16": digest(y)}
    assert got == meta["outputs"]


# ---------------------------------------------------------------- on the GPU
@pytest.mark.gpu
def test_gpu_reproduces_config0_digests(dev):
    import phi_qlinear as Q
    from phi_qlinear import synth

    meta = json.load(open(os.path.join(GOLD, "config0_digest.json")))
    x = synth.activations(256, 3072, seed=0).to(dev)
    W = synth.int8_weight(3072, 3072, seed=1).to(dev)
    b = synth.bias(3072, seed=2).to(dev)
    q8 = torch.empty((256, 3072), dtype=torch.int8, device=dev)
    s8 = torch.empty((256,), dtype=torch.float32, device=dev)
    y = Q.q8_linear(x, W, synth.weight_scale(0.002, device=dev), b, q8=q8, s8=s8)
    acc = Q.i8_gemm(q8, W, None, None, out_dtype=torch.int32)
    torch.cuda.synchronize()
    got = {"q": digest(q8.cpu().numpy()), "s": digest(s8.cpu().numpy()),
           "acc": digest(acc.cpu().numpy()), "y_bf16": digest(u16(y))}
    assert got == meta["outputs"]


@pytest.mark.gpu
def test_gpu_reproduces_small_fixtures(dev):
    import phi_qlinear as Q

    f = load("quant_small.npz")
    q, s = Q.quant_rotate(torch.from_numpy(f["x"]).to(dev))
    assert np.array_equal(q.cpu().numpy(), f["q_rot"]) and np.array_equal(s.cpu().numpy(), f["s_rot"])
    q, s = Q.quant_rotate(torch.from_numpy(f["x"]).to(dev), rotate=False)
    assert np.array_equal(q.cpu().numpy(), f["q_plain"]) and np.array_equal(s.cpu().numpy(), f["s_plain"])
    q, s = Q.quant_rotate(torch.from_numpy(f["x"]).to(dev), rotate=False, round_mode=Q.ROUND_HALF_EVEN)
    assert np.array_equal(q.cpu().numpy(), f["q_even"])

    f = load("linear_small.npz")
    x = torch.from_numpy(f["x_bf16"].view(np.int16)).view(torch.bfloat16).to(dev)
    b = torch.from_numpy(f["bias_bf16"].view(np.int16)).view(torch.bfloat16).to(dev)
    q8 = torch.empty((16, 512), dtype=torch.int8, device=dev)
    s8 = torch.empty((16,), dtype=torch.float32, device=dev)
    y = Q.q8_linear(x, torch.from_numpy(f["w"]).to(dev), torch.from_numpy(f["sw"]).to(dev), b, q8=q8, s8=s8)
    assert np.array_equal(u16(y), f["y_bf16"]) and np.array_equal(q8.cpu().numpy(), f["q"])

    f = load("w4a8_small.npz")
    q, s = Q.w4a8_expand(torch.from_numpy(f["codes"]).to(dev), torch.from_numpy(f["s_rel"]).to(dev), Q.F32,
                         torch.from_numpy(f["s_channel"]).to(dev), k=256, group=128,
                         correction=torch.from_numpy(f["correction"]).to(dev))
    assert np.array_equal(q.cpu().numpy(), f["q"]) and np.array_equal(s.cpu().numpy(), f["s"])
