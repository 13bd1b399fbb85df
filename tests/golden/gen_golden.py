"""Writes the golden fixtures under tests/golden/ from the oracle.

Each fixture is data only: seeded inputs and the expected outputs.  Before a
fixture is written, every output the reference's own CPU path can produce
(oracle/_ref, core/host/quant.cpp compiled from its sources) is checked
against it; the script refuses to write when that build is missing.

    python tests/golden/gen_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "phi-agent_amd")]

import torch  # noqa: E402

import oracle as O  # noqa: E402
from phi_qlinear import synth  # noqa: E402


def u16(t):
    return t.view(torch.int16).numpy().view(np.uint16)


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    if not O.ref_available():
        sys.exit("gen_golden: oracle/_ref/phiref is missing (build oracle/ with the reference mounted)")

    # 1. rotate + quantise, fp32 input with outliers, crafted ties in the last row
    rng = np.random.default_rng(20240912)
    x = rng.standard_normal((8, 512)).astype(np.float32)
    x[:, rng.choice(512, 6, replace=False)] *= 20
    x[7] = 0
    x[7, :8] = [0.5, -0.5, 1.5, -2.5, 126.5, -126.5, 127.0, 0.49999997]
    q_rot, s_rot = O.quantize_rows(x)
    q_ref, s_ref = O.ref_quantize(x)
    assert np.array_equal(q_rot, q_ref) and np.array_equal(s_rot.view(np.uint32), s_ref.view(np.uint32))
    q_plain, s_plain = O.quantize_rows(x, rotate=False)
    qp_ref, sp_ref = O.ref_quantize(x, rotate=False)
    assert np.array_equal(q_plain, qp_ref) and np.array_equal(s_plain.view(np.uint32), sp_ref.view(np.uint32))
    q_even, s_even = O.quantize_rows(x, rotate=False, round_mode=O.ROUND_HALF_EVEN)
    np.savez_compressed(os.path.join(HERE, "quant_small.npz"), x=x, q_rot=q_rot, s_rot=s_rot,
                        q_plain=q_plain, s_plain=s_plain, q_even=q_even, s_even=s_even)

    # 2. a small W8A8 linear, bf16 activations and bias, per-tensor weight scale
    xb = synth.activations(16, 512, seed=7)
    W = synth.int8_weight(64, 512, seed=8).numpy()
    sW = np.array([0.002], np.float32)
    b = synth.bias(64, seed=9)
    y, q, s, acc = O.q8_linear(u16(xb), W, sW, u16(b))
    qr, sr = O.ref_quantize(O.bf16_to_f32(u16(xb)))
    assert np.array_equal(q, qr) and np.array_equal(s.view(np.uint32), sr.view(np.uint32))
    yf_ref = O.ref_gemm(q, s, W, np.full(64, 0.002, np.float32))
    assert np.array_equal(O.epilogue(acc, s, sW, out="f32").view(np.uint32), yf_ref.view(np.uint32))
    np.savez_compressed(os.path.join(HERE, "linear_small.npz"), x_bf16=u16(xb), w=W, sw=sW,
                        bias_bf16=u16(b), q=q, s=s, acc=acc, y_bf16=y)

    # 3. grouped 4-bit weight with codebook-free levels, fp32 relative scales
    #    (the form the reference build decodes) and a correction plane
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 256, (16, 128), dtype=np.uint8)
    s_rel = rng.uniform(0.25, 14, (16, 2)).astype(np.float32)
    sch = rng.uniform(1e-3, 1e-2, 16).astype(np.float32)
    corr = (rng.standard_normal((2, 16)) * 1e-3).astype(np.float32)
    wq, ws, wv = O.w4a8_expand(codes, s_rel, O.F32, sch, k=256, group=128, correction=corr,
                               return_values=True)
    vr = O.ref_grouped_decode(codes, s_rel, sch, k=256, group=128, correction=corr)
    assert np.array_equal(wv.view(np.uint32), vr.view(np.uint32))
    qr, sr = O.ref_quantize(vr, rotate=False)
    assert np.array_equal(wq, qr) and np.array_equal(ws.view(np.uint32), sr.view(np.uint32))
    np.savez_compressed(os.path.join(HERE, "w4a8_small.npz"), codes=codes, s_rel=s_rel, s_channel=sch,
                        correction=corr, q=wq, s=ws)

    # 4. config 0 at full size: digests of every output (inputs are the seeded
    #    synth tensors: activations seed 0, weight seed 1, bias seed 2)
    x0 = synth.activations(256, 3072, seed=0)
    W0 = synth.int8_weight(3072, 3072, seed=1).numpy()
    b0 = synth.bias(3072, seed=2)
    y0, q0, s0, acc0 = O.q8_linear(u16(x0), W0, np.array([0.002], np.float32), u16(b0))
    qr, sr = O.ref_quantize(O.bf16_to_f32(u16(x0)))
    assert np.array_equal(q0, qr) and np.array_equal(s0.view(np.uint32), sr.view(np.uint32))
    rows = np.arange(0, 256, 51)
    yr = O.ref_gemm(q0[rows], s0[rows], W0, np.full(3072, 0.002, np.float32))
    assert np.array_equal(O.epilogue(acc0[rows], s0[rows], np.array([0.002], np.float32), out="f32")
                          .view(np.uint32), yr.view(np.uint32))
    meta = {"config": "BASELINE.json configs[0]: M=256, K=3072, N=3072, bf16 activations seed 0 "
                      "(0.1% outlier channels x20), int8 weight seed 1, scale 0.002, bf16 bias seed 2",
            "inputs": {"x_bf16": digest(u16(x0)), "w": digest(W0), "bias_bf16": digest(u16(b0))},
            "outputs": {"q": digest(q0), "s": digest(s0), "acc": digest(acc0), "y_bf16": digest(y0)},
            "y_bf16_first_row_head": [int(v) for v in y0[0, :16]]}
    with open(os.path.join(HERE, "config0_digest.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print("golden fixtures written")


if __name__ == "__main__":
    main()
