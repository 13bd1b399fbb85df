"""Seeded synthetic operands with the distributions of the benchmark configs.

* activations: N(0, 1) with 0.1 % of the K channels scaled x20 (outlier
  channels), stored as bf16;
* int8 weights: uniform integers in [-127, 127];
* per-tensor weight scale 0.002; bias N(0, 0.02) as bf16;
* W4A8 weights: codes U{0..15}, per-group (group 128) fp16 scale U(0.001, 0.01)
  and zero point U{6..9}, expressed in the reference's grouped parameterisation
  (level = code - 8, s_rel fp16, s_channel fp32, additive correction plane).

The same seed gives the same tensors on every machine: generation runs on the
CPU generator for small shapes (tests) and on the device generator for the
large benchmark shapes.
"""
from __future__ import annotations

import torch


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def activations(M: int, K: int, seed: int = 0, device="cpu", outlier_frac: float = 0.001,
                outlier_scale: float = 20.0, dtype=torch.bfloat16) -> torch.Tensor:
    g = _gen(seed, device)
    x = torch.randn((M, K), generator=g, device=device, dtype=torch.float32)
    n_out = max(1, int(round(K * outlier_frac)))
    cols = torch.randperm(K, generator=g, device=device)[:n_out]
    x[:, cols] *= outlier_scale
    return x.to(dtype)


def int8_weight(N: int, K: int, seed: int = 1, device="cpu") -> torch.Tensor:
    g = _gen(seed, device)
    return torch.randint(-127, 128, (N, K), generator=g, device=device, dtype=torch.int8)


def weight_scale(value: float = 0.002, device="cpu") -> torch.Tensor:
    return torch.full((1,), value, dtype=torch.float32, device=device)


def bias(N: int, seed: int = 2, device="cpu") -> torch.Tensor:
    g = _gen(seed, device)
    return (torch.randn((N,), generator=g, device=device) * 0.02).to(torch.bfloat16)


def w4a8_weight(N: int, K: int, group: int = 128, seed: int = 3, device="cpu"):
    """(codes u8 [N, K/2], s_rel f16 [N, K/group], s_channel f32 [N], correction
    f32 [K/group, N]) for w[n,k] = (code - zp_g) * s_g.

    s_channel[n] = max_g(s_g * 9) / 127 and s_rel = fp16(s_g / s_channel), so
    level * s_rel lands inside the +-127 int8 grid; the zero point enters through
    correction[g][n] = (8 - zp_g) * s_g (core/host/st.cpp:447-491 applies it).
    """
    g = _gen(seed, device)
    groups = K // group
    codes = torch.randint(0, 16, (N, K), generator=g, device=device, dtype=torch.int32)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).to(torch.uint8)
    s_g = (torch.rand((N, groups), generator=g, device=device) * 0.009 + 0.001).to(torch.float16)
    zp = torch.randint(6, 10, (N, groups), generator=g, device=device, dtype=torch.int32)
    s_g32 = s_g.float()
    s_channel = (s_g32 * 9.0).amax(dim=1) / 127.0
    s_rel = (s_g32 / s_channel[:, None]).to(torch.float16)
    correction = ((8 - zp).float() * s_g32).t().contiguous()
    return packed.contiguous(), s_rel.contiguous(), s_channel.contiguous(), correction
