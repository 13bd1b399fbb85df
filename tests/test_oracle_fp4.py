"""Pins for the oracle's fp8 and nvfp4 / mxfp4 weight decoders
(oracle.dequant_fp8_rows, oracle.dequant_fp4_rows; the reference's
dequant_fp8_row and dequant_nvfp4_row, core/host/quant.cpp:390-439).

The reference's own build cannot pin them: they call the f8 and e2m1 decoders
of core/util/media_common.cpp, which includes <windows.h>.  What pins them here:
* E2M1 from its definition (sign, two exponent bits with bias 1, one mantissa
  bit, exponent 0 subnormal), every one of the 16 codes, with the even column
  in the high nibble;
* the block-scale table's cuBLAS tiled layout, built independently with
  numpy's reshapes in the steps the layout is defined by (pad to 128 x 4
  tiles, tiles row-tile-major, each 128 x 4 tile as 32 x (4 x 4)); every
  element of a decoded weight must carry its own (row, block) scale, for row
  counts and block counts that are and are not multiples of the tile;
* fp8 codes against torch's float8_e4m3fn / float8_e5m2 conversion (a library
  routine), times the row scale;
* the product order (e2m1 * block scale) * global, checked with values whose
  two orders round differently.
"""
import numpy as np
import pytest
import torch

import oracle as O


def e2m1_definition(nib: int) -> float:
    s, e, m = nib >> 3, (nib >> 1) & 3, nib & 1
    mag = 0.5 * m if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)
    return -mag if s else mag


def to_blocked(scales: np.ndarray) -> np.ndarray:
    """The cuBLAS block-scale layout: [rows, blocks] -> [R, C] stored table."""
    rows, cols = scales.shape
    R, C = -(-rows // 128) * 128, -(-cols // 4) * 4
    pad = np.zeros((R, C), scales.dtype)
    pad[:rows, :cols] = scales
    t = pad.reshape(R // 128, 128, C // 4, 4).transpose(0, 2, 1, 3)    # tiles, row-tile-major
    t = t.reshape(-1, 4, 32, 4).transpose(0, 2, 1, 3)                  # each 128 x 4 tile as 32 x (4 x 4)
    return t.reshape(R, C)


def test_e2m1_every_code_high_nibble_first():
    codes = np.array([[(a << 4) | b for a in range(16) for b in range(16)]], np.uint8)
    out = O.dequant_fp4_rows(codes, 512)
    want = np.array([[e2m1_definition(a), e2m1_definition(b)] for a in range(16) for b in range(16)],
                    np.float32).reshape(1, 512)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))  # -0 included


@pytest.mark.parametrize("rows,k,block", [(1, 32, 16), (128, 256, 16), (200, 512, 16), (300, 1088, 32),
                                          (129, 64, 32), (256, 4096, 16)])
def test_tiled_block_scales(rows, k, block):
    """Each element carries its own (row, block) scale through the tiled table."""
    nblk = -(-k // block)
    scales = (np.arange(rows * nblk) % 251 + 1).astype(np.float32).reshape(rows, nblk)
    table = to_blocked(scales)
    codes = np.full((rows, k // 2), 0x22, np.uint8)  # every code 2: value 1.0
    out = O.dequant_fp4_rows(codes, k, table=table, table_dtype=O.F32, block=block)
    want = np.repeat(scales, block, axis=1)[:, :k]
    assert np.array_equal(out, want)
    # rows decoded from row0: the table is indexed by the weight's own row
    r0 = rows // 2
    part = O.dequant_fp4_rows(codes[r0:], k, table=table, table_dtype=O.F32, block=block, row0=r0)
    assert np.array_equal(part, want[r0:])


def test_fp8_table_and_global_scale_order():
    """An E4M3 block table in a byte container and a global scale: the decode is
    (e2m1 * s) * g, two roundings, which (e2m1 * (s * g)) would not match."""
    rng = np.random.default_rng(5)
    rows, k, block = 130, 256, 16
    nblk = k // block
    s8 = rng.integers(0x08, 0x77, size=(rows, nblk), dtype=np.uint8)  # positive finite E4M3 codes
    sf = torch.from_numpy(s8).view(torch.float8_e4m3fn).float().numpy()
    codes = rng.integers(0, 256, size=(rows, k // 2), dtype=np.uint8)
    g = np.float32(1.1)
    out = O.dequant_fp4_rows(codes, k, table=to_blocked(s8), table_dtype=O.U8_E4M3, block=block, global_scale=g)
    hi, lo = codes >> 4, codes & 15
    nib = np.stack([hi, lo], axis=2).reshape(rows, k)
    v = np.vectorize(e2m1_definition)(nib).astype(np.float32)
    want = (v * np.repeat(sf, block, axis=1)).astype(np.float32) * g
    assert np.array_equal(out, want)
    other = v * (np.repeat(sf, block, axis=1) * g).astype(np.float32)
    assert not np.array_equal(out, other)


@pytest.mark.parametrize("dtype,tdt", [(O.F8_E4M3, torch.float8_e4m3fn), (O.F8_E5M2, torch.float8_e5m2)])
def test_fp8_rows_against_torch(dtype, tdt):
    codes = np.arange(256, dtype=np.uint8).reshape(4, 64)
    if tdt == torch.float8_e4m3fn:
        codes[(codes & 0x7F) == 0x7F] = 0  # the NaN codes
    scale = np.array([1.0, 0.5, 3.0, 0.001], np.float32)
    out = O.dequant_fp8_rows(codes, dtype, scale)
    ref = torch.from_numpy(codes).view(tdt).float().numpy() * scale[:, None]
    fin = np.isfinite(ref)
    assert np.array_equal(out[fin], ref[fin]) and np.array_equal(np.isnan(out), np.isnan(ref))
    assert np.array_equal(O.dequant_fp8_rows(codes, dtype)[fin], torch.from_numpy(codes).view(tdt).float().numpy()[fin])
