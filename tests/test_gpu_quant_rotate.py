"""GPU parity: rotate + per-token quantise (phi_hip_quant_rotate) vs the oracle.

Bar: int8 codes and fp32 scales bit-exact (reference core/host/quant.cpp:109-169),
for finite and non-finite rows alike."""
import os

import numpy as np
import pytest
import torch

import phi_qlinear as Q
from phi_qlinear import synth

pytestmark = pytest.mark.gpu


def bits_u16(t: torch.Tensor) -> np.ndarray:
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def run(dev, orc, x, **kw):
    q, s = Q.quant_rotate(x.to(dev), **kw)
    torch.cuda.synchronize()
    xin = bits_u16(x) if x.dtype == torch.bfloat16 else x.numpy()
    rot = kw.get("rotate", True)
    qo, so = orc.quantize_rows(xin, rotate=rot, qmax=kw.get("qmax", 127.0),
                               round_mode=kw.get("round_mode", 0))
    return q.cpu().numpy(), s.cpu().numpy(), qo, so


@pytest.mark.parametrize("M,K", [(1, 256), (3, 768), (256, 3072), (17, 5120), (8, 12288),
                                 (2, 24576), (65, 1024)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rotate_quant_bit_exact(dev, orc, M, K, dtype):
    x = synth.activations(M, K, seed=M * 131 + K, dtype=dtype)
    q, s, qo, so = run(dev, orc, x)
    assert np.array_equal(q, qo), f"{(q != qo).sum()} code mismatches"
    assert np.array_equal(s.view(np.uint32), so.view(np.uint32))


@pytest.mark.parametrize("G", list(range(1, 50)))
def test_every_group_count(dev, orc, G):
    """Each 256-group count up to 49 (the register-resident kernel's rounds of
    four groups, its partial last round, and the first count past it), with a
    row count that leaves a partial block of rows."""
    M, K = 5, 256 * G
    dtype = torch.float32 if G % 7 == 3 else torch.bfloat16
    x = synth.activations(M, K, seed=G, dtype=dtype)
    q, s, qo, so = run(dev, orc, x)
    assert np.array_equal(q, qo), f"{(q != qo).sum()} code mismatches"
    assert np.array_equal(s.view(np.uint32), so.view(np.uint32))


@pytest.mark.parametrize("rounds", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("G", [1, 7, 12, 20, 33, 48, 64])
def test_forced_rounds(dev, orc, monkeypatch, rounds, G):
    """Every rounds-per-wave instance of the register-resident kernel
    (PHI_QR_ROUNDS), bf16 and fp32 input, with dead groups and rows."""
    monkeypatch.setenv("PHI_QR_ROUNDS", str(rounds))
    for dtype in (torch.bfloat16, torch.float32):
        x = synth.activations(11, 256 * G, seed=100 * rounds + G, dtype=dtype)
        q, s, qo, so = run(dev, orc, x)
        assert np.array_equal(q, qo), f"{(q != qo).sum()} code mismatches"
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32))
    x = synth.activations(6, 256 * G, seed=7 + G, dtype=torch.bfloat16)
    q, s, qo, so = run(dev, orc, x, round_mode=Q.ROUND_HALF_EVEN, qmax=7.0)
    assert np.array_equal(q, qo) and np.array_equal(s.view(np.uint32), so.view(np.uint32))
    q, s, qo, so = run(dev, orc, x, rotate=False)
    assert np.array_equal(q, qo) and np.array_equal(s.view(np.uint32), so.view(np.uint32))


def test_c0_activation_block(dev, orc):
    """config 0's activation: [256, 3072] bf16 with outlier channels, seed 0."""
    x = synth.activations(256, 3072, seed=0)
    q, s, qo, so = run(dev, orc, x)
    assert np.array_equal(q, qo) and np.array_equal(s.view(np.uint32), so.view(np.uint32))
    assert np.abs(q).max() == 127


@pytest.mark.parametrize("rotate", [True, False])
@pytest.mark.parametrize("qmax", [127.0, 7.0])
@pytest.mark.parametrize("round_mode", [Q.ROUND_HALF_AWAY, Q.ROUND_HALF_EVEN])
def test_modes(dev, orc, rotate, qmax, round_mode):
    x = synth.activations(33, 2048, seed=5, dtype=torch.float32) * 3
    q, s, qo, so = run(dev, orc, x, rotate=rotate, qmax=qmax, round_mode=round_mode)
    assert np.array_equal(q, qo)
    assert np.array_equal(s.view(np.uint32), so.view(np.uint32))


def test_exact_ties_and_the_half_boundary(dev, orc):
    """Rows with amax 127 quantise with inv == 1, so the input is the value that
    is rounded.  Exact .5 ties separate half-away from half-even, and
    0.5 - 2^-25 is the fp32 value where a float d + 0.5f rounding gives 1 while
    the reference's double rule gives 0."""
    K = 256
    vals = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5,
                     np.float32(0.5) - np.float32(2.0 ** -25), -(np.float32(0.5) - np.float32(2.0 ** -25)),
                     0.49999997, 1.4999999, 127.0, -127.0, 0.0, -0.0], np.float32)
    row = np.zeros(K, np.float32)
    row[:vals.size] = vals
    row[-1] = 127.0
    x = torch.from_numpy(np.stack([row, row * 0.5]))
    for mode in (Q.ROUND_HALF_AWAY, Q.ROUND_HALF_EVEN):
        q, s, qo, so = run(dev, orc, x, rotate=False, round_mode=mode)
        assert np.array_equal(q, qo)
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32))
    q, _, _, _ = run(dev, orc, x, rotate=False)
    assert list(q[0, :10]) == [1, -1, 2, -2, 3, -3, 127, -127, 0, 0]


def near_ties(lo=-128, hi=128, ulps=3):
    """Every half-integer in [lo, hi) and its fp32 neighbours within `ulps`
    (the same set the oracle's own rounding pins use)."""
    centres = np.arange(lo, hi) + 0.5
    out = [centres.astype(np.float32)]
    up = dn = centres.astype(np.float32)
    for _ in range(ulps):
        up = np.nextafter(up, np.float32(np.inf))
        dn = np.nextafter(dn, np.float32(-np.inf))
        out += [up, dn]
    v = np.concatenate(out)
    return v[np.abs(v) <= 127]


def half_away(v):
    """Round half away from zero, exactly (float64 holds every fp32 value)."""
    d = v.astype(np.float64)
    return np.clip(np.sign(d) * np.floor(np.abs(d) + 0.5), -127, 127).astype(np.int8)


@pytest.mark.parametrize("round_mode", [Q.ROUND_HALF_AWAY, Q.ROUND_HALF_EVEN])
@pytest.mark.parametrize("inv_pow", [0, 3, -2])
def test_every_near_tie_unrotated(dev, orc, round_mode, inv_pow):
    """The whole near-tie set in one row per scale: amax 127 * 2^-inv_pow makes
    inv = 2^inv_pow exactly, so v * inv is exact and the rounding alone decides
    each code (the kernel's add-0.49999997-then-truncate shortcut included)."""
    v = near_ties()
    K = 256 * ((v.size + 1 + 255) // 256)
    row = np.zeros(K, np.float32)
    row[:v.size] = v
    row[-1] = 127.0
    row *= np.float32(2.0 ** -inv_pow)
    x = torch.from_numpy(np.stack([row, -row]))
    q, s, qo, so = run(dev, orc, x, rotate=False, round_mode=round_mode)
    assert np.array_equal(s.view(np.uint32), so.view(np.uint32))
    assert s[0] == np.float32(2.0 ** -inv_pow)
    assert np.array_equal(q, qo), f"{(q != qo).sum()} code mismatches"
    if round_mode == Q.ROUND_HALF_AWAY:
        assert np.array_equal(q[0, :v.size], half_away(v))


@pytest.mark.parametrize("rotate", [False, True])
def test_rounding_contract_at_the_device_floor_edge(dev, orc, rotate):
    """The library rounds by the reference's host rule (core/host/quant.cpp:163-166),
    not by its device kernel's fp32 floorf(d + 0.5f) (core/kernels/int8_gemm.cpp:777-780).
    The two differ only at d = +-(0.5 - 2^-25): 0 by the host rule, +-1 by the
    device form.  Rows put exactly those products through both kernels, without
    and with the rotation (one non-zero per 256-group rotates to +-c/16 in every
    element, exactly)."""
    edge = np.float32(0.5 - 2.0 ** -25)
    K = 1024
    row = np.zeros(K, np.float32)
    if rotate:
        row[0], row[256], row[512], row[768] = 16 * edge, -16 * edge, 16 * 127.0, 16 * 1.5
    else:
        row[:4] = [edge, -edge, 127.0, 1.5]
    x = torch.from_numpy(np.stack([row, row * np.float32(0.25)]))
    q, s, qo, so = run(dev, orc, x, rotate=rotate)
    assert np.array_equal(q, qo) and np.array_equal(s.view(np.uint32), so.view(np.uint32))
    qd, sd = orc.quantize_rows(x.numpy(), rotate=rotate, round_mode=orc.ROUND_DEVICE_FLOOR)
    codes = q[0, [0, 256, 512, 768]] if rotate else q[0, :4]
    dcodes = qd[0, [0, 256, 512, 768]] if rotate else qd[0, :4]
    assert s[0] == 1.0
    assert list(codes[:2].astype(int)) == [0, 0] and abs(int(codes[2])) == 127
    assert [abs(int(c)) for c in dcodes[:2]] == [1, 1]
    # both rows (the second scaled by 1/4, so inv = 4 and the products are the same)
    # differ at their edge products only: two groups of 256 rotated, two elements not
    assert (q != qd).sum() == (2 * 2 * 256 if rotate else 2 * 2), "the forms differ only at the edge products"


@pytest.mark.parametrize("round_mode", [Q.ROUND_HALF_AWAY, Q.ROUND_HALF_EVEN])
@pytest.mark.parametrize("groups", [96, 64, 12])
def test_every_near_tie_through_the_rotation(dev, orc, round_mode, groups):
    """The near-tie set through the rotation and the folded inv/16.  A 256-group
    holding one non-zero c at position p rotates to +-c in every element, times
    1/16, with no rounding; with c = 16 t the group's values are exactly +-t.
    One group per row holds 16 * 127, so amax = 127, scale = 1 and the kernel's
    folded multiplier is 1/16: every code is the rounding of +-t.  96 groups a
    row run the row kernel; 64 and 12 the register-resident kernel's fast rows
    (its exact scale divisions and unclamped codes), with 16 and 3 waves
    sharing a row (12 groups is config 1's K)."""
    v = near_ties()
    per_row = groups - 1  # groups left in a row after the amax group
    rows = (v.size + per_row - 1) // per_row
    K = groups * 256
    x = np.zeros((rows, K), np.float32)
    want = np.zeros((rows, per_row), np.float32)
    for i, t in enumerate(v):
        r, g = divmod(i, per_row)
        x[r, g * 256 + (i * 37) % 256] = np.float32(16.0) * t
        want[r, g] = t
    x[:, per_row * 256 + 5] = np.float32(16.0 * 127.0)
    q, s, qo, so = run(dev, orc, torch.from_numpy(x), round_mode=round_mode)
    assert np.array_equal(s.view(np.uint32), so.view(np.uint32))
    assert np.all(s == 1.0)
    assert np.array_equal(q, qo), f"{(q != qo).sum()} code mismatches"
    if round_mode == Q.ROUND_HALF_AWAY:
        # Each group's codes are +-round(t); the sign pattern is the column's.
        mag = np.abs(q[:, :per_row * 256].reshape(rows, per_row, 256).astype(np.int16))
        n = v.size
        got = mag.max(axis=2).reshape(-1)[:n]
        assert np.array_equal(got, np.abs(half_away(want.reshape(-1)[:n])).astype(np.int16))


def test_huge_rows(dev, orc):
    """Rows whose amax is so large that inv/16 would be subnormal (qmax 1,
    amax 1e37): the kernel then scales each element by 1/16 before inv, as the
    reference does.  A constant group rotates to 16 c before the 1/16."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((3, 1024)) * 1e35).astype(np.float32)
    x[0, :256] = 1e37
    x[1, 256:512] = -6e36
    x = torch.from_numpy(x)
    for qmax in (1.0, 7.0, 127.0):
        for mode in (Q.ROUND_HALF_AWAY, Q.ROUND_HALF_EVEN):
            q, s, qo, so = run(dev, orc, x, qmax=qmax, round_mode=mode)
            assert np.array_equal(q, qo), (qmax, mode, (q != qo).sum())
            assert np.array_equal(s.view(np.uint32), so.view(np.uint32))


def nonfinite_rows(K):
    """Finite rows beside rows with a NaN, an inf of either sign, both infs,
    and values that overflow inside the rotation (to inf, or to +inf and -inf
    that meet as NaN)."""
    rng = np.random.default_rng(K)
    x = rng.standard_normal((9, K)).astype(np.float32)
    x[1, 300] = np.nan
    x[2, 5] = np.inf
    x[3, K - 68] = -np.inf
    x[4, 10], x[4, K - 1] = np.inf, -np.inf
    x[5, 256:260] = 3e38
    x[6, 0], x[6, 1] = 3e38, -3e38
    x[7, :] = np.nan
    return torch.from_numpy(x)


@pytest.mark.parametrize("rounds", [0, 1, 3, 5])
@pytest.mark.parametrize("K", [768, 3072, 16640])
def test_nonfinite_rows(dev, orc, monkeypatch, rounds, K):
    """Rows holding inf or NaN take the clamped path and give the reference's
    codes (a NaN product is -qmax); the finite rows of the same launch take
    the unclamped one.  Every rounds-per-wave instance (0: the library's
    choice), the row kernel past 64 groups, both rounding modes, bf16 and
    fp32 input, row-major and K-tiled output."""
    if rounds:
        monkeypatch.setenv("PHI_QR_ROUNDS", str(rounds))
    x32 = nonfinite_rows(K)
    for dtype in (torch.float32, torch.bfloat16):
        x = x32.to(dtype)
        for mode in (Q.ROUND_HALF_AWAY, Q.ROUND_HALF_EVEN):
            q, s, qo, so = run(dev, orc, x, round_mode=mode)
            assert np.array_equal(q, qo), (dtype, mode, np.argwhere(q != qo)[:5])
            assert np.array_equal(s.view(np.uint32), so.view(np.uint32))
            if K <= 16384:
                qk, sk = Q.quant_rotate_kt(x.to(dev), round_mode=mode)
                assert torch.equal(qk.cpu(), Q.pack_k_tiled(torch.from_numpy(qo).to(dev)).cpu())
                assert np.array_equal(sk.cpu().numpy().view(np.uint32), so.view(np.uint32))


def test_zero_rows_and_tiny_rows(dev, orc):
    x = torch.zeros((4, 512), dtype=torch.float32)
    x[1, 7] = 1e-31  # amax below 1e-30 -> scale 1
    x[2, 3] = 3e-30
    q, s, qo, so = run(dev, orc, x)
    assert np.array_equal(q, qo)
    assert np.array_equal(s.view(np.uint32), so.view(np.uint32))
    assert s[0] == 1.0 and not q[0].any()


def test_strided_rows_and_empty(dev, orc):
    big = synth.activations(9, 1280, seed=11, dtype=torch.float32).to(dev)
    x = big[:, :1024]
    q = torch.empty((9, 1024 + 64), dtype=torch.int8, device=dev)
    s = torch.empty((9,), dtype=torch.float32, device=dev)
    Q.quant_rotate(x, q=q, s=s)
    torch.cuda.synchronize()
    qo, so = orc.quantize_rows(x.cpu().numpy())
    assert np.array_equal(q[:, :1024].cpu().numpy(), qo)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    e = torch.empty((0, 256), device=dev)
    Q.quant_rotate(e)  # rows == 0 is a no-op


def test_contract_errors(dev):
    with pytest.raises(Q.QLinearError, match="multiple of 256"):
        Q.quant_rotate(torch.zeros((2, 300), device=dev))
    with pytest.raises(Q.QLinearError, match="exceeds"):
        Q.quant_rotate(torch.zeros((1, 24576 + 256), device=dev))


def _all_significands(exp: int) -> np.ndarray:
    return ((np.arange(1 << 23, dtype=np.uint32)) | np.uint32((127 + exp) << 23)).view(np.float32)


def test_scale_divisions_on_device(dev):
    """The fast row-scale divisions (csrc/qt_scale.hpp) on the GPU, every
    significand at the ends of their ranges and at 1, against IEEE division
    (numpy's float32 divide): rmax / qmax from the rounded 1/qmax with one fma
    correction, and 1 / scale from v_rcp_f32's estimate with two Newton steps
    (the all-ones significand fixed).  The estimate is the hardware's own; the
    CPU check (test_host_logic.py) covers any estimate within 2 ulps."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(os.path.dirname(Q.LIB_PATH), "libphi_probe.so"))
    f = lib.phi_probe_qt_scale
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_void_p]
    st = torch.cuda.current_stream().cuda_stream
    for mode, exps, qmaxes in ((0, (-90, 0, 121), (127.0, 7.0, 1.0, 100.0)), (1, (-97, 0, 121), (127.0,))):
        for e in exps:
            a = _all_significands(e)
            x = torch.from_numpy(a).to(dev)
            out = torch.empty_like(x)
            for qm in qmaxes:
                assert f(st, x.data_ptr(), a.size, mode, qm, out.data_ptr()) == 0
                torch.cuda.synchronize()
                want = a / np.float32(qm) if mode == 0 else np.float32(1.0) / a
                got = out.cpu().numpy()
                bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
                assert bad.size == 0, f"mode {mode} exp {e} qmax {qm}: {bad.size} mismatches, first b={a[bad[0]]!r}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("round_mode", [Q.ROUND_HALF_AWAY, Q.ROUND_HALF_EVEN])
def test_row_scales_across_the_division_ranges(dev, orc, dtype, round_mode):
    """Rows whose amax spans the fast divisions' range and its edges: rotated
    amax around 2^-86 (below it the kernel divides as IEEE does), near the
    1e-30 scale floor, ordinary, and up to just under 2^126 (the fast-row
    limit).  Codes and scales bit-exact against the oracle."""
    x = synth.activations(24, 3072, seed=7, dtype=torch.float32)
    exps = [-120, -100, -90, -88, -87, -86, -85, -84, -80, -40, -5, 0, 3, 20, 60, 100, 110, 118, 119, 120, 121, 122,
            -99, -98]
    for i, e in enumerate(exps):
        x[i] *= float(2.0 ** e)
    x = x.to(dtype)
    q, s, qo, so = run(dev, orc, x, round_mode=round_mode)
    assert np.array_equal(s.view(np.uint32), so.view(np.uint32))
    assert np.array_equal(q, qo), f"{(q != qo).sum()} code mismatches"
