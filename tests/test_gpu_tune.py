"""GPU checks of the GEMM tuning table (phi_hip_gemm_plan_*, the host layer's
GemmTuneStore and autotune_int8_gemm; the reference's autotune store and sweep,
core/kernels/autotune.hpp:30-88, core/kernels/autotune.cpp:158-334).

* Every plan a caller can set gives the default plan's output bit for bit
  (bf16 with a bias, row-major and K-tiled operands), and the library reports
  the plan it runs.
* The sweep checks the default plan's accumulators against host integer sums
  on sampled rows, finds every candidate bit-identical to the default, and its
  winner survives the JSON round trip into the library's table.
"""
import json

import numpy as np
import pytest
import torch

import ckpt_util as C
import phi_qlinear as Q
from phi_qlinear import synth

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kt", [False, True])
def test_tuned_plans_give_the_same_bits(dev, kt):
    M, N, K = 2304, 6144, 1024
    A = synth.int8_weight(M, K, seed=5, device=dev)
    B = synth.int8_weight(N, K, seed=6, device=dev)
    sA = torch.rand(M, device=dev) * 0.01 + 1e-3
    sB = torch.rand(N, device=dev) * 0.01 + 1e-3
    bias = synth.bias(N, seed=7, device=dev)
    Ak, Bk = (Q.pack_k_tiled(A), Q.pack_k_tiled(B)) if kt else (None, None)

    def run():
        if kt:
            return Q.i8_gemm_kt(Ak, Bk, M, N, K, sA, sB, bias)
        return Q.i8_gemm(A, B, sA, sB, bias)

    Q.gemm_plan_clear()
    try:
        assert not Q.gemm_plan_get(M, N, K, k_tiled=kt)["tuned"]
        want = run()
        plans = [dict(big_rows=2304, group_m=2), dict(big_rows=2048, group_m=8, split=True),
                 dict(big_rows=0, group_m=4), dict(big_rows=1792, group_m=1), dict(big_rows=-1, group_m=16),
                 dict(big_rows=1792, group_m=4, tile=Q.PLAN_TILE_SQUARE)]
        plans += [dict(big_rows=-1, group_m=g, tile=Q.PLAN_TILE_272) for g in (1, 4, 8)]
        for plan in plans:
            Q.gemm_plan_set(M, N, K, k_tiled=kt, **plan)
            got = run()
            torch.cuda.synchronize()
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), plan
            now = Q.gemm_plan_get(M, N, K, k_tiled=kt)
            assert now["tuned"] and now["group_m"] == plan["group_m"]
            if plan.get("tile", Q.PLAN_TILE_AUTO) != Q.PLAN_TILE_AUTO:
                assert now["tile"] == plan["tile"]
            if plan["big_rows"] >= 0:
                assert now["big_rows"] == plan["big_rows"]
            else:
                assert now["big_rows"] == Q.big_tile_rows(M, N)
    finally:
        Q.gemm_plan_clear()


@pytest.mark.parametrize("kt", [0, 1])
@pytest.mark.parametrize("M,N,K", [(1280, 4096, 768), (4352, 12288, 3072)])
def test_autotune_sweep_round_trip(dev, tmp_path, kt, M, N, K):
    path = tmp_path / "gemm_plans.json"
    out = C.run("tune", M, N, K, 2, kt, str(path))
    r = json.loads(out.stdout)
    assert r["ok"] and r["default_exact"]
    assert r["exact"] == r["tried"] >= 6, r
    assert r["applied"] == r["best"] and r["tuned"] == 1 and r["entries"] == 1
    assert r["best_us"] == pytest.approx(min(r["us"]), rel=1e-6)
    saved = json.loads(path.read_text())
    (e,) = saved["plans"]
    assert (e["M"], e["N"], e["K"], e["k_tiled"]) == (M, N, K, kt)
    assert [e["big_rows"], e["group_m"], e["split"], e["tile"]] == r["best"]
    # 272 x 192 candidates where they apply (K % 512 == 0), one a group height
    assert r["tiles"].count(Q.PLAN_TILE_272) == (3 if K % 512 == 0 else 0)
    assert len(r["tiles"]) == r["tried"]
    if K % 512 == 0:
        assert r["best"][3] in (Q.PLAN_TILE_SQUARE, Q.PLAN_TILE_272)
    else:
        assert r["best"][3] == Q.PLAN_TILE_SQUARE
