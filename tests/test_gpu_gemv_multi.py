"""Multi-vector decode GEMV (small-M batched GEMV for speculative decode
verification) vs the oracle and vs the single-vector GEMV, both paths:
the MFMA path (exact=False) and the VALU path (exact=True).

Tolerance: normwise max|y - ref| / max|ref| <= 1e-3 (fp16 y) and 2e-5
(fp32 y) per vector against the oracle's fp32 product with exact fp32
dequantized weights (Y[m] = gemv_ref(x[m])). For exact=True, where the
single GEMV runs unsplit (N >= 1920 rows), every row of Y must also be
bit-identical to the single GEMV of that x row: that path keeps its block
order and reduction order, so speculative verification scores exactly what
token-by-token decode would. The MFMA path's rows must agree with the
single GEMV to 2e-5 (fp32 outputs).
"""
import numpy as np
import pytest
import torch

from oracle import q4_oracle as O
from tests.helpers import synth_int4, to_np, upload_int4

pytestmark = pytest.mark.gpu
TOL = {torch.float16: 1e-3, torch.float32: 2e-5}


def _x(rng, M, K):
    return rng.standard_normal((M, K)).astype(np.float16)


@pytest.mark.parametrize("N,K", [(15360, 3840), (3840, 15360), (4096, 3840), (2048, 256), (100, 96), (1000, 3072)])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 11, 16])
@pytest.mark.parametrize("exact", [True, False])
def test_gemv_multi_vs_oracle_and_single(gpu, N, K, M, exact):
    rng = np.random.default_rng(N + K + M)
    q, s = synth_int4(rng, N, K)
    X = _x(rng, M, K)
    wq, sc = upload_int4(q, s)
    ref = O.gemm_w4a16_ref(X, q, s)
    Xd = torch.from_numpy(X).cuda()
    unsplit = gpu.auto_split(N, K) == 1
    for ydt in (torch.float16, torch.float32):
        Y = gpu.gemv_multi(Xd, wq, sc, N, K, y_dtype=ydt, exact=exact)
        assert tuple(Y.shape) == (M, N)
        Yh = to_np(Y).astype(np.float32)
        for m in range(M):
            assert O.normwise_rel_err(Yh[m], ref[m]) <= TOL[ydt], (ydt, m)
            y1 = gpu.gemv(Xd[m].contiguous(), wq, sc, N, K, y_dtype=ydt)
            if exact and unsplit:
                assert torch.equal(Y[m], y1), (ydt, m)
            elif ydt == torch.float32:
                assert O.normwise_rel_err(Yh[m], to_np(y1)) <= TOL[ydt], m


@pytest.mark.parametrize("rows", ["8", "16", "32", "64"])
@pytest.mark.parametrize("units", ["4", "8"])
def test_gemv_multi_plan_variants_bit_identical(gpu, rows, units, tune):
    """Every rows-per-workgroup x units-in-flight variant, with a block count
    (37) that leaves the last round of the load ring partly empty: each row
    equals the single GEMV under the same plan."""
    tune("gemv_rows", rows)
    tune("gemv_units", units)
    N, K, M = 2048, 32 * 37, 6
    rng = np.random.default_rng(int(rows) * 10 + int(units))
    q, s = synth_int4(rng, N, K)
    X = _x(rng, M, K)
    wq, sc = upload_int4(q, s)
    Xd = torch.from_numpy(X).cuda()
    Y = gpu.gemv_multi(Xd, wq, sc, N, K, y_dtype=torch.float32, exact=True)
    ref = O.gemm_w4a16_ref(X, q, s)
    for m in range(M):
        assert O.normwise_rel_err(to_np(Y[m]), ref[m]) <= TOL[torch.float32]
        assert torch.equal(Y[m], gpu.gemv(Xd[m].contiguous(), wq, sc, N, K, y_dtype=torch.float32, split=1))


@pytest.mark.parametrize("exact", [True, False])
def test_gemv_multi_e4m3(gpu, exact):
    rng = np.random.default_rng(9)
    for N, K, M in [(15360, 3840, 4), (3840, 15360, 8), (256, 256, 3)]:
        q, s = synth_int4(rng, N, K)
        e8, inv, _ = O.e4m3_lift(s)
        X = _x(rng, M, K)
        ref = O.gemm_w4a16_ref(X, q, O.e4m3_decode(e8)) * np.float32(inv)
        wq, _ = upload_int4(q, s)
        sc8 = torch.from_numpy(O.scales_dev(e8)).cuda()
        Xd = torch.from_numpy(X).cuda()
        Y = gpu.gemv_multi(Xd, wq, sc8, N, K, scale_fmt=gpu.SCALE_E4M3, inv=inv, y_dtype=torch.float32, exact=exact)
        for m in range(M):
            assert O.normwise_rel_err(to_np(Y[m]), ref[m]) <= TOL[torch.float32], (N, K, m)
            if exact and N >= 1920:
                y1 = gpu.gemv(Xd[m].contiguous(), wq, sc8, N, K, scale_fmt=gpu.SCALE_E4M3, inv=inv,
                              y_dtype=torch.float32)
                assert torch.equal(Y[m], y1)


def test_gemv_multi_largest_staging_and_limits(gpu):
    """The largest K per launch size of the exact path (8 vectors at K = 8192,
    4 at 16384, 2 at 32768) against the oracle, both paths; a K whose
    two-vector staging does not fit the LDS (exact path) and M outside
    1..16 are rejected by the host."""
    rng = np.random.default_rng(4)
    for K, M in [(8192, 8), (16384, 5), (32768, 3)]:
        N = 2048
        q, s = synth_int4(rng, N, K)
        X = _x(rng, M, K)
        wq, sc = upload_int4(q, s)
        ref = O.gemm_w4a16_ref(X, q, s)
        for exact in (True, False):
            Y = gpu.gemv_multi(torch.from_numpy(X).cuda(), wq, sc, N, K, y_dtype=torch.float32, exact=exact)
            for m in range(M):
                assert O.normwise_rel_err(to_np(Y[m]), ref[m]) <= TOL[torch.float32], (K, m, exact)
    N, K = 256, 65536
    q, s = synth_int4(rng, N, K)
    wq, sc = upload_int4(q, s)
    with pytest.raises(RuntimeError, match="LDS"):
        gpu.gemv_multi(torch.zeros(2, K, dtype=torch.float16, device="cuda"), wq, sc, N, K, exact=True)
    with pytest.raises(ValueError):
        gpu.gemv_multi(torch.zeros(17, K, dtype=torch.float16, device="cuda"), wq, sc, N, K)


@pytest.mark.parametrize("tiles", ["1", "2", "4"])
@pytest.mark.parametrize("deep", ["0", "1"])
def test_gemv_multi_mfma_plan_variants(gpu, tiles, deep, tune):
    """Every row-tile count x load depth of the MFMA path against the oracle,
    with block counts that leave waves without blocks (3: wave 3 idle) and
    the last round of the load ring partly empty (37, 200). The blocks and
    partial sums are added in the same order whatever the depth, so both
    depths give bit-identical outputs."""
    tune("gemv_mm_tiles", tiles)
    tune("gemv_mm_deep", deep)
    for N, nblk, M in [(256, 3, 16), (320, 37, 7), (4096, 200, 13)]:
        K = 32 * nblk
        rng = np.random.default_rng(N + nblk + int(tiles))
        q, s = synth_int4(rng, N, K)
        X = _x(rng, M, K)
        wq, sc = upload_int4(q, s)
        Y = gpu.gemv_multi(torch.from_numpy(X).cuda(), wq, sc, N, K, y_dtype=torch.float32)
        ref = O.gemm_w4a16_ref(X, q, s)
        for m in range(M):
            assert O.normwise_rel_err(to_np(Y[m]), ref[m]) <= TOL[torch.float32], (N, nblk, m)
        tune("gemv_mm_deep", "1" if deep == "0" else "0")
        Y2 = gpu.gemv_multi(torch.from_numpy(X).cuda(), wq, sc, N, K, y_dtype=torch.float32)
        tune("gemv_mm_deep", deep)
        assert torch.equal(Y, Y2)


def test_gemv_multi_mfma_zero_and_extreme_codes(gpu):
    """Codes 0 and 15 everywhere (the dequant's end points, -8 and +7) and a
    zero matrix, against the oracle, fp16 and e4m3 scales."""
    rng = np.random.default_rng(12)
    N, K, M = 2048, 512, 9
    X = _x(rng, M, K)
    for code in (0, 15, 8):
        q = np.full((N, K), code, np.uint8)
        s = (rng.random((N, K // 32)) + 0.5).astype(np.float16).astype(np.float32)
        wq, sc = upload_int4(q, s)
        Y = gpu.gemv_multi(torch.from_numpy(X).cuda(), wq, sc, N, K, y_dtype=torch.float32)
        ref = O.gemm_w4a16_ref(X, q, s)
        if code == 8:
            assert not to_np(Y).any()
        else:
            for m in range(M):
                assert O.normwise_rel_err(to_np(Y[m]), ref[m]) <= TOL[torch.float32], (code, m)


@pytest.mark.parametrize("split", ["1", "2", "3", "5", "8"])
def test_gemv_multi_ksplit_variants(gpu, split, tune):
    """K split across workgroups (T = 4 tiles, fp32 partials, split-order
    reduce) at forced split counts, with block counts that leave the last
    split shorter (203 blocks) and M * N not a multiple of 4 (the reduce's
    one-output-per-thread path), fp16 and fp32 y, against the oracle and
    against the unsplit launch."""
    tune("gemv_mm_split", split)
    for N, nblk, M in [(3840, 203, 16), (1001, 96, 3), (4096, 120, 5)]:
        K = 32 * nblk
        rng = np.random.default_rng(N + nblk + int(split))
        q, s = synth_int4(rng, N, K)
        X = _x(rng, M, K)
        wq, sc = upload_int4(q, s)
        Xd = torch.from_numpy(X).cuda()
        ref = O.gemm_w4a16_ref(X, q, s)
        need = gpu.gemv_multi_workspace_bytes(M, N, K)
        assert need == (int(split) * M * N * 4 if split != "1" else 0)
        for ydt in (torch.float16, torch.float32):
            Y = gpu.gemv_multi(Xd, wq, sc, N, K, y_dtype=ydt)
            tune("gemv_mm_split", "1")
            Y1 = gpu.gemv_multi(Xd, wq, sc, N, K, y_dtype=ydt)
            tune("gemv_mm_split", split)
            Yh = to_np(Y).astype(np.float32)
            for m in range(M):
                assert O.normwise_rel_err(Yh[m], ref[m]) <= TOL[ydt], (N, nblk, m, ydt)
                if ydt == torch.float32:
                    assert O.normwise_rel_err(Yh[m], to_np(Y1[m])) <= TOL[ydt], (N, nblk, m)


def test_gemv_multi_ksplit_down_shape_reuses_workspace(gpu):
    """The down shape (3840 x 15360) at M = 16 and then M = 4 through one
    workspace sized for M = 16: the second call's partials are all written
    by the second call (the reduce reads only [split][4][N])."""
    N, K = 3840, 15360
    rng = np.random.default_rng(77)
    q, s = synth_int4(rng, N, K)
    wq, sc = upload_int4(q, s)
    ws = torch.empty(gpu.gemv_multi_workspace_bytes(16, N, K), dtype=torch.uint8, device="cuda")
    assert ws.numel() > 0
    for M in (16, 4):
        X = _x(rng, M, K)
        Y = gpu.gemv_multi(torch.from_numpy(X).cuda(), wq, sc, N, K, y_dtype=torch.float32, ws=ws)
        ref = O.gemm_w4a16_ref(X, q, s)
        for m in range(M):
            assert O.normwise_rel_err(to_np(Y[m]), ref[m]) <= TOL[torch.float32], (M, m)
