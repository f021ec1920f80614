"""Prefill GEMMs and the int8 activation quantizer vs the oracle.

Bit-exact: int8 activation codes and scales, W8A8/W4A8 int32 accumulators
and their fp16 epilogue. W4A16: normwise <= 1e-3 against the oracle's exact
fp32 dequant + fp32 matmul (the kernel rounds each dequantized weight to
fp16 as the reference shader does, then accumulates in fp32).
"""
import numpy as np
import pytest
import torch

from oracle import decode_ops_oracle as D
from oracle import q4_oracle as O
from tests.helpers import W8A8_EPILOGUE_KATS, synth_int4, to_np, upload_int4, w8a8_dot_operands

pytestmark = pytest.mark.gpu


# ------------------------------------------------------ activation quant
@pytest.mark.parametrize("M,K", [(1, 4), (3, 64), (128, 3840), (2048, 3840), (17, 15360)])
@pytest.mark.parametrize("dt", [np.float32, np.float16])
def test_quant_act_i8_bit_exact(gpu, M, K, dt):
    rng = np.random.default_rng(M + K)
    X = rng.standard_normal((M, K)).astype(dt)
    if M >= 3:
        X[0] = 0                                   # zero row -> 1e-12 scale
        X[1, :4] = [127, 2.5, -3.5, 0.5] if K >= 4 else X[1, :4]   # absmax 127 -> exact ties
    A, sa = O.quant_act_i8(X)
    gA, gsa = gpu.quant_act_i8(torch.from_numpy(X).cuda())
    assert (to_np(gsa) == sa).all()
    assert (to_np(gA) == A).all()


# ------------------------------------------------------------------ W8A8
def _w8a8_case(rng, M, N, K):
    W = (rng.standard_normal((N, K)) * 0.08).astype(np.float32)
    q, sc = O.quant_codes(W)
    W8, sw = O.w8_fold(q, sc)
    X = rng.standard_normal((M, K)).astype(np.float16)
    A, sa = O.quant_act_i8(X)
    return A, sa, W8, sw


@pytest.mark.parametrize("M,N,K", [(64, 256, 64), (100, 320, 128), (70, 300, 192), (256, 512, 3840),
                                   (128, 15360, 3840), (300, 3840, 15360), (1024, 2048, 320)])
@pytest.mark.parametrize("swdt", [np.float32, np.float16])
def test_w8a8_bit_exact(gpu, M, N, K, swdt):
    rng = np.random.default_rng(M * 3 + N + K)
    A, sa, W8, sw = _w8a8_case(rng, M, N, K)
    sw_used = sw.astype(swdt)
    C, Y = O.gemm_w8a8_ref(A, W8, sa, sw_used.astype(np.float32))
    gY, gC = gpu.gemm_w8a8(torch.from_numpy(A).cuda(), torch.from_numpy(W8).cuda(), torch.from_numpy(sa).cuda(),
                           torch.from_numpy(sw_used).cuda(), want_c=True)
    assert (to_np(gC) == C).all()
    assert (to_np(gY).view(np.uint16) == Y.view(np.uint16)).all()


def test_w8a8_config_size_rows(gpu):
    """Prefill shape M=2048, N=15360, K=3840. The whole int32 accumulator and
    every fp16 output are checked bit-exactly against the oracle."""
    rng = np.random.default_rng(0)
    M, N, K = 2048, 15360, 3840
    codes = rng.integers(-8, 8, (N, K))
    s = np.abs(rng.normal(0, 0.02, (N, K // 32))).astype(np.float16).astype(np.float32)
    q = (codes + 8).astype(np.uint8)
    W8, sw = O.w8_fold(q, s)
    X = rng.standard_normal((M, K)).astype(np.float16)
    A, sa = O.quant_act_i8(X)
    gA, gsa = gpu.quant_act_i8(torch.from_numpy(X).cuda())
    assert (to_np(gA) == A).all() and (to_np(gsa) == sa).all()
    gY, gC = gpu.gemm_w8a8(gA, torch.from_numpy(W8).cuda(), gsa, torch.from_numpy(sw).cuda(), want_c=True)
    C = O.int_matmul_exact(A, W8)
    assert (to_np(gC) == C).all()
    Y = O.w8a8_epilogue(C, sa, sw)
    assert (to_np(gY).view(np.uint16) == Y.view(np.uint16)).all()


# ------------------------------------------------------ W8A8, packed weights
@pytest.mark.parametrize("N,K", [(256, 64), (300, 192), (15360, 3840), (40, 320)])
def test_w8_pack_layout(gpu, N, K):
    rng = np.random.default_rng(N + K)
    W8 = rng.integers(-127, 128, (N, K), dtype=np.int8)
    got = to_np(gpu.w8_pack(torch.from_numpy(W8).cuda()))
    assert (got == O.pack_w8_dev(W8)).all()


@pytest.mark.parametrize("M,N,K", [(64, 256, 64), (100, 320, 128), (70, 300, 192), (256, 512, 3840),
                                   (128, 15360, 3840), (300, 3840, 15360), (1024, 2048, 320), (520, 600, 4096)])
@pytest.mark.parametrize("swdt", [np.float32, np.float16])
def test_w8a8_packed_bit_exact(gpu, M, N, K, swdt):
    """Same cases as the [N][K] kernel (K % 128 == 64 included: the last k-step
    then runs on zero-padded weights), plus bit-identity with that kernel."""
    rng = np.random.default_rng(M * 3 + N + K)
    A, sa, W8, sw = _w8a8_case(rng, M, N, K)
    sw_used = sw.astype(swdt)
    C, Y = O.gemm_w8a8_ref(A, W8, sa, sw_used.astype(np.float32))
    gA, gsa, gsw = torch.from_numpy(A).cuda(), torch.from_numpy(sa).cuda(), torch.from_numpy(sw_used).cuda()
    W8p = torch.from_numpy(O.pack_w8_dev(W8)).cuda()
    gY, gC = gpu.gemm_w8a8_packed(gA, W8p, gsa, gsw, N, want_c=True)
    assert (to_np(gC) == C).all()
    assert (to_np(gY).view(np.uint16) == Y.view(np.uint16)).all()
    gY2 = gpu.gemm_w8a8(gA, torch.from_numpy(W8).cuda(), gsa, gsw)
    assert (to_np(gY2).view(np.uint16) == to_np(gY).view(np.uint16)).all()


def test_w8a8_packed_config_size_rows(gpu):
    """M=2048, N=15360, K=3840 on packed weights packed on the GPU: the whole
    int32 accumulator and every fp16 output vs the oracle."""
    rng = np.random.default_rng(0)
    M, N, K = 2048, 15360, 3840
    codes = rng.integers(-8, 8, (N, K))
    s = np.abs(rng.normal(0, 0.02, (N, K // 32))).astype(np.float16).astype(np.float32)
    W8, sw = O.w8_fold((codes + 8).astype(np.uint8), s)
    X = rng.standard_normal((M, K)).astype(np.float16)
    A, sa = O.quant_act_i8(X)
    gA, gsa = gpu.quant_act_i8(torch.from_numpy(X).cuda())
    W8p = gpu.w8_pack(torch.from_numpy(W8).cuda())
    gY, gC = gpu.gemm_w8a8_packed(gA, W8p, gsa, torch.from_numpy(sw).cuda(), N, want_c=True)
    C = O.int_matmul_exact(A, W8)
    assert (to_np(gC) == C).all()
    Y = O.w8a8_epilogue(C, sa, sw)
    assert (to_np(gY).view(np.uint16) == Y.view(np.uint16)).all()
    # Y only: every tile takes the full-tile epilogue (16-byte stores)
    gY1 = gpu.gemm_w8a8_packed(gA, W8p, gsa, torch.from_numpy(sw).cuda(), N)
    assert (to_np(gY1).view(np.uint16) == Y.view(np.uint16)).all()


@pytest.mark.parametrize("M,N,K,wgs", [
    (128, 320, 384, 1),         # one tile, three k-steps
    (512, 1280, 320, 16),       # K % 128 == 64: the last k-step of each tile has two slices
    (2048, 5760, 384, 256),     # 288 tiles in XCD eighths: 1 or 2 per workgroup, tiles shorter than their drain
    (1664, 13120, 384, 256),    # 533 tiles (not a multiple of 8): 2 or 3 per workgroup
    (1920, 12800, 2688, 256),   # 600 tiles, 2 or 3 per workgroup, 21 k-steps (drain ends a k-step early)
    (1024, 12800, 384, 256),    # 320 tiles in groups of 8 m-tiles x 4 n-tiles, 1 or 2 per workgroup
])
def test_w8a8_persistent_tiles_bit_exact(gpu, tune, M, N, K, wgs):
    """The persistent 128 x 320-tile kernel (forced through the plan override,
    also where the default plan keeps 256-row tiles): every int32 of C and
    every fp16 of Y vs the oracle, fp32 and fp16 s_w, and Y bit-identical to
    the 256-row kernel's (forced the same way)."""
    rng = np.random.default_rng(M + N + K)
    A, sa, W8, sw = _w8a8_case(rng, M, N, K)
    gA, gsa = torch.from_numpy(A).cuda(), torch.from_numpy(sa).cuda()
    W8p = torch.from_numpy(O.pack_w8_dev(W8)).cuda()
    C = O.int_matmul_exact(A, W8)
    for swdt in (np.float32, np.float16):
        sw_used = sw.astype(swdt)
        Y = O.w8a8_epilogue(C, sa, sw_used.astype(np.float32))
        gsw = torch.from_numpy(sw_used).cuda()
        tune("w8a8_tiles", 1)
        assert gpu.w8a8_workgroups(M, N, K) == wgs
        gY, gC = gpu.gemm_w8a8_packed(gA, W8p, gsa, gsw, N, want_c=True)
        assert (to_np(gC) == C).all()
        assert (to_np(gY).view(np.uint16) == Y.view(np.uint16)).all()
        gY1 = gpu.gemm_w8a8_packed(gA, W8p, gsa, gsw, N)
        assert (to_np(gY1).view(np.uint16) == Y.view(np.uint16)).all()
        tune("w8a8_tiles", 0)
        assert gpu.w8a8_workgroups(M, N, K) != wgs
        gY0 = gpu.gemm_w8a8_packed(gA, W8p, gsa, gsw, N)
        assert (to_np(gY0).view(np.uint16) == to_np(gY1).view(np.uint16)).all()


def test_w8a8_packed_unaligned_scales_fall_back(gpu):
    """A shape the persistent plan takes by default, called with sa and sw
    offset from 16-byte alignment (4-byte aligned views one element into
    larger buffers): the entry point runs the per-tile plan instead, with the
    same bits."""
    rng = np.random.default_rng(31)
    M, N, K = 1024, 12800, 384
    A, sa, W8, sw = _w8a8_case(rng, M, N, K)
    C, Y = O.gemm_w8a8_ref(A, W8, sa, sw)
    gA, W8p = torch.from_numpy(A).cuda(), torch.from_numpy(O.pack_w8_dev(W8)).cuda()
    sa_b = torch.zeros(M + 1, dtype=torch.float32, device="cuda")
    sw_b = torch.zeros(N + 1, dtype=torch.float32, device="cuda")
    sa_b[1:] = torch.from_numpy(sa).cuda()
    sw_b[1:] = torch.from_numpy(sw).cuda()
    gY = gpu.gemm_w8a8_packed(gA, W8p, sa_b[1:], sw_b[1:], N)
    assert (to_np(gY).view(np.uint16) == Y.view(np.uint16)).all()
    gY2, gC = gpu.gemm_w8a8_packed(gA, W8p, torch.from_numpy(sa).cuda(), torch.from_numpy(sw).cuda(), N,
                                   want_c=True)
    assert gpu.w8a8_workgroups(M, N, K) == 256 and (to_np(gC) == C).all()
    assert (to_np(gY2).view(np.uint16) == Y.view(np.uint16)).all()


@pytest.mark.parametrize("M,N", [(2304, 7432), (2100, 7424)])
def test_w8a8_packed_y_only_ragged(gpu, M, N):
    """Y-only launches with 256-row tiles (>= 256 tiles) whose grid has both
    full tiles (16-byte-store epilogue) and ragged edge tiles (M % 256 and
    N % 256 != 0; N % 8 == 0): every fp16 output vs the oracle, fp32 and fp16
    s_w."""
    rng = np.random.default_rng(M + N)
    K = 512
    A, sa, W8, sw = _w8a8_case(rng, M, N, K)
    assert gpu.w8a8_workgroups(M, N, K) >= 256
    gA, gsa = torch.from_numpy(A).cuda(), torch.from_numpy(sa).cuda()
    W8p = torch.from_numpy(O.pack_w8_dev(W8)).cuda()
    for swdt in (np.float32, np.float16):
        sw_used = sw.astype(swdt)
        _, Y = O.gemm_w8a8_ref(A, W8, sa, sw_used.astype(np.float32))
        gY = gpu.gemm_w8a8_packed(gA, W8p, gsa, torch.from_numpy(sw_used).cuda(), N)
        assert (to_np(gY).view(np.uint16) == Y.view(np.uint16)).all()


@pytest.mark.parametrize("M,N,K,wgs", [(2048, 8192, 256, 256), (2048, 10240, 384, 256)])
def test_w8a8_packed_epilogue_known_answers(gpu, M, N, K, wgs):
    """The kernel's epilogue order is the reference's, f16((f32(C) * sa) * sw)
    (vk/coopgemm_w8a8.comp:35): rows i < 3 of A and W8 are built so that
    C[i, i] is exactly the C of a known answer whose fp16 result differs under
    every other evaluation order, with its sa and sw bits. N = 8192: 256 tiles
    of 256 rows, so the Y-only launch takes the full-tile epilogue and the
    launch with C the general one; N = 10240: 512 persistent tiles of
    128 x 320 (two per workgroup). Against the oracle everywhere and against
    the known answers on the diagonal."""
    rng = np.random.default_rng(11)
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    W8 = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sa = (rng.random(M) * 0.05 + 0.005).astype(np.float32)
    sw = (rng.random(N) * 2e-4 + 1e-5).astype(np.float32)
    A[:3] = 0
    W8[:3] = 0
    k0 = 0
    for i, (c, sab, swb, _) in enumerate(W8A8_EPILOGUE_KATS):
        a, w = w8a8_dot_operands(c)
        A[i, k0:k0 + len(a)] = a
        W8[i, k0:k0 + len(a)] = w
        k0 += len(a)
        sa[i] = np.array([sab], np.uint32).view(np.float32)[0]
        sw[i] = np.array([swb], np.uint32).view(np.float32)[0]
    assert k0 <= K and gpu.w8a8_workgroups(M, N, K) == wgs
    C, Y = O.gemm_w8a8_ref(A, W8, sa, sw)
    assert [int(C[i, i]) for i in range(3)] == [k[0] for k in W8A8_EPILOGUE_KATS]
    assert [float(Y[i, i]) for i in range(3)] == [k[3] for k in W8A8_EPILOGUE_KATS]
    gA, gsa, gsw = torch.from_numpy(A).cuda(), torch.from_numpy(sa).cuda(), torch.from_numpy(sw).cuda()
    W8p = torch.from_numpy(O.pack_w8_dev(W8)).cuda()
    gY = gpu.gemm_w8a8_packed(gA, W8p, gsa, gsw, N)
    gY2, gC = gpu.gemm_w8a8_packed(gA, W8p, gsa, gsw, N, want_c=True)
    assert (to_np(gC) == C).all()
    for y in (gY, gY2):
        assert (to_np(y).view(np.uint16) == Y.view(np.uint16)).all()


@pytest.mark.parametrize("M,N,K", [(100, 320, 192), (2048, 15360, 3840)])
def test_w8a8_packed_stamped(gpu, M, N, K):
    """The stamped launch (per-workgroup clocks) gives the plain launch's
    results bit for bit, with 128-row tiles below 256 tiles and with the
    persistent 128 x 320 tiles at the full size, and its stamps are ordered:
    start <= end of the (last) k-loop <= end, cycles > 0."""
    rng = np.random.default_rng(M + N + K)
    A, sa, W8, sw = _w8a8_case(rng, M, N, K)
    gA, gsa, gsw = torch.from_numpy(A).cuda(), torch.from_numpy(sa).cuda(), torch.from_numpy(sw).cuda()
    W8p = torch.from_numpy(O.pack_w8_dev(W8)).cuda()
    wgs = gpu.w8a8_workgroups(M, N, K)
    assert wgs == (256 if (M, N, K) == (2048, 15360, 3840) else -(-M // 128) * -(-N // 256))
    stamps = torch.zeros((wgs, 4), dtype=torch.int64, device="cuda")
    gY, gC = gpu.gemm_w8a8_packed(gA, W8p, gsa, gsw, N, want_c=True)
    sY, sC = gpu.gemm_w8a8_packed(gA, W8p, gsa, gsw, N, want_c=True, stamps=stamps)
    assert (to_np(sC) == to_np(gC)).all()
    assert (to_np(sY).view(np.uint16) == to_np(gY).view(np.uint16)).all()
    s = to_np(stamps)
    assert (s[:, 0] > 0).all() and (s[:, 0] <= s[:, 1]).all() and (s[:, 1] <= s[:, 2]).all() and (s[:, 3] > 0).all()
    with pytest.raises(RuntimeError, match="stamps"):
        gpu.gemm_w8a8_packed(gA, W8p, gsa, gsw, N, stamps=stamps[: wgs - 1])


# ------------------------------------------------------------------ W4A8
@pytest.mark.parametrize("M,N,K", [(64, 256, 64), (100, 512, 3840), (33, 300, 320), (128, 15360, 3840)])
def test_w4a8_bit_exact(gpu, M, N, K):
    rng = np.random.default_rng(M + N + K + 1)
    W = (rng.standard_normal((N, K)) * 0.08).astype(np.float32)
    q, sc = O.quant_codes(W)
    _, sw = O.w8_fold(q, sc)
    ratio = O.w4a8_ratio(sc, sw)
    B = O.w4a8_weights(q, ratio)
    X = (rng.standard_normal((M, K)) * 0.3).astype(np.float32)
    A, sa = O.quant_act_i8(X)
    sw16 = sw.astype(np.float16)
    C, Y = O.gemm_w8a8_ref(A, B, sa, sw16.astype(np.float32))
    wq = torch.from_numpy(O.pack_dev(q).view(np.int32)).cuda()
    r = torch.from_numpy(O.scales_dev(ratio)).cuda()
    gY, gC = gpu.gemm_w4a8(torch.from_numpy(A).cuda(), wq, r, torch.from_numpy(sa).cuda(),
                           torch.from_numpy(sw16).cuda(), N, want_c=True)
    assert (to_np(gC) == C).all()
    assert (to_np(gY).view(np.uint16) == Y.view(np.uint16)).all()


@pytest.mark.parametrize("N,K", [(256, 64), (300, 256), (15360, 3840)])
def test_w4a8_weights_once_then_w8a8_bit_identical(gpu, N, K):
    """W4A8's int8 weights formed once (q4_w4a8_weights) equal the oracle's
    requant bit for bit, and packed W8A8 on them gives q4_gemm_w4a8's Y and C
    bit for bit."""
    rng = np.random.default_rng(N + K + 7)
    W = (rng.standard_normal((N, K)) * 0.08).astype(np.float32)
    q, sc = O.quant_codes(W)
    _, sw = O.w8_fold(q, sc)
    ratio = O.w4a8_ratio(sc, sw)
    wq = torch.from_numpy(O.pack_dev(q).view(np.int32)).cuda()
    r = torch.from_numpy(O.scales_dev(ratio)).cuda()
    W8 = gpu.w4a8_weights(wq, r, N, K)
    assert (to_np(W8) == O.w4a8_weights(q, ratio)).all()
    M = 128
    X = (rng.standard_normal((M, K)) * 0.3).astype(np.float32)
    A, sa = O.quant_act_i8(X)
    tA, tsa = torch.from_numpy(A).cuda(), torch.from_numpy(sa).cuda()
    sw16 = torch.from_numpy(sw.astype(np.float16)).cuda()
    Y4, C4 = gpu.gemm_w4a8(tA, wq, r, tsa, sw16, N, want_c=True)
    Y8, C8 = gpu.gemm_w8a8_packed(tA, gpu.w8_pack(W8), tsa, sw16, N, want_c=True)
    assert torch.equal(C4, C8) and torch.equal(Y4, Y8)


# ----------------------------------------------------------------- W4A16
@pytest.mark.parametrize("M,N,K", [(64, 256, 32), (100, 320, 96), (40, 300, 224), (128, 3840, 15360),
                                   (512, 15360, 3840), (512, 3840, 15360), (1024, 8192, 256), (2048, 8192, 96),
                                   (37, 70, 15360)])   # split K with M N not a multiple of 4: scalar reduce
def test_w4a16(gpu, M, N, K):
    rng = np.random.default_rng(M + 2 * N + K)
    q, s = synth_int4(rng, N, K)
    X = rng.standard_normal((M, K)).astype(np.float16)
    ref = O.gemm_w4a16_ref(X, q, s)
    wq, sc = upload_int4(q, s)
    Y = gpu.gemm_w4a16(torch.from_numpy(X).cuda(), wq, sc, N)
    Yh = to_np(Y).astype(np.float32)
    err = O.normwise_rel_err(Yh, ref)
    assert err <= 1e-3, err
    assert O.cosine(Yh, ref) > 0.99999


@pytest.mark.parametrize("M,N,K", [(128, 3840, 15360), (512, 3840, 1920), (100, 320, 96), (256, 1024, 224)])
def test_w4a16_two_kgroups_match_one(gpu, M, N, K, tune):
    """128-row tiles can run two groups of 4 waves over the two halves of
    each workgroup's k-steps (forced here with the w4a16_kg override = 2) and add group
    1's sums into group 0's. Against the one-group kernel (w4a16_kg = 1)
    only the fp32 summation order differs. The shapes cover an odd k-step count per workgroup (group 1's
    surplus step reads zero scales), a one-block last k-step, and split-K."""
    rng = np.random.default_rng(M + N + K)
    q, s = synth_int4(rng, N, K)
    X = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).cuda()
    wq, sc = upload_int4(q, s)
    tune("w4a16_kg", "2")
    Y2 = to_np(gpu.gemm_w4a16(X, wq, sc, N)).astype(np.float64)
    tune("w4a16_kg", "1")
    Y1 = to_np(gpu.gemm_w4a16(X, wq, sc, N)).astype(np.float64)
    assert np.isfinite(Y2).all()
    assert np.abs(Y2 - Y1).max() <= np.abs(Y1).max() * 2.0 ** -9
    ref = O.gemm_w4a16_ref(to_np(X), q, s)
    assert O.normwise_rel_err(Y2.astype(np.float32), ref) <= 1e-3


def test_w4a16_two_kgroups_nonfinite_x(gpu, tune):
    """An Inf in X in the last k-step of group 1's range (each of the 16 K
    splits at M=128, N=3840, K=15360 gives group 1 an odd 7 of 15 k-steps):
    two k-groups give the one-group kernel's Inf/NaN pattern (NaN only where
    the dequantized weight is 0), so the odd group multiplies nothing extra."""
    M, N, K = 128, 3840, 15360
    rng = np.random.default_rng(5)
    q, s = synth_int4(rng, N, K)
    Xh = rng.standard_normal((M, K)).astype(np.float16)
    Xh[3, K - 1] = np.inf
    Xh[70, K - 40] = -np.inf
    X = torch.from_numpy(Xh).cuda()
    wq, sc = upload_int4(q, s)
    tune("w4a16_kg", "2")
    Y2 = to_np(gpu.gemm_w4a16(X, wq, sc, N)).astype(np.float64)
    tune("w4a16_kg", "1")
    Y1 = to_np(gpu.gemm_w4a16(X, wq, sc, N)).astype(np.float64)
    for m, k in ((3, K - 1), (70, K - 40)):
        zero_w = (q[:, k] == 8) | (s[:, k // 32] == 0)  # a dequantized weight of 0: Inf * 0
        assert np.isnan(Y1[m]).tolist() == zero_w.tolist()
        assert np.isinf(Y1[m][~zero_w]).all()
    assert (np.isnan(Y2) == np.isnan(Y1)).all()
    fin = np.isfinite(Y1)
    assert (Y2[~fin & ~np.isnan(Y1)] == Y1[~fin & ~np.isnan(Y1)]).all()
    assert np.isfinite(Y2[fin]).all()
    assert np.abs(Y2[fin] - Y1[fin]).max() <= np.abs(Y1[fin]).max() * 2.0 ** -9


@pytest.mark.parametrize("M,I,K,dev_interleave", [(128, 15360, 3840, True), (128, 512, 256, True),
                                                  (100, 330, 96, False), (37, 7, 224, False),
                                                  (512, 1024, 1920, True), (37, 35, 15360, False)])
def test_w4a16_gated_equals_separate_gemms_and_gelumul(gpu, M, I, K, dev_interleave, tune):
    """The gated W4A16 GEMM over interleaved gate/up rows gives the separate
    route's activations bit for bit (gate GEMM, up GEMM, each rounded to
    fp16, then gelumul) when both split K the same way (the w4a16_split override),
    and matches the oracle: gelu_tanh(f16(X Wg^T)) * f16(X Wu^T), rounded to
    fp16, within an fp16 step of the largest output. Shapes: the prefill
    chunk's gate/up (I 15360), a one-block last k-step (K % 64 = 32), an
    output count that is no multiple of 4 (the reduce's scalar tail; rows
    interleaved on the host, as q4_interleave_rows takes multiples of 32),
    and two k-groups at M = 512."""
    rng = np.random.default_rng(M + I + K)
    qg, sg = synth_int4(rng, I, K)
    qu, su = synth_int4(rng, I, K)
    X = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).cuda()
    wg, scg = upload_int4(qg, sg)
    wu, scu = upload_int4(qu, su)
    if dev_interleave:
        wi, si = gpu.interleave_rows(wg, scg, wu, scu, I, K)
    else:
        qi, s_i = np.empty((2 * I, K), qg.dtype), np.empty((2 * I, K // 32), sg.dtype)
        qi[0::2], qi[1::2], s_i[0::2], s_i[1::2] = qg, qu, sg, su
        wi, si = upload_int4(qi, s_i)
    split = max(1, gpu.gemm_workspace_bytes(M, 2 * I, K) // (M * 2 * I * 4))
    tune("w4a16_split", str(split))
    A = to_np(gpu.gemm_w4a16_gated(X, wi, si, 2 * I))
    G = gpu.gemm_w4a16(X, wg, scg, I)
    U = gpu.gemm_w4a16(X, wu, scu, I)
    sep = to_np(gpu.pre_gelumul(G.reshape(-1), U.reshape(-1), torch.empty(M * I, dtype=torch.float16,
                                                                            device="cuda"))).reshape(M, I)
    assert np.array_equal(A.view(np.uint16), sep.view(np.uint16))
    Xn = to_np(X)
    g16 = O.gemm_w4a16_ref(Xn, qg, sg).astype(np.float16).astype(np.float64)
    u16 = O.gemm_w4a16_ref(Xn, qu, su).astype(np.float16).astype(np.float64)
    act = D.gelumul_ref(g16, u16)
    assert np.abs(A.astype(np.float64) - act).max() <= np.abs(act).max() * 2.0 ** -9


@pytest.mark.parametrize("M,N,K,fuse_norm", [(128, 3840, 4096, True), (128, 3840, 15360, True),
                                              (100, 320, 96, False), (37, 256, 224, True), (512, 1024, 1920, True)])
def test_w4a16_normadd_equals_gemm_then_normadd(gpu, M, N, K, fuse_norm):
    """The GEMM handing its split-K partials to the normadd (and the rmsnorm
    after it) gives h and y bit for bit as q4_gemm_w4a16_ws (fp16 output)
    followed by q4_pre_normadd(_rmsnorm): the normadd sums the partials in
    split order and rounds to fp16 as the reduce does. Shapes: the prefill
    o (K 4096) and down (K 15360) projections, a one-block last k-step, a
    row count that is no multiple of the tile, two k-groups at M = 512."""
    rng = np.random.default_rng(M + N + K)
    q, s = synth_int4(rng, N, K)
    wq, sc = upload_int4(q, s)
    X = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).cuda()
    w = torch.from_numpy((rng.random(N) + 0.5).astype(np.float32)).cuda()
    w2 = torch.from_numpy((rng.random(N) + 0.5).astype(np.float32)).cuda()
    h0 = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).cuda()
    h1, h2 = h0.clone(), h0.clone()
    Y = gpu.gemm_w4a16(X, wq, sc, N)
    if fuse_norm:
        y1 = gpu.pre_normadd(Y, w, h1, M=M, D=N, scale=0.5, w2=w2, y_dtype=torch.float16)
        y2 = gpu.gemm_w4a16_normadd(X, wq, sc, N, w, h2, scale=0.5, w2=w2, y_dtype=torch.float16)
        assert torch.equal(y1, y2)
    else:
        gpu.pre_normadd(Y, w, h1, M=M, D=N, scale=0.5)
        gpu.gemm_w4a16_normadd(X, wq, sc, N, w, h2, scale=0.5)
    assert torch.equal(h1, h2)


@pytest.mark.parametrize("M,nH,nkv,hd,keqv,window,stride,p0", [
    (128, 16, 8, 256, False, 1024, 1024, 3968),   # a sliding layer of the prefill chunk
    (128, 16, 1, 512, True, 0, 4096, 3968),       # a global layer (k == v)
    (37, 4, 2, 64, False, 16, 16, 5),             # ragged M; the chunk wraps the 16-slot ring
    (64, 4, 2, 128, True, 0, 80, 40),             # global, positions past the cache depth write nothing
])
def test_w4a16_qkv_prepkv_equals_gemm_then_prepkv(gpu, M, nH, nkv, hd, keqv, window, stride, p0):
    """The stacked q/k/v GEMM with its reduce and the prepkv in one launch
    gives the q rows and both caches bit for bit as q4_gemm_w4a16_ws (fp16
    output) followed by q4_pre_prepkv on its k/v columns."""
    rng = np.random.default_rng(M + nH + hd + p0)
    nq, nk = nH * hd, nkv * hd
    N, K = nq + nk * (1 if keqv else 2), 512
    q, s = synth_int4(rng, N, K)
    wq, sc = upload_int4(q, s)
    X = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).cuda()
    knw = torch.from_numpy((rng.random(hd) + 0.5).astype(np.float32)).cuda()
    cosM = torch.from_numpy((rng.random(M * hd) - 0.5).astype(np.float32)).cuda()
    sinM = torch.from_numpy((rng.random(M * hd) - 0.5).astype(np.float32)).cuda()
    dyn = torch.tensor([p0, M, 0, 0], dtype=torch.int32, device="cuda")
    kc0 = torch.from_numpy(rng.standard_normal(nkv * stride * hd).astype(np.float16)).cuda()
    vc0 = torch.from_numpy(rng.standard_normal(nkv * stride * hd).astype(np.float16)).cuda()
    kc1, vc1, kc2, vc2 = kc0.clone(), vc0.clone(), kc0.clone(), vc0.clone()
    Y = gpu.gemm_w4a16(X, wq, sc, N)
    Yf = Y.reshape(-1)
    gpu.pre_prepkv(Yf[nq:], Yf[nq if keqv else nq + nk:], knw, cosM, sinM, kc1, vc1, M=M, ld=N, nkv=nkv, hd=hd,
                   stride=stride, window=window, dyn=dyn)
    Q = torch.zeros(M, N, dtype=torch.float16, device="cuda")
    gpu.gemm_w4a16_qkv_prepkv(X, wq, sc, N, Q, knw, cosM, sinM, kc2, vc2, nq=nq, ldq=N, nkv=nkv, hd=hd, keqv=keqv,
                              stride=stride, window=window, dyn=dyn)
    assert torch.equal(Q[:, :nq], Y[:, :nq])
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)


def test_w4a16_matches_f16_rounded_weights(gpu):
    """The kernel's dequant is f16((q-8)*s) per weight: against that exact
    product (computed in float64) the only remaining error is fp32
    accumulation and the final fp16 rounding."""
    rng = np.random.default_rng(31)
    M, N, K = 96, 384, 512
    q, s = synth_int4(rng, N, K)
    X = rng.standard_normal((M, K)).astype(np.float16)
    Wh = O.dequant(q, s).astype(np.float16).astype(np.float64)
    ref = X.astype(np.float64) @ Wh.T
    wq, sc = upload_int4(q, s)
    Y = to_np(gpu.gemm_w4a16(torch.from_numpy(X).cuda(), wq, sc, N)).astype(np.float64)
    assert np.abs(Y - ref).max() <= np.abs(ref).max() * 2.0 ** -11 * 1.01
