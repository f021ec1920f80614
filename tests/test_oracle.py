"""Pins of the CPU oracle (oracle/q4_oracle.py).

The reference ships no golden vectors or known-answer tests for this path
(its checks are cosine thresholds in benchmarks/*.py), so each oracle
function is pinned here by hand-computed known answers, closed forms,
exhaustive tables, a third-party library routine (torch's float8_e4m3fn for
the e4m3 codec, the dependency src/vk_engine.py:136 calls), or brute force
on tiny inputs. Each check is chosen so that a plausible slip (dropped
term, wrong sign/index, transposed operand, wrong rounding) fails it.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import q4_oracle as O
from tests.helpers import W8A8_EPILOGUE_KATS


# ------------------------------------------------------------ quant codes
def test_quant_codes_known_answer_with_ties():
    # block max 7 -> scale exactly 1, so codes are rint(W) + 8 (half-to-even)
    row = np.zeros(32, np.float32)
    row[:9] = [7.0, -7.0, 3.5, -3.5, 0.5, 1.5, 2.5, -2.5, 6.49]
    q, sc = O.quant_codes(row[None, :])
    assert sc.dtype == np.float32 and sc[0, 0] == np.float32(1.0)
    assert list(q[0, :9]) == [15, 1, 12, 4, 8, 10, 10, 6, 14]
    assert (q[0, 9:] == 8).all()


def test_quant_codes_zero_block_and_scale_floor():
    W = np.zeros((2, 64), np.float32)
    W[1, 32] = 0.7  # second block of row 1: scale 0.1 (fp32 0.7/7)
    q, sc = O.quant_codes(W)
    assert sc[0, 0] == np.float32(1e-8) and sc[0, 1] == np.float32(1e-8)
    assert sc[1, 1] == np.float32(0.7) / np.float32(7.0)
    assert (q[0] == 8).all() and q[1, 32] == 15 and (q[1, 33:] == 8).all()


def test_quant_codes_reconstruction_bound():
    rng = np.random.default_rng(1)
    W = rng.standard_normal((16, 256)).astype(np.float32)
    q, sc = O.quant_codes(W)
    Wdq = O.dequant(q, sc)
    # rounding to the nearest code: error at most half a step per element
    step = np.repeat(sc, 32, axis=1)
    assert (np.abs(Wdq - W) <= 0.5 * step * (1 + 1e-6)).all()
    assert q.min() >= 1 and q.max() <= 15  # symmetric quantizer never emits code 0


# ------------------------------------------------------- reference packing
def test_pack_ref_known_word():
    q = np.arange(8, dtype=np.uint8).reshape(8, 1)  # q[n, 0] = n
    assert O.pack_ref(q)[0, 0] == 0x76543210


def test_pack_ref_bruteforce_and_roundtrip():
    rng = np.random.default_rng(2)
    N, K = 24, 5
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    wp = O.pack_ref(q)
    assert wp.shape == (K, N // 8)
    for k in range(K):
        for n in range(N):
            assert (int(wp[k, n // 8]) >> (4 * (n % 8))) & 15 == q[n, k]
    assert (O.unpack_ref(wp, N) == q).all()


def test_pack_ref_exhaustive_codes_positions():
    # every code at every nibble position survives the round trip
    q = np.array([[(c + j) % 16 for c in range(16)] for j in range(8)], np.uint8)  # [8, 16]
    assert (O.unpack_ref(O.pack_ref(q), 8) == q).all()


# ----------------------------------------------------------- device layout
def test_pack_dev_known_word():
    q = np.zeros((64, 32), np.uint8)
    q[0, :8] = np.arange(8)      # elements e = 0..7 of word 0 of (row 0, block 0)
    q[1, 8:16] = 0xF             # word 1 of row 1 all ones
    words = O.pack_dev(q).reshape(1, 1, 64, 4)   # p, b, r, i
    assert words[0, 0, 0, 0] == 0x75316420       # nibble pos (e&1)*4 + (e>>1)
    assert words[0, 0, 1, 1] == 0xFFFFFFFF and words[0, 0, 1, 0] == 0


def test_pack_dev_unit_order_and_padding():
    N, K = 70, 64                                  # 2 panels (second one padded), 2 blocks
    q = np.zeros((N, K), np.uint8)
    q[65, 32] = 9                                  # row 65 = panel 1 lane 1, block 1, word 0, e 0
    words = O.pack_dev(q)
    nblk = 2
    unit = ((65 // 64) * nblk + 1) * 64 + 65 % 64
    assert words[4 * unit] == 9
    assert words.size == 128 * nblk * 4
    w = words.reshape(2, nblk, 64, 4)
    assert (w[1, :, 6:, :] == 0x88888888).all()   # padded rows hold code 8


def test_pack_dev_roundtrip_random():
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, (100, 96), dtype=np.uint8)
    assert (O.unpack_dev(O.pack_dev(q), 100, 96) == q).all()
    s = rng.standard_normal((100, 3)).astype(np.float16)
    assert (O.unscales_dev(O.scales_dev(s), 100, 3) == s).all()


def test_pack_w8_dev_known_positions():
    """Chunk l of block (t, s) = row 32t + l % 32, bytes 32s + 16 (l // 32) .. +16."""
    N, K = 70, 192                                  # 3 n-tiles (last padded), K padded to 256
    W8 = np.zeros((N, K), np.int8)
    W8[33, 2 * 32 + 16 + 5] = 7                     # t=1, r=1, s=2, h=1, byte 5
    W8[69, 191] = -3                                # t=2, r=5, s=5, h=1, byte 15
    flat = O.pack_w8_dev(W8)
    kp = 256 // 32
    assert flat.size == 96 * 256
    assert flat[(1 * kp + 2) * 1024 + (32 + 1) * 16 + 5] == 7
    assert flat[(2 * kp + 5) * 1024 + (32 + 5) * 16 + 15] == -3
    assert np.count_nonzero(flat) == 2              # padding (rows 70..95, bytes 192..255) is zero


def test_pack_w8_dev_roundtrip_random():
    rng = np.random.default_rng(5)
    for N, K in [(64, 128), (100, 320), (32, 3840)]:
        W8 = rng.integers(-127, 128, (N, K), dtype=np.int8)
        assert (O.unpack_w8_dev(O.pack_w8_dev(W8), N, K) == W8).all()


def test_scales_f16_ref_layout():
    sc = np.array([[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], np.float32)  # [N=3, nblk=2]
    assert O.scales_f16_ref(sc).tolist() == [[1.0, 3.0, 5.0], [2.0, 4.0, 6.0]]


def test_split_ref_matches_reference_comments():
    # src/vk_engine.py:138-142 quote: lm_head -> 1, down (rows 8) -> 48, gate (rows 30) -> 12
    assert O.split_ref(262144, 120) == 1
    assert O.split_ref(3840, 480) == 48
    assert O.split_ref(15360, 120) == 12


# ---------------------------------------------------------------- e4m3
def _torch_decode_all():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    return codes.view(torch.float8_e4m3fn).to(torch.float32).numpy()


def test_e4m3_decode_exhaustive_vs_torch():
    ours = O.e4m3_decode(np.arange(256))
    ref = _torch_decode_all()
    finite = np.isfinite(ref)
    assert finite.sum() == 254  # 0x7F and 0xFF are NaN in e4m3fn
    assert (ours[finite] == ref[finite]).all()
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9 and ours[0x08] == 2.0 ** -6


def test_e4m3_encode_exact_values_roundtrip():
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)])
    vals = O.e4m3_decode(codes)
    enc = O.e4m3_encode(vals)
    assert (enc == codes).all()


def test_e4m3_encode_midpoints_tie_to_even():
    codes = np.arange(0, 0x7E)  # consecutive positive codes
    lo, hi = O.e4m3_decode(codes), O.e4m3_decode(codes + 1)
    mid = ((lo.astype(np.float64) + hi) / 2).astype(np.float32)
    assert (mid.astype(np.float64) == (lo.astype(np.float64) + hi) / 2).all()  # exact midpoints
    enc = O.e4m3_encode(mid)
    want = np.where(codes % 2 == 0, codes, codes + 1)
    assert (enc == want).all()


def test_e4m3_encode_dense_sweep_vs_torch():
    rng = np.random.default_rng(4)
    v = np.concatenate([
        rng.uniform(0, 448, 200000), np.exp2(rng.uniform(-14, 8.8, 200000)),
        rng.uniform(0, 2.0 ** -6, 50000)]).astype(np.float32)
    v = np.clip(v, 0, 448).astype(np.float32)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert (O.e4m3_encode(v) == ref).all()
    assert (O.e4m3_encode(-v[:1000]) == torch.from_numpy(-v[:1000]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()).all()


def test_e4m3_lift_known_shift():
    sc = np.full((4, 2), 0.01, np.float32)
    sc[2, 1] = 0.1
    e8, inv, shift = O.e4m3_lift(sc)
    assert shift == 11 and inv == 2.0 ** -11          # floor(log2(256 / 0.1)) = floor(11.32)
    assert O.e4m3_decode(e8[2, 1]) == O.e4m3_decode(O.e4m3_encode(np.float32(0.1) * np.float32(2048)))
    # max scale lands in [128, 256): inside e4m3's normal band
    assert 128 <= O.e4m3_decode(e8).max() < 256


def test_e4m3_lift_power_of_two_edge():
    sc = np.array([[0.5, 0.25]], np.float32)         # 256 / 0.5 = 512 exactly -> shift 9
    _, inv, shift = O.e4m3_lift(sc)
    assert shift == 9 and inv == 2.0 ** -9


# -------------------------------------------------------- GEMV / W4A16
def _brute_gemv(q, s, x):
    N, K = q.shape
    y = np.zeros(N)
    for n in range(N):
        for k in range(K):
            y[n] += (int(q[n, k]) - 8) * float(s[n, k // 32]) * float(x[k])
    return y


def test_gemv_ref_bruteforce():
    rng = np.random.default_rng(5)
    N, K = 8, 64
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    s = np.abs(rng.normal(0, 0.02, (N, 2))).astype(np.float16).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float16)
    y = O.gemv_ref(q, s, x)
    assert O.normwise_rel_err(y, _brute_gemv(q, s, x)) < 1e-6
    # inv is a plain output factor
    assert np.allclose(O.gemv_ref(q, s, x, inv=0.25), 0.25 * y, rtol=0, atol=0)


def test_gemv_ref_code8_is_zero_and_sign():
    q = np.full((2, 32), 8, np.uint8)
    q[0, 3] = 9      # +1
    q[1, 5] = 0      # -8
    s = np.array([[2.0], [0.5]], np.float32)
    x = np.arange(32, dtype=np.float32)
    assert O.gemv_ref(q, s, x).tolist() == [2.0 * 3, -8 * 0.5 * 5]


def test_gemm_w4a16_ref_bruteforce_and_transpose():
    rng = np.random.default_rng(6)
    M, N, K = 3, 4, 64
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    s = rng.uniform(0.01, 0.03, (N, 2)).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float16)
    Y = O.gemm_w4a16_ref(X, q, s)
    assert Y.shape == (M, N)
    for m in range(M):
        assert O.normwise_rel_err(Y[m], _brute_gemv(q, s, X[m])) < 1e-6


# ------------------------------------------------------ int8 activations
def test_quant_act_i8_ties_and_extremes():
    # absmax 127 -> scale exactly 1: codes are rint(x) with ties to even
    X = np.array([[127.0, 2.5, 3.5, -2.5, -0.5, 0.49, -127.0, 1.5]], np.float32)
    A, sa = O.quant_act_i8(X)
    assert sa[0] == np.float32(1.0)
    assert A[0].tolist() == [127, 2, 4, -2, 0, 0, -127, 2]


def test_quant_act_i8_zero_row_and_fp16_input():
    X = np.zeros((2, 8), np.float16)
    X[1] = [1, -2, 0.5, 0, 0, 0, 0, 0.25]
    A, sa = O.quant_act_i8(X)
    assert sa[0] == np.float32(1e-12) and (A[0] == 0).all()
    assert sa[1] == np.float32(2.0) / np.float32(127.0)
    assert A[1, 1] == -127 and A[1, 0] == 64   # 1 / (2/127) = 63.5 -> 64 (tie to even)


def test_quant_act_i8_uses_division_not_reciprocal():
    # choose x, s where x/s and x*(1/s) round to different integers
    rng = np.random.default_rng(7)
    hits = 0
    for _ in range(2000):
        mx = np.float32(rng.uniform(1, 100))
        s = np.maximum(mx / np.float32(127.0), np.float32(1e-12))
        k = rng.integers(-126, 126)
        x = np.float32((k + 0.5) * s)
        a_div = np.rint(x / s)
        a_rcp = np.rint(x * (np.float32(1.0) / s))
        if a_div != a_rcp:
            A, _ = O.quant_act_i8(np.array([[mx, x]], np.float32))
            assert A[0, 1] == a_div
            hits += 1
    assert hits > 0


# ------------------------------------------------------------ W8 fold
def test_w8_fold_known_answer():
    q = np.full((1, 64), 8, np.uint8)
    q[0, 0] = 15     # +7
    q[0, 1] = 1      # -7
    q[0, 40] = 12    # +4 in block 1
    sc = np.array([[1.0, 2.0]], np.float32)   # deq: 7, -7, ..., 8 (block 1)
    W8, sw = O.w8_fold(q, sc)
    assert sw[0] == np.float32(8.0) / np.float32(127.0)
    assert W8[0, 40] == 127
    assert W8[0, 0] == int(np.rint(np.float32(7.0) / sw[0])) == 111
    assert W8[0, 1] == -111 and (W8[0, 2:40] == 0).all()


def test_w8_fold_uses_unrounded_scale():
    q = np.full((1, 32), 8, np.uint8)
    q[0, 0], q[0, 1] = 15, 9
    sc = np.array([[np.float32(1.0) / np.float32(3.0)]], np.float32)  # not an fp16 value
    W8, sw = O.w8_fold(q, sc)
    deq1 = np.float32(1.0) * sc[0, 0]
    assert W8[0, 1] == np.rint(deq1 / sw[0])
    assert O.w4a8_ratio(sc, sw).dtype == np.float16


def _rne(x: Fraction, p: int) -> Fraction:
    """x > 0 rounded to p significant bits, ties to even (normal range)."""
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    ulp = Fraction(2) ** (e - p + 1)
    m = x / ulp
    f = m.numerator // m.denominator
    rem = m - f
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and f % 2):
        f += 1
    return f * ulp


def _f32(bits: int) -> np.float32:
    return np.array([bits], np.uint32).view(np.float32)[0]


def _f16_bits(v: Fraction) -> int:
    return int(np.array([float(v)], np.float64).astype(np.float16).view(np.uint16)[0])


# W4A8 ratio (benchmarks/coopgemm_w4a8.py:84): fp32 sc / fp32 s_w, rounded to
# fp32 by the division, then to fp16. Known answers worked out with exact
# rational arithmetic (quotient of the two fp32 values, round to 24 bits, then
# to 11 bits); each value pair is chosen so that a plausible mistake gives a
# different fp16 pattern.
#   pair A (sc 0x3c82ed64 = 0.015982337, s_w 0x3b1909c5 = 0.002335177):
#     f16(sc/s_w) = 0x46d8, swapped f16(s_w/sc) = 0x30ad,
#     f16(f16(sc)/s_w) = 0x46d7, f16(sc/f16(s_w)) = 0x46d9
#   pair B (sc 0x3a384351, s_w 0x3a382c4b): the fp32 quotient is exactly the
#     fp16 midpoint 1 + 2^-11, which ties to even (0x3c00); rounding the exact
#     quotient straight to fp16 would give 0x3c01, and f16(s_w/sc) 0x3bff.
_RATIO_PINS = [(0x3C82ED64, 0x3B1909C5, 0x46D8, (0x30AD, 0x46D7, 0x46D9)),
               (0x3A384351, 0x3A382C4B, 0x3C00, (0x3BFF, 0x3C01))]


@pytest.mark.parametrize("sc_bits,sw_bits,want,wrong", _RATIO_PINS)
def test_w4a8_ratio_known_answer(sc_bits, sw_bits, want, wrong):
    sc, sw = _f32(sc_bits), _f32(sw_bits)
    # the known answer from exact arithmetic: two roundings, fp32 then fp16
    exact = Fraction(float(sc)) / Fraction(float(sw))
    assert _f16_bits(_rne(_rne(exact, 24), 11)) == want
    got = O.w4a8_ratio(np.array([[sc]], np.float32), np.array([sw], np.float32))
    assert got.dtype == np.float16 and got.shape == (1, 1)
    assert int(got.view(np.uint16)[0, 0]) == want
    assert want not in wrong
    # the alternatives really are the patterns quoted above
    alts = [_f16_bits(_rne(_rne(Fraction(float(sw)) / Fraction(float(sc)), 24), 11))]
    if len(wrong) == 3:
        sc16 = Fraction(float(np.float16(sc)))
        sw16 = Fraction(float(np.float16(sw)))
        alts += [_f16_bits(_rne(_rne(sc16 / Fraction(float(sw)), 24), 11)),
                 _f16_bits(_rne(_rne(Fraction(float(sc)) / sw16, 24), 11))]
    else:
        alts += [_f16_bits(_rne(exact, 11))]
    assert tuple(alts) == wrong


def test_w4a8_ratio_layout():
    # row n divides by s_w[n], block b takes sc[n, b]: [N, nblk] out, no transpose
    sc = np.array([[0.5, 1.0, 2.0], [3.0, 6.0, 12.0]], np.float32)
    sw = np.array([0.25, 1.5], np.float32)
    got = O.w4a8_ratio(sc, sw)
    assert got.shape == (2, 3)
    np.testing.assert_array_equal(got.astype(np.float32), np.array([[2, 4, 8], [2, 4, 8]], np.float32))
    sw2 = np.array([0.25, 0.5], np.float32)
    np.testing.assert_array_equal(O.w4a8_ratio(sc, sw2).astype(np.float32),
                                  np.array([[2, 4, 8], [6, 12, 24]], np.float32))


def test_w4a8_weights_known_answer():
    q = np.array([[15, 1, 8, 10, 11] + [8] * 27], np.uint8)
    r = np.array([[np.float16(1.25)]])
    B = O.w4a8_weights(q, r)
    # (7, -7, 0, 2, 3) * 1.25 = 8.75, -8.75, 0, 2.5, 3.75 -> 9, -9, 0, 2 (tie to even), 4
    assert B[0, :5].tolist() == [9, -9, 0, 2, 4]
    B2 = O.w4a8_weights(q, np.array([[np.float16(100.0)]]))
    assert B2[0, 0] == 127 and B2[0, 1] == -127


# --------------------------------------------------------- int matmul
def test_int_matmul_exact_vs_int64():
    rng = np.random.default_rng(8)
    A = rng.integers(-127, 128, (17, 256), dtype=np.int8)
    B = rng.integers(-127, 128, (9, 256), dtype=np.int8)
    C = O.int_matmul_exact(A, B)
    assert C.dtype == np.int32
    assert (C == (A.astype(np.int64) @ B.astype(np.int64).T)).all()
    # worst case magnitude at K = 15360 stays exact
    Aw = np.full((1, 15360), 127, np.int8)
    assert O.int_matmul_exact(Aw, -Aw)[0, 0] == -127 * 127 * 15360
    with pytest.raises(ValueError):
        O.int_matmul_exact(np.zeros((1, 140000), np.int8), np.zeros((1, 140000), np.int8))


def test_w8a8_epilogue_order_and_rounding():
    C = np.array([[3, -5], [1000, 7]], np.int32)
    sa = np.array([0.5, 0.25], np.float32)
    sw = np.array([2.0, 0.125], np.float32)
    Y = O.w8a8_epilogue(C, sa, sw)
    # powers of two: exact products, one f16 rounding; row scale sa[m], column scale sw[n]
    assert Y.tolist() == [[3.0, -0.3125], [500.0, 0.21875]]
    # 2049 is a tie between 2048 and 2050 in f16 -> even
    C1 = np.array([[2049]], np.int32)
    Y1 = O.w8a8_epilogue(C1, np.array([1.0], np.float32), np.array([1.0], np.float32))
    assert Y1[0, 0] == np.float16(2048.0)


def test_w8a8_epilogue_known_answers_separate_orders():
    for C, sab, swb, want in W8A8_EPILOGUE_KATS:
        sa = np.array([sab], np.uint32).view(np.float32)
        sw = np.array([swb], np.uint32).view(np.float32)
        Y = O.w8a8_epilogue(np.array([[C]], np.int32), sa, sw)
        assert Y[0, 0] == np.float16(want)
        Cf = np.float32(C)
        exact = float(C) * float(sa[0]) * float(sw[0])
        others = [np.float16(Cf * (sa[0] * sw[0])), np.float16((Cf * sw[0]) * sa[0]), np.float16(exact),
                  np.float16(np.float32(exact))]
        assert all(o.view(np.uint16) != Y[0, 0].view(np.uint16) for o in others), (C, others)


def test_normwise_metric():
    assert O.normwise_rel_err([1.0, 2.0], [1.0, 2.0]) == 0.0
    assert O.normwise_rel_err([1.1, 2.0], [1.0, 2.0]) == pytest.approx(0.05)
    assert O.cosine([1, 0], [0, 1]) == pytest.approx(0.0)
