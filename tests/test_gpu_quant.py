"""GPU quantizer / repack kernels vs the oracle: bit-exact."""
import numpy as np
import pytest
import torch

from oracle import q4_oracle as O
from tests.helpers import to_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,K,scale", [(64, 32, 1.0), (100, 96, 0.08), (256, 3840, 0.05), (8, 64, 1e-7)])
def test_quantize_bit_exact(gpu, N, K, scale):
    rng = np.random.default_rng(N + K)
    W = (rng.standard_normal((N, K)) * scale).astype(np.float32)
    W[0, :32] = 0.0                                   # zero block -> 1e-8 floor
    if N > 3:
        W[3, :32] = np.linspace(-7, 7, 32) * scale    # exact ties after scaling
    q, sc = O.quant_codes(W)
    wq, sc16, sc32 = gpu.quantize(torch.from_numpy(W).cuda())
    assert (to_np(wq).view(np.uint32) == O.pack_dev(q)).all()
    assert (to_np(sc32) == sc).all()
    want16 = O.scales_dev(sc.astype(np.float16))
    assert (to_np(sc16).view(np.uint16) == want16.view(np.uint16)).all()


@pytest.mark.parametrize("N,K", [(64, 64), (300, 256), (4096, 3840)])
def test_scales_e4m3_bit_exact(gpu, N, K):
    rng = np.random.default_rng(11)
    sc = np.abs(rng.normal(0, 0.02, (N, K // 32))).astype(np.float32)
    sc[0, 0] = 1e-8
    e8, inv, _ = O.e4m3_lift(sc)
    sc8, inv_gpu = gpu.scales_e4m3(torch.from_numpy(sc).cuda(), N, K)
    assert inv_gpu == inv
    assert (to_np(sc8) == O.scales_dev(e8)).all()


def test_e4m3_encoder_exhaustive_band(gpu):
    # every e4m3 value and every midpoint between neighbours, through the lift kernel
    codes = np.arange(0, 0x7F)
    vals = O.e4m3_decode(codes).astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    keep = vals <= 256.0                            # max 256 -> shift 0: values encode as themselves
    v = np.concatenate([vals[keep], mids[keep[1:]]]).astype(np.float32)
    v = np.concatenate([v, np.zeros(256 - v.size, np.float32)])
    N = v.size // 2
    sc = v.reshape(N, 2)                            # K = 64 -> 2 blocks per row
    e8, inv, shift = O.e4m3_lift(sc)
    assert shift == 0
    sc8, inv_gpu = gpu.scales_e4m3(torch.from_numpy(sc).cuda(), N, 64)
    assert inv_gpu == 1.0 and (to_np(sc8) == O.scales_dev(e8)).all()


@pytest.mark.parametrize("N,K", [(64, 64), (130, 96), (512, 3840)])
def test_w8_fold_and_ratio_bit_exact(gpu, N, K):
    rng = np.random.default_rng(12)
    W = (rng.standard_normal((N, K)) * 0.08).astype(np.float32)
    q, sc = O.quant_codes(W)
    W8, sw = O.w8_fold(q, sc)
    wq, _sc16, sc32 = gpu.quantize(torch.from_numpy(W).cuda())
    gW8, gsw32, gsw16 = gpu.w8_fold(wq, sc32, N, K)
    assert (to_np(gW8) == W8).all()
    assert (to_np(gsw32) == sw).all()
    assert (to_np(gsw16) == sw.astype(np.float16)).all()
    ratio = O.w4a8_ratio(sc, sw)
    gr = gpu.w4a8_ratio(sc32, gsw32, N, K)
    assert (to_np(gr).view(np.uint16) == O.scales_dev(ratio).view(np.uint16)).all()


@pytest.mark.parametrize("N,K", [(64, 32), (104, 96), (1024, 256)])
def test_repack_ref_bit_exact(gpu, N, K):
    rng = np.random.default_rng(13)
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    s = np.abs(rng.normal(0, 0.02, (N, K // 32))).astype(np.float16)
    wp = O.pack_ref(q)                                  # [K, N/8]
    sc_ref = O.scales_f16_ref(s.astype(np.float32))     # [nblk, N]
    wq, scd = gpu.repack_ref(torch.from_numpy(wp.view(np.int32)).cuda(), torch.from_numpy(sc_ref).cuda(), N, K)
    assert (to_np(wq).view(np.uint32) == O.pack_dev(q)).all()
    assert (to_np(scd).view(np.uint16) == O.scales_dev(s).view(np.uint16)).all()
    e8 = rng.integers(0, 0x7F, (K // 32, N), dtype=np.uint8)
    d8 = gpu.repack_e4m3_ref(torch.from_numpy(e8).cuda(), N, K)
    assert (to_np(d8) == O.scales_dev(np.ascontiguousarray(e8.T))).all()
    w8 = rng.integers(-127, 128, (K, N), dtype=np.int8)
    assert (to_np(gpu.repack_w8_ref(torch.from_numpy(w8).cuda(), N, K)) == w8.T).all()


def test_casts_bit_exact(gpu):
    rng = np.random.default_rng(14)
    x = (rng.standard_normal(1003) * 1000).astype(np.float32)
    x[:4] = [65520.0, 1e-8, -0.0, 3e-5]
    h = gpu.cast_f32_f16(torch.from_numpy(x).cuda())
    assert (to_np(h).view(np.uint16) == x.astype(np.float16).view(np.uint16)).all()
    back = gpu.cast_f16_f32(h)
    assert (to_np(back) == x.astype(np.float16).astype(np.float32)).all()
