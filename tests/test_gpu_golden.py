"""Every step of the HIP path on the committed golden fixture
(``tests/golden/q4_small.npz``), through the C ABI: bit-exact for codes,
scales, int8 weights and activations and int32 accumulators; normwise
``max|y - ref| / max|ref|`` within 2e-5 (fp32 outputs) or 1e-3 (fp16
outputs) for the fp32-accumulated products."""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import q4_oracle as O
from tests.helpers import to_np

pytestmark = pytest.mark.gpu

FIX = Path(__file__).resolve().parent / "golden" / "q4_small.npz"


@pytest.fixture(scope="module")
def gold():
    with np.load(FIX, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_golden_quantizer_and_formats(gpu, gold):
    N, K = int(gold["N"]), int(gold["K"])
    nblk = K // 32
    print(f"golden quantizer N={N} K={K}", flush=True)
    wq, sc16, sc32 = gpu.quantize(_dev(gold["W"]))
    assert (O.unpack_dev(to_np(wq).view(np.uint32), N, K) == gold["q"]).all()
    assert (to_np(sc32) == gold["sc"]).all()
    assert (O.unscales_dev(to_np(sc16), N, nblk).view(np.uint16) == gold["scb16_ref"].T.view(np.uint16)).all()
    # the reference's own storage layouts convert to the same device words
    wq2, sc2 = gpu.repack_ref(_dev(gold["wp_ref"].view(np.int32)), _dev(gold["scb16_ref"]), N, K)
    assert (to_np(wq2) == to_np(wq)).all() and (to_np(sc2).view(np.uint16) == to_np(sc16).view(np.uint16)).all()
    sc8, inv = gpu.scales_e4m3(sc32, N, K)
    assert inv == float(gold["e4m3_inv"])
    assert (O.unscales_dev(to_np(sc8), N, nblk) == gold["e8"]).all()
    W8, sw32, sw16 = gpu.w8_fold(wq, sc32, N, K)
    assert (to_np(W8) == gold["W8"]).all()
    assert (to_np(sw32) == gold["sw32"]).all()
    assert (to_np(sw16).view(np.uint16) == gold["sw16"].view(np.uint16)).all()
    ratio = gpu.w4a8_ratio(sc32, sw32, N, K)
    assert (O.unscales_dev(to_np(ratio), N, nblk).view(np.uint16) == gold["ratio"].view(np.uint16)).all()
    assert (to_np(gpu.w4a8_weights(wq, ratio, N, K)) == gold["W8_w4a8"]).all()


def test_golden_gemv(gpu, gold):
    N, K = int(gold["N"]), int(gold["K"])
    print(f"golden gemv N={N} K={K}", flush=True)
    wq, sc16, sc32 = gpu.quantize(_dev(gold["W"]))
    x = _dev(gold["x"])
    y32 = gpu.gemv(x, wq, sc16, N, K, y_dtype=torch.float32)
    assert O.normwise_rel_err(to_np(y32), gold["y_f16s"]) <= 2e-5
    y16 = gpu.gemv(x, wq, sc16, N, K, y_dtype=torch.float16)
    assert O.normwise_rel_err(to_np(y16), gold["y_f16s"]) <= 1e-3
    sc8, inv = gpu.scales_e4m3(sc32, N, K)
    y8 = gpu.gemv(x, wq, sc8, N, K, scale_fmt=gpu.SCALE_E4M3, inv=inv, y_dtype=torch.float32)
    assert O.normwise_rel_err(to_np(y8), gold["y_e4m3"]) <= 2e-5


def test_golden_prefill_gemms(gpu, gold):
    N, K = int(gold["N"]), int(gold["K"])
    print(f"golden prefill GEMMs M={int(gold['M'])} N={N} K={K}", flush=True)
    A, sa = gpu.quant_act_i8(_dev(gold["X"]))
    assert (to_np(A) == gold["A"]).all() and (to_np(sa) == gold["sa"]).all()
    W8 = _dev(gold["W8"])
    for sw, want in ((gold["sw32"], gold["Y_w8a8_sw32"]), (gold["sw16"], gold["Y_w8a8_sw16"])):
        Y, C = gpu.gemm_w8a8(A, W8, sa, _dev(sw), want_c=True)
        assert (to_np(C) == gold["C_w8a8"]).all()
        assert (to_np(Y).view(np.uint16) == want.view(np.uint16)).all()
        Yp, Cp = gpu.gemm_w8a8_packed(A, gpu.w8_pack(W8), sa, _dev(sw), N, want_c=True)
        assert (to_np(Cp) == gold["C_w8a8"]).all()
        assert (to_np(Yp).view(np.uint16) == want.view(np.uint16)).all()
    wq, sc16, sc32 = gpu.quantize(_dev(gold["W"]))
    ratio = gpu.w4a8_ratio(sc32, _dev(gold["sw32"]), N, K)
    Y4, C4 = gpu.gemm_w4a8(A, wq, ratio, sa, _dev(gold["sw32"]), N, want_c=True)
    assert (to_np(C4) == gold["C_w4a8"]).all()
    assert (to_np(Y4).view(np.uint16) == gold["Y_w4a8"].view(np.uint16)).all()
    Yh = gpu.gemm_w4a16(_dev(gold["X"]), wq, sc16, N)
    assert O.normwise_rel_err(to_np(Yh), gold["Y_w4a16"]) <= 1e-3
