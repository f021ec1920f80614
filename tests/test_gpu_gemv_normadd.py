"""GEMVs with the normadd + rmsnorm before them fused into their launch
(q4_gemv_normadd, q4_gemv_batch_normadd) against the oracle (float64
normadd and rmsnorm, then the fp32 GEMV of the fp16-rounded norm output)
and against the two-launch sequence they replace (q4_normadd_rmsnorm, then
q4_gemv / q4_gemv_batch / q4_gemv_gated)."""
import ctypes as C
import os

import numpy as np
import pytest
import torch

from oracle import decode_ops_oracle as D
from oracle import q4_oracle as O
from tests.helpers import synth_int4, to_np, upload_int4

pytestmark = pytest.mark.gpu


def _norm_inputs(rng, K):
    a = (rng.standard_normal(K) * 3.0).astype(np.float32)
    h = (rng.standard_normal(K) * 20.0).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    w2 = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    return a, h, w, w2


def _oracle_x(a, w, h, w2, scale):
    hn = D.normadd_ref(a, w, h, scale)
    return hn, D.rmsnorm_ref(hn, w2).astype(np.float16).astype(np.float32)


def _cuda(*arrs):
    return [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in arrs]


@pytest.mark.parametrize("pair", ["0", "1"])
@pytest.mark.parametrize("N,K,scale", [(1024, 3840, 0.0), (300, 96, 0.5), (640, 4096, 0.0), (2048, 800, 1.25),
                                       (15360, 3840, 0.0)])
def test_gemv_normadd(gpu, N, K, scale, pair, tune):
    tune("gemv_pair", pair)
    print(f"gemv_normadd N={N} K={K} scale={scale} pair={pair}", flush=True)
    rng = np.random.default_rng(N + K)
    q, s = synth_int4(rng, N, K)
    wq, sc = upload_int4(q, s)
    a, h, w, w2 = _norm_inputs(rng, K)
    ta, th, tw, tw2 = _cuda(a, h, w, w2)
    h_out = torch.full((K,), float("nan"), dtype=torch.float32, device="cuda")
    y = gpu.gemv_normadd(ta, tw, th, h_out, tw2, wq, sc, N, K, scale=scale, y_dtype=torch.float32)
    hn, xr = _oracle_x(a, w, h, w2, scale)
    assert (to_np(th) == h).all()                           # h is read, not written
    assert O.normwise_rel_err(to_np(h_out), hn) <= 2e-6
    assert O.normwise_rel_err(to_np(y), O.gemv_ref(q, s, xr)) <= 1e-3
    # against the two launches it replaces
    h2 = th.clone()
    xn = gpu.normadd_rmsnorm(ta, tw, h2, tw2, scale, y_dtype=torch.float16)
    y2 = gpu.gemv(xn, wq, sc, N, K, y_dtype=torch.float32)
    assert O.normwise_rel_err(to_np(h_out), to_np(h2)) <= 1e-6
    assert O.normwise_rel_err(to_np(y), to_np(y2)) <= 1e-3
    # deterministic
    y3 = gpu.gemv_normadd(ta, tw, th, h_out, tw2, wq, sc, N, K, scale=scale, y_dtype=torch.float32)
    assert (to_np(y3) == to_np(y)).all()


@pytest.mark.parametrize("e4m3", [False, True])
def test_gemv_batch_normadd_qkv(gpu, e4m3):
    K, Ns = 3840, (4096, 2048, 2048)
    print(f"gemv_batch_normadd qkv e4m3={e4m3}", flush=True)
    rng = np.random.default_rng(7)
    a, h, w, w2 = _norm_inputs(rng, K)
    ta, th, tw, tw2 = _cuda(a, h, w, w2)
    hn, xr = _oracle_x(a, w, h, w2, 0.0)
    mats, refs = [], []
    for N in Ns:
        q, s = synth_int4(rng, N, K)
        if e4m3:
            sc32 = torch.from_numpy(s).cuda()
            sc8, inv = gpu.scales_e4m3(sc32, N, K)
            e8, inv_o, _ = O.e4m3_lift(s)
            assert inv == inv_o
            wq, _ = upload_int4(q, s)
            mats.append((wq, sc8, N, None, inv))
            refs.append(O.gemv_ref(q, O.e4m3_decode(e8), xr, inv=inv))
        else:
            wq, sc = upload_int4(q, s)
            mats.append((wq, sc, N, None, None))
            refs.append(O.gemv_ref(q, s, xr))
    h_out = torch.empty_like(th)
    fmt = gpu.SCALE_E4M3 if e4m3 else gpu.SCALE_F16
    ys = gpu.gemv_batch_normadd(ta, tw, th, h_out, tw2, mats, K, scale_fmt=fmt, y_dtype=torch.float32)
    assert O.normwise_rel_err(to_np(h_out), hn) <= 2e-6
    xn = gpu.normadd_rmsnorm(ta, tw, th.clone(), tw2, 0.0, y_dtype=torch.float16)
    plain = gpu.gemv_batch(xn, mats, K, scale_fmt=fmt, y_dtype=torch.float32)
    for y, ref, y2 in zip(ys, refs, plain):
        assert O.normwise_rel_err(to_np(y), ref) <= 1e-3
        assert O.normwise_rel_err(to_np(y), to_np(y2)) <= 1e-3


def test_gemv_normadd_gated(gpu):
    K, I = 3840, 2048
    print(f"gemv_normadd gated I={I}", flush=True)
    rng = np.random.default_rng(9)
    qg, sg = synth_int4(rng, I, K)
    qu, su = synth_int4(rng, I, K)
    wg, scg = upload_int4(qg, sg)
    wu, scu = upload_int4(qu, su)
    wo, so = gpu.interleave_rows(wg, scg, wu, scu, I, K)
    a, h, w, w2 = _norm_inputs(rng, K)
    ta, th, tw, tw2 = _cuda(a, h, w, w2)
    h_out = torch.empty_like(th)
    act = gpu.gemv_normadd(ta, tw, th, h_out, tw2, wo, so, 2 * I, K, scale=0.0, y_dtype=torch.float16, gated=True)
    hn, xr = _oracle_x(a, w, h, w2, 0.0)
    ref = D.gelumul_ref(O.gemv_ref(qg, sg, xr), O.gemv_ref(qu, su, xr))
    assert O.normwise_rel_err(to_np(act).astype(np.float32), ref) <= 1e-3
    xn = gpu.normadd_rmsnorm(ta, tw, th.clone(), tw2, 0.0, y_dtype=torch.float16)
    act2 = gpu.gemv_gated(xn, wo, so, 2 * I, K, act_dtype=torch.float16)
    assert O.normwise_rel_err(to_np(act).astype(np.float32), to_np(act2).astype(np.float32)) <= 1e-3


def test_gemv_normadd_rejects_bad_operands(gpu):
    K, N = 256, 64
    rng = np.random.default_rng(3)
    q, s = synth_int4(rng, N, K)
    wq, sc = upload_int4(q, s)
    a, h, w, w2 = _cuda(*_norm_inputs(rng, K))
    with pytest.raises(ValueError, match="overlap"):
        gpu.gemv_normadd(a, w, h, h, w2, wq, sc, N, K)
    big = torch.zeros(8192, dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="K <="):
        gpu.gemv_normadd(big, big, big, big.clone(), big, wq, sc, N, 8192)
    # the C ABI checks the same (called directly, past the Python checks)
    from g4mi import _lib
    lib = _lib.lib()
    rc = lib.q4_gemv_normadd(a.data_ptr(), w.data_ptr(), h.data_ptr(), a.data_ptr() + 16, 0.0, w2.data_ptr(),
                             wq.data_ptr(), sc.data_ptr(), 0, 1.0, h.data_ptr(), 0, N, K, 0, None)
    assert rc == _lib.Q4_ERR_ARG and b"overlap" in lib.q4_last_error()
    # y may not overlap a norm operand or h_out (early workgroups write y while others read them)
    h_out = torch.empty_like(h)
    for tgt, nm in ((a, "a"), (h, "h"), (w, "w"), (w2, "w2"), (h_out, "h_out")):
        with pytest.raises(ValueError, match=f"y must not overlap {nm}"):
            gpu.gemv_normadd(a, w, h, h_out, w2, wq, sc, N, K, y=tgt)
        rc = lib.q4_gemv_normadd(a.data_ptr(), w.data_ptr(), h.data_ptr(), h_out.data_ptr(), 0.0, w2.data_ptr(),
                                 wq.data_ptr(), sc.data_ptr(), 0, 1.0, tgt.data_ptr() + 8, 0, N, K, 0, None)
        assert rc == _lib.Q4_ERR_ARG and b"y must not overlap" in lib.q4_last_error()
    with pytest.raises(ValueError, match="y must not overlap h"):
        gpu.gemv_batch_normadd(a, w, h, h_out, w2, [(wq, sc, N, None, None), (wq, sc, N, h[32:], None)], K)
    ys = (C.c_void_p * 2)(h_out.data_ptr() + 4 * K, h.data_ptr())
    ptrs = (C.c_void_p * 2)(wq.data_ptr(), wq.data_ptr())
    scs = (C.c_void_p * 2)(sc.data_ptr(), sc.data_ptr())
    Ns = (C.c_int * 2)(N, N)
    tmp = torch.empty(4 * K, dtype=torch.float32, device="cuda")
    ys[0] = tmp.data_ptr()
    rc = lib.q4_gemv_batch_normadd(a.data_ptr(), w.data_ptr(), h.data_ptr(), h_out.data_ptr(), 0.0, w2.data_ptr(),
                                   K, 0, 0, 2, ptrs, scs, None, ys, Ns, None)
    assert rc == _lib.Q4_ERR_ARG and b"y must not overlap" in lib.q4_last_error()
    torch.cuda.synchronize()


@pytest.mark.parametrize("pair", ["0", "1"])
@pytest.mark.parametrize("gated", [False, True])
def test_gemv_normadd_rows64(gpu, pair, gated, tune):
    """64 rows per workgroup: one block slot per wave in nx_stage's LDS mapping,
    the plan the real gate/up launch (30720 x 3840, gated, paired) takes."""
    tune("gemv_pair", pair)
    K, I = 3840, 15360 if gated else 2048
    N = 2 * I if gated else 4096
    if not gated:
        tune("gemv_rows", "64")
    print(f"gemv_normadd rows64 N={N} gated={gated} pair={pair}", flush=True)
    rng = np.random.default_rng(21 + int(gated))
    a, h, w, w2 = _norm_inputs(rng, K)
    ta, th, tw, tw2 = _cuda(a, h, w, w2)
    hn, xr = _oracle_x(a, w, h, w2, 0.0)
    h_out = torch.empty_like(th)
    if gated:
        qg, sg = synth_int4(rng, I, K)
        qu, su = synth_int4(rng, I, K)
        wg, scg = upload_int4(qg, sg)
        wu, scu = upload_int4(qu, su)
        wo, so = gpu.interleave_rows(wg, scg, wu, scu, I, K)
        y = gpu.gemv_normadd(ta, tw, th, h_out, tw2, wo, so, N, K, y_dtype=torch.float16, gated=True)
        ref = D.gelumul_ref(O.gemv_ref(qg, sg, xr), O.gemv_ref(qu, su, xr))
        xn = gpu.normadd_rmsnorm(ta, tw, th.clone(), tw2, 0.0, y_dtype=torch.float16)
        y2 = gpu.gemv_gated(xn, wo, so, N, K, act_dtype=torch.float16)
    else:
        q, s = synth_int4(rng, N, K)
        wq, sc = upload_int4(q, s)
        y = gpu.gemv_normadd(ta, tw, th, h_out, tw2, wq, sc, N, K, y_dtype=torch.float32)
        ref = O.gemv_ref(q, s, xr)
        xn = gpu.normadd_rmsnorm(ta, tw, th.clone(), tw2, 0.0, y_dtype=torch.float16)
        y2 = gpu.gemv(xn, wq, sc, N, K, y_dtype=torch.float32)
    yn = to_np(y).astype(np.float32)
    assert O.normwise_rel_err(to_np(h_out), hn) <= 2e-6
    assert O.normwise_rel_err(yn, ref) <= 1e-3
    assert O.normwise_rel_err(yn, to_np(y2).astype(np.float32)) <= 1e-3
