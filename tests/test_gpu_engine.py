"""The reference-signature host helpers (vk_engine mirror) on the GPU, used the
way src/vk_engine.py uses its own: quant -> gemv_ds/gemv into fp32 buffers,
gemm_ds/gmm for a prefill chunk, and a recorded token graph replayed with a
bounded wait."""
import importlib

import numpy as np
import pytest
import torch

from oracle import q4_oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def E(gpu):
    return importlib.import_module("g4mi.vk_engine")


def _w(rng, N, K, scale=0.05):
    return (rng.standard_normal((N, K)) * scale).astype(np.float32)


@pytest.mark.parametrize("fp8", [False, True])
def test_quant_gemv_ds_gemv(E, fp8):
    rng = np.random.default_rng(41)
    N, K = 4096, 3840
    W = _w(rng, N, K)
    qw = E.quant(W, fp8=fp8, prefill_i8=False)
    bw, bs, split, nblk, inv, bs16, w8, sw8 = qw
    assert nblk == K // 32 and w8 is None and split >= 1
    q, sc = O.quant_codes(W)
    assert (bw.t.cpu().numpy().view(np.uint32) == O.pack_dev(q)).all()
    x = rng.standard_normal(K).astype(np.float32)
    inbuf, outbuf = E.Buf(K * 4), E.Buf((N + 16) * 4)
    inbuf.write(x)
    g = E.gemv_ds((qw, (N, K)), inbuf, outbuf, out_off=64)
    E.gemv(g)
    torch.cuda.synchronize()
    y = np.frombuffer(outbuf.read((N + 16) * 4), np.float32)[16:16 + N]
    if fp8:
        e8, inv_o, _ = O.e4m3_lift(sc)
        assert inv == inv_o
        ref = O.gemv_ref(q, O.e4m3_decode(e8), x, inv=inv)
    else:
        ref = O.gemv_ref(q, sc.astype(np.float16).astype(np.float32), x)
    assert O.normwise_rel_err(y, ref) <= 2e-5
    # the reference's own quality check: cosine vs the ORIGINAL weights (benchmarks/vk_gemv.py:143)
    assert O.cosine(y, W @ x) > 0.98


@pytest.mark.parametrize("fp8", [False, True])
def test_gemv_many_qkv_into_one_buffer(E, fp8):
    """q/k/v descriptors on one input buffer, written at their offsets of one
    qkv buffer (src/vk_engine.py:232-234), launched as one batch: the same
    values as three gemv() calls (both compared with the oracle)."""
    rng = np.random.default_rng(43)
    K = 3840
    shapes = [4096, 2048, 2048]
    x = rng.standard_normal(K).astype(np.float32)
    inbuf, qkv = E.Buf(K * 4), E.Buf(sum(shapes) * 4)
    inbuf.write(x)
    descs, refs, off = [], [], 0
    for N in shapes:
        W = _w(rng, N, K)
        qw = E.quant(W, fp8=fp8, prefill_i8=False)
        descs.append(E.gemv_ds((qw, (N, K)), inbuf, qkv, out_off=off * 4))
        q, sc = O.quant_codes(W)
        if fp8:
            e8, inv, _ = O.e4m3_lift(sc)
            refs.append(O.gemv_ref(q, O.e4m3_decode(e8), x, inv=inv))
        else:
            refs.append(O.gemv_ref(q, sc.astype(np.float16).astype(np.float32), x))
        off += N
    E.gemv_many(descs)
    torch.cuda.synchronize()
    y = np.frombuffer(qkv.read(sum(shapes) * 4), np.float32)
    off = 0
    for N, ref in zip(shapes, refs):
        assert O.normwise_rel_err(y[off:off + N], ref) <= 2e-5
        off += N


@pytest.mark.parametrize("i8", [False, True])
def test_gemm_ds_gmm_prefill_chunk(E, i8):
    rng = np.random.default_rng(42)
    N, K, MC = 3840, 4096, E.MC
    W = _w(rng, N, K)
    qw = E.quant(W, fp8=False, prefill_i8=i8)
    q, sc = O.quant_codes(W)
    X = rng.standard_normal((MC, K)).astype(np.float32)
    inbuf, outbuf = E.Buf(MC * K * 4), E.Buf(MC * N * 4)
    inbuf.write(X)
    t = E.gemm_ds((qw, (N, K)), inbuf, outbuf, prefill_i8=i8)
    E.gmm(None, t, tag="o")
    torch.cuda.synchronize()
    Y = np.frombuffer(outbuf.read(MC * N * 4), np.float32).reshape(MC, N)
    if i8:
        W8, sw = O.w8_fold(q, sc)
        A, sa = O.quant_act_i8(X)
        _, Yref = O.gemm_w8a8_ref(A, W8, sa, sw.astype(np.float16).astype(np.float32))
        assert (Y == Yref.astype(np.float32)).all()
    else:
        ref = O.gemm_w4a16_ref(X.astype(np.float16), q, sc.astype(np.float16).astype(np.float32))
        assert O.normwise_rel_err(Y, ref) <= 1e-3


def test_record_once_token_graph(E):
    """A small 'token': q/k/v/o/gate_up/down GEMVs of 2 layers + lm_head,
    recorded once, replayed 3 times with fresh inputs written between replays."""
    rng = np.random.default_rng(43)
    H, I, V = 512, 1536, 4096
    shapes = {"q": (1024, H), "k": (256, H), "v": (256, H), "o": (H, 1024), "gu": (2 * I, H), "d": (H, I)}
    layers = []
    for _ in range(2):
        L = {}
        for name, (N, K) in shapes.items():
            W = _w(rng, N, K)
            L[name] = ((E.quant(W, fp8=False, prefill_i8=False), (N, K)), W)
        layers.append(L)
    lmW = _w(rng, V, H)
    lm = (E.quant(lmW, fp8=False, prefill_i8=False), (V, H))
    xin = E.Buf(I * 4)
    outs = {}
    descs = []
    for li, L in enumerate(layers):
        for name, (qw, W) in L.items():
            outs[(li, name)] = E.Buf(qw[1][0] * 4)
            descs.append(E.gemv_ds(qw, xin, outs[(li, name)]))
    lmout = E.Buf(V * 4)
    descs.append(E.gemv_ds(lm, xin, lmout))
    graph = E.record(lambda: [E.gemv(d) for d in descs])
    for rep in range(3):
        x = rng.standard_normal(I).astype(np.float32)
        xin.write(x)
        E.submit(graph, label=f"token {rep}", timeout_ms=60000)
        for li, L in enumerate(layers):
            for name, (qw, W) in L.items():
                N, K = qw[1]
                q, sc = O.quant_codes(W)
                y = np.frombuffer(outs[(li, name)].read(N * 4), np.float32)
                ref = O.gemv_ref(q, sc.astype(np.float16).astype(np.float32), x[:K])
                assert O.normwise_rel_err(y, ref) <= 2e-5, (rep, li, name)
        y = np.frombuffer(lmout.read(V * 4), np.float32)
        q, sc = O.quant_codes(lmW)
        assert O.normwise_rel_err(y, O.gemv_ref(q, sc.astype(np.float16).astype(np.float32), x[:H])) <= 2e-5
    graph.destroy()
