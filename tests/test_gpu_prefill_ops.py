"""GPU parity of the batched-prefill layer ops (row norms, normadd, gelumul,
prepkv and causal MFMA attention over a chunk of M tokens) against the
oracle (oracle/prefill_ops_oracle.py, float64).

Tolerances: normwise max|y - ref| / max|ref| <= 2e-6 for the fp32 norms and
gelumul (fp32 arithmetic against float64), <= 1e-3 for fp16 outputs; KV
cache entries within one fp16 ulp of the float64 value; attention <= 2e-4
(fp32 out) and <= 1e-3 (fp16 out): q . k is exact to fp32 rounding (q split
into fp16 hi + lo), but the softmax weights enter the V product rounded to
fp16 (relative error <= 2^-11 per weight; the row maximum's weight, 1, is
exact), and the scores are unscaled.
"""
import numpy as np
import pytest
import torch

from oracle import decode_ops_oracle as D
from oracle import prefill_ops_oracle as P
from oracle import q4_oracle as O

pytestmark = pytest.mark.gpu


def _t(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).cuda()


def _np(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def _dyn(p0, M):
    return torch.tensor([p0, M, 0, 0], dtype=torch.int32, device="cuda")


def _rope_rows(M, hd, p0):
    inv = 1.0 / (10000.0 ** (np.arange(0, hd, 2) / hd))
    ang = (p0 + np.arange(M))[:, None] * inv[None, :]
    return (np.concatenate([np.cos(ang)] * 2, 1).astype(np.float32),
            np.concatenate([np.sin(ang)] * 2, 1).astype(np.float32))


def _within_one_f16_ulp(got16, ref64):
    ref16 = ref64.astype(np.float16)
    up = np.nextafter(ref16, np.float16(np.inf))
    dn = np.nextafter(ref16, np.float16(-np.inf))
    g = got16.astype(np.float16)
    return bool(np.all((g == ref16) | (g == up) | (g == dn)))


@pytest.mark.parametrize("M,D_", [(5, 3840), (128, 3840), (3, 100)])
def test_pre_rmsnorm_rows(gpu, M, D_):
    rng = np.random.default_rng(M + D_)
    X = (rng.standard_normal((M, D_)) * 3).astype(np.float32)
    w = (rng.random(D_) + 0.5).astype(np.float32)
    ref = P.pre_rmsnorm_ref(X, w)
    Y = gpu.pre_rmsnorm(_t(X), _t(w), M=M, D=D_)
    assert O.normwise_rel_err(_np(Y), ref) <= 2e-6
    Yh = gpu.pre_rmsnorm(_t(X), _t(w), M=M, D=D_, y_dtype=torch.float16)
    assert O.normwise_rel_err(_np(Yh).astype(np.float64), ref) <= 1e-3
    # each row is the decode rmsnorm of that row, bit for bit (the same kernel, one row per workgroup)
    y1 = gpu.rmsnorm(_t(X[M - 1]), _t(w))
    assert torch.equal(Y[M - 1], y1)


@pytest.mark.parametrize("xdt", [torch.float32, torch.float16])
@pytest.mark.parametrize("scale", [0.0, 0.5])
def test_pre_normadd_rows_and_fused(gpu, xdt, scale):
    rng = np.random.default_rng(int(scale * 10) + (xdt == torch.float16))
    M, D_ = 7, 3840
    X = rng.standard_normal((M, D_)).astype(np.float32)
    if xdt == torch.float16:
        X = X.astype(np.float16).astype(np.float32)  # what the GEMM hands over
    Hm = rng.standard_normal((M, D_)).astype(np.float32)
    w, w2 = (rng.random((2, D_)) + 0.5).astype(np.float32)
    ref = P.pre_normadd_ref(X, w, Hm, scale)
    h = _t(Hm)
    gpu.pre_normadd(_t(X, xdt), _t(w), h, M=M, D=D_, scale=scale)
    assert O.normwise_rel_err(_np(h), ref) <= 2e-6
    h2 = _t(Hm)
    y = gpu.pre_normadd(_t(X, xdt), _t(w), h2, M=M, D=D_, scale=scale, w2=_t(w2), y_dtype=torch.float16)
    assert torch.equal(h2, h)  # the fused launch leaves h exactly as the plain one
    assert O.normwise_rel_err(_np(y).astype(np.float64), P.pre_rmsnorm_ref(_np(h), w2)) <= 1e-3


def test_pre_gelumul_f16_inputs(gpu):
    rng = np.random.default_rng(5)
    n = 128 * 1000 + 7
    g, u = (rng.standard_normal((2, n)) * 2).astype(np.float16)
    ref = D.gelumul_ref(g.astype(np.float64), u.astype(np.float64))
    out = gpu.pre_gelumul(_t(g, torch.float16), _t(u, torch.float16))
    assert O.normwise_rel_err(_np(out), ref) <= 2e-6
    outh = gpu.pre_gelumul(_t(g, torch.float16), _t(u, torch.float16), out_dtype=torch.float16)
    assert O.normwise_rel_err(_np(outh).astype(np.float64), ref) <= 1e-3


@pytest.mark.parametrize("hd,nkv,stride,window,M,p0,keqv,kvdt", [
    (256, 8, 1024, 1024, 128, 1000, False, torch.float32),  # the ring wraps inside the chunk
    (512, 2, 300, 0, 40, 17, True, torch.float16),          # global layer, k == v, fp16 GEMM outputs
    (64, 3, 16, 16, 16, 5, False, torch.float16),           # a chunk as long as the ring
])
def test_pre_prepkv(gpu, hd, nkv, stride, window, M, p0, keqv, kvdt):
    rng = np.random.default_rng(hd + M)
    ld = nkv * hd + 8
    K = (rng.standard_normal((M, ld)) * 2).astype(np.float32)
    V = None if keqv else (rng.standard_normal((M, ld)) * 2).astype(np.float32)
    if kvdt == torch.float16:
        K = K.astype(np.float16).astype(np.float32)
        V = None if V is None else V.astype(np.float16).astype(np.float32)
    knw = (rng.random(hd) + 0.5).astype(np.float32)
    cosM, sinM = _rope_rows(M, hd, p0)
    kc0 = rng.standard_normal(nkv * stride * hd).astype(np.float16)
    vc0 = rng.standard_normal(nkv * stride * hd).astype(np.float16)
    rk, rv = P.pre_prepkv_ref(K[:, :nkv * hd], None if V is None else V[:, :nkv * hd], knw, cosM, sinM, kc0, vc0,
                              nkv=nkv, hd=hd, stride=stride, window=window, p0=p0)
    kc, vc = _t(kc0, torch.float16), _t(vc0, torch.float16)
    tk = _t(K, kvdt)
    gpu.pre_prepkv(tk, tk if V is None else _t(V, kvdt), _t(knw), _t(cosM), _t(sinM), kc, vc, M=M, ld=ld, nkv=nkv,
                   hd=hd, stride=stride, window=window, dyn=_dyn(p0, M))
    gk, gv = _np(kc).reshape(-1, hd), _np(vc).reshape(-1, hd)
    slots = {D.kv_slot(p0 + m, window): m for m in range(M)}  # the last token of each slot
    written = np.zeros(nkv * stride, bool)
    for s, m in slots.items():
        for h in range(nkv):
            r = h * stride + s
            written[r] = True
            k = K[m, h * hd:(h + 1) * hd].astype(np.float64)
            v = (K if V is None else V)[m, h * hd:(h + 1) * hd].astype(np.float64)
            assert _within_one_f16_ulp(gk[r], D.rope_ref(k * D.rms_inv(k) * knw, cosM[m], sinM[m])), (m, h)
            assert _within_one_f16_ulp(gv[r], v * D.rms_inv(v)), (m, h)
    assert np.array_equal(gk[~written], kc0.reshape(-1, hd)[~written])  # other slots untouched
    assert np.array_equal(gv[~written], vc0.reshape(-1, hd)[~written])
    assert np.mean(gk[written] == rk.reshape(-1, hd)[written]) > 0.99


def _attn_case(rng, *, M, nH, nkv, hd, stride, window, p0, qdt, peaky=False):
    """A cache of random fp16 rows (earlier tokens) with the chunk's own
    rows written by the oracle's prepkv, and the chunk's q rows."""
    kc = rng.standard_normal(nkv * stride * hd).astype(np.float16)
    vc = rng.standard_normal(nkv * stride * hd).astype(np.float16)
    cosM, sinM = _rope_rows(M, hd, p0)
    K = rng.standard_normal((M, nkv * hd))
    knw = rng.random(hd) + 0.5
    kc, vc = P.pre_prepkv_ref(K, rng.standard_normal((M, nkv * hd)), knw, cosM, sinM, kc, vc, nkv=nkv, hd=hd,
                              stride=stride, window=window, p0=p0)
    Q = (rng.standard_normal((M, nH * hd)) * 2).astype(np.float32)
    if qdt == torch.float16:
        Q = Q.astype(np.float16).astype(np.float32)
    qnw = (rng.random(hd) + 0.5) if peaky else (rng.random(hd) * 0.2 + 0.05)
    return Q, qnw.astype(np.float32), cosM, sinM, kc, vc


@pytest.mark.parametrize("hd,nH,nkv,stride,window,M,p0,max_keys,qdt,odt,peaky", [
    (256, 16, 8, 1024, 1024, 128, 1000, 1024, torch.float32, torch.float32, False),  # sliding layer, ring wraps
    (256, 16, 8, 1024, 1024, 128, 0, 1024, torch.float16, torch.float16, False),     # first chunk of a prompt
    (512, 16, 2, 2048, 0, 32, 600, 640, torch.float32, torch.float32, False),        # global layer, grp 8
    (512, 16, 1, 4096, 0, 128, 3968, 4096, torch.float16, torch.float16, False),     # last chunk of 4096, MQA
    (512, 4, 1, 300, 256, 40, 500, 256, torch.float16, torch.float32, True),         # hd 512 ring, ragged tiles
    (512, 2, 2, 100, 0, 3, 90, 100, torch.float32, torch.float32, False),           # grp 1; last tile past the cache
    (512, 8, 1, 77, 64, 5, 200, 77, torch.float16, torch.float16, True),            # ring of 64 in a 77-slot cache
    (128, 4, 2, 96, 64, 40, 130, 64, torch.float16, torch.float32, True),            # unscaled large scores
    (64, 6, 3, 300, 0, 21, 257, 300, torch.float32, torch.float32, False),           # ragged rows and splits
])
def test_pre_attn_vs_oracle(gpu, hd, nH, nkv, stride, window, M, p0, max_keys, qdt, odt, peaky):
    rng = np.random.default_rng(hd + M + p0)
    Q, qnw, cosM, sinM, kc, vc = _attn_case(rng, M=M, nH=nH, nkv=nkv, hd=hd, stride=stride, window=window, p0=p0,
                                            qdt=qdt, peaky=peaky)
    ref = P.pre_attn_ref(Q, qnw, cosM, sinM, kc, vc, nH=nH, hd=hd, stride=stride, window=window, grp=nH // nkv,
                         p0=p0)
    out = gpu.pre_attn(_t(Q, qdt), _t(qnw), _t(cosM), _t(sinM), _t(kc, torch.float16), _t(vc, torch.float16),
                       M=M, ldq=nH * hd, nH=nH, nkv=nkv, hd=hd, stride=stride, window=window, max_keys=max_keys,
                       dyn=_dyn(p0, M), out_dtype=odt)
    got = _np(out).astype(np.float64)
    tol = 2e-4 if odt == torch.float32 else 1e-3
    for m in range(M):
        err = O.normwise_rel_err(got[m], ref[m])
        assert err <= tol, (m, err)


def test_pre_attn_graph_replay_follows_p0(gpu):
    """prepkv + attention of a chunk captured once; p0 lives in device memory
    and advances by M between replays (three chunks of one prompt). Every
    replay matches eager calls at the same p0 bit for bit, and the oracle."""
    rng = np.random.default_rng(21)
    nH, nkv, hd, stride, window, M = 8, 4, 128, 256, 256, 64
    kc0 = np.zeros(nkv * stride * hd, np.float16)
    knw = (rng.random(hd) + 0.5).astype(np.float32)
    qnw = (rng.random(hd) * 0.2 + 0.05).astype(np.float32)
    kc, vc = _t(kc0, torch.float16), _t(kc0, torch.float16)
    kc_e, vc_e = kc.clone(), vc.clone()
    K, V, Q = _t(np.zeros((M, nkv * hd))), _t(np.zeros((M, nkv * hd))), _t(np.zeros((M, nH * hd)))
    cs, sn = _t(np.zeros((M, hd))), _t(np.zeros((M, hd)))
    t_knw, t_qnw = _t(knw), _t(qnw)
    dyn = _dyn(0, M)
    ws = gpu.pre_attn_workspace(M, nH, nkv, hd, window)
    out = torch.empty(M, nH * hd, device="cuda")
    kw = dict(M=M, nkv=nkv, hd=hd, stride=stride, window=window, dyn=dyn)
    akw = dict(M=M, ldq=nH * hd, nH=nH, nkv=nkv, hd=hd, stride=stride, window=window, max_keys=window)
    g = gpu.Graph()
    with g.capture():
        gpu.pre_prepkv(K, V, t_knw, cs, sn, kc, vc, ld=nkv * hd, **kw)
        gpu.pre_attn(Q, t_qnw, cs, sn, kc, vc, out, dyn=dyn, ws=ws, **akw)
    rkc, rvc = kc0.copy(), kc0.copy()
    for chunk in range(5):
        p0 = chunk * M
        Kn, Vn = rng.standard_normal((2, M, nkv * hd)).astype(np.float32)
        Qn = (rng.standard_normal((M, nH * hd)) * 2).astype(np.float32)
        c, s = _rope_rows(M, hd, p0)
        for t, a in ((K, Kn), (V, Vn), (Q, Qn), (cs, c), (sn, s)):
            t.copy_(_t(a))
        dyn.copy_(_dyn(p0, M))
        g.launch()
        got = _np(out).copy()
        de = _dyn(p0, M)
        gpu.pre_prepkv(K, V, t_knw, cs, sn, kc_e, vc_e, ld=nkv * hd, **dict(kw, dyn=de))
        eager = gpu.pre_attn(Q, t_qnw, cs, sn, kc_e, vc_e, dyn=de, ws=ws, **akw)
        assert np.array_equal(got, _np(eager)), chunk
        assert torch.equal(kc, kc_e) and torch.equal(vc, vc_e)
        rkc, rvc = P.pre_prepkv_ref(Kn, Vn, knw, c, s, rkc, rvc, nkv=nkv, hd=hd, stride=stride, window=window, p0=p0)
        ref = P.pre_attn_ref(Qn, qnw, c, s, rkc, rvc, nH=nH, hd=hd, stride=stride, window=window, grp=nH // nkv,
                             p0=p0)
        assert O.normwise_rel_err(got, ref) <= 2e-4, chunk
        rkc, rvc = _np(kc).copy(), _np(vc).copy()  # carry the device caches (fp16 rounding ties aside)
    g.destroy()
