"""GPU parity of the decode-token ops (rmsnorm, normadd, gelumul, prepkv,
attention) against the oracle (oracle/decode_ops_oracle.py, float64).

Tolerances (fp32 arithmetic against the float64 value of the shaders'
formulas): normwise max|y - ref| / max|ref| <= 2e-6 for the fp32 norms and
gelumul, <= 1e-3 for fp16 outputs, KV-cache entries within one fp16 ulp of
the oracle's rounding (the fp32 value can sit on the other side of an fp16
rounding boundary), attention normwise <= 1e-4 (scores of ~|q||k| without
scaling amplify fp32 rounding in the softmax).
"""
import numpy as np
import pytest
import torch

from oracle import decode_ops_oracle as D
from oracle import q4_oracle as O

pytestmark = pytest.mark.gpu


def _t(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).cuda()


def _np(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("D_", [3840, 15360, 100, 1])
def test_rmsnorm(gpu, D_):
    rng = np.random.default_rng(D_)
    x = (rng.standard_normal(D_) * 3).astype(np.float32)
    w = (rng.random(D_) + 0.5).astype(np.float32)
    ref = D.rmsnorm_ref(x, w)
    y = gpu.rmsnorm(_t(x), _t(w))
    assert O.normwise_rel_err(_np(y), ref) <= 2e-6
    yh = gpu.rmsnorm(_t(x), _t(w), y_dtype=torch.float16)
    assert yh.dtype == torch.float16 and O.normwise_rel_err(_np(yh).astype(np.float64), ref) <= 1e-3


@pytest.mark.parametrize("scale,n", [(0.0, 3840), (0.37, 3840), (0.5, 5000), (0.0, 100)])
def test_normadd(gpu, scale, n):
    rng = np.random.default_rng(7)
    x, h = rng.standard_normal((2, n)).astype(np.float32)
    w = rng.random(n).astype(np.float32)
    ref = D.normadd_ref(x, w, h, scale)
    ht = _t(h)
    gpu.normadd(_t(x), _t(w), ht, scale)
    assert O.normwise_rel_err(_np(ht), ref) <= 2e-6


@pytest.mark.parametrize("scale,n,ydt", [(0.0, 3840, torch.float32), (0.5, 3840, torch.float16),
                                         (0.25, 5000, torch.float32), (0.0, 1, torch.float32)])
def test_normadd_rmsnorm_fused(gpu, scale, n, ydt):
    """One launch = normadd then rmsnorm of the new h: h as q4_normadd leaves
    it (bit for bit), y against the oracle's rmsnorm of the oracle's h."""
    rng = np.random.default_rng(n)
    x, h = rng.standard_normal((2, n)).astype(np.float32)
    w, w2 = (rng.random((2, n)) + 0.5).astype(np.float32)
    href = D.normadd_ref(x, w, h, scale)
    yref = D.rmsnorm_ref(href, w2)
    ht, ht2 = _t(h), _t(h)
    y = gpu.normadd_rmsnorm(_t(x), _t(w), ht, _t(w2), scale, y_dtype=ydt)
    gpu.normadd(_t(x), _t(w), ht2, scale)
    assert torch.equal(ht, ht2)
    assert O.normwise_rel_err(_np(ht), href) <= 2e-6
    assert O.normwise_rel_err(_np(y).astype(np.float64), yref) <= (2e-6 if ydt == torch.float32 else 1e-3)


@pytest.mark.parametrize("n", [15360, 37])
def test_gelumul(gpu, n):
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 3).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    ref = D.gelumul_ref(g, u)
    assert O.normwise_rel_err(_np(gpu.gelumul(_t(g), _t(u))), ref) <= 2e-6
    assert O.normwise_rel_err(_np(gpu.gelumul(_t(g), _t(u), out_dtype=torch.float16)).astype(np.float64), ref) <= 1e-3


def _rope_tables(rng, hd):
    ang = rng.random(hd // 2) * 6.0
    return (np.concatenate([np.cos(ang), np.cos(ang)]).astype(np.float32),
            np.concatenate([np.sin(ang), np.sin(ang)]).astype(np.float32))


def _within_one_f16_ulp(got, ref):
    g = got.astype(np.float64)
    r = ref.astype(np.float16).astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    return np.all(np.abs(g - r) <= ulp)


@pytest.mark.parametrize("hd,nkv,stride,window,pos,keqv", [(256, 8, 64, 64, 100, False), (512, 2, 300, 0, 257, True),
                                                           (256, 8, 64, 64, 0, False)])
def test_prepkv(gpu, hd, nkv, stride, window, pos, keqv):
    rng = np.random.default_rng(hd + pos)
    nq = 16 * hd
    qkv = (rng.standard_normal(nq + 2 * nkv * hd) * 2).astype(np.float32)
    knw = (rng.random(hd) + 0.5).astype(np.float32)
    cs, sn = _rope_tables(rng, hd)
    kc0 = rng.standard_normal(nkv * stride * hd).astype(np.float16)
    vc0 = rng.standard_normal(nkv * stride * hd).astype(np.float16)
    koff, voff = nq, nq + nkv * hd
    rk, rv = D.prepkv_ref(qkv, knw, cs, sn, kc0, vc0, nkv=nkv, hd=hd, koff=koff, voff=voff, keqv=keqv,
                          stride=stride, window=window, pos=pos)
    kc, vc = _t(kc0, torch.float16), _t(vc0, torch.float16)
    dyn = torch.tensor([pos, pos + 1, 0, 0], dtype=torch.int32, device="cuda")
    gpu.prepkv(_t(qkv), _t(knw), _t(cs), _t(sn), kc, vc, nkv=nkv, hd=hd, koff=koff, voff=voff, keqv=keqv,
               stride=stride, window=window, dyn=dyn)
    gk, gv = _np(kc), _np(vc)
    slot = D.kv_slot(pos, window)
    rows = [h * stride + slot for h in range(nkv)]
    mask = np.ones(nkv * stride, bool)
    mask[rows] = False
    assert np.array_equal(gk.reshape(-1, hd)[mask], kc0.reshape(-1, hd)[mask])  # other slots untouched
    assert np.array_equal(gv.reshape(-1, hd)[mask], vc0.reshape(-1, hd)[mask])
    # the written rows against the oracle's float64 values, within one fp16 ulp
    vo = koff if keqv else voff
    for h in range(nkv):
        k = qkv[koff + h * hd: koff + (h + 1) * hd].astype(np.float64)
        kref = D.rope_ref(k * D.rms_inv(k) * knw, cs, sn)
        v = qkv[vo + h * hd: vo + (h + 1) * hd].astype(np.float64)
        vref = v * D.rms_inv(v)
        r = rows[h]
        assert _within_one_f16_ulp(gk.reshape(-1, hd)[r], kref)
        assert _within_one_f16_ulp(gv.reshape(-1, hd)[r], vref)
        assert np.mean(gk.reshape(-1, hd)[r] == rk.reshape(-1, hd)[r]) > 0.99


def _attn_case(rng, nH, nkv, hd, stride):
    qkv = (rng.standard_normal(nH * hd + 2 * nkv * hd) * 2).astype(np.float32)
    qnw = (rng.random(hd) * 0.2 + 0.05).astype(np.float32)   # scores of a few units, as after q/k norms
    cs, sn = _rope_tables(rng, hd)
    kc = rng.standard_normal(nkv * stride * hd).astype(np.float16)
    vc = rng.standard_normal(nkv * stride * hd).astype(np.float16)
    return qkv, qnw, cs, sn, kc, vc


@pytest.mark.parametrize("nH,nkv,hd,stride,window,pos", [
    (16, 8, 256, 1024, 1024, 0),      # one key
    (16, 8, 256, 1024, 1024, 300),    # two splits, ragged
    (16, 8, 256, 1024, 1024, 5000),   # ring full: T = window
    (16, 2, 512, 2048, 0, 1500),      # global layer, hd 512, grp 8
    (16, 1, 512, 4096, 0, 4095),      # one KV head for 16 query heads: four head groups, 128 splits
    (6, 2, 128, 100, 0, 77),          # grp 3: one query head per workgroup
    (4, 4, 64, 40, 0, 39),            # tiny, last slot
    (4, 2, 64, 9000, 0, 8999),        # 282 live splits: the merging workgroup takes the weights 256 at a time
])
def test_attn(gpu, nH, nkv, hd, stride, window, pos):
    rng = np.random.default_rng(nH * hd + pos)
    qkv, qnw, cs, sn, kc, vc = _attn_case(rng, nH, nkv, hd, stride)
    kw = dict(nH=nH, hd=hd, stride=stride, window=window, qoff=0, grp=nH // nkv, pos=pos)
    ref = D.attn_ref(qkv, qnw, cs, sn, kc, vc, **kw)
    dyn = torch.tensor([pos, pos + 1, 0, 0], dtype=torch.int32, device="cuda")
    out = gpu.attn(_t(qkv), _t(qnw), _t(cs), _t(sn), _t(kc, torch.float16), _t(vc, torch.float16), nH=nH, nkv=nkv,
                   hd=hd, stride=stride, window=window, qoff=0, grp=nH // nkv, dyn=dyn)
    got = _np(out)
    assert O.normwise_rel_err(got, ref) <= 1e-4
    assert O.cosine(got, ref) > 0.999999


def test_prepkv_attn_graph_replay_follows_position(gpu):
    """prepkv + attention captured once; the position lives in device memory
    and advances between replays (as the engine's DYN buffer does). Every
    replay matches the eager result of the same position bit for bit, and
    the oracle."""
    rng = np.random.default_rng(11)
    nH, nkv, hd, stride, window = 8, 4, 256, 512, 512
    qkv, qnw, cs, sn, kc0, vc0 = _attn_case(rng, nH, nkv, hd, stride)
    knw = (rng.random(hd) + 0.5).astype(np.float32)
    koff, voff = nH * hd, nH * hd + nkv * hd
    args = dict(nkv=nkv, hd=hd, koff=koff, voff=voff, keqv=False, stride=stride, window=window)
    akw = dict(nH=nH, nkv=nkv, hd=hd, stride=stride, window=window, qoff=0, grp=nH // nkv)
    t_qkv, t_knw, t_qnw, t_cs, t_sn = _t(qkv), _t(knw), _t(qnw), _t(cs), _t(sn)
    kc, vc = _t(kc0, torch.float16), _t(vc0, torch.float16)
    kc_e, vc_e = kc.clone(), vc.clone()
    dyn = torch.zeros(4, dtype=torch.int32, device="cuda")
    dyn_e = torch.zeros(4, dtype=torch.int32, device="cuda")
    ws = gpu.attn_workspace(nH, hd, stride)
    out = torch.empty(nH * hd, device="cuda")
    g = gpu.Graph()
    with g.capture():
        gpu.prepkv(t_qkv, t_knw, t_cs, t_sn, kc, vc, dyn=dyn, **args)
        gpu.attn(t_qkv, t_qnw, t_cs, t_sn, kc, vc, out, dyn=dyn, ws=ws, **akw)
    for pos in [0, 1, 255, 256, 600]:
        dyn.copy_(torch.tensor([pos, pos + 1, 0, 0], dtype=torch.int32))
        dyn_e.copy_(dyn)
        torch.cuda.synchronize()
        g.launch()
        torch.cuda.synchronize()
        gpu.prepkv(t_qkv, t_knw, t_cs, t_sn, kc_e, vc_e, dyn=dyn_e, **args)
        oe = gpu.attn(t_qkv, t_qnw, t_cs, t_sn, kc_e, vc_e, dyn=dyn_e, **akw)
        torch.cuda.synchronize()
        assert torch.equal(out, oe) and torch.equal(kc, kc_e) and torch.equal(vc, vc_e), pos
        ref = D.attn_ref(qkv, qnw, cs, sn, _np(kc), _np(vc), nH=nH, hd=hd, stride=stride, window=window, qoff=0,
                         grp=nH // nkv, pos=pos)
        assert O.normwise_rel_err(_np(out), ref) <= 1e-4, pos
    g.destroy()


@pytest.mark.parametrize("nH,nkv,hd,stride,window,pos,keqv", [
    (16, 8, 256, 1024, 1024, 0, False),      # first token
    (16, 8, 256, 1024, 1024, 700, False),    # slot in the middle split
    (16, 8, 256, 1024, 1024, 2500, False),   # ring wrapped: slot 452, all 1024 keys live
    (16, 2, 512, 2048, 0, 1500, True),       # global layer, k == v, grp 8
    (4, 4, 64, 40, 0, 45, False),            # global layer past its cache depth: nothing written
])
def test_prepkv_attn_fused_equals_separate(gpu, nH, nkv, hd, stride, window, pos, keqv):
    """q4_prepkv_attn (prepkv folded into the attention split kernel) leaves
    the same caches and the same output, bit for bit, as q4_prepkv followed
    by q4_attn."""
    rng = np.random.default_rng(nH + hd + pos)
    qkv, qnw, cs, sn, kc, vc = _attn_case(rng, nH, nkv, hd, stride)
    knw = (rng.random(hd) + 0.5).astype(np.float32)
    koff, voff = nH * hd, nH * hd + nkv * hd
    dyn = torch.tensor([pos, pos + 1, 0, 0], dtype=torch.int32, device="cuda")
    t = dict(qkv=_t(qkv), knw=_t(knw), qnw=_t(qnw), cs=_t(cs), sn=_t(sn))
    kc1, vc1 = _t(kc, torch.float16), _t(vc, torch.float16)
    kc2, vc2 = kc1.clone(), vc1.clone()
    kw = dict(nH=nH, nkv=nkv, hd=hd, stride=stride, window=window, qoff=0, grp=nH // nkv, dyn=dyn)
    for odt in (torch.float32, torch.float16):
        gpu.prepkv(t["qkv"], t["knw"], t["cs"], t["sn"], kc1, vc1, nkv=nkv, hd=hd, koff=koff, voff=voff, keqv=keqv,
                   stride=stride, window=window, dyn=dyn)
        o1 = gpu.attn(t["qkv"], t["qnw"], t["cs"], t["sn"], kc1, vc1, out_dtype=odt, **kw)
        o2 = gpu.prepkv_attn(t["qkv"], t["knw"], t["qnw"], t["cs"], t["sn"], kc2, vc2, koff=koff, voff=voff, keqv=keqv,
                             out_dtype=odt, **kw)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2) and torch.equal(kc1, kc2) and torch.equal(vc1, vc2), odt
