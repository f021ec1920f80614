"""Pins of the decode-op oracle (oracle/decode_ops_oracle.py).

The reference has no known-answer tests for these shaders either; each
function is pinned by closed forms and invariants (a constant vector
normalises to the weight, RoPE preserves the norm of each rotated pair and
is the identity at angle 0), by library routines (the erf GELU that the
tanh form approximates), and attention by special cases (one key, equal
keys, a dominant key) plus the direct softmax against the shader's tiled
online softmax restated loop by loop.
"""
import math

import numpy as np
import pytest

from oracle import decode_ops_oracle as D


def test_rmsnorm_constant_vector_gives_weight():
    x = np.full(3840, -2.5)
    w = np.linspace(0.5, 1.5, 3840)
    y = D.rmsnorm_ref(x, w)
    # mean(x^2) = 6.25: y = -2.5 / sqrt(6.25 + 1e-6) * w
    assert np.allclose(y, -2.5 / math.sqrt(6.25 + 1e-6) * w, rtol=1e-15)


def test_rmsnorm_zero_and_scale_invariance():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(512)
    w = rng.random(512) + 0.5
    assert (D.rmsnorm_ref(np.zeros(512), w) == 0).all()
    # scale invariance up to eps: mean(x^2) ~ 1, so eps = 1e-6 moves the result by ~5e-7 relative
    assert np.allclose(D.rmsnorm_ref(100 * x, w), D.rmsnorm_ref(x, w), rtol=1e-6)
    assert not np.allclose(D.rmsnorm_ref(100 * x, w), D.rmsnorm_ref(x, w), rtol=1e-8)
    # with unit weights the output has mean square 1 (up to eps)
    y = D.rmsnorm_ref(x, np.ones(512))
    assert abs(np.mean(y * y) - 1.0) < 1e-5


def test_normadd_residual_and_scale_rule():
    rng = np.random.default_rng(2)
    x, h = rng.standard_normal(256), rng.standard_normal(256)
    w = rng.random(256)
    n = D.rmsnorm_ref(x, w)
    assert np.allclose(D.normadd_ref(x, w, h), h + n, rtol=1e-15)
    assert np.allclose(D.normadd_ref(x, w, h, 0.0), h + n, rtol=1e-15)  # 0 means unscaled
    assert np.allclose(D.normadd_ref(x, w, h, 0.25), 0.25 * (h + n), rtol=1e-15)


def test_gelumul_known_values():
    g = np.array([0.0, 1.0, -1.0, 8.0, -8.0, 0.5])
    out = D.gelumul_ref(g, np.ones(6))
    assert out[0] == 0.0
    assert abs(out[1] - 0.8411919906082768) < 1e-12  # tanh form at 1
    assert abs(out[1] - out[2] - 1.0) < 1e-12        # gelu(x) - gelu(-x) = x
    assert abs(out[3] - 8.0) < 1e-12 and abs(out[4]) < 1e-12
    # the tanh form approximates x * Phi(x) to ~1e-3
    erf_gelu = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in g])
    assert np.max(np.abs(out - erf_gelu)) < 1e-3
    up = np.array([2.0, -3.0, 1.0, 0.5, 1.0, 4.0])
    assert np.allclose(D.gelumul_ref(g, up), out * up, rtol=1e-15)


def test_rope_identity_rotation_and_norm():
    rng = np.random.default_rng(3)
    v = rng.standard_normal(256)
    assert np.allclose(D.rope_ref(v, np.ones(256), np.zeros(256)), v, rtol=0)
    # 90 degrees: (a, b) -> (-b, a) for pairs (i, i + 128)
    r = D.rope_ref(v, np.zeros(256), np.ones(256))
    assert np.allclose(r[:128], -v[128:]) and np.allclose(r[128:], v[:128])
    ang = rng.random(128) * 6.0
    c = np.concatenate([np.cos(ang), np.cos(ang)])
    s = np.concatenate([np.sin(ang), np.sin(ang)])
    r = D.rope_ref(v, c, s)
    assert np.allclose(r[:128] ** 2 + r[128:] ** 2, v[:128] ** 2 + v[128:] ** 2, rtol=1e-12)


def test_kv_slot_ring_and_global():
    assert D.kv_slot(5, 0) == 5 and D.kv_slot(1029, 1024) == 5 and D.kv_slot(1023, 1024) == 1023


def _kv_case(rng, nkv, hd, stride, window, pos, keqv=False):
    nq = 4 * hd
    qkv = rng.standard_normal(nq + 2 * nkv * hd)
    knw = rng.random(hd) + 0.5
    ang = rng.random(hd // 2) * 3
    c = np.concatenate([np.cos(ang), np.cos(ang)])
    s = np.concatenate([np.sin(ang), np.sin(ang)])
    kc = rng.standard_normal(nkv * stride * hd).astype(np.float16)
    vc = rng.standard_normal(nkv * stride * hd).astype(np.float16)
    return dict(qkv=qkv, knw=knw, cosb=c, sinb=s, kc=kc, vc=vc, nq=nq)


@pytest.mark.parametrize("keqv", [False, True])
def test_prepkv_writes_one_slot_per_head(keqv):
    rng = np.random.default_rng(4)
    nkv, hd, stride, window, pos = 2, 64, 8, 8, 13
    c = _kv_case(rng, nkv, hd, stride, window, pos)
    koff, voff = c["nq"], c["nq"] + nkv * hd
    kc, vc = D.prepkv_ref(c["qkv"], c["knw"], c["cosb"], c["sinb"], c["kc"], c["vc"], nkv=nkv, hd=hd, koff=koff,
                          voff=voff, keqv=keqv, stride=stride, window=window, pos=pos)
    slot = 13 % 8
    for h in range(nkv):
        o = (h * stride + slot) * hd
        k = c["qkv"][koff + h * hd: koff + (h + 1) * hd]
        v = c["qkv"][(koff if keqv else voff) + h * hd:][:hd]
        # K: norm then weight then RoPE; the rotated pairs keep the normed pair norms
        kn = k / np.sqrt(np.mean(k * k) + 1e-6) * c["knw"]
        got = kc[o: o + hd].astype(np.float64)
        assert np.allclose(got[:32] ** 2 + got[32:] ** 2, kn[:32] ** 2 + kn[32:] ** 2, rtol=2e-3, atol=1e-3)
        # V: norm only, fp16
        assert np.array_equal(vc[o: o + hd], (v / np.sqrt(np.mean(v * v) + 1e-6)).astype(np.float16))
    # every other slot untouched
    mask = np.ones(nkv * stride, bool)
    mask[[h * stride + slot for h in range(nkv)]] = False
    assert np.array_equal(kc.reshape(-1, hd)[mask], c["kc"].reshape(-1, hd)[mask])
    assert np.array_equal(vc.reshape(-1, hd)[mask], c["vc"].reshape(-1, hd)[mask])


def _attn_args(rng, nH=4, nkv=2, hd=64, stride=40, window=0, pos=29):
    qkv = rng.standard_normal(nH * hd + 2 * nkv * hd)
    qnw = rng.random(hd) * 0.3 + 0.2  # keeps the scores moderate
    ang = rng.random(hd // 2) * 3
    c = np.concatenate([np.cos(ang), np.cos(ang)])
    s = np.concatenate([np.sin(ang), np.sin(ang)])
    kc = (rng.standard_normal(nkv * stride * hd) * 0.3).astype(np.float16)
    vc = rng.standard_normal(nkv * stride * hd).astype(np.float16)
    kw = dict(nH=nH, hd=hd, stride=stride, window=window, qoff=0, grp=nH // nkv, pos=pos)
    return qkv, qnw, c, s, kc, vc, kw


@pytest.mark.parametrize("window,pos,tile", [(0, 29, 8), (0, 29, 256), (16, 29, 5), (16, 7, 3)])
def test_attn_direct_equals_online(window, pos, tile):
    rng = np.random.default_rng(5 + pos)
    qkv, qnw, c, s, kc, vc, kw = _attn_args(rng, window=window, pos=pos)
    a = D.attn_ref(qkv, qnw, c, s, kc, vc, **kw)
    b = D.attn_online_ref(qkv, qnw, c, s, kc, vc, tile=tile, **kw)
    assert np.allclose(a, b, rtol=1e-12, atol=1e-12)


def test_attn_special_cases():
    rng = np.random.default_rng(6)
    qkv, qnw, c, s, kc, vc, kw = _attn_args(rng, pos=0)
    # one key: the output is that key's V row (KV head h // grp, slot 0)
    out = D.attn_ref(qkv, qnw, c, s, kc, vc, **kw)
    hd, stride = kw["hd"], kw["stride"]
    for h in range(kw["nH"]):
        kvh = h // kw["grp"]
        assert np.allclose(out[h * hd:(h + 1) * hd], vc[kvh * stride * hd:][:hd].astype(np.float64), rtol=1e-12)
    # identical keys: the output is the mean of the V rows of the window
    kw2 = dict(kw, pos=9, window=4)
    kc2 = np.tile(kc[:hd], kw["stride"] * 2)
    out = D.attn_ref(qkv, qnw, c, s, kc2, vc, **kw2)
    V = vc.astype(np.float64).reshape(2, stride, hd)
    assert np.allclose(out[:hd], V[0, :4].mean(axis=0), rtol=1e-12)
    # a dominant key takes the whole weight
    kc3 = np.zeros_like(kc)
    q0 = D.rope_ref(qkv[:hd] / np.sqrt(np.mean(qkv[:hd] ** 2) + 1e-6) * qnw, c, s)
    kc3[3 * hd: 4 * hd] = (q0 / np.linalg.norm(q0) * 8).astype(np.float16)  # score ~ 8 |q|, others 0
    out = D.attn_ref(qkv, qnw, c, s, kc3, vc, **dict(kw, pos=9))
    assert np.allclose(out[:hd], vc[3 * hd: 4 * hd].astype(np.float64), rtol=1e-6, atol=1e-6)
