"""numpy restatement of the reference's decode-token ops between the GEMVs.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the shipped package
never imports this file; tests use it as the checker.

The reference records, per layer (``src/vk_engine.py:277-287``): rmsnorm ->
q/k/v GEMVs -> prepkv (k-norm + RoPE into the fp16 KV cache, v-norm) ->
attention (q-norm + RoPE, softmax over the cached keys) -> o GEMV ->
normadd -> rmsnorm -> gate/up GEMVs -> gelumul -> down GEMV -> normadd. The
shaders are ``vk/rmsnorm.comp``, ``vk/normadd.comp``, ``vk/gelumul.comp``,
``vk/prepkv.comp`` and ``vk/attn.comp``; citations are relative to the
reference repository root.

Everything is computed in float64 (the mathematical value of each shader's
fp32 arithmetic); KV-cache entries are rounded to fp16 exactly where the
shaders round them. Parity status: every function is pinned in
``tests/test_oracle_decode.py`` by closed forms, invariants and special
cases, and ``attn_ref`` (direct softmax) against ``attn_online_ref`` (the
shader's tiled online softmax restated loop by loop).
"""
from __future__ import annotations

import numpy as np

EPS = 1e-6  # every norm in the shaders: inversesqrt(mean(x^2) + 1e-6)


def _f64(a):
    return np.asarray(a, dtype=np.float64)


def rms_inv(x) -> float:
    """``inversesqrt(sum(x^2) / D + 1e-6)`` (``vk/rmsnorm.comp:9-11``)."""
    x = _f64(x)
    return 1.0 / np.sqrt(np.dot(x, x) / x.size + EPS)


def rmsnorm_ref(x, w) -> np.ndarray:
    """``y = x * inv * w`` (``vk/rmsnorm.comp:8-12``)."""
    x = _f64(x)
    return x * rms_inv(x) * _f64(w)


def normadd_ref(x, w, h, scale: float = 0.0) -> np.ndarray:
    """``h = (h + x * inv * w) * sc`` with ``sc = scale`` unless it is 0, then 1
    (``vk/normadd.comp:8-12``: the uniform's second word holds the scale's
    bits, 0 meaning unscaled). Returns the new ``h``."""
    x = _f64(x)
    sc = 1.0 if scale == 0.0 else float(scale)
    return (_f64(h) + x * rms_inv(x) * _f64(w)) * sc


def gelumul_ref(gate, up) -> np.ndarray:
    """``0.5 x (1 + tanh(0.7978845608028654 (x + 0.044715 x^3))) * up``
    (``vk/gelumul.comp:7-8``)."""
    x = _f64(gate)
    g = 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)))
    return g * _f64(up)


def rope_ref(v, cosb, sinb) -> np.ndarray:
    """Rotate-half RoPE of one head (``vk/prepkv.comp:24``, ``vk/attn.comp:29``):
    ``out[i] = v[i] cos[i] + r[i] sin[i]`` with ``r[i] = -v[i + hd/2]`` for the
    first half and ``v[i - hd/2]`` for the second."""
    v = _f64(v)
    hf = v.size // 2
    r = np.concatenate([-v[hf:], v[:hf]])
    return v * _f64(cosb)[: v.size] + r * _f64(sinb)[: v.size]


def kv_slot(pos: int, window: int) -> int:
    """Cache slot of token ``pos``: a ring of ``window`` slots for sliding
    layers, ``pos`` itself for global ones (``vk/prepkv.comp:18``)."""
    return pos % window if window > 0 else pos


def prepkv_ref(qkv, knw, cosb, sinb, kc, vc, *, nkv, hd, koff, voff, keqv, stride, window, pos):
    """Write this token's K (k-norm, weight, RoPE) and V (v-norm, no weight)
    of every KV head into the fp16 caches ``kc``/``vc`` (``[nkv, stride, hd]``
    flattened) at the token's slot (``vk/prepkv.comp:16-30``). With ``keqv``
    V is read from the K part of ``qkv``. Returns new copies of the caches."""
    qkv = _f64(qkv)
    kc = np.array(kc, dtype=np.float16, copy=True)
    vc = np.array(vc, dtype=np.float16, copy=True)
    slot = kv_slot(pos, window)
    vo = koff if keqv else voff
    for h in range(nkv):
        k = qkv[koff + h * hd: koff + (h + 1) * hd]
        kn = k * rms_inv(k) * _f64(knw)[:hd]
        o = (h * stride + slot) * hd
        kc[o: o + hd] = rope_ref(kn, cosb, sinb).astype(np.float16)
        v = qkv[vo + h * hd: vo + (h + 1) * hd]
        vc[o: o + hd] = (v * rms_inv(v)).astype(np.float16)
    return kc, vc


def _attn_inputs(qkv, qnw, cosb, sinb, kc, *, h, hd, stride, window, qoff, grp, pos):
    q = _f64(qkv)[qoff + h * hd: qoff + (h + 1) * hd]
    q = rope_ref(q * rms_inv(q) * _f64(qnw)[:hd], cosb, sinb)
    T = min(pos + 1, window) if window > 0 else pos + 1
    kvh = h // grp
    base = kvh * stride * hd
    K = _f64(np.asarray(kc, dtype=np.float16)[base: base + T * hd]).reshape(T, hd)
    return q, T, base, K


def attn_ref(qkv, qnw, cosb, sinb, kc, vc, *, nH, hd, stride, window, qoff, grp, pos) -> np.ndarray:
    """Decode attention of every query head (``vk/attn.comp:18-53``): q from
    ``qkv`` (q-norm with weight, RoPE), scores ``q . k_j`` over the first
    ``T`` cache slots of KV head ``h // grp`` (``T = pos + 1``, or
    ``min(pos + 1, window)`` for a ring), no score scaling, softmax, weighted
    sum of the fp16 V rows. Direct softmax; returns ``[nH * hd]``."""
    out = np.zeros(nH * hd)
    for h in range(nH):
        q, T, base, K = _attn_inputs(qkv, qnw, cosb, sinb, kc, h=h, hd=hd, stride=stride, window=window,
                                     qoff=qoff, grp=grp, pos=pos)
        V = _f64(np.asarray(vc, dtype=np.float16)[base: base + T * hd]).reshape(T, hd)
        s = K @ q
        p = np.exp(s - s.max())
        out[h * hd: (h + 1) * hd] = (p @ V) / p.sum()
    return out


def attn_online_ref(qkv, qnw, cosb, sinb, kc, vc, *, nH, hd, stride, window, qoff, grp, pos,
                    tile: int = 256) -> np.ndarray:
    """The shader's own algorithm, loop by loop (``vk/attn.comp:31-52``):
    tiles of ``tile`` keys, running max ``m`` and sum ``l``, accumulator
    rescaled by ``exp(m_old - m_new)`` per tile. Kept to pin ``attn_ref``."""
    out = np.zeros(nH * hd)
    vcf = _f64(np.asarray(vc, dtype=np.float16))
    for h in range(nH):
        q, T, base, K = _attn_inputs(qkv, qnw, cosb, sinb, kc, h=h, hd=hd, stride=stride, window=window,
                                     qoff=qoff, grp=grp, pos=pos)
        m, l = -1e30, 0.0
        acc = np.zeros(hd)
        t0 = 0
        while t0 < T:
            n = min(tile, T - t0)
            sc = [float(np.dot(q, K[t0 + j])) for j in range(n)]
            mn = max(m, max(sc))
            corr = np.exp(m - mn)
            m = mn
            p = [np.exp(s - mn) for s in sc]
            l = l * corr + sum(p)
            for i in range(hd):
                a = acc[i] * corr
                for j in range(n):
                    a += p[j] * vcf[base + (t0 + j) * hd + i]
                acc[i] = a
            t0 += tile
        out[h * hd: (h + 1) * hd] = acc / l
    return out
