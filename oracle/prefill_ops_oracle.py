"""numpy restatement of the reference's batched-prefill layer ops.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the shipped package
never imports this file; tests use it as the checker.

The reference prefills a chunk of M tokens (positions p0 .. p0+M-1) per
layer as (``src/vk_engine.py:410-424``): pre_norm -> q/k/v GEMMs ->
pre_prepkv (every token's K and V into the fp16 cache) -> pre_attn (every
token's causal attention over the cache) -> o GEMM -> pre_na -> pre_norm ->
gate/up GEMMs -> gelumul -> down GEMM -> pre_na. The shaders are
``vk/pre_norm.comp``, ``vk/pre_na.comp``, ``vk/pre_prepkv.comp`` and
``vk/pre_attn.comp`` (one workgroup per token, or per (head, token)); the
row arithmetic is the decode shaders', restated in
``oracle/decode_ops_oracle.py``, applied per token with the token's own
position and RoPE row. The one new rule is pre_attn's ring mask: the whole
chunk's K/V are written before any token attends, so in a sliding layer a
ring slot can hold a key from later in the chunk than the query; such keys
are skipped (``vk/pre_attn.comp:39-41``).

Everything is in float64; cache entries are rounded to fp16 where the
shaders round them. Parity status: pinned in ``tests/test_oracle_prefill.py``
(per-row equality with the pinned decode functions, the ring-mask closed
form, causality, brute-force softmax).
"""
from __future__ import annotations

import numpy as np

from oracle import decode_ops_oracle as D


def _f64(a):
    return np.asarray(a, dtype=np.float64)


def pre_rmsnorm_ref(X, w) -> np.ndarray:
    """Every row of ``X`` [M, D] through rmsnorm (``vk/pre_norm.comp:9-13``)."""
    return np.stack([D.rmsnorm_ref(x, w) for x in _f64(X)])


def pre_normadd_ref(X, w, Hm, scale: float = 0.0) -> np.ndarray:
    """``h[m] = (h[m] + rmsnorm(x[m]) * w) * sc`` per row (``vk/pre_na.comp:9-14``)."""
    return np.stack([D.normadd_ref(x, w, h, scale) for x, h in zip(_f64(X), _f64(Hm))])


def pre_prepkv_ref(K, V, knw, cosM, sinM, kc, vc, *, nkv, hd, stride, window, p0):
    """K (k-norm with weight, RoPE with the token's cos/sin row) and V
    (v-norm) of tokens m = 0 .. M-1 at positions p0 + m into the caches, in
    token order, so a later token overwrites an earlier one's ring slot
    (``vk/pre_prepkv.comp:18-32``). ``K``, ``V`` [M, nkv * hd] (``V`` None:
    k == v, V read from K). Returns new copies of the caches."""
    K = _f64(K)
    V = K if V is None else _f64(V)
    M = K.shape[0]
    nk = nkv * hd
    for m in range(M):
        row = np.concatenate([K[m], V[m]])
        kc, vc = D.prepkv_ref(row, knw, _f64(cosM)[m], _f64(sinM)[m], kc, vc, nkv=nkv, hd=hd, koff=0, voff=nk,
                              keqv=False, stride=stride, window=window, pos=p0 + m)
    return kc, vc


def slot_position(slot: int, base: int, window: int) -> int:
    """Absolute position of the key a ring slot holds once positions up to
    ``base`` (the chunk's last token) are written: ``base - ((base + window -
    slot) mod window)`` (``vk/pre_attn.comp:40``)."""
    return base - ((base + window - slot) % window)


def pre_attn_ref(Q, qnw, cosM, sinM, kc, vc, *, nH, hd, stride, window, grp, p0) -> np.ndarray:
    """Causal attention of tokens m = 0 .. M-1 (positions p0 + m), every
    query head, over the cache after the whole chunk was written
    (``vk/pre_attn.comp:18-53``): q-norm with weight and RoPE with the
    token's row, scores over the first ``T`` slots of KV head ``h // grp``
    (``T = pos + 1``, or ``min(pos + 1, window)`` for a ring), slots whose
    key position is after the token's skipped (ring layers only), no score
    scaling, softmax, fp16 V rows. Returns ``[M, nH * hd]``."""
    Q = _f64(Q)
    M = Q.shape[0]
    base_pos = p0 + M - 1
    kch = _f64(np.asarray(kc, dtype=np.float16)).reshape(-1, stride, hd)
    vch = _f64(np.asarray(vc, dtype=np.float16)).reshape(-1, stride, hd)
    out = np.zeros((M, nH * hd))
    for m in range(M):
        pos = p0 + m
        T = min(pos + 1, window) if window > 0 else pos + 1
        T = min(T, stride)
        live = np.array([s for s in range(T) if window == 0 or slot_position(s, base_pos, window) <= pos])
        for h in range(nH):
            q = Q[m, h * hd: (h + 1) * hd]
            q = D.rope_ref(q * D.rms_inv(q) * _f64(qnw)[:hd], _f64(cosM)[m], _f64(sinM)[m])
            Kr = kch[h // grp][live]
            Vr = vch[h // grp][live]
            sc = Kr @ q
            p = np.exp(sc - sc.max())
            out[m, h * hd: (h + 1) * hd] = (p @ Vr) / p.sum()
    return out
