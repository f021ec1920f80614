"""Pins of oracle/prefill_ops_oracle.py (CPU): each prefill op against the
pinned decode oracle applied token by token, the ring-slot closed form
against a simulated ring, causality, and a brute-force visible-key set."""
import numpy as np

from oracle import decode_ops_oracle as D
from oracle import prefill_ops_oracle as P


def _rope_rows(M, hd, p0, rng):
    inv = 1.0 / (10000.0 ** (np.arange(0, hd, 2) / hd))
    ang = (p0 + np.arange(M))[:, None] * inv[None, :]
    return np.concatenate([np.cos(ang)] * 2, 1), np.concatenate([np.sin(ang)] * 2, 1)


def test_pre_norms_are_row_wise_decode_norms():
    rng = np.random.default_rng(0)
    X, Hm, w = rng.standard_normal((5, 96)), rng.standard_normal((5, 96)), rng.random(96) + 0.5
    Y = P.pre_rmsnorm_ref(X, w)
    H2 = P.pre_normadd_ref(X, w, Hm, 0.75)
    for m in range(5):
        assert np.array_equal(Y[m], D.rmsnorm_ref(X[m], w))
        assert np.array_equal(H2[m], D.normadd_ref(X[m], w, Hm[m], 0.75))
    # rows are independent: a permutation of the rows permutes the outputs
    perm = rng.permutation(5)
    assert np.array_equal(P.pre_rmsnorm_ref(X[perm], w), Y[perm])
    # constant rows normalise to the weight (closed form, eps aside)
    c = P.pre_rmsnorm_ref(np.full((2, 96), 3.0), w)
    assert np.allclose(c, w * 3.0 / np.sqrt(9.0 + D.EPS))


def test_slot_position_matches_a_simulated_ring():
    for window in (4, 7, 16):
        for base in range(0, 3 * window):
            ring = {}
            for pos in range(base + 1):
                ring[pos % window] = pos
            for slot, pos in ring.items():
                assert P.slot_position(slot, base, window) == pos, (window, base, slot)


def test_pre_prepkv_equals_decode_prepkv_token_by_token_and_last_writer_wins():
    rng = np.random.default_rng(1)
    nkv, hd, M, window, stride, p0 = 2, 16, 6, 4, 4, 3
    K, V = rng.standard_normal((M, nkv * hd)), rng.standard_normal((M, nkv * hd))
    knw = rng.random(hd) + 0.5
    cosM, sinM = _rope_rows(M, hd, p0, rng)
    kc0 = np.zeros(nkv * stride * hd, np.float16)
    kc, vc = P.pre_prepkv_ref(K, V, knw, cosM, sinM, kc0, kc0, nkv=nkv, hd=hd, stride=stride, window=window, p0=p0)
    # the ring holds, per slot, the last of the chunk's tokens mapped to it
    for m in range(M - window, M):
        slot = (p0 + m) % window
        for h in range(nkv):
            k = K[m, h * hd:(h + 1) * hd]
            want = D.rope_ref(k * D.rms_inv(k) * knw, cosM[m], sinM[m]).astype(np.float16)
            o = (h * stride + slot) * hd
            assert np.array_equal(kc[o:o + hd], want)
            v = V[m, h * hd:(h + 1) * hd]
            assert np.array_equal(vc[o:o + hd], (v * D.rms_inv(v)).astype(np.float16))
    # k == v: V taken from K
    kc2, vc2 = P.pre_prepkv_ref(K, None, knw, cosM, sinM, kc0, kc0, nkv=nkv, hd=hd, stride=stride, window=window,
                                p0=p0)
    assert np.array_equal(kc2, kc)
    kv = K[M - 1, :hd]
    slot = (p0 + M - 1) % window
    assert np.array_equal(vc2[slot * hd:(slot + 1) * hd], (kv * D.rms_inv(kv)).astype(np.float16))


def _chunk(rng, *, M, nH, nkv, hd, stride, window, p0, prior):
    """Caches holding `prior` earlier random keys, then the chunk written."""
    kc = np.zeros(nkv * stride * hd, np.float16)
    vc = np.zeros(nkv * stride * hd, np.float16)
    for pos in range(p0 - prior, p0):
        s = pos % window if window else pos
        for h in range(nkv):
            o = (h * stride + s) * hd
            kc[o:o + hd] = rng.standard_normal(hd).astype(np.float16)
            vc[o:o + hd] = rng.standard_normal(hd).astype(np.float16)
    K, V = rng.standard_normal((M, nkv * hd)), rng.standard_normal((M, nkv * hd))
    cosM, sinM = _rope_rows(M, hd, p0, rng)
    knw = rng.random(hd) + 0.5
    kc, vc = P.pre_prepkv_ref(K, V, knw, cosM, sinM, kc, vc, nkv=nkv, hd=hd, stride=stride, window=window, p0=p0)
    Q = rng.standard_normal((M, nH * hd))
    qnw = (rng.random(hd) + 0.5) * (2.0 / hd)
    return Q, qnw, cosM, sinM, kc, vc, K, V, knw


def test_pre_attn_without_wrap_is_causal_decode_attention():
    """No ring wrap inside the chunk (and a global layer): token m's output
    equals the pinned decode attention at pos = p0 + m on the cache as it
    stood right after token m was written."""
    rng = np.random.default_rng(2)
    for window, stride, p0 in [(0, 64, 5), (32, 32, 4)]:
        nH, nkv, hd, M = 4, 2, 16, 8
        Q, qnw, cosM, sinM, kc, vc, K, V, knw = _chunk(rng, M=M, nH=nH, nkv=nkv, hd=hd, stride=stride,
                                                       window=window, p0=p0, prior=p0)
        out = P.pre_attn_ref(Q, qnw, cosM, sinM, kc, vc, nH=nH, hd=hd, stride=stride, window=window,
                             grp=nH // nkv, p0=p0)
        for m in range(M):
            # decode attention reads slots 0 .. pos only, so later tokens of the chunk are invisible to it
            ref = D.attn_ref(Q[m], qnw, cosM[m], sinM[m], kc, vc, nH=nH, hd=hd, stride=stride, window=window,
                             qoff=0, grp=nH // nkv, pos=p0 + m)
            assert np.allclose(out[m], ref, rtol=0, atol=1e-12), (window, m)


def test_pre_attn_ring_wrap_brute_force_visible_keys():
    """A chunk that wraps the ring: the keys a token sees are exactly the
    slots whose current occupant (simulated) is at or before it; a token
    whose only visible key is one slot returns that V row."""
    rng = np.random.default_rng(3)
    nH, nkv, hd, M, window, p0 = 2, 1, 8, 4, 4, 9
    Q, qnw, cosM, sinM, kc, vc, K, V, knw = _chunk(rng, M=M, nH=nH, nkv=nkv, hd=hd, stride=window, window=window,
                                                   p0=p0, prior=window)
    out = P.pre_attn_ref(Q, qnw, cosM, sinM, kc, vc, nH=nH, hd=hd, stride=window, window=window, grp=2, p0=p0)
    occupant = {}
    for pos in range(p0 + M):
        occupant[pos % window] = pos
    kch, vch = kc.astype(np.float64), vc.astype(np.float64)
    for m in range(M):
        pos = p0 + m
        vis = [s for s in range(min(pos + 1, window)) if occupant[s] <= pos]
        for h in range(nH):
            q = Q[m, h * hd:(h + 1) * hd]
            q = D.rope_ref(q * D.rms_inv(q) * qnw, cosM[m], sinM[m])
            sc = np.array([np.dot(q, kch[s * hd:(s + 1) * hd]) for s in vis])
            p = np.exp(sc - sc.max())
            want = sum(p[i] * vch[s * hd:(s + 1) * hd] for i, s in enumerate(vis)) / p.sum()
            assert np.allclose(out[m, h * hd:(h + 1) * hd], want, rtol=0, atol=1e-12)
            if len(vis) == 1:
                assert np.allclose(want, vch[vis[0] * hd:(vis[0] + 1) * hd])
    # a chunk as long as the ring: its first token sees only its own key (the
    # earlier positions' slots were overwritten by the chunk's later tokens)
    assert [s for s in range(window) if occupant[s] <= p0] == [p0 % window]
