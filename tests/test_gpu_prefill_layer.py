"""Prefill of a prompt through the engine mirror (vk_engine.py): a small
Gemma-style model (one sliding-window layer, one global k==v layer) built
with the reference's prefill descriptor helpers, recorded once in the
reference's per-layer order (src/vk_engine.py:410-424) and replayed per
128-token chunk with p0 and the RoPE rows written to device buffers
(src/vk_engine.py:482-487), against the oracle's chunk: W4A16 GEMMs as
f16(f16(x) @ f16((q-8) s)^T) (the reference's casts and its shader's fp16
weights), the prefill ops of oracle/prefill_ops_oracle.py, fp16 KV caches
carried across chunks. Three chunks: the sliding layer's 256-slot ring
fills and wraps.

Tolerance: the residual stream after each chunk, normwise
max|x - ref| / max|ref| <= 1e-3 (fp32 device arithmetic and fp16 GEMM
outputs against float64 with the same fp16 roundings; a GEMM output can
round to the neighbouring fp16 value). The KV caches within 2e-3: a k
element that rounded to its neighbouring fp16 value moves the RoPE outputs
it feeds by up to one fp16 ulp of that element (2^-11 relative), and each
cache entry is rounded to fp16 again, so entries can sit up to two ulps of
the largest entries (~2e-3 normwise) from the float64 value.
"""
import importlib

import numpy as np
import pytest
import torch

from oracle import decode_ops_oracle as D
from oracle import prefill_ops_oracle as P
from oracle import q4_oracle as O

pytestmark = pytest.mark.gpu

H, NH, I = 256, 4, 512
LAYERS = [dict(hd=64, nkv=2, keqv=False, window=256, stride=256, scl=0.5),
          dict(hd=128, nkv=1, keqv=True, window=0, stride=512, scl=1.0)]
CHUNKS = 3


def _rope_rows(M, hd, p0):
    inv = 1.0 / (10000.0 ** (np.arange(0, hd, 2) / hd))
    ang = (p0 + np.arange(M))[:, None] * inv[None, :]
    return (np.concatenate([np.cos(ang)] * 2, 1).astype(np.float32),
            np.concatenate([np.sin(ang)] * 2, 1).astype(np.float32))


def _f16(a):
    return np.asarray(a, np.float64).astype(np.float16).astype(np.float64)


@pytest.mark.parametrize("fast,stacked", [(False, False), (True, False), (True, True)])
def test_prefill_chunks_through_the_engine_mirror(g4, gpu, fast, stacked):
    """fast: fp16 buffers between producers and GEMMs (no cast launches) and
    each pre_na fused with the pre_norm after it; otherwise the reference's
    fp32 buffers, casts and separate launches. stacked: q/k/v as one GEMM
    over their stacked rows (p_qkv; prepkv and attention read q, k, v at
    column offsets of its rows), gate/up with the gelumul as one gated
    W4A16 GEMM over interleaved rows (p_gu), the o and down GEMMs' split-K
    partials summed inside the normadd after them, and the q/k/v GEMM's inside
    the q store + prepkv after it (gemm_norms)."""
    E = importlib.import_module("g4mi.vk_engine")
    MC = E.MC
    rng = np.random.default_rng(0)
    f32 = lambda a: np.asarray(a, np.float32)
    h16 = torch.float16 if fast else torch.float32

    def lin(N, K):
        W = f32(rng.standard_normal((N, K)) * (1.0 / np.sqrt(K)))
        q, sc = O.quant_codes(W)
        wd16 = _f16(O.dequant(q, sc.astype(np.float16).astype(np.float32)))
        return E.quant(W, pf=True, fp8=False, prefill_i8=False), (N, K), wd16

    def wbuf(a):
        b = E.Buf(f32(a).nbytes)
        b.write(f32(a))
        return b

    fb = lambda n: E.Buf(n * 4)
    maxq = max(NH * L["hd"] for L in LAYERS)
    maxk = max(L["nkv"] * L["hd"] for L in LAYERS)
    Xp, Np, Tp = fb(MC * H), fb(MC * H), fb(MC * H)
    Qp, Ap, Kp, Vp = fb(MC * maxq), fb(MC * maxq), fb(MC * maxk), fb(MC * maxk)
    Gp, Upp, ACp = fb(MC * I), fb(MC * I), fb(MC * I)
    QKVp = fb(MC * (maxq + 2 * maxk))
    cosM = {hd: fb(MC * hd) for hd in (64, 128)}
    sinM = {hd: fb(MC * hd) for hd in (64, 128)}
    DYNP = E.buf_u32([0, MC, 0, 0])
    DUH = E.buf_u32([H, 0, 0, 0])
    DUIp = E.buf_u32([MC * I, 0, 0, 0])
    layers, ref_layers = [], []
    for cfg in LAYERS:
        hd, nkv, keqv = cfg["hd"], cfg["nkv"], cfg["keqv"]
        nq, nk = NH * hd, nkv * hd
        qp, kp = lin(nq, H), lin(nk, H)
        vp = None if keqv else lin(nk, H)
        op, gp, up, dp = lin(H, nq), lin(I, H), lin(I, H), lin(H, I)
        norms = {k: f32(rng.random(n) + 0.5) for k, n in dict(qnw=hd, knw=hd, inw=H, paw=H, pfw=H, ofw=H).items()}
        norms["qnw"] = f32(norms["qnw"] * (2.0 / hd))   # scores of a few units, as in the decode tests
        kc, vc = E.Buf(nkv * cfg["stride"] * hd * 2), E.Buf(nkv * cfg["stride"] * hd * 2)
        kc.write(np.zeros(nkv * cfg["stride"] * hd, np.float16))
        vc.write(np.zeros(nkv * cfg["stride"] * hd, np.float16))
        nb = {k: wbuf(v) for k, v in norms.items()}
        gk = dict(x_dtype=h16, y_dtype=h16)
        vsrc = Kp if keqv else Vp
        Pp = [nkv, hd, nk, 0, cfg["stride"], cfg["window"], 0, 0]
        Aa = [NH, nq, hd, cfg["stride"], cfg["window"], NH // nkv, 0, 0]
        ldc = nq + (nk if keqv else 2 * nk)
        qsrc, ksrc = (QKVp, QKVp) if stacked else (Qp, Kp)
        vsrc = QKVp if stacked else vsrc
        kv_at = dict(ld=ldc, koff=nq, voff=nq if keqv else nq + nk) if stacked else {}
        q_at = dict(ldq=ldc) if stacked else {}
        nas = E.buf_u32([H, int(np.array([cfg["scl"]], np.float32).view(np.uint32)[0]), 0, 0])
        L = dict(p_in=E.pre_norm_ds(Xp, nb["inw"], Np, DUH, out_dtype=h16),
                 p_q=E.gemm_ds(qp[:2], Np, Qp, **gk), p_k=E.gemm_ds(kp[:2], Np, Kp, **gk),
                 p_v=None if keqv else E.gemm_ds(vp[:2], Np, Vp, **gk),
                 p_qkv=E.gemm_cat_ds([qp[:2], kp[:2]] + ([] if keqv else [vp[:2]]), Np, QKVp, **gk)
                 if stacked else None,
                 p_prep=E.pre_prepkv_ds(ksrc, vsrc, nb["knw"], cosM[hd], sinM[hd], kc, vc, Pp, DYNP, kv_dtype=h16,
                                        **kv_at),
                 p_attn=E.pre_attn_ds(qsrc, nb["qnw"], cosM[hd], sinM[hd], kc, vc, Ap, Aa, DYNP, nkv, q_dtype=h16,
                                      out_dtype=h16, **q_at),
                 p_o=E.gemm_ds(op[:2], Ap, Tp, **gk),
                 p_na=E.pre_na_ds(Tp, nb["paw"], Xp, DUH, x_dtype=h16),
                 p_pfn=E.pre_norm_ds(Xp, nb["pfw"], Np, DUH, out_dtype=h16),
                 p_g=E.gemm_ds(gp[:2], Np, Gp, **gk), p_u=E.gemm_ds(up[:2], Np, Upp, **gk),
                 p_gm=E.pre_gelumul_ds(Gp, Upp, ACp, DUIp, in_dtype=h16, out_dtype=h16),
                 p_gu=E.pre_gate_up_ds(gp[:2], up[:2], Np, ACp) if stacked else None,
                 p_d=E.gemm_ds(dp[:2], ACp, Tp, **gk),
                 p_nas=E.pre_na_ds(Tp, nb["ofw"], Xp, nas, x_dtype=h16))
        layers.append((L, kc, vc))
        ref_layers.append(dict(cfg, nq=nq, nk=nk, q=qp[2], k=kp[2], v=None if keqv else vp[2], o=op[2], g=gp[2],
                               u=up[2], d=dp[2], kc=np.zeros(nkv * cfg["stride"] * hd, np.float16),
                               vc=np.zeros(nkv * cfg["stride"] * hd, np.float16), **norms))
    graph = E.record_prefill([L for L, _, _ in layers], fuse=fast, gemm_norms=stacked)
    if stacked:  # every o/down GEMM fused into its normadd, every q/k/v GEMM into its prepkv
        fns = [getattr(op, "fn", None) for op in graph.seq]
        assert fns.count(g4.ops.gemm_w4a16_normadd) == 2 * len(layers)
        assert fns.count(g4.ops.gemm_w4a16_qkv_prepkv) == len(layers)

    gemm = lambda x, wd16: _f16(_f16(x) @ wd16.T)
    for chunk in range(CHUNKS):
        p0 = chunk * MC
        emb = f32(rng.standard_normal((MC, H)))
        Xp.write(emb)
        DYNP.write(np.array([p0, MC, 0, 0], np.uint32))
        tabs = {hd: _rope_rows(MC, hd, p0) for hd in (64, 128)}
        for hd, (c, s) in tabs.items():
            cosM[hd].write(c)
            sinM[hd].write(s)
        E.submit(graph, label=f"prefill p0={p0}", timeout_ms=20000)
        x_dev = np.frombuffer(Xp.read(MC * H * 4), np.float32).reshape(MC, H)

        X = emb.astype(np.float64)
        for R in ref_layers:
            hd = R["hd"]
            c, s = tabs[hd]
            Xn = P.pre_rmsnorm_ref(X, R["inw"])
            q, k = gemm(Xn, R["q"]), gemm(Xn, R["k"])
            v = None if R["keqv"] else gemm(Xn, R["v"])
            R["kc"], R["vc"] = P.pre_prepkv_ref(k, v, R["knw"], c, s, R["kc"], R["vc"], nkv=R["nkv"], hd=hd,
                                                stride=R["stride"], window=R["window"], p0=p0)
            A = P.pre_attn_ref(q, R["qnw"], c, s, R["kc"], R["vc"], nH=NH, hd=hd, stride=R["stride"],
                               window=R["window"], grp=NH // R["nkv"], p0=p0)
            X = P.pre_normadd_ref(gemm(A, R["o"]), R["paw"], X)
            Xn2 = P.pre_rmsnorm_ref(X, R["pfw"])
            act = D.gelumul_ref(gemm(Xn2, R["g"]), gemm(Xn2, R["u"]))
            X = P.pre_normadd_ref(gemm(act, R["d"]), R["ofw"], X, R["scl"])
        assert O.normwise_rel_err(x_dev, X) <= 1e-3, chunk
        for (L, kc, vc), R in zip(layers, ref_layers):
            n = R["nkv"] * R["stride"] * R["hd"]
            gk = np.frombuffer(kc.read(n * 2), np.float16).astype(np.float64)
            gv = np.frombuffer(vc.read(n * 2), np.float16).astype(np.float64)
            assert O.normwise_rel_err(gk, R["kc"].astype(np.float64)) <= 2e-3, chunk
            assert O.normwise_rel_err(gv, R["vc"].astype(np.float64)) <= 2e-3, chunk
            # carry the device caches so later chunks compare like with like
            R["kc"], R["vc"] = gk.astype(np.float16), gv.astype(np.float16)
    graph.destroy()
