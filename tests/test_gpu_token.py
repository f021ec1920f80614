"""A whole decode token through the engine mirror (vk_engine.py): a small
Gemma-style model (one sliding-window layer, one global k==v layer) built
with the reference's descriptor helpers, recorded once in the reference's
dispatch order (src/vk_engine.py:274-287) and replayed per token with the
position and RoPE tables written to device buffers, against the oracle's
token step (oracle GEMV on the same int4 codes and fp16 scales, oracle
decode ops, fp16 KV caches carried along).

Tolerance: logits normwise max|y - ref| / max|ref| <= 1e-3 over 20 tokens
(the ring of the sliding layer wraps at 16), fp32 device arithmetic against
float64 (with fp16 GEMV inputs, the oracle rounds the same inputs).
"""
import importlib

import numpy as np
import pytest
import torch

from oracle import decode_ops_oracle as D
from oracle import q4_oracle as O
from tests.helpers import to_np

pytestmark = pytest.mark.gpu

H, NH, I, V = 256, 4, 512, 1024
LAYERS = [dict(hd=64, nkv=2, keqv=False, window=16, stride=16, scl=0.5),
          dict(hd=128, nkv=1, keqv=True, window=0, stride=64, scl=1.0)]


def _rope(pos, hd):
    inv = 1.0 / (10000.0 ** (np.arange(0, hd, 2) / hd))
    ang = pos * inv
    return (np.concatenate([np.cos(ang)] * 2).astype(np.float32), np.concatenate([np.sin(ang)] * 2).astype(np.float32))


@pytest.mark.parametrize("fuse,half,gated,fg", [(False, False, False, False), (True, False, False, True),
                                                (True, True, False, False), (True, True, False, True),
                                                (True, True, True, False), (True, True, True, True),
                                                (False, False, True, False)])
def test_decode_token_through_the_engine_mirror(g4, gpu, fuse, half, gated, fg):
    """fuse: normadd + next rmsnorm as one launch; half: fp16 GEMV inputs
    (norm, gelumul and attention write fp16, the residual stream stays
    fp32): the oracle rounds the same GEMV inputs to fp16; gated: gate/up
    interleaved with the gelumul in the GEMV epilogue; fg: the fused norms
    with fp16 outputs inside the GEMV launches that read them."""
    _token_steps(gpu, fuse, half, gated, fg)


@pytest.mark.parametrize("fuse,half,gated,fg", [(True, True, True, True), (False, False, False, False)])
def test_decode_token_forward_with_device_inputs(g4, gpu, fuse, half, gated, fg):
    """forward(): the token id and position go into a pinned step buffer and
    the graph's first launch gathers the embedding row, the DYN words and
    both layer types' RoPE rows on the device (src/vk_engine.py:312-314 done
    in the graph): one launch and one bounded wait per token, same oracle
    tolerance over 20 tokens of random ids."""
    _token_steps(gpu, fuse, half, gated, fg, device_inputs=True)


def test_token_inputs_gather_and_clamp(g4, gpu):
    """q4_token_inputs alone, step in pinned host memory and in device memory:
    h, DYN and every table's cos/sin rows are the selected rows bit for bit,
    the host's later rewrite of the pinned step is what the next launch
    reads, and out-of-range values written past forward()'s check are
    clamped to the last row / position 0 (nothing is read outside the
    tables)."""
    rng = np.random.default_rng(3)
    vocab, Hh, max_pos = 300, 260, 50
    emb = torch.from_numpy(rng.standard_normal((vocab, Hh)).astype(np.float32)).cuda()
    tabs = []
    for hd in (64, 128):
        ct = torch.from_numpy(rng.standard_normal((max_pos, hd)).astype(np.float32)).cuda()
        st = torch.from_numpy(rng.standard_normal((max_pos, hd)).astype(np.float32)).cuda()
        tabs.append((ct, st, hd, torch.empty(hd, device="cuda"), torch.empty(hd, device="cuda")))
    h = torch.empty(Hh, device="cuda")
    dyn = torch.zeros(4, dtype=torch.int32, device="cuda")
    for pinned in (True, False):
        step = torch.zeros(2, dtype=torch.int32, pin_memory=True) if pinned else torch.zeros(2, dtype=torch.int32,
                                                                                              device="cuda")
        for tid, pos, want_t, want_p in [(7, 3, 7, 3), (299, 49, 299, 49), (0, 0, 0, 0), (305, -3, 299, 0)]:
            if pinned:
                step[0], step[1] = tid, pos
            else:
                step.copy_(torch.tensor([tid, pos], dtype=torch.int32))
            gpu.token_inputs(step, emb, h, dyn, tabs, vocab=vocab, H=Hh, max_pos=max_pos)
            torch.cuda.synchronize()
            assert (to_np(h) == to_np(emb[want_t])).all()
            assert to_np(dyn)[:2].tolist() == [want_p, want_p + 1]
            for ct, st, hd, co, so in tabs:
                assert (to_np(co) == to_np(ct[want_p])).all() and (to_np(so) == to_np(st[want_p])).all()


@pytest.mark.parametrize("gated", [False, True])
def test_decode_token_lm_head_keeps_its_norm_launch(g4, gpu, gated, monkeypatch):
    """The real model's case: lm_head is too tall for a norm-fused launch,
    so the fused launches are odd in number (here 3: gate/up of both layers
    and the second layer's q/k/v), the final normadd + norm acts on the
    residual's twin buffer and a copy at the end of the graph puts it back.
    Logits and the residual h after every token are checked."""
    E = importlib.import_module("g4mi.vk_engine")
    monkeypatch.setattr(E, "_NX_MAX_ROWS", 1536)
    _token_steps(gpu, True, True, gated, True, V=2048, lm_fused=False)


def test_decode_token_profile(g4, gpu):
    """PROFILE=1's counterpart (src/vk_engine.py:37-46,263-265,321-335): a
    GPU timestamp after every op of the recorded token; every submit adds
    each op's time to its label. The oracle bar holds with the timestamps in
    the graph, and the report covers every op of the token once per submit."""
    E = importlib.import_module("g4mi.vk_engine")
    rep, seq, runs = _token_steps(gpu, True, True, True, True, profile=True)
    assert runs == 20
    labels = set(rep) - {"TOTAL"}
    assert labels == {E.op_label(op) for op in seq}
    assert "prepkv_attn" in labels and any(k.startswith("gemv+norm ") for k in labels)
    assert all(v > 0 for v in rep.values()) and abs(rep["TOTAL"] - sum(rep[k] for k in labels)) < 1e-6 * rep["TOTAL"]


def _token_steps(gpu, fuse, half, gated, fg, V=V, lm_fused=True, device_inputs=False, profile=False):
    E = importlib.import_module("g4mi.vk_engine")
    xdt = torch.float16 if half else torch.float32
    rx = (lambda v: np.asarray(v).astype(np.float16).astype(np.float64)) if half else (lambda v: v)
    rng = np.random.default_rng(0)
    f32 = lambda a: np.asarray(a, np.float32)

    def lin(N, K):
        W = f32(rng.standard_normal((N, K)) * (1.0 / np.sqrt(K)))
        q, sc = O.quant_codes(W)
        return E.quant(W, pf=False, fp8=False, prefill_i8=False), (N, K), (q, sc.astype(np.float16).astype(np.float32))

    def wbuf(a):
        b = E.Buf(f32(a).nbytes)
        b.write(f32(a))
        return b

    fb = lambda n: E.Buf(n * 4)
    maxq = max(NH * L["hd"] for L in LAYERS)
    B = {k: fb(n) for k, n in dict(h=H, normed=H, normed2=H, o=H, down=H, normed_f=H, attn=maxq, gate=I, up=I,
                                   act=I, logits=V, qkv=maxq + 2 * 2 * 128).items()}
    cosb = {hd: fb(hd) for hd in (64, 128)}
    sinb = {hd: fb(hd) for hd in (64, 128)}
    DYN = E.buf_u32([0, 0, 0, 0])
    DUH, DUI = E.buf_u32([H, 0, 0, 0]), E.buf_u32([I, 0, 0, 0])
    layers, ref_layers = [], []
    for cfg in LAYERS:
        hd, nkv, keqv = cfg["hd"], cfg["nkv"], cfg["keqv"]
        nq, nk = NH * hd, nkv * hd
        qp, kp = lin(nq, H), lin(nk, H)
        vp = None if keqv else lin(nk, H)
        op, gp, up, dp = lin(H, nq), lin(I, H), lin(I, H), lin(H, I)
        norms = {k: f32(rng.random(n) + 0.5) for k, n in dict(qnw=hd, knw=hd, inw=H, paw=H, pfw=H, ofw=H).items()}
        # unscaled q.k scores: a small q-norm weight keeps them at a few units, so the
        # softmax does not amplify fp32-vs-float64 rounding flips of the fp16 inputs
        norms["qnw"] = f32(norms["qnw"] * (2.0 / hd))
        kc, vc = E.Buf(nkv * cfg["stride"] * hd * 2), E.Buf(nkv * cfg["stride"] * hd * 2)
        nb = {k: wbuf(v) for k, v in norms.items()}
        P = [nkv, hd, nq, nq + nk, int(keqv), cfg["stride"], cfg["window"], 0]
        A = [NH, nkv, hd, cfg["stride"], cfg["window"], 0, NH // nkv, 0]
        nas = E.buf_u32([H, int(np.array([cfg["scl"]], np.float32).view(np.uint32)[0]), 0, 0])
        L = dict(d_in=E.normbg(B["h"], nb["inw"], B["normed"], DUH, out_dtype=xdt),
                 d_q=E.gemv_ds(qp[:2], B["normed"], B["qkv"], 0, x_dtype=xdt),
                 d_k=E.gemv_ds(kp[:2], B["normed"], B["qkv"], nq * 4, x_dtype=xdt),
                 d_v=None if keqv else E.gemv_ds(vp[:2], B["normed"], B["qkv"], (nq + nk) * 4, x_dtype=xdt),
                 d_prep=E.prepkv_ds(B["qkv"], nb["knw"], cosb[hd], sinb[hd], kc, vc, P, DYN),
                 d_attn=E.attn_ds(B["qkv"], nb["qnw"], cosb[hd], sinb[hd], kc, vc, B["attn"], A, DYN, out_dtype=xdt),
                 d_o=E.gemv_ds(op[:2], B["attn"], B["o"], 0, x_dtype=xdt),
                 d_na=E.normadd_ds(B["o"], nb["paw"], B["h"], DUH),
                 d_pfn=E.normbg(B["h"], nb["pfw"], B["normed2"], DUH, out_dtype=xdt),
                 d_g=E.gemv_ds(gp[:2], B["normed2"], B["gate"], 0, x_dtype=xdt),
                 d_u=E.gemv_ds(up[:2], B["normed2"], B["up"], 0, x_dtype=xdt),
                 d_gm=E.gelumul_ds(B["gate"], B["up"], B["act"], DUI, out_dtype=xdt),
                 d_d=E.gemv_ds(dp[:2], B["act"], B["down"], 0, x_dtype=xdt),
                 d_nas=E.normadd_ds(B["down"], nb["ofw"], B["h"], nas))
        if gated:
            L["d_gu"] = E.gate_up_ds(gp[:2], up[:2], B["normed2"], B["act"], x_dtype=xdt, act_dtype=xdt)
            assert L["d_gu"] is not None
        layers.append(L)
        ref_layers.append(dict(cfg, nq=nq, nk=nk, q=qp[2], k=kp[2], v=None if keqv else vp[2], o=op[2], g=gp[2],
                               u=up[2], d=dp[2], kc=np.zeros(nkv * cfg["stride"] * hd, np.float16),
                               vc=np.zeros(nkv * cfg["stride"] * hd, np.float16), **norms))
    lm = lin(V, H)
    finw = f32(rng.random(H) + 0.5)
    d_fin = E.normbg(B["h"], wbuf(finw), B["normed_f"], DUH, out_dtype=xdt)
    d_lm = E.gemv_ds(lm[:2], B["normed_f"], B["logits"], 0, x_dtype=xdt)
    d_tok = step = EMB = None
    VOC, MAXP = 512, 64
    if device_inputs:  # embedding rows and RoPE tables on the device, (tid, pos) in pinned host memory
        EMB = f32(rng.standard_normal((VOC, H)))
        step = torch.zeros(2, dtype=torch.int32, pin_memory=True)
        rope = {hd: [wbuf(np.stack([_rope(p, hd)[i] for p in range(MAXP)])) for i in (0, 1)] for hd in (64, 128)}
        d_tok = E.token_inputs_ds(step, wbuf(EMB), B["h"], DYN, [(rope[hd][0], rope[hd][1], hd, cosb[hd], sinb[hd])
                                                                 for hd in (64, 128)], vocab=VOC, H=H, max_pos=MAXP)
    graph = E.record_decode(layers, d_fin, d_lm, fuse=fuse, fuse_gemv=fg, d_tok=d_tok, profile=profile)
    n_nx = sum(1 for op in graph.seq if (isinstance(op, tuple) and op[0] == "gemvs_nx")
               or getattr(op, "fn", None) is gpu.gemv_normadd)
    # per layer: the gate/up GEMV(s) and the next layer's q/k/v or (last layer) the 1024-row lm_head
    assert n_nx == ((2 * len(layers) - (0 if lm_fused else 1)) if (fuse and half and fg) else 0)
    if not lm_fused:
        assert getattr(graph.seq[-1], "fn", None) is E._copy_into   # the residual goes back home
    print(f"token fuse={fuse} half={half} gated={gated} fg={fg}: {n_nx} fused norm GEMVs", flush=True)

    gv = lambda qs, x: O.gemv_ref(qs[0], qs[1], x).astype(np.float64)
    for pos in range(20):
        tabs = {hd: _rope(pos, hd) for hd in (64, 128)}
        if device_inputs:
            tid = int(rng.integers(0, VOC))
            emb = EMB[tid]
            E.forward(graph, step, tid, pos, vocab=VOC, max_pos=MAXP, timeout_ms=20000)
        else:
            emb = f32(rng.standard_normal(H))
            B["h"].write(emb)
            DYN.write(np.array([pos, pos + 1, 0, 0], np.uint32))
            for hd, (c, s) in tabs.items():
                cosb[hd].write(c)
                sinb[hd].write(s)
            E.submit(graph, label=f"decode pos={pos}", timeout_ms=20000)
        logits = np.frombuffer(B["logits"].read(V * 4), np.float32)

        h = emb.astype(np.float64)
        for R in ref_layers:
            hd, nq, nk = R["hd"], R["nq"], R["nk"]
            c, s = tabs[hd]
            x = rx(D.rmsnorm_ref(h, R["inw"]))
            qkv = np.concatenate([gv(R["q"], x), gv(R["k"], x)] + ([] if R["keqv"] else [gv(R["v"], x)]))
            R["kc"], R["vc"] = D.prepkv_ref(qkv, R["knw"], c, s, R["kc"], R["vc"], nkv=R["nkv"], hd=hd, koff=nq,
                                            voff=nq + nk, keqv=R["keqv"], stride=R["stride"], window=R["window"],
                                            pos=pos)
            att = D.attn_ref(qkv, R["qnw"], c, s, R["kc"], R["vc"], nH=NH, hd=hd, stride=R["stride"],
                             window=R["window"], qoff=0, grp=NH // R["nkv"], pos=pos)
            h = D.normadd_ref(gv(R["o"], rx(att)), R["paw"], h)
            x2 = rx(D.rmsnorm_ref(h, R["pfw"]))
            act = rx(D.gelumul_ref(gv(R["g"], x2), gv(R["u"], x2)))
            h = D.normadd_ref(gv(R["d"], act), R["ofw"], h, R["scl"])
        ref = gv(lm[2], rx(D.rmsnorm_ref(h, finw)))
        assert O.normwise_rel_err(logits, ref) <= 1e-3, pos
        if not lm_fused:
            hdev = np.frombuffer(B["h"].read(H * 4), np.float32)
            assert O.normwise_rel_err(hdev, h) <= 1e-3, pos
    out = (E.profile_report(graph), graph.seq, graph.prof_runs) if profile else None
    graph.destroy()
    return out
