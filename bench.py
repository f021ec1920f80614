"""Benchmark of the int4/int8 quantized matmul path on one MI355X.

Default workload (the headline, one "step" = one decoded token): the decode
GEMV set of 48 distinct Gemma-style layers {q 4096x3840, k 2048x3840,
v 2048x3840, o 3840x4096, fused gate_up 30720x3840, down 3840x15360} plus
lm_head 262144x3840, int4 block-32 codes with fp16 scales, fp16 activations
and outputs, captured once as a hipGraph and replayed per token. Every
weight byte is distinct (6.6 GB per token), so the 256 MB Infinity Cache
cannot serve repeats. value = algorithmic bytes per token / time per token.

Also measured in the same run: single GEMV shapes on their own (15360x3840
with fp16 and with e4m3 scales, lm_head 262144x3840), the per-token time
distribution, the W8A8 prefill GEMM at M=2048, N=15360,
K=3840 (int8 MFMA) and the W4A16 GEMM at M=512 (f16 MFMA), each as a
fraction of MI355X's dense peak, and the CPU baseline (the oracle's numpy
dequant+matmul, the reference's own formulation) on a bounded sample.

Data are synthetic (random codes/scales/activations of the stated shapes).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "int4 GEMV HBM GB/s (% of 8 TB/s) + W8A8 prefill GEMM TOPS (% int8 MFMA peak)"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0      # dense int8 MFMA, MI355X
F16_PEAK_TFLOPS = 2500.0     # dense f16 MFMA, MI355X
H, QN, KVN, I, V = 3840, 4096, 2048, 15360, 262144
LAYERS = 48
LAYER_SHAPES = [("q", QN, H), ("k", KVN, H), ("v", KVN, H), ("o", H, QN), ("gate_up", 2 * I, H), ("down", H, I)]


def gemv_bytes(N: int, K: int, scale_bytes: int = 2) -> int:
    """Algorithmic bytes of one int4 GEMV: weights, block scales, fp16 x, fp16 y."""
    return N * K // 2 + (N * K // 32) * scale_bytes + 2 * K + 2 * N


def load_ops():
    import importlib

    import __graft_entry__ as G

    G.load_package()
    return importlib.import_module("g4mi.ops")


# ------------------------------------------------------------- GPU legs
def bench_decode(ops, steps: int, warmup: int, e4m3: bool = False):
    """The decode GEMV set (see the module docstring). ``e4m3``: the same
    set with e4m3 block scales (codes as e4m3 bytes of values 2^-2 .. 2^2;
    timing does not depend on the values), one byte per block instead of
    two: 5.5% fewer algorithmic bytes."""
    import torch

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    mats = []
    fmt = ops.SCALE_E4M3 if e4m3 else ops.SCALE_F16

    def make(N, K):
        words = torch.randint(-2 ** 31, 2 ** 31 - 1, (N * K // 8,), dtype=torch.int64, device=dev,
                              generator=gen).to(torch.int32)
        if e4m3:
            sc = torch.randint(0x28, 0x48, (N * K // 32,), dtype=torch.int32, device=dev,
                               generator=gen).to(torch.uint8)
        else:
            sc = (torch.randn(N * K // 32, device=dev, generator=gen) * 0.02).abs().to(torch.float16)
        return words, sc

    xs = {K: torch.randn(K, device=dev, generator=gen).to(torch.float16) for K in (H, QN, I)}
    ys = {}
    for _ in range(LAYERS):
        for name, N, K in LAYER_SHAPES:
            w, s = make(N, K)
            ys.setdefault(name, torch.empty(N, dtype=torch.float16, device=dev))
            mats.append((name, N, K, w, s))
    w, s = make(V, H)
    ys["lm_head"] = torch.empty(V, dtype=torch.float16, device=dev)
    mats.append(("lm_head", V, H, w, s))
    ws = ops.Workspace(max(ops.Workspace.bytes_for(N, K) for _, N, K, _, _ in mats))
    torch.cuda.synchronize()
    # q, k and v read the same normed activation: one batched launch per layer
    # (the reference dispatches them back to back on one input buffer)
    launches = []
    i = 0
    while i < len(mats):
        if mats[i][0] == "q":
            launches.append(("qkv", mats[i:i + 3]))
            i += 3
        else:
            launches.append((mats[i][0], [mats[i]]))
            i += 1

    def launch(sel):
        if len(sel) == 1:
            _, N, K, w, s = sel[0]
            ops.gemv(xs[K], w, s, N, K, y=ys[sel[0][0]], ws=ws, scale_fmt=fmt, inv=0.5)
        else:
            K = sel[0][2]
            ops.gemv_batch(xs[K], [(w, s, N, ys[nm], 0.5) for nm, N, _, w, s in sel], K, scale_fmt=fmt)

    def token():
        for _, sel in launches:
            launch(sel)

    graph = ops.Graph()
    with graph.capture():
        token()
    st = graph.stream
    for _ in range(warmup):
        graph.launch()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(st)
    for _ in range(steps):
        graph.launch()
    t1.record(st)
    t1.synchronize()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    # distribution: every replay between its own pair of events (a separate pass)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    evs[0].record(st)
    for i in range(steps):
        graph.launch()
        evs[i + 1].record(st)
    evs[-1].synchronize()
    per = sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(steps))
    pct = {f"p{q}": round(per[min(steps - 1, int(q / 100 * steps))], 4) for q in (10, 50, 90)}
    nbytes = sum(gemv_bytes(N, K, 1 if e4m3 else 2) for _, N, K, _, _ in mats)
    # per-shape kernel time: one graph of the 48 same-shape launches per shape, same stream
    per_shape = {}
    for name in ["qkv", "o", "gate_up", "down", "lm_head"]:
        sel = [lz for nm, lz in launches if nm == name]
        g2 = ops.Graph(st)
        with g2.capture():
            for lz in sel:
                launch(lz)
        reps = max(3, 480 // len(sel))
        for _ in range(2):
            g2.launch()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(st)
        for _ in range(reps):
            g2.launch()
        b.record(st)
        b.synchronize()
        us = a.elapsed_time(b) * 1e3 / (reps * len(sel))
        lb = sum(gemv_bytes(N, K, 1 if e4m3 else 2) for _, N, K, _, _ in sel[0])
        per_shape[name] = {"N": "+".join(str(m[1]) for m in sel[0]), "K": sel[0][0][2],
                           "us_per_launch": round(us, 3), "GBps": round(lb / us / 1e3, 1),
                           "bytes_per_launch": lb, "launches_per_token": len(sel)}
        g2.destroy()
    graph.destroy()
    del mats, ws
    torch.cuda.empty_cache()
    return {"ms_per_step": ms, "bytes_per_step": nbytes, "launches": len(launches),
            "GBps": nbytes / (ms * 1e-3) / 1e9, "per_shape": per_shape, "ms_per_step_percentiles": pct}


def bench_gemv_single(ops, N: int, K: int, e4m3: bool, reps: int = 10):
    """One GEMV shape on its own: a graph of launches over distinct weights
    (>= 1.5 GB, so the 256 MB Infinity Cache cannot serve repeats), HIP events
    around the replays; time per launch, GB/s of algorithmic bytes."""
    import torch

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(3)
    sb = 1 if e4m3 else 2
    per = gemv_bytes(N, K, sb)
    n = max(4, (1536 << 20) // per)
    x = torch.randn(K, device=dev, generator=gen).to(torch.float16)
    y = torch.empty(N, dtype=torch.float16, device=dev)
    mats = []
    for _ in range(n):
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (N * K // 8,), dtype=torch.int64, device=dev,
                          generator=gen).to(torch.int32)
        if e4m3:  # e4m3 codes of scale values 2^-2 .. 2^2 (timing does not depend on the values)
            s = torch.randint(0x28, 0x48, (N * K // 32,), dtype=torch.int32, device=dev, generator=gen).to(torch.uint8)
        else:
            s = (torch.randn(N * K // 32, device=dev, generator=gen) * 0.02).abs().to(torch.float16)
        mats.append((w, s))
    fmt = ops.SCALE_E4M3 if e4m3 else ops.SCALE_F16
    g = ops.Graph()
    with g.capture():
        for w, s in mats:
            ops.gemv(x, w, s, N, K, scale_fmt=fmt, inv=0.5, y=y)
    g.launch()
    g.launch()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(g.stream)
    for _ in range(reps):
        g.launch()
    b.record(g.stream)
    b.synchronize()
    us = a.elapsed_time(b) * 1e3 / (reps * n)
    g.destroy()
    del mats
    torch.cuda.empty_cache()
    return {"N": N, "K": K, "scales": "e4m3" if e4m3 else "f16", "us_per_launch": round(us, 3),
            "bytes_per_launch": per, "GBps": round(per / us / 1e3, 1),
            "frac_of_hbm_peak": round(per / us / 1e3 / HBM_PEAK_GBS, 4), "distinct_weight_sets": n}


def bench_small_m(ops, reps: int = 6):
    """Small-M GEMV (speculative-decode verification: M tokens against one
    matrix) on the decode shapes, each path timed as a graph of launches over
    distinct weights (>= 1.5 GB): the MFMA path (K split where planned, and
    unsplit beside it), the bit-exact VALU path, the
    W4A16 prefill GEMM at the same M, and M single-vector GEMVs. GB/s counts
    the weight and scale bytes once per launch (what one GEMV reads)."""
    import torch

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(4)

    def timed(fn, n):
        g = ops.Graph()
        with g.capture():
            for i in range(n):
                fn(i)
        g.launch()
        g.launch()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(g.stream)
        for _ in range(reps):
            g.launch()
        b.record(g.stream)
        b.synchronize()
        g.destroy()
        return a.elapsed_time(b) * 1e3 / (reps * n)

    out = {}
    for name, N, K in [("c1", I, H), ("gate_up", 2 * I, H), ("down", H, I)]:
        per = gemv_bytes(N, K)
        n = max(4, (1536 << 20) // per)
        mats = []
        for _ in range(n):
            w = torch.randint(-2 ** 31, 2 ** 31 - 1, (N * K // 8,), dtype=torch.int64, device=dev,
                              generator=gen).to(torch.int32)
            s = (torch.randn(N * K // 32, device=dev, generator=gen) * 0.02).abs().to(torch.float16)
            mats.append((w, s))
        x1 = torch.randn(K, device=dev, generator=gen).to(torch.float16)
        y1 = torch.empty(N, dtype=torch.float16, device=dev)
        t1 = timed(lambda i: ops.gemv(x1, mats[i][0], mats[i][1], N, K, y=y1), n)
        for M in (4, 8, 16):
            X = torch.randn((M, K), device=dev, generator=gen).to(torch.float16)
            Y = torch.empty((M, N), dtype=torch.float16, device=dev)
            mws = ops.gemv_multi_workspace_bytes(M, N, K)
            mws = torch.empty(mws, dtype=torch.uint8, device=dev) if mws else None
            t_mm = timed(lambda i: ops.gemv_multi(X, mats[i][0], mats[i][1], N, K, y=Y, ws=mws), n)
            t_mm1 = timed(lambda i: ops.gemv_multi(X, mats[i][0], mats[i][1], N, K, y=Y, ksplit=False), n) \
                if mws is not None else t_mm
            t_ex = timed(lambda i: ops.gemv_multi(X, mats[i][0], mats[i][1], N, K, y=Y, exact=True), n)
            need = ops.gemm_workspace_bytes(M, N, K)
            ws = torch.empty(need, dtype=torch.uint8, device=dev) if need else None
            t_w4 = timed(lambda i: ops.gemm_w4a16(X, mats[i][0], mats[i][1], N, Y=Y, ws=ws), n)
            out[f"{name}_{N}x{K}_M{M}"] = {
                "mfma_us": round(t_mm, 2), "mfma_GBps": round(per / t_mm / 1e3, 1),
                "mfma_k_split": ops.gemv_multi_workspace_bytes(M, N, K) // (4 * M * N),
                "mfma_unsplit_us": round(t_mm1, 2),
                "exact_us": round(t_ex, 2), "w4a16_gemm_us": round(t_w4, 2),
                "m_single_gemvs_us": round(M * t1, 2), "speedup_vs_w4a16": round(t_w4 / t_mm, 2),
                "speedup_vs_m_gemvs": round(M * t1 / t_mm, 2)}
        del mats
        torch.cuda.empty_cache()
    return out


def bench_prefill(ops, reps: int = 5, p0: int = 3968, stacked: bool = True, gemm_norms: bool = True):
    """One 128-token prefill chunk through the 48-layer stack with the
    batched-prefill layer graph (vk_engine.record_prefill: per layer
    pre_norm, q/k/v W4A16 GEMMs, pre_prepkv, pre_attn, o GEMM, pre_na +
    pre_norm, gate/up GEMMs, gelumul, down GEMM, pre_na), fp16 buffers
    between producers and GEMMs, fused norms; with ``stacked``, q/k/v run as
    one GEMM over their stacked rows, gate/up and the gelumul as one gated
    W4A16 GEMM over interleaved gate/up rows, and the GEMMs hand their
    split-K partials straight to the op after them (o and down: the normadd;
    q/k/v: the q store and prepkv). Layers: 40 sliding (16 query
    and 8 KV heads of 256, 1024-slot ring) and 8 global (16 query heads and
    one k == v head of 512, every sixth layer), H 3840, I 15360; the chunk
    is the last of a 4096-token prompt (p0 = 3968: sliding layers attend
    1024 keys, global layers 4096). Synthetic int4 weights (distinct per
    layer), HIP events over graph replays. Also times the attention
    launches alone (their own graph)."""
    import importlib

    import numpy as np
    import torch

    E = importlib.import_module("g4mi.vk_engine")
    MC = E.MC
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(5)

    def qw(N, K):
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (N * K // 8,), dtype=torch.int64, device=dev,
                          generator=gen).to(torch.int32)
        sc = (torch.randn(N * K // 32, device=dev, generator=gen) * 0.02).abs().to(torch.float16)
        b = E.Buf(tensor=sc)
        return E.QW(E.Buf(tensor=w), b, 1, K // 32, 1.0, b, None, None), (N, K)

    def fbuf(n, scale=1.0, dtype=torch.float32):
        return E.Buf(tensor=(torch.rand(n, device=dev, generator=gen) * scale + 0.5 * scale).to(dtype))

    h16 = torch.float16
    NHq, prompt = 16, p0 + MC
    Xp = E.Buf(tensor=torch.randn(MC * H, device=dev, generator=gen))
    Np, Tp = E.Buf(MC * H * 4), E.Buf(MC * H * 4)
    Qp, Ap = E.Buf(MC * NHq * 512 * 4), E.Buf(MC * NHq * 512 * 4)
    Kp, Vp = E.Buf(MC * 8 * 256 * 4), E.Buf(MC * 8 * 256 * 4)
    Gp, Upp, ACp = E.Buf(MC * I * 4), E.Buf(MC * I * 4), E.Buf(MC * I * 4)
    QKVp = E.Buf(MC * (NHq * 512 + 512) * 2)   # the stacked q/k/v GEMM's fp16 rows
    cosM = {hd: fbuf(MC * hd) for hd in (256, 512)}
    sinM = {hd: fbuf(MC * hd) for hd in (256, 512)}
    DYNP = E.buf_u32([p0, MC, 0, 0])
    DUH = E.buf_u32([H, 0, 0, 0])
    DUIp = E.buf_u32([MC * I, 0, 0, 0])
    gk = dict(x_dtype=h16, y_dtype=h16)
    layers, weight_bytes = [], 0
    for li in range(LAYERS):
        glob = li % 6 == 5
        hd, nkv, window, stride = (512, 1, 0, prompt) if glob else (256, 8, 1024, 1024)
        nq, nk = NHq * hd, nkv * hd
        kc = E.Buf(tensor=torch.randn(nkv * stride * hd, device=dev, generator=gen).to(h16))
        vc = E.Buf(tensor=torch.randn(nkv * stride * hd, device=dev, generator=gen).to(h16))
        q, k = qw(nq, H), qw(nk, H)
        v = None if glob else qw(nk, H)
        o, g, u, d = qw(H, nq), qw(I, H), qw(I, H), qw(H, I)
        weight_bytes += sum(N * K // 2 + N * K // 16 for _, (N, K) in [q, k, o, g, u, d] + ([v] if v else []))
        nb = {kk: fbuf(n, 0.1) for kk, n in dict(qnw=hd, knw=hd, inw=H, paw=H, pfw=H, ofw=H).items()}
        Pp = [nkv, hd, nk, 0, stride, window, 0, 0]
        Aa = [NHq, nq, hd, stride, window, NHq // nkv, 0, 0]
        # stacked q/k/v: one GEMM, q, k (and v) at column offsets of one row
        ldc = nq + (nk if glob else 2 * nk)
        qsrc, ksrc, vsrc = (QKVp, QKVp, QKVp) if stacked else (Qp, Kp, Kp if glob else Vp)
        kv_at = dict(ld=ldc, koff=nq, voff=nq if glob else nq + nk) if stacked else {}
        q_at = dict(ldq=ldc) if stacked else {}
        nas = E.buf_u32([H, int(np.array([0.5], np.float32).view(np.uint32)[0]), 0, 0])
        layers.append(dict(
            p_in=E.pre_norm_ds(Xp, nb["inw"], Np, DUH, out_dtype=h16),
            p_q=E.gemm_ds(q, Np, Qp, **gk), p_k=E.gemm_ds(k, Np, Kp, **gk),
            p_v=None if glob else E.gemm_ds(v, Np, Vp, **gk),
            p_qkv=E.gemm_cat_ds([q, k] + ([] if glob else [v]), Np, QKVp, **gk) if stacked else None,
            p_prep=E.pre_prepkv_ds(ksrc, vsrc, nb["knw"], cosM[hd], sinM[hd], kc, vc, Pp, DYNP, kv_dtype=h16,
                                   **kv_at),
            p_attn=E.pre_attn_ds(qsrc, nb["qnw"], cosM[hd], sinM[hd], kc, vc, Ap, Aa, DYNP, nkv,
                                 max_keys=prompt if glob else window, q_dtype=h16, out_dtype=h16, **q_at),
            p_o=E.gemm_ds(o, Ap, Tp, **gk),
            p_na=E.pre_na_ds(Tp, nb["paw"], Xp, DUH, x_dtype=h16),
            p_pfn=E.pre_norm_ds(Xp, nb["pfw"], Np, DUH, out_dtype=h16),
            p_g=E.gemm_ds(g, Np, Gp, **gk), p_u=E.gemm_ds(u, Np, Upp, **gk),
            p_gm=E.pre_gelumul_ds(Gp, Upp, ACp, DUIp, in_dtype=h16, out_dtype=h16),
            p_gu=E.pre_gate_up_ds(g, u, Np, ACp) if stacked else None,
            p_d=E.gemm_ds(d, ACp, Tp, **gk),
            p_nas=E.pre_na_ds(Tp, nb["ofw"], Xp, nas, x_dtype=h16)))
    graph = E.record_prefill(layers, fuse=True, gemm_norms=stacked and gemm_norms)
    att = E.record(lambda: [E.disp(L["p_attn"]) for L in layers])

    def timed(gr, n):
        gr.launch()
        gr.launch()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(gr.stream)
        for _ in range(n):
            gr.launch()
        b.record(gr.stream)
        b.synchronize()
        return a.elapsed_time(b) / n

    ms = timed(graph, reps)
    ms_att = timed(att, reps)
    graph.destroy()
    att.destroy()
    del layers
    torch.cuda.empty_cache()
    return {"chunk_tokens": MC, "p0": p0, "layers": LAYERS, "global_layers": LAYERS // 6,
            "ms_per_chunk": round(ms, 3), "prompt_tok_per_s": round(MC / (ms * 1e-3), 1),
            "attention_ms_per_chunk": round(ms_att, 3), "attention_share": round(ms_att / ms, 3),
            "weight_bytes": weight_bytes, "weight_GBps": round(weight_bytes / (ms * 1e-3) / 1e9, 1)}


def bench_token_step(ops, steps: int, warmup: int, pos: int = 1023, fast: bool = False,
                     fuse_gemv: bool = True, host_loop: bool = False, profile: bool = False, e4m3: bool = False):
    """A whole decode token through the engine mirror (vk_engine.py): the
    reference's per-layer dispatch order (norm, q/k/v, prepkv, attention, o,
    normadd, norm, gate/up, gelumul, down, normadd) for 48 layers of the
    decode-set shapes (16 query heads and 8 KV heads of 256, a 1024-slot
    sliding-window fp16 KV cache per layer) plus the final norm and
    lm_head, recorded once and replayed with the position in device
    memory. Synthetic int4 weights. ``fast=False``: fp32 activations
    everywhere and one launch per reference dispatch (the reference's
    buffers); ``fast=True``: every normadd fused with the rmsnorm that
    follows it, gate/up interleaved with the gelumul in their GEMV's
    epilogue, and fp16 GEMV inputs (the residual stream stays fp32); with
    ``fuse_gemv`` too, each fused norm runs inside the q/k/v or gate/up GEMV
    launch that reads it. With ``host_loop``, the graph starts with the
    token-inputs launch (embedding row from a device table of all 262144
    tokens, position, RoPE rows from a table) and each token is one
    ``vk_engine.forward`` call at the next position: pinned-memory write of
    (tid, pos), graph launch, bounded wait, timed on the host clock
    (``ms_per_token``) beside the back-to-back replays of the same graph
    (``graph_replay_ms_per_token``). With ``profile``, the graph carries a
    GPU timestamp after every launch (the engine's PROFILE=1 mode) and the
    result adds ``profile_us``: GPU time per token by op label, each op with
    one stamp launch's gap. ``e4m3``: every matrix with e4m3 block scales
    (the engine's GEMV_FP8=1 decode, one scale byte per block; values
    2^-2 .. 2^2, timing does not depend on them)."""
    import importlib

    import numpy as np
    import torch

    E = importlib.import_module("g4mi.vk_engine")
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(4)
    nH, nkv, hd, win = 16, 8, 256, 1024
    nq, nk = nH * hd, nkv * hd

    def qw(N, K):
        words = torch.randint(-2 ** 31, 2 ** 31 - 1, (N * K // 8,), dtype=torch.int64, device=dev,
                              generator=gen).to(torch.int32)
        sc = (torch.randn(N * K // 32, device=dev, generator=gen) * 0.02).abs().to(torch.float16)
        b = E.Buf(tensor=sc)
        bs = E.Buf(tensor=torch.randint(0x28, 0x48, (N * K // 32,), dtype=torch.int32, device=dev,
                                        generator=gen).to(torch.uint8)) if e4m3 else b
        return E.QW(E.Buf(tensor=words), bs, ops.auto_split(N, K), K // 32, 1.0, b, None, None), (N, K)

    def vec(n, lo=0.5):
        return E.Buf(tensor=(torch.rand(n, device=dev, generator=gen) + lo).to(torch.float32))

    fb = lambda n: E.Buf(n * 4)
    xdt = torch.float16 if fast else torch.float32
    B = {k: fb(n) for k, n in dict(h=H, normed=H, normed2=H, o=H, down=H, normed_f=H, attn=nq, gate=I, up=I, act=I,
                                   logits=V, qkv=nq + 2 * nk).items()}
    cosb, sinb = vec(hd, -0.5), vec(hd, -0.5)
    DYN = E.buf_u32([pos, pos + 1, 0, 0])
    DUH, DUI = E.buf_u32([H, 0, 0, 0]), E.buf_u32([I, 0, 0, 0])
    nas = E.buf_u32([H, int(np.array([0.5], np.float32).view(np.uint32)[0]), 0, 0])
    layers = []
    for _ in range(LAYERS):
        kc, vc = E.Buf(tensor=torch.randn(nkv * win * hd, device=dev, generator=gen).to(torch.float16)), \
            E.Buf(tensor=torch.randn(nkv * win * hd, device=dev, generator=gen).to(torch.float16))
        P = [nkv, hd, nq, nq + nk, 0, win, win, 0]
        A = [nH, nkv, hd, win, win, 0, nH // nkv, 0]
        qg, qu = qw(I, H), qw(I, H)
        layers.append(dict(
            d_in=E.normbg(B["h"], vec(H), B["normed"], DUH, out_dtype=xdt),
            d_q=E.gemv_ds(qw(nq, H), B["normed"], B["qkv"], 0, x_dtype=xdt),
            d_k=E.gemv_ds(qw(nk, H), B["normed"], B["qkv"], nq * 4, x_dtype=xdt),
            d_v=E.gemv_ds(qw(nk, H), B["normed"], B["qkv"], (nq + nk) * 4, x_dtype=xdt),
            d_prep=E.prepkv_ds(B["qkv"], vec(hd), cosb, sinb, kc, vc, P, DYN),
            d_attn=E.attn_ds(B["qkv"], vec(hd, 0.05), cosb, sinb, kc, vc, B["attn"], A, DYN, out_dtype=xdt),
            d_o=E.gemv_ds(qw(H, nq), B["attn"], B["o"], 0, x_dtype=xdt),
            d_na=E.normadd_ds(B["o"], vec(H), B["h"], DUH),
            d_pfn=E.normbg(B["h"], vec(H), B["normed2"], DUH, out_dtype=xdt),
            d_g=E.gemv_ds(qg, B["normed2"], B["gate"], 0, x_dtype=xdt),
            d_u=E.gemv_ds(qu, B["normed2"], B["up"], 0, x_dtype=xdt),
            d_gm=E.gelumul_ds(B["gate"], B["up"], B["act"], DUI, out_dtype=xdt),
            d_d=E.gemv_ds(qw(H, I), B["act"], B["down"], 0, x_dtype=xdt),
            d_nas=E.normadd_ds(B["down"], vec(H), B["h"], nas)))
        if fast:  # gate/up interleaved once, gelumul in the GEMV epilogue; the separate copies are dropped
            layers[-1]["d_gu"] = E.gate_up_ds(qg, qu, B["normed2"], B["act"], x_dtype=xdt, act_dtype=xdt)
            layers[-1]["d_g"] = layers[-1]["d_u"] = None
        del qg, qu
    d_fin = E.normbg(B["h"], vec(H), B["normed_f"], DUH, out_dtype=xdt)
    d_lm = E.gemv_ds(qw(V, H), B["normed_f"], B["logits"], 0, x_dtype=xdt)
    B["h"].write(np.ones(H, np.float32))
    d_tok = step = None
    max_pos = pos + 2 * (warmup + steps) + 2
    if host_loop:
        emb = E.Buf(tensor=torch.randn(V * H, device=dev, generator=gen) * 0.05)
        ctab, stab = vec(max_pos * hd, -0.5), vec(max_pos * hd, -0.5)
        step = torch.zeros(2, dtype=torch.int32, pin_memory=True)
        d_tok = E.token_inputs_ds(step, emb, B["h"], DYN, [(ctab, stab, hd, cosb, sinb)], vocab=V, H=H,
                                  max_pos=max_pos)
    graph = E.record_decode(layers, d_fin, d_lm, fuse=fast, fuse_gemv=fuse_gemv, d_tok=d_tok, profile=profile)
    # one launch per recorded descriptor, plus the split merge of every attention
    launches = len(graph.seq) + sum(1 for op in graph.seq if getattr(op, "fn", None) in (ops.attn, ops.prepkv_attn))
    host = None
    if host_loop:
        tids = torch.randint(0, V, (warmup + steps,), generator=torch.Generator().manual_seed(5)).tolist()
        p = pos
        for i in range(warmup):
            E.forward(graph, step, tids[i], p, vocab=V, max_pos=max_pos, timeout_ms=20000)
            p += 1
        t0 = time.perf_counter()
        for i in range(steps):
            E.forward(graph, step, tids[warmup + i], p, vocab=V, max_pos=max_pos, timeout_ms=20000)
            p += 1
        host = (time.perf_counter() - t0) * 1e3 / steps
    for _ in range(warmup):
        graph.launch()
    torch.cuda.synchronize()
    prof = None
    if profile:  # one wait per token, so every token's stamps are read
        for _ in range(steps):
            E.submit(graph, timeout_ms=20000)
        prof = {k: round(v, 2) for k, v in E.profile_report(graph).items()}
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(graph.stream)
    for _ in range(steps):
        graph.launch()
    b.record(graph.stream)
    b.synchronize()
    ms = a.elapsed_time(b) / steps
    T = min(pos + 1, win)
    xb = 0 if fast else 1  # fp32 x: 2K more bytes than the fp16 count
    sb = 1 if e4m3 else 2
    wbytes = LAYERS * sum(gemv_bytes(N, K, sb) + 2 * K * xb for N, K in
                          [(nq, H), (nk, H), (nk, H), (H, nq), (I, H), (I, H), (H, I)]) + gemv_bytes(V, H, sb) + 2 * H * xb
    kvbytes = LAYERS * 2 * nkv * T * hd * 2
    graph.destroy()
    del layers, B
    E.KEEP.clear()
    torch.cuda.empty_cache()
    out = {"ms_per_token": round(host if host_loop else ms, 4), "position": pos, "keys_attended": T,
            "activations": (("fp32 residual stream, fp16 GEMV inputs, fused norms, gelumul in the gate/up GEMV"
                             + (", norms inside the q/k/v and gate/up GEMV launches" if fuse_gemv else ""))
                            if fast else "fp32 (reference)"),
            "weight_bytes": wbytes, "kv_cache_bytes_read": kvbytes,
            "GBps": round((wbytes + kvbytes) / (ms * 1e-3) / 1e9, 1),
            "kernels_per_token": launches}
    if host_loop:
        out.update(timing="vk_engine.forward per token on the host clock (pinned (tid, pos) write, graph launch, "
                          "bounded wait), positions advancing from " + str(pos),
                   graph_replay_ms_per_token=round(ms, 4))
    if prof is not None:
        out["profile_us"] = prof
    return out


def counter_workload(ops):
    """The decode-token GEMV launches, for hardware-counter runs: 16 launches
    of each layer shape (qkv batched, o, gate_up, down; distinct weights) and
    2 lm_head launches, then one 512 MiB device copy whose FETCH_SIZE /
    WRITE_SIZE readings calibrate the counters' units."""
    import torch

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)

    def make(N, K):
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (N * K // 8,), dtype=torch.int64, device=dev,
                          generator=gen).to(torch.int32)
        s = (torch.randn(N * K // 32, device=dev, generator=gen) * 0.02).abs().to(torch.float16)
        return w, s

    xs = {K: torch.randn(K, device=dev, generator=gen).to(torch.float16) for K in (H, QN, I)}
    reps = 16
    src = torch.ones(512 * 2 ** 20 // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for name, shapes in [("qkv", [(QN, H), (KVN, H), (KVN, H)]), ("o", [(H, QN)]), ("gate_up", [(2 * I, H)]),
                         ("down", [(H, I)]), ("lm_head", [(V, H)])]:
        n = 2 if name == "lm_head" else reps
        mats = [[make(N, K) for N, K in shapes] for _ in range(n)]
        K = shapes[0][1]
        ys = [torch.empty(N, dtype=torch.float16, device=dev) for N, _ in shapes]
        torch.cuda.synchronize()
        for m in mats:
            if len(shapes) == 1:
                ops.gemv(xs[K], m[0][0], m[0][1], shapes[0][0], K, y=ys[0])
            else:
                ops.gemv_batch(xs[K], [(w, s, N, y, None) for (w, s), (N, _), y in zip(m, shapes, ys)], K)
        torch.cuda.synchronize()
        del mats
        print(f"[bench] counter workload: {n} x {name}", flush=True)
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[bench] counter workload done: copy {src.numel() * 4} B", flush=True)


ROTATE_BYTES = 1 << 30     # distinct weights a GEMM leg cycles through (4x the 256 MB Infinity Cache)


def bench_w8a8(ops, iters: int = 50):
    """W8A8 at M=2048, N=15360, K=3840 on packed weights (the product path:
    weights are packed once at load time), 50 back-to-back launches cycling
    through >= 1 GB of distinct weight sets (so the Infinity Cache cannot
    serve repeats). The weights are what the workload defines: int4 block
    codes uniform in [-8, 7] with |N(0, 0.02)| fp16 block scales, folded on
    the GPU into int8 weights and a per-row fp32 scale (q4_w8_fold, the
    reference's quant() fold). Beside it: the same kernel on uniformly random
    int8 weights (every bit of the operands toggles: a harsher power load),
    the row-major kernel, W4A8 and the activation quantizer."""
    import torch

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(1)
    M, N, K = 2048, 15360, 3840
    X = torch.randn((M, K), device=dev, generator=gen).to(torch.float16)
    nw = -(-ROTATE_BYTES // (N * K))

    def int4_set():
        wq = torch.randint(-2 ** 31, 2 ** 31 - 1, (N * K // 8,), dtype=torch.int64, device=dev,
                           generator=gen).to(torch.int32)
        sc = (torch.randn((N, K // 32), device=dev, generator=gen) * 0.02).abs().to(torch.float16).float()
        return wq, sc

    folded = []
    for _ in range(nw):
        wq, sc = int4_set()
        W8, sw32, _ = ops.w8_fold(wq, sc, N, K)
        folded.append((ops.w8_pack(W8), sw32, W8))
    ratio = ops.w4a8_ratio(sc, sw32, N, K)   # the last set's requant ratio, for the W4A8 legs
    A, sa = ops.quant_act_i8(X)
    Y = torch.empty((M, N), dtype=torch.float16, device=dev)
    st = torch.cuda.current_stream()

    def timed(fn):
        for i in range(5):
            fn(i)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(st)
        for i in range(iters):
            fn(i)
        b.record(st)
        b.synchronize()
        return a.elapsed_time(b) * 1e3 / iters

    def packed(i, stp=None):
        W8p, sw32, _ = folded[i % nw]
        return ops.gemm_w8a8_packed(A, W8p, sa, sw32, N, Y=Y, stamps=stp)

    us = timed(packed)
    stamped = w8a8_stamped(ops, packed, M, N, K, iters)
    us_nk = timed(lambda i: ops.gemm_w8a8(A, folded[i % nw][2], sa, folded[i % nw][1], Y=Y))
    del folded
    torch.cuda.empty_cache()
    # the same kernel on uniformly random int8 weights
    sw_u = (torch.rand(N, device=dev, generator=gen) * 1e-3 + 1e-4).to(torch.float32)
    W8u = [ops.w8_pack(torch.randint(-127, 128, (N, K), device=dev, generator=gen, dtype=torch.int8))
           for _ in range(nw)]
    us_u = timed(lambda i: ops.gemm_w8a8_packed(A, W8u[i % nw], sa, sw_u, N, Y=Y))
    del W8u
    # W4A8: the same product with B requantized to int8 on the fly from the int4 codes
    n4 = -(-ROTATE_BYTES // (N * K // 2))
    wq4 = [int4_set()[0] for _ in range(n4)]
    us_w4 = timed(lambda i: ops.gemm_w4a8(A, wq4[i % n4], ratio, sa, sw32, N, Y=Y))
    # ... or with its int8 weights formed once (q4_w4a8_weights) and packed: the W8A8 kernel, same results
    W8w4 = [ops.w8_pack(ops.w4a8_weights(w, ratio, N, K)) for w in wq4[:nw]]
    us_w4o = timed(lambda i: ops.gemm_w8a8_packed(A, W8w4[i % nw], sa, sw32, N, Y=Y))
    del wq4, W8w4
    # activation quantizer (bandwidth-bound: 2MK read + MK write)
    us_q = timed(lambda i: ops.quant_act_i8(X, A, sa))
    tops = 2.0 * M * N * K / (us * 1e-6) / 1e12
    tops_u = 2.0 * M * N * K / (us_u * 1e-6) / 1e12
    torch.cuda.empty_cache()
    return {"M": M, "N": N, "K": K, "weights": "int4 block codes folded to int8 (q4_w8_fold), packed (tile-32)",
            "launches": iters, "distinct_weight_sets": nw, "rotated_bytes": nw * N * K, "us": round(us, 2),
            "TOPS": round(tops, 1), "frac_of_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
            "stamped": stamped,
            "uniform_random_int8_weights": {"us": round(us_u, 2), "TOPS": round(tops_u, 1),
                                            "frac_of_int8_peak": round(tops_u / INT8_PEAK_TOPS, 4)},
            "us_row_major_weights": round(us_nk, 2),
            "w4a8_us": round(us_w4, 2), "w4a8_TOPS": round(2.0 * M * N * K / (us_w4 * 1e-6) / 1e12, 1),
            "w4a8_int8_weights_once_us": round(us_w4o, 2),
            "quant_act_us": round(us_q, 2), "quant_act_GBps": round(3 * M * K / (us_q * 1e-6) / 1e9, 1)}


def w8a8_stamped(ops, run, M: int, N: int, K: int, iters: int):
    """``iters`` back-to-back launches of the stamped W8A8 (each workgroup
    reads the wall clock at its start, after its k-loop and at its end, and
    counts shader cycles): the clock the chip held, how a launch's time
    splits into k-loop and epilogue, and the gap between launches, measured
    from inside the run."""
    import numpy as np
    import torch

    wgs = ops.w8a8_workgroups(M, N, K)
    stamps = torch.zeros((iters, wgs, 4), dtype=torch.int64, device="cuda:0")
    for i in range(5):
        run(i, stamps[0])
    torch.cuda.synchronize()
    for i in range(iters):
        run(i, stamps[i])
    torch.cuda.synchronize()
    tick_us = 1e3 / ops.probe_wall_clock_khz()
    s = stamps.cpu().numpy().astype(np.int64)
    w0, w1, w2, cyc = s[..., 0], s[..., 1], s[..., 2], s[..., 3]
    ghz = cyc / ((w2 - w0) * tick_us * 1e3)
    span = (w2.max(1) - w0.min(1)) * tick_us
    gaps = (w0.min(1)[1:] - w2.max(1)[:-1]) * tick_us
    half = iters // 2   # the second half: the sustained state
    return {"launches": iters, "workgroups": wgs,
            "shader_clock_GHz_median": round(float(np.median(ghz[half:])), 3),
            "shader_clock_GHz_first_launch": round(float(np.median(ghz[0])), 3),
            "span_us_median": round(float(np.median(span[half:])), 2),
            "kloop_us_median": round(float(np.median((w1 - w0)[half:]) * tick_us), 2),
            "epilogue_us_median": round(float(np.median((w2 - w1)[half:]) * tick_us), 2),
            "gap_between_launches_us_median": round(float(np.median(gaps[half - 1:])), 2)}


def bench_w4a16(ops, iters: int = 50):
    """W4A16 at the two M=512 prefill shapes, back-to-back launches cycling
    through >= 1 GB of distinct int4 weight sets."""
    import torch

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(2)
    out = {}
    for M, N, K in [(512, 15360, 3840), (512, 3840, 15360)]:
        X = torch.randn((M, K), device=dev, generator=gen).to(torch.float16)
        per = N * K // 2 + N * K // 16
        nw = -(-ROTATE_BYTES // per)
        mats = [(torch.randint(-2 ** 31, 2 ** 31 - 1, (N * K // 8,), dtype=torch.int64, device=dev,
                               generator=gen).to(torch.int32),
                 (torch.randn(N * K // 32, device=dev, generator=gen) * 0.02).abs().to(torch.float16))
                for _ in range(nw)]
        need = ops.gemm_workspace_bytes(M, N, K)
        ws = torch.empty(need, dtype=torch.uint8, device=dev) if need else None
        Y = torch.empty((M, N), dtype=torch.float16, device=dev)
        st = torch.cuda.current_stream()
        for i in range(5):
            ops.gemm_w4a16(X, mats[i % nw][0], mats[i % nw][1], N, Y=Y, ws=ws)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(st)
        for i in range(iters):
            ops.gemm_w4a16(X, mats[i % nw][0], mats[i % nw][1], N, Y=Y, ws=ws)
        b.record(st)
        b.synchronize()
        us = a.elapsed_time(b) * 1e3 / iters
        tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
        out[f"M{M}_N{N}_K{K}"] = {"us": round(us, 2), "TFLOPS": round(tf, 1),
                                 "frac_of_f16_peak": round(tf / F16_PEAK_TFLOPS, 4), "launches": iters,
                                 "distinct_weight_sets": nw}
        del mats
        torch.cuda.empty_cache()
    return out


def _timed_graph(ops, fn, n: int, reps: int) -> float:
    """us per call of fn(i), i < n, captured once as a graph and replayed reps times (HIP events on the graph's
    stream)."""
    import torch

    g = ops.Graph()
    with g.capture():
        for i in range(n):
            fn(i)
    g.launch()
    g.launch()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(g.stream)
    for _ in range(reps):
        g.launch()
    b.record(g.stream)
    b.synchronize()
    g.destroy()
    return a.elapsed_time(b) * 1e3 / (reps * n)


def bench_ceilings(ops):
    """Ceilings measured on this part (the denominators worth quoting beside
    the data-sheet peaks):
    - stream_read: the probe streaming-read kernel at each decode GEMV's byte
      count, as a graph of launches over distinct buffers (>= 1 GB, so every
      launch reads from HBM) - the best time for a dependent launch that
      reads that many bytes once; best of a sweep of grid sizes, loads in
      flight and chunked/strided order; at the 15360x3840 size also with
      each launch prefetching its successor's first bytes into L2;
    - mfma: MFMA-only loops (int8 32x32x32, f16 32x32x16), on the same
      operands every time and on random operands that change with every
      MFMA, one short launch and 50 back-to-back launches, with the shader
      clock read back;
    - hipblaslt: torch's int8 (_int_mm) and fp16 (matmul) GEMMs at the W8A8
      and W4A16 shapes, cycling through >= 1 GB of distinct weights."""
    import torch

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(7)
    out = {}
    sink = torch.empty(65536, dtype=torch.int32, device=dev)
    sizes = {"o_3840x4096": gemv_bytes(H, QN), "qkv_8192x3840": gemv_bytes(QN + 2 * KVN, H),
             "c1_15360x3840": gemv_bytes(I, H), "gate_up_30720x3840": gemv_bytes(2 * I, H),
             "lm_head_262144x3840": gemv_bytes(V, H)}
    sweep = [(w, u, c) for w in (256, 512, 1024, 2048) for u in (4, 8, 16) for c in (True, False)]
    sr = {}
    for name, nbytes in sizes.items():
        nbytes = -(-nbytes // 16) * 16
        n = max(3, ROTATE_BYTES // nbytes + 1)
        bufs = [torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), dtype=torch.int32, device=dev, generator=gen)
                for _ in range(n)]
        reps = 3 if nbytes > (256 << 20) else 5
        res = {}
        for w, u, c in sweep:
            res[(w, u, c)] = _timed_graph(ops, lambda i: ops.probe_stream_read(bufs[i], w, units=u, chunked=c,
                                                                               sink=sink), n, reps)
        (w, u, c), us = min(res.items(), key=lambda kv: kv[1])
        ent = {"bytes": nbytes, "us_per_launch": round(us, 3), "GBps": round(nbytes / us / 1e3, 1),
               "frac_of_hbm_peak": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
               "best": {"wgs": w, "units": u, "order": "chunked" if c else "strided"}, "distinct_buffers": n}
        # the GEMV's own access pattern: 16-byte loads over the code bytes
        # (8/9 of the bytes) and, with every one, a 2-byte companion load from
        # a second buffer of 1/8 their size (the fp16 block scales): the same
        # bytes as the GEMV, twice the load instructions; best of the chunked
        # grids
        if name != "lm_head_262144x3840":
            nu = nbytes * 8 // 9 // 16 * 16
            comps = [torch.randint(-2 ** 31, 2 ** 31 - 1, (-(-nu // 32),), dtype=torch.int32, device=dev,
                                   generator=gen) for _ in range(n)]
            rc = {}
            for w2 in (256, 512, 1024, 2048):
                for u2 in (4, 8):
                    rc[(w2, u2)] = _timed_graph(ops, lambda i: ops.probe_stream_read(
                        bufs[i][: nu // 4], w2, units=u2, chunked=True, comp=comps[i], sink=sink), n, reps)
            (w2, u2), us2 = min(rc.items(), key=lambda kv: kv[1])
            ent["with_scale_companion_loads"] = {"us_per_launch": round(us2, 3),
                                                 "bytes_incl_companion": nu + nu // 8,
                                                 "best": {"wgs": w2, "units": u2}}
            del comps
        if name == "c1_15360x3840":
            pf = {}
            for mb in (2, 4, 8, 16):
                t = _timed_graph(ops, lambda i: ops.probe_stream_read(
                    bufs[i], w, units=u, chunked=c, next=bufs[(i + 1) % n], prefetch_bytes=mb << 20, sink=sink),
                    n, reps)
                pf[f"{mb}MB"] = {"us_per_launch": round(t, 3), "GBps": round(nbytes / t / 1e3, 1)}
            ent["with_successor_prefetch"] = pf
        sr[name] = ent
        print(f"[bench] ceiling stream_read {name}: {ent}", flush=True)
        del bufs
        torch.cuda.empty_cache()
    out["stream_read"] = sr

    khz = ops.probe_wall_clock_khz()
    mf = {}
    # random operand bytes (int8 values / f16 values of either sign below 1
    # in magnitude), a different fragment for every MFMA of a round
    rnd = torch.randint(-2 ** 31, 2 ** 31 - 1, (16384,), dtype=torch.int32, device=dev, generator=gen)
    rnd_f16 = rnd & (0xBBFFBBFF - 2 ** 32)
    for kind, nm, per_mfma, peak in ((0, "int8_32x32x32", 65536, INT8_PEAK_TOPS), (1, "f16_32x32x16", 32768,
                                                                                 F16_PEAK_TFLOPS)):
        for wgs in (256, 512):
            iters = 2000
            clocks = torch.zeros((wgs, 2), dtype=torch.int64, device=dev)
            st = torch.cuda.current_stream()
            ops_per = wgs * 4 * iters * 4 * per_mfma
            res = {}
            for opn, operands in (("same_operands", None), ("random_operands", rnd if kind == 0 else rnd_f16)):
                for label, launches in (("short", 1), ("sustained_50", 50)):
                    for _ in range(3):
                        ops.probe_mfma(kind, wgs, iters, clocks, sink, operands)
                    torch.cuda.synchronize()
                    a = torch.cuda.Event(enable_timing=True)
                    b = torch.cuda.Event(enable_timing=True)
                    a.record(st)
                    for _ in range(launches):
                        ops.probe_mfma(kind, wgs, iters, clocks, sink, operands)
                    b.record(st)
                    b.synchronize()
                    us = a.elapsed_time(b) * 1e3 / launches
                    c = clocks.cpu().double()
                    ghz = float((c[:, 0] / (c[:, 1] / (khz * 1e3))).median()) / 1e9
                    t = ops_per / (us * 1e-6) / 1e12
                    res[f"{opn}_{label}"] = {"us_per_launch": round(us, 2), "T_per_s": round(t, 1),
                                             "frac_of_peak": round(t / peak, 4), "shader_clock_GHz": round(ghz, 3),
                                             "frac_of_peak_at_measured_clock": round(t / (peak * ghz / 2.4), 4)}
            mf[f"{nm}_{wgs // 256}wave_per_simd"] = res
    out["mfma"] = mf
    out["wall_clock_khz"] = khz
    print(f"[bench] ceiling mfma {mf}", flush=True)

    hb = {}
    st = torch.cuda.current_stream()

    def timed(fn, iters=50):
        for i in range(5):
            fn(i)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(st)
        for i in range(iters):
            fn(i)
        b.record(st)
        b.synchronize()
        return a.elapsed_time(b) * 1e3 / iters

    try:
        M, N, K = 2048, 15360, 3840
        A8 = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=gen)
        nw = -(-ROTATE_BYTES // (N * K))
        Bs = [torch.randint(-127, 128, (K, N), dtype=torch.int8, device=dev, generator=gen) for _ in range(nw)]
        us = timed(lambda i: torch._int_mm(A8, Bs[i % nw]))
        t = 2.0 * M * N * K / (us * 1e-6) / 1e12
        hb["int8_M2048_N15360_K3840"] = {"us": round(us, 2), "TOPS": round(t, 1),
                                         "frac_of_int8_peak": round(t / INT8_PEAK_TOPS, 4), "op": "torch._int_mm"}
        del Bs
    except Exception as e:  # noqa: BLE001 - a ceiling that cannot be measured is reported as such
        hb["int8_M2048_N15360_K3840"] = {"error": repr(e)[:200]}
    for M, N, K in ((512, 15360, 3840), (512, 3840, 15360), (2048, 15360, 3840)):
        try:
            X = torch.randn((M, K), device=dev, generator=gen).to(torch.float16)
            nw = -(-ROTATE_BYTES // (2 * N * K))
            Bs = [torch.randn((K, N), device=dev, generator=gen).to(torch.float16) for _ in range(nw)]
            us = timed(lambda i: torch.matmul(X, Bs[i % nw]))
            t = 2.0 * M * N * K / (us * 1e-6) / 1e12
            hb[f"f16_M{M}_N{N}_K{K}"] = {"us": round(us, 2), "TFLOPS": round(t, 1),
                                         "frac_of_f16_peak": round(t / F16_PEAK_TFLOPS, 4), "op": "torch.matmul"}
            del Bs
        except Exception as e:  # noqa: BLE001
            hb[f"f16_M{M}_N{N}_K{K}"] = {"error": repr(e)[:200]}
    torch.cuda.empty_cache()
    out["hipblaslt"] = hb
    print(f"[bench] ceiling hipblaslt {hb}", flush=True)
    return out


def committed_traffic(shape: str):
    """HBM bytes per launch of a decode GEMV shape from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE summary (calibrated by a copy of known
    size), or None when the summary does not cover the current kernel."""
    import re

    f = ROOT / "profiles" / "gemv_decode_hbm_traffic.md"
    if not f.exists():
        return None
    m = re.search(rf"^traffic {shape}: (\d+) B per launch$", f.read_text(), flags=re.M)
    return int(m.group(1)) if m else None


# --------------------------------------------------------- CPU baseline
def _cpu_info():
    """Host cores the numpy legs can use: os.cpu_count(), the affinity mask and
    the BLAS thread pool (threadpoolctl when present, else OMP_NUM_THREADS)."""
    threads = None
    try:
        from threadpoolctl import threadpool_info

        threads = max((p.get("num_threads") or 0) for p in threadpool_info()) or None
    except Exception:  # noqa: BLE001 - the count is informational
        pass
    if threads is None:
        threads = int(os.environ.get("OMP_NUM_THREADS", "1"))
    return {"cpu_count": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)), "blas_threads": threads}


def cpu_baseline(budget_s: float = 15.0):
    """The reference's numpy formulations, through the oracle, on the host cores:
    - value: GEMV dequant + matmul (benchmarks/coopgemm_i4.py:51-52 pattern)
      over whole decode layers of the decode-set shapes, ~half the budget;
    - gemv_matmul_only: the same GEMVs with the fp32 dequantized weights
      formed beforehand, only Wdq @ x timed (GB/s of the same int4 bytes);
    - w4a16: X.f32 @ Wdq.T at M=512, N=15360, K=3840 (dequant outside and
      inside the timed region);
    - w8a8: M=2048, N=15360, K=3840: per-row int8 activation quant
      (benchmarks/coopgemm_w4a8.py:87-88), the exact product as
      A.f64 @ W8.f64.T, and the f16((C sa) sw) epilogue."""
    import numpy as np

    from oracle import q4_oracle as O

    info = _cpu_info()
    rng = np.random.default_rng(0)
    x = {K: rng.standard_normal(K).astype(np.float16) for K in (H, QN, I)}
    layer = []
    for name, N, K in LAYER_SHAPES:
        q = rng.integers(0, 16, (N, K), dtype=np.uint8)
        s = np.abs(rng.normal(0, 0.02, (N, K // 32))).astype(np.float16).astype(np.float32)
        layer.append((N, K, q, s))
    t_total, nbytes, gemvs, layers = 0.0, 0, 0, 0
    while t_total < budget_s / 2 and layers < 64:
        for N, K, q, s in layer:
            t0 = time.perf_counter()
            O.gemv_ref(q, s, x[K]).astype(np.float16)
            t_total += time.perf_counter() - t0
            nbytes += gemv_bytes(N, K)
            gemvs += 1
        layers += 1
    # matmul only: Wdq formed outside the timed region
    wdq = [(N, K, O.dequant(q, s)) for N, K, q, s in layer]
    xf = {K: v.astype(np.float32) for K, v in x.items()}
    t_mm, b_mm, l_mm = 0.0, 0, 0
    while t_mm < budget_s / 6 and l_mm < 64:
        for N, K, W in wdq:
            t0 = time.perf_counter()
            (W @ xf[K]).astype(np.float16)
            t_mm += time.perf_counter() - t0
            b_mm += gemv_bytes(N, K)
        l_mm += 1
    del wdq
    # W4A16 at M=512, N=15360, K=3840
    M4, N4, K4 = 512, I, H
    q4 = rng.integers(0, 16, (N4, K4), dtype=np.uint8)
    s4 = np.abs(rng.normal(0, 0.02, (N4, K4 // 32))).astype(np.float16).astype(np.float32)
    X4 = rng.standard_normal((M4, K4)).astype(np.float16)
    t0 = time.perf_counter()
    Wd = O.dequant(q4, s4)
    t_dq = time.perf_counter() - t0
    t0 = time.perf_counter()
    (X4.astype(np.float32) @ Wd.T).astype(np.float16)
    t_w4 = time.perf_counter() - t0
    del Wd, q4
    # W8A8 at M=2048, N=15360, K=3840
    M8, N8, K8 = 2048, I, H
    W8 = rng.integers(-127, 128, (N8, K8), dtype=np.int8)
    sw = (rng.random(N8) * 1e-3 + 1e-4).astype(np.float32)
    X8 = rng.standard_normal((M8, K8)).astype(np.float16)
    t0 = time.perf_counter()
    A, sa = O.quant_act_i8(X8)
    t_q = time.perf_counter() - t0
    t0 = time.perf_counter()
    C = O.int_matmul_exact(A, W8)
    t_c = time.perf_counter() - t0
    t0 = time.perf_counter()
    O.w8a8_epilogue(C, sa, sw)
    t_e = time.perf_counter() - t0
    del W8, C
    f4 = 2.0 * M4 * N4 * K4
    f8 = 2.0 * M8 * N8 * K8
    return {"value": round(nbytes / t_total / 1e9, 3), "unit": "GB/s", "cores": info["blas_threads"], "kind": "port",
            "sample": f"{layers} decode layers ({gemvs} GEMVs, {nbytes / 1e9:.2f} GB algorithmic) of the same "
                      f"shapes through the oracle's numpy dequant+matmul in {t_total:.1f} s",
            **info,
            "gemv_matmul_only_GBps": round(b_mm / t_mm / 1e9, 3),
            "gemv_matmul_only_sample": f"{l_mm} decode layers, fp32 Wdq formed beforehand, {t_mm:.1f} s",
            "w4a16": {"shape": f"M{M4}_N{N4}_K{K4}", "matmul_s": round(t_w4, 3), "dequant_s": round(t_dq, 3),
                      "TFLOPS": round(f4 / t_w4 / 1e12, 4), "TFLOPS_with_dequant": round(f4 / (t_w4 + t_dq) / 1e12, 4)},
            "w8a8": {"shape": f"M{M8}_N{N8}_K{K8}", "quant_act_s": round(t_q, 3), "exact_matmul_f64_s": round(t_c, 3),
                     "epilogue_s": round(t_e, 3), "TOPS": round(f8 / (t_q + t_c + t_e) / 1e12, 4)}}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM legs")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--counters", action="store_true",
                    help="run only the decode GEMV launches (16 per layer shape, 2 lm_head) and a 512 MiB "
                         "calibration copy, for rocprofv3 --pmc passes; prints no JSON line")
    ap.add_argument("--no-token", action="store_true", help="skip the whole-token legs")
    ap.add_argument("--no-ceilings", action="store_true", help="skip the measured-ceiling probes")
    ap.add_argument("--ceilings-only", action="store_true",
                    help="run only the measured-ceiling probes; prints their results, no JSON line")
    ap.add_argument("--gemm-only", action="store_true",
                    help="run only the W8A8 and W4A16 legs; prints their results, no JSON line")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the prefill-chunk leg; prints its result, no JSON line")
    ap.add_argument("--small-m-only", action="store_true",
                    help="run only the small-M GEMV leg; prints its result, no JSON line")
    ap.add_argument("--token-profile", action="store_true",
                    help="only the fused decode token with a GPU timestamp after every launch: time per op label")
    ap.add_argument("--token-only", action="store_true",
                    help="run only the whole-token legs (reference dispatches, then fused) for --steps replays; "
                         "prints their results, no JSON line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this path is a single-GPU kernel set (multi-GPU sharding is "
              "design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    torch.cuda.set_device(0)
    ops = load_ops()
    if args.counters:
        counter_workload(ops)
        return
    if args.prefill_only:
        print(f"[bench] prefill chunk {bench_prefill(ops, reps=max(1, args.steps // 40))}", flush=True)
        print(f"[bench] prefill chunk, GEMMs with their own split-K reduce (no normadd/prepkv fusion) "
              f"{bench_prefill(ops, reps=max(1, args.steps // 40), gemm_norms=False)}", flush=True)
        print(f"[bench] prefill chunk, separate q/k/v and gate/up GEMMs and gelumul "
              f"{bench_prefill(ops, reps=max(1, args.steps // 40), stacked=False)}", flush=True)
        return
    if args.ceilings_only:
        bench_ceilings(ops)
        return
    if args.small_m_only:
        print(f"[bench] small-M gemv {bench_small_m(ops)}", flush=True)
        return
    if args.gemm_only:
        print(f"[bench] w8a8 {bench_w8a8(ops)}", flush=True)
        print(f"[bench] w4a16 {bench_w4a16(ops)}", flush=True)
        return
    if args.token_only:
        for fast in (False, True):
            print(f"[bench] token step {bench_token_step(ops, args.steps, args.warmup, fast=fast, host_loop=fast)}",
                  flush=True)
        return
    if args.token_profile:
        t = bench_token_step(ops, args.steps, args.warmup, fast=True, profile=True)
        print(f"[bench] token profile (us per token, in-graph stamps) {t['profile_us']}", flush=True)
        return
    print(f"[bench] decode graph: {LAYERS} layers + lm_head, {args.steps} steps after {args.warmup} warmup",
          flush=True)
    dec = bench_decode(ops, args.steps, args.warmup)
    print(f"[bench] decode {dec['ms_per_step']:.3f} ms/token, {dec['GBps']:.0f} GB/s "
          f"(per-token {dec['ms_per_step_percentiles']})", flush=True)
    dec8 = bench_decode(ops, args.steps, args.warmup, e4m3=True)
    print(f"[bench] decode, e4m3 scales {dec8['ms_per_step']:.3f} ms/token, {dec8['GBps']:.0f} GB/s "
          f"(per-shape us {json.dumps({k: v['us_per_launch'] for k, v in dec8['per_shape'].items()})})", flush=True)
    tok = None
    if not args.no_token:
        tok = {"reference_dispatches": bench_token_step(ops, max(20, args.steps // 4), 5),
               "fused": bench_token_step(ops, max(20, args.steps // 4), 5, fast=True, host_loop=True),
               "fused_norm_launches": bench_token_step(ops, max(20, args.steps // 4), 5, fast=True,
                                                       fuse_gemv=False),
               "fused_e4m3_scales": bench_token_step(ops, max(20, args.steps // 4), 5, fast=True, host_loop=True,
                                                     e4m3=True)}
        print(f"[bench] token step {tok}", flush=True)
    single = {"c1_15360x3840_f16_scales": bench_gemv_single(ops, I, H, False),
              "c3_15360x3840_e4m3_scales": bench_gemv_single(ops, I, H, True),
              "lm_head_262144x3840_f16_scales": bench_gemv_single(ops, V, H, False, reps=4)}
    print(f"[bench] single-shape gemv {single}", flush=True)
    small = bench_small_m(ops)
    print(f"[bench] small-M gemv {small}", flush=True)
    pre = bench_prefill(ops)
    pre["separate_qkv_gate_up_ms_per_chunk"] = bench_prefill(ops, stacked=False)["ms_per_chunk"]
    print(f"[bench] prefill chunk {pre}", flush=True)
    w8 = w4 = None
    if not args.no_gemm:
        w8 = bench_w8a8(ops)
        print(f"[bench] w8a8 {w8}", flush=True)
        w4 = bench_w4a16(ops)
        print(f"[bench] w4a16 {w4}", flush=True)
    ceil = None
    if not args.no_ceilings:
        ceil = bench_ceilings(ops)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_budget)
        print(f"[bench] cpu {cpu}", flush=True)

    ms = dec["ms_per_step"]
    # roofline kernel: the gate_up GEMV (30720x3840, 48 launches per token), the largest single-shape share
    # of the token; its average launch duration is measured above with HIP events over a graph of its 48
    # launches on the decode stream
    gu = dec["per_shape"]["gate_up"]
    gu_bytes = gu["bytes_per_launch"]
    achieved = gu_bytes / (gu["us_per_launch"] * 1e-6) / 1e9
    roof = {"bound": "hbm", "kernel": "gemv_kernel gate_up 30720x3840 (f16 x, f16 scales, f16 y)",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": committed_traffic("gate_up"),
            "bytes_per_launch": gu_bytes, "avg_launch_us": gu["us_per_launch"]}
    if ceil:
        # the token as dependent launches that each read their bytes once at the probe's best rate
        sr = {k: v["us_per_launch"] for k, v in ceil["stream_read"].items()}
        ach = (LAYERS * (sr["qkv_8192x3840"] + sr["o_3840x4096"] + sr["gate_up_30720x3840"] + sr["c1_15360x3840"])
               + sr["lm_head_262144x3840"]) / 1e3
        roof["achievable_ms_per_step"] = round(ach, 4)
        roof["frac_of_achievable"] = round(ach / ms, 4)
        # ... and with the GEMV's own access pattern (separate 2-byte scale loads; lm_head at its plain read)
        sc = {k: v.get("with_scale_companion_loads", v)["us_per_launch"] for k, v in ceil["stream_read"].items()}
        ach2 = (LAYERS * (sc["qkv_8192x3840"] + sc["o_3840x4096"] + sc["gate_up_30720x3840"] + sc["c1_15360x3840"])
                + sc["lm_head_262144x3840"]) / 1e3
        roof["achievable_scale_pattern_ms_per_step"] = round(ach2, 4)
    line = {
        "metric": METRIC,
        "value": round(dec["GBps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i4xf16->f32",
        "data": "synthetic",
        "config": {"workload": "decode GEMV set: 48 layers {q,k,v,o,gate_up,down} + lm_head 262144x3840, "
                               "int4 block-32 fp16 scales, one hipGraph per token",
                   "bytes_per_step": dec["bytes_per_step"], "kernels_per_step": dec["launches"],
                   "frac_of_hbm_peak": round(dec["GBps"] / HBM_PEAK_GBS, 4)},
        "roofline": roof,
        "cpu_baseline": None if cpu is None else {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample")},
        "per_shape_us": {k: v["us_per_launch"] for k, v in dec["per_shape"].items()},
        "decode_set_e4m3_ms": round(dec8["ms_per_step"], 4),
        "c1_us": single["c1_15360x3840_f16_scales"]["us_per_launch"],
        "c3_us": single["c3_15360x3840_e4m3_scales"]["us_per_launch"],
        "lm_head_us": single["lm_head_262144x3840_f16_scales"]["us_per_launch"],
        "token_ms": None if tok is None else tok["fused"]["ms_per_token"],
        "token_graph_ms": None if tok is None else tok["fused"]["graph_replay_ms_per_token"],
        "token_e4m3_ms": None if tok is None else tok["fused_e4m3_scales"]["ms_per_token"],
        "prefill_chunk_ms": pre["ms_per_chunk"],
    }
    if w8 is not None:
        line["w8a8_us"] = w8["us"]
        line["w8a8_frac_of_int8_peak"] = w8["frac_of_int8_peak"]
        line["w8a8_shader_clock_GHz"] = w8["stamped"]["shader_clock_GHz_median"]
        if ceil:
            mc = ceil["mfma"]["int8_32x32x32_1wave_per_simd"]["random_operands_sustained_50"]["T_per_s"]
            line["w8a8_frac_of_mfma_ceiling"] = round(w8["TOPS"] / mc, 4)
    if w4 is not None:
        line["w4a16_us"] = {k: v["us"] for k, v in w4.items()}
    if cpu is not None:
        line["cpu_w8a8_TOPS"] = cpu["w8a8"]["TOPS"]
        line["cpu_w4a16_TFLOPS"] = cpu["w4a16"]["TFLOPS"]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
