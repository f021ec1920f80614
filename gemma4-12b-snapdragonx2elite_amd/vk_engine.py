"""Drop-in host helpers for the quantized matmul path, with the reference
engine's call signatures (src/vk_engine.py of
monstercameron/Gemma4-12B-SnapdragonX2Elite).

The reference records Vulkan dispatches of GLSL shaders; here the same calls
enqueue HIP kernels of libq4mi.so on torch's current stream, and "recording
once" is a hipGraph capture (:func:`record`), replayed per token with a
bounded, labelled wait (:func:`submit`).

=====================  ====================================================
reference              here
=====================  ====================================================
``quant(W, pf)``       same tuple ``(bw, bs, split, nblk, inv, bs16, w8,
  :125-159             sw8)``; buffers are device :class:`Buf` in the
                       panel-64 layout, quantized on the GPU bit-exactly
``i4(lin, pf)`` :186   same
``Buf`` :56-69         device buffer with ``write``/``read``/``size``
``gemv_ds`` :214-226   same arguments; returns ``(dp, dr, N, split, WGx)``
                       with ``dr`` always None (the split-K reduce is
                       fused into the GEMV launch)
``gemv(g)`` :270-272   launches (or, inside :func:`record`, captures)
``gemv_many(gs)``      (new) descriptors on one input buffer as one
                       batched launch, e.g. q/k/v :232-234, gate/up :242-243
``gemm_ds`` :351-365   same arguments/return shape ``(cin, gem, cout, N, K)``
``gmm(C, t, L, tag)``  ``C`` is a torch stream or None (current stream)
  :391-400
``normbg`` :227-228,   :func:`normbg`, :func:`normadd_ds`, :func:`gelumul_ds`,
``ds(LN/LP/LA, ..)``   :func:`prepkv_ds`, :func:`attn_ds` build the non-GEMV
  :235-249             descriptors of a layer with the reference's buffers
                       and uniforms; :func:`disp` enqueues one
``buf_u32`` :71-73     same (the DYN position buffer is one)
``d_g/d_u/d_gm``       :func:`gate_up_ds`: gate/up rows interleaved once, the
  :242-246             gelumul in the GEMV epilogue (one launch)
fence wait :293-302    :func:`submit` / :func:`wait` raise
                       ``RuntimeError('GPU fence TIMEOUT after ..ms at [..]')``
=====================  ====================================================

Flags are read at import like the reference: ``GEMV_FP8=1`` selects e4m3
decode scales, ``PREFILL_I8=1`` the W8A8 prefill GEMM,
``GEMMA4_FENCE_TIMEOUT_MS`` the wait bound, ``PROFILE=1`` / ``PREPROF=1`` a
GPU timestamp after every op of the decode / prefill graph, summed per op
label at every submit (:func:`profile_report`, :func:`print_profile`).
"""
from __future__ import annotations

import os
import weakref
from typing import NamedTuple

import numpy as np
import torch

from . import ops
from ._lib import SCALE_E4M3, SCALE_F16

FP8 = os.environ.get("GEMV_FP8") == "1"
PREFILL_I8 = os.environ.get("PREFILL_I8") == "1"
PROFILE = os.environ.get("PROFILE") == "1"   # per-op GPU timestamps in the decode graph (src/vk_engine.py:37)
PREPROF = os.environ.get("PREPROF") == "1"   # ... and in the prefill graph (:38)
BLK = 32
MC = 128                    # prefill chunk (rows per prefill GEMM), src/vk_engine.py:339
_FENCE_MS = int(os.environ.get("GEMMA4_FENCE_TIMEOUT_MS", "0"))
KEEP: list = []             # buffers owned for the process lifetime (src/vk_engine.py:71)


class Buf:
    """Device buffer of ``nbytes`` (src/vk_engine.py:56-69)."""

    __slots__ = ("t", "size")

    def __init__(self, nbytes: int = 0, device=None, tensor: torch.Tensor | None = None):
        if tensor is not None:
            self.t = tensor.contiguous()
            self.size = self.t.numel() * self.t.element_size()
        else:
            self.t = torch.zeros(max(16, int(nbytes)), dtype=torch.uint8, device=device or "cuda")
            self.size = int(nbytes)

    @property
    def ptr(self) -> int:
        return self.t.data_ptr()

    def write(self, arr) -> None:
        a = np.ascontiguousarray(arr)
        src = torch.from_numpy(a.reshape(-1).view(np.uint8))
        dst = self.t.view(torch.uint8).reshape(-1)[: a.nbytes]
        dst.copy_(src)
        torch.cuda.current_stream().synchronize()

    def read(self, nbytes: int) -> bytes:
        return self.t.view(torch.uint8).reshape(-1)[:nbytes].cpu().numpy().tobytes()

    def view(self, dtype, count: int | None = None, byte_off: int = 0) -> torch.Tensor:
        u8 = self.t.view(torch.uint8).reshape(-1)
        esz = torch.empty((), dtype=dtype).element_size()
        n = count if count is not None else (u8.numel() - byte_off) // esz
        return u8[byte_off: byte_off + n * esz].view(dtype)


class QW(NamedTuple):
    bw: Buf
    bs: Buf
    split: int
    nblk: int
    inv: float
    bs16: Buf
    w8: Buf | None
    sw8: Buf | None


def quant(W, pf: bool = True, fp8: bool | None = None, prefill_i8: bool | None = None) -> QW:
    """int4 block quantization of ``W[N, K]`` on the GPU (src/vk_engine.py:125-159)."""
    fp8 = FP8 if fp8 is None else fp8
    prefill_i8 = PREFILL_I8 if prefill_i8 is None else prefill_i8
    Wt = torch.as_tensor(W).to(device="cuda", dtype=torch.float32).contiguous()
    N, K = Wt.shape
    nblk = K // BLK
    wq, sc16, sc32 = ops.quantize(Wt)
    del Wt
    inv = 1.0
    bs16 = Buf(tensor=sc16)
    bs = bs16
    if fp8:
        sc8, inv = ops.scales_e4m3(sc32, N, K)
        bs = Buf(tensor=sc8)
    split = ops.auto_split(N, K)
    w8 = sw8 = None
    if prefill_i8 and pf:
        W8, _sw32, sw16 = ops.w8_fold(wq, sc32, N, K)
        # int8 weights kept in the packed layout the W8A8 kernel reads (the
        # reference keeps Wi8T [K, N], src/vk_engine.py:155)
        w8, sw8 = Buf(tensor=ops.w8_pack(W8)), Buf(tensor=sw16)
        del W8
    return QW(Buf(tensor=wq), bs, split, nblk, float(inv), bs16, w8, sw8)


def i4(lin, pf: bool = True):
    """Quantize an ``nn.Linear`` and drop its fp weight (src/vk_engine.py:186)."""
    W = lin.weight.detach().float()
    lin.weight = None
    return quant(W, pf), tuple(W.shape)


# ------------------------------------------------- on-disk quantized weights
QUANT_FORMAT = "q4mi-panel64-v1"


def save_quant(path, mats: dict) -> None:
    """Write quantized matrices ``{name: (QW, (N, K))}`` (as :func:`quant`/:func:`i4`
    return them) to one safetensors file, in the device layouts the kernels
    read, so a restart loads them instead of re-quantizing (the reference
    re-quantizes every model load, ~4 minutes; JOURNEY.md:634-635 names a
    saved format as the follow-up). Per matrix ``name``: ``name.wq`` (panel-64
    int4 words, int32), ``name.sc16`` (panel-64 fp16 scales), ``name.sc8``
    (panel-64 e4m3 scale bytes, when the matrix uses them), ``name.w8`` and
    ``name.sw8`` (packed int8 weights and fp16 row scales, when present);
    shape, split, e4m3 ``inv`` and the format tag go in the header metadata.
    Only tensors and JSON-like metadata are stored: loading executes nothing
    from the file."""
    import json

    from safetensors.torch import save_file

    tensors, meta = {}, {"format": QUANT_FORMAT}
    for name, ((bw, bs, split, nblk, inv, bs16, w8, sw8), (N, K)) in mats.items():
        if "." in name:
            raise ValueError(f"matrix name {name!r} may not contain '.'")
        tensors[f"{name}.wq"] = bw.t.contiguous().cpu()
        tensors[f"{name}.sc16"] = bs16.t.contiguous().cpu()
        e4m3 = bs.t.dtype == torch.uint8
        if e4m3:
            tensors[f"{name}.sc8"] = bs.t.contiguous().cpu()
        if w8 is not None:
            tensors[f"{name}.w8"] = w8.t.contiguous().cpu()
            tensors[f"{name}.sw8"] = sw8.t.contiguous().cpu()
        meta[name] = json.dumps({"N": int(N), "K": int(K), "split": int(split), "nblk": int(nblk), "inv": float(inv),
                                 "e4m3": e4m3})
    save_file(tensors, str(path), metadata=meta)


def load_quant(path, device="cuda") -> dict:
    """Read a file written by :func:`save_quant`: ``{name: (QW, (N, K))}`` with
    the buffers on ``device``, ready for :func:`gemv_ds` / :func:`gemm_ds`."""
    import json

    from safetensors import safe_open

    out = {}
    with safe_open(str(path), framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != QUANT_FORMAT:
            raise ValueError(f"{path}: not a {QUANT_FORMAT} file (format {meta.get('format')!r})")
        keys = set(f.keys())
        for name, js in meta.items():
            if name == "format":
                continue
            m = json.loads(js)
            N, K = int(m["N"]), int(m["K"])
            if N <= 0 or K <= 0 or K % BLK or int(m["nblk"]) != K // BLK:
                raise ValueError(f"{path}: matrix {name!r} has a bad shape N={N} K={K} nblk={m['nblk']}")
            get = lambda k: Buf(tensor=f.get_tensor(f"{name}.{k}").to(device)) if f"{name}.{k}" in keys else None
            bw, bs16 = get("wq"), get("sc16")
            if bw is None or bs16 is None:
                raise ValueError(f"{path}: matrix {name!r} lacks its words or scales")
            wb, se = ops.dev_sizes(N, K)
            if bw.size != wb or bs16.size != 2 * se:
                raise ValueError(f"{path}: matrix {name!r} has the wrong size for {N}x{K}")
            bs = get("sc8") if m["e4m3"] else bs16
            if bs is None:
                raise ValueError(f"{path}: matrix {name!r} lacks its e4m3 scales")
            if m["e4m3"] and (bs.size != se or bs.t.dtype != torch.uint8):
                raise ValueError(f"{path}: matrix {name!r} has e4m3 scales of the wrong size for {N}x{K}")
            w8, sw8 = get("w8"), get("sw8")
            if (w8 is None) != (sw8 is None):
                raise ValueError(f"{path}: matrix {name!r} has only one of its int8 weights and row scales")
            if w8 is not None and (w8.size != int(ops.lib().q4_w8_packed_bytes(N, K)) or sw8.size != 2 * N):
                raise ValueError(f"{path}: matrix {name!r} has int8 weights of the wrong size for {N}x{K}")
            out[name] = (QW(bw, bs, int(m["split"]), int(m["nblk"]), float(m["inv"]), bs16, w8, sw8), (N, K))
    return out


class GemvDesc(NamedTuple):
    dp: tuple
    dr: None
    N: int
    split: int
    WGx: int


def gemv_ds(qw, inbuf: Buf, outbuf: Buf, out_off: int = 0, x_dtype=torch.float32) -> GemvDesc:
    """Bind a quantized matrix to fp32 input/output buffers (src/vk_engine.py:214-226).
    ``x_dtype=torch.float16`` reads an fp16 input buffer instead (written by a
    producer with an fp16 output: :func:`normbg`, :func:`gelumul_ds`,
    :func:`attn_ds`)."""
    (bw, bs, split, nblk, inv, _bs16, _w8, _sw8), (N, K) = qw
    fmt = SCALE_E4M3 if bs.t.dtype == torch.uint8 else SCALE_F16
    ws = ops.default_workspace(N, K, split, bw.t.device)
    if ws is not None:
        KEEP.append(ws)
    x = inbuf.view(x_dtype, K)
    y = outbuf.view(torch.float32, N, out_off)
    dp = (x, bw.t, bs.t, fmt, inv, y, N, K, split, ws)
    return GemvDesc(dp, None, N, split, (N + 63) // 64)


def gemv(g: GemvDesc) -> None:
    """Enqueue (or capture) one GEMV (src/vk_engine.py:270-272)."""
    x, wq, sc, fmt, inv, y, N, K, split, ws = g.dp
    ops.gemv(x, wq, sc, N, K, scale_fmt=fmt, inv=inv, y=y, split=split, ws=ws)


def gemv_many(gs) -> None:
    """Enqueue several :func:`gemv_ds` descriptors that read the same input
    buffer (q/k/v into the qkv buffer, gate/up: src/vk_engine.py:232-234,
    242-243) as one batched launch. Descriptors that cannot share a launch
    (different inputs, K, scale format, more than the batch limit) are
    launched one by one; the results are the same either way."""
    gs = list(gs)
    groups: list = []
    for g in gs:
        x, _wq, sc, fmt, _inv, _y, _N, K, _split, _ws = g.dp
        last = groups[-1] if groups else None
        if (last is not None and len(last) < ops.GEMV_MAX_BATCH and last[0].dp[0].data_ptr() == x.data_ptr()
                and last[0].dp[0].dtype == x.dtype and last[0].dp[7] == K and last[0].dp[3] == fmt and last[0].dp[5].dtype == g.dp[5].dtype
                and K <= ops.gemv_batch_max_k(x.dtype)):
            last.append(g)
        else:
            groups.append([g])
    for grp in groups:
        if len(grp) == 1:
            gemv(grp[0])
            continue
        x, _, _, fmt, _, _, _, K, _, _ = grp[0].dp
        ops.gemv_batch(x, [(d.dp[1], d.dp[2], d.dp[6], d.dp[5], d.dp[4]) for d in grp], K, scale_fmt=fmt)


_STAGE: dict = {}


def _stage(name: str, nbytes: int) -> Buf:
    b = _STAGE.get(name)
    if b is None or b.size < nbytes:
        b = Buf(nbytes)
        KEEP.append(b)
        _STAGE[name] = b
    return b


def gemm_ds(qw, inbuf: Buf, outbuf: Buf, prefill_i8: bool | None = None, x_dtype=torch.float32,
            y_dtype=torch.float32):
    """Prefill GEMM wiring for an ``MC``-row chunk (src/vk_engine.py:351-365).

    f16 route: cast f32->f16, W4A16 GEMM, cast f16->f32. W8A8 route
    (``PREFILL_I8``): per-row int8 quant, W8A8 GEMM, cast f16->f32.
    ``x_dtype=float16``: ``inbuf`` already holds the fp16 rows (its producer
    wrote them; the cast the reference runs would give the same values) and
    the f16 route skips its down-cast; ``y_dtype=float16``: the GEMM writes
    ``outbuf`` directly (its consumer reads fp16) and the up-cast is skipped.
    """
    prefill_i8 = PREFILL_I8 if prefill_i8 is None else prefill_i8
    (bw, _bs, _s, _n, _inv, bs16, w8, sw8), (N, K) = qw
    xin = inbuf.view(x_dtype, MC * K).view(MC, K)
    yout = outbuf.view(y_dtype, MC * N).view(MC, N)
    y16 = yout if y_dtype == torch.float16 else \
        _stage("Yf16", MC * max(N, K) * 2).view(torch.float16, MC * N).view(MC, N)
    if prefill_i8:
        if w8 is None:
            raise ValueError("PREFILL_I8 needs int8 weights: quantize with pf=True and prefill_i8=True")
        a8 = _stage("Ai8", MC * max(N, K)).view(torch.int8, MC * K).view(MC, K)
        sa = _stage("SAb", MC * 4).view(torch.float32, MC)
        W8p = w8.t
        sw = sw8.t
        cin = ("quant_act_i8", xin, a8, sa)
        gem = ("w8a8", a8, W8p, sa, sw, y16, N)
    else:
        if x_dtype == torch.float16:
            x16, cin = xin, None
        else:
            x16 = _stage("Xf16", MC * max(N, K) * 2).view(torch.float16, MC * K).view(MC, K)
            cin = ("cast_dn", xin, x16)
        need = ops.gemm_workspace_bytes(MC, N, K)   # split-K partials, allocated here so recording can capture
        ws = _stage("W4ws", need).view(torch.uint8, need) if need else None
        gem = ("w4a16", x16, bw.t, bs16.t, N, y16, ws)
    cout = None if y_dtype == torch.float16 else ("cast_up", y16, yout)
    return (cin, gem, cout, N, K)


def _run(op):
    kind = op[0]
    if kind == "cast_dn":
        ops.cast_f32_f16(op[1], op[2])
    elif kind == "cast_up":
        ops.cast_f16_f32(op[1], op[2])
    elif kind == "quant_act_i8":
        ops.quant_act_i8(op[1], op[2], op[3])
    elif kind == "w8a8":
        ops.gemm_w8a8_packed(op[1], op[2], op[3], op[4], op[6], Y=op[5])
    elif kind == "w4a16":
        ops.gemm_w4a16(op[1], op[2], op[3], op[4], Y=op[5], ws=op[6])
    else:
        raise ValueError(kind)


def gmm(C, t, L=None, tag: str = "") -> None:
    """cast -> GEMM -> cast for one prefill matmul (src/vk_engine.py:391-400).
    ``C``: torch stream to enqueue on (None = current stream)."""
    cin, gem, cout, _N, _K = t
    seq = [op for op in (cin, gem, cout) if op is not None]
    if C is None:
        for op in seq:
            _run(op)
    else:
        with torch.cuda.stream(C):
            for op in seq:
                _run(op)


# ------------------------------------------------- decode-token ops (non-GEMV)
def buf_u32(vals) -> Buf:
    """Small uint32 buffer (uniforms, the DYN position buffer), kept alive
    for the process (src/vk_engine.py:71-73)."""
    b = Buf(max(16, len(vals) * 4))
    b.write(np.array(vals, np.uint32))
    KEEP.append(b)
    return b


def _u32(du) -> np.ndarray:
    """Words of a small uniform given as a Buf (read once, at descriptor time) or a sequence."""
    if isinstance(du, Buf):
        return np.frombuffer(du.read(16), np.uint32)
    return np.asarray(list(du) + [0] * (4 - len(du)), np.uint32)


class OpDesc(NamedTuple):
    """A recorded non-GEMV dispatch: ``disp(d)`` enqueues it."""
    fn: object
    args: tuple
    kw: dict


def disp(d: OpDesc) -> None:
    """Enqueue (or, inside :func:`record`, capture) one op descriptor
    (the reference's ``disp``, src/vk_engine.py:265-269)."""
    d.fn(*d.args, **d.kw)


def _f32v(b: Buf, n: int, byte_off: int = 0) -> torch.Tensor:
    return b.view(torch.float32, n, byte_off)


def normbg(inbuf: Buf, wb: Buf, outbuf: Buf, du, out_dtype=torch.float32) -> OpDesc:
    """RMS norm of ``du[0]`` floats of ``inbuf`` times ``wb`` into ``outbuf``
    (src/vk_engine.py:227-228, vk/rmsnorm.comp); ``out_dtype`` fp32 (the
    reference) or fp16."""
    D = int(_u32(du)[0])
    return OpDesc(ops.rmsnorm, (_f32v(inbuf, D), _f32v(wb, D), outbuf.view(out_dtype, D)), {})


def normadd_ds(xbuf: Buf, wb: Buf, hbuf: Buf, du) -> OpDesc:
    """``h = (h + norm(x) * w) * sc``, ``sc`` the float whose bits are
    ``du[1]`` (0: unscaled) (d_na / d_nas, src/vk_engine.py:242,248-249)."""
    u = _u32(du)
    D, sc = int(u[0]), float(u[1:2].view(np.float32)[0])
    return OpDesc(ops.normadd, (_f32v(xbuf, D), _f32v(wb, D), _f32v(hbuf, D), sc), {})


def gelumul_ds(gate: Buf, up: Buf, out: Buf, du, out_dtype=torch.float32) -> OpDesc:
    """``out = gelu_tanh(gate) * up`` over ``du[0]`` floats (d_gm, src/vk_engine.py:246)."""
    n = int(_u32(du)[0])
    return OpDesc(ops.gelumul, (_f32v(gate, n), _f32v(up, n), out.view(out_dtype, n)), {})


_INTERLEAVED: dict = {}


def _interleaved(wg, sg, wu, su, N: int, K: int):
    """The gate/up matrices interleaved row by row (:func:`ops.interleave_rows`),
    made once per set of source arrays: the decode gated GEMV and the prefill
    gated GEMM share it when they read the same scale array. KEEP owns the
    copy; the cache holds weak references only, and an entry counts only
    while its sources and its copy are all alive (so a reused address never
    returns a stale copy, and clearing KEEP frees the copies)."""
    key = (wg.data_ptr(), sg.data_ptr(), wu.data_ptr(), su.data_ptr(), N, K)
    hit = _INTERLEAVED.get(key)
    if hit is not None:
        refs = [r() for r in hit]
        if all(t is not None for t in refs) and all(a is b for a, b in zip(refs[2:], (wg, sg, wu, su))):
            return refs[0], refs[1]
    wo, so = ops.interleave_rows(wg, sg, wu, su, N, K)
    KEEP.extend([wo, so])
    _INTERLEAVED[key] = tuple(weakref.ref(t) for t in (wo, so, wg, sg, wu, su))
    return wo, so


def gate_up_ds(qg, qu, inbuf: Buf, actbuf: Buf, x_dtype=torch.float32, act_dtype=torch.float32) -> OpDesc | None:
    """The gate and up GEMVs and the gelumul after them (src/vk_engine.py:242-243,
    246) as one launch: the two matrices are interleaved row by row here (a
    copy of their weights, made once) and the GEMV's epilogue writes
    ``act = gelu_tanh(gate) * up``. Returns None when the two cannot share
    one matrix (different shapes, scale formats or e4m3 lifts); then record
    the separate descriptors."""
    (bwg, bsg, _sg, _nb, invg, _a, _b, _c), (N, K) = qg
    (bwu, bsu, _su, _nb2, invu, _d, _e, _f), (N2, K2) = qu
    if (N, K) != (N2, K2) or bsg.t.dtype != bsu.t.dtype or invg != invu or N % 32:
        return None
    fmt = SCALE_E4M3 if bsg.t.dtype == torch.uint8 else SCALE_F16
    wo, so = _interleaved(bwg.t, bsg.t, bwu.t, bsu.t, N, K)
    split = ops.auto_split(2 * N, K)
    ws = ops.default_workspace(2 * N, K, split, wo.device)
    if ws is not None:
        KEEP.append(ws)
    return OpDesc(ops.gemv_gated, (inbuf.view(x_dtype, K), wo, so, 2 * N, K),
                  dict(scale_fmt=fmt, inv=invg, act=actbuf.view(act_dtype, N), split=split, ws=ws))


def prepkv_ds(qkv: Buf, knw: Buf, cosb: Buf, sinb: Buf, kc: Buf, vc: Buf, P, dyn: Buf) -> OpDesc:
    """This token's K/V into the fp16 caches (d_prep, src/vk_engine.py:235-237);
    ``P`` = (nkv, hd, koff, voff, keqv, stride, window, 0) in floats/slots."""
    nkv, hd, koff, voff, keqv, stride, window = (int(v) for v in np.asarray(P, np.uint32)[:7])
    kw = dict(nkv=nkv, hd=hd, koff=koff, voff=voff, keqv=bool(keqv), stride=stride, window=window,
              dyn=dyn.view(torch.int32, 4))
    return OpDesc(ops.prepkv, (qkv.view(torch.float32), _f32v(knw, hd), _f32v(cosb, hd), _f32v(sinb, hd),
                               kc.view(torch.float16), vc.view(torch.float16)), kw)


def attn_ds(qkv: Buf, qnw: Buf, cosb: Buf, sinb: Buf, kc: Buf, vc: Buf, out: Buf, A, dyn: Buf,
            out_dtype=torch.float32) -> OpDesc:
    """Decode attention (d_attn, src/vk_engine.py:238-239); ``A`` = (nH, nkv,
    hd, stride, window, qoff, grp, 0). The split-key scratch is allocated
    here, before any recording."""
    nH, nkv, hd, stride, window, qoff, grp = (int(v) for v in np.asarray(A, np.uint32)[:7])
    ws = ops.attn_workspace(nH, hd, stride, qkv.t.device)
    KEEP.append(ws)
    kw = dict(nH=nH, nkv=nkv, hd=hd, stride=stride, window=window, qoff=qoff, grp=grp,
              dyn=dyn.view(torch.int32, 4), ws=ws)
    return OpDesc(ops.attn, (qkv.view(torch.float32), _f32v(qnw, hd), _f32v(cosb, hd), _f32v(sinb, hd),
                             kc.view(torch.float16), vc.view(torch.float16), out.view(out_dtype, nH * hd)), kw)


# ----------------------------------------------- batched-prefill layer ops
def pre_norm_ds(inbuf: Buf, wb: Buf, outbuf: Buf, du, out_dtype=torch.float32) -> OpDesc:
    """RMS norm of the ``MC`` rows of ``du[0]`` floats (p_in, p_pfn:
    src/vk_engine.py:369,377, vk/pre_norm.comp)."""
    D = int(_u32(du)[0])
    return OpDesc(ops.pre_rmsnorm, (_f32v(inbuf, MC * D), _f32v(wb, D), outbuf.view(out_dtype, MC * D)),
                  dict(M=MC, D=D))


def pre_na_ds(xbuf: Buf, wb: Buf, hbuf: Buf, du, x_dtype=torch.float32) -> OpDesc:
    """``h = (h + norm(x) * w) * sc`` per row (p_na, p_nas: :376,382-383,
    vk/pre_na.comp); ``x_dtype=float16`` reads a GEMM's fp16 output."""
    u = _u32(du)
    D, sc = int(u[0]), float(u[1:2].view(np.float32)[0])
    return OpDesc(ops.pre_normadd, (xbuf.view(x_dtype, MC * D), _f32v(wb, D), _f32v(hbuf, MC * D)),
                  dict(M=MC, D=D, scale=sc))


def pre_gelumul_ds(gate: Buf, up: Buf, out: Buf, du, in_dtype=torch.float32, out_dtype=torch.float32) -> OpDesc:
    """``out = gelu_tanh(gate) * up`` over ``du[0]`` (= MC * I) elements (p_gm, :380)."""
    n = int(_u32(du)[0])
    return OpDesc(ops.pre_gelumul, (gate.view(in_dtype, n), up.view(in_dtype, n), out.view(out_dtype, n)), {})


def gemm_cat_ds(qws, inbuf: Buf, outbuf: Buf, **kw):
    """The prefill GEMMs of several matrices that read the same rows (the
    q, k and v projections, p_q/p_k/p_v: src/vk_engine.py:370-371, 414-415)
    as one GEMM over their rows stacked (a copy made once): ``outbuf`` gets
    rows of sum(N) elements, matrix i's outputs at column offset sum(N[:i]).
    Each N must be a multiple of 64 (whole weight panels). ``kw`` as
    :func:`gemm_ds`; returns its tuple (for :func:`gmm`). The stacked copy
    stays beside the separate matrices (the decode GEMVs read those): one more
    copy of the q/k/v weights in all."""
    Ns = [N for _, (N, _K) in qws]
    K = qws[0][1][1]
    if any(N % 64 for N in Ns) or any(k != K for _, (_n, k) in qws):
        raise ValueError("stacked GEMMs need a common K and N multiples of 64")
    parts = [q for q, _ in qws]

    def cat(field):
        vals = [getattr(q, field) for q in parts]
        if any(v is None for v in vals):
            return None
        t = torch.cat([v.t.reshape(-1) for v in vals])
        KEEP.append(t)
        return Buf(tensor=t)
    bw, bs16 = cat("bw"), cat("bs16")
    bs = cat("bs") if len({q.bs.t.dtype for q in parts}) == 1 else None
    w8, sw8 = cat("w8"), cat("sw8")
    q0 = parts[0]
    qw = QW(bw, bs if bs is not None else bs16, q0.split, q0.nblk, q0.inv, bs16, w8, sw8)
    return gemm_ds((qw, (sum(Ns), K)), inbuf, outbuf, **kw)


def pre_gate_up_ds(qg, qu, inbuf: Buf, actbuf: Buf) -> OpDesc | None:
    """The prefill gate and up GEMMs and the gelumul after them (p_g, p_u,
    p_gm: src/vk_engine.py:381-382, 421-422) as one gated W4A16 product
    (:func:`ops.gemm_w4a16_gated`) over the two matrices interleaved row by
    row (a copy made once): ``actbuf`` gets the fp16 activations the
    separate route's gelumul writes, from fp16 normed rows in ``inbuf``.
    Returns None when the two cannot share one matrix (different shapes) or
    on the W8A8 route; then record the separate descriptors. The interleaved
    copy is shared with :func:`gate_up_ds` on the same fp16 scales and stays
    beside the separate matrices (one more copy of gate and up in all); the
    split-K workspace is the shared prefill stage buffer (the gated GEMM
    reduces it inside its own call, and recorded ops run in order on one
    stream)."""
    (bwg, _bsg, _sg, _nb, _ig, bs16g, _a, _b), (N, K) = qg
    (bwu, _bsu, _su, _nb2, _iu, bs16u, _c, _d), (N2, K2) = qu
    if (N, K) != (N2, K2) or PREFILL_I8 or bs16g is None or bs16u is None:
        return None
    wo, so = _interleaved(bwg.t, bs16g.t, bwu.t, bs16u.t, N, K)
    need = ops.gemm_gated_workspace_bytes(MC, 2 * N, K)
    ws = _stage("W4nws", need).view(torch.uint8, need)
    return OpDesc(ops.gemm_w4a16_gated, (inbuf.view(torch.float16, MC * K).view(MC, K), wo, so, 2 * N),
                  dict(Y=actbuf.view(torch.float16, MC * N).view(MC, N), ws=ws))


def pre_prepkv_ds(kbuf: Buf, vbuf: Buf, knw: Buf, cosM: Buf, sinM: Buf, kc: Buf, vc: Buf, Pp, dyn: Buf,
                  kv_dtype=torch.float32, ld: int | None = None, koff: int = 0, voff: int = 0) -> OpDesc:
    """The chunk's K/V into the caches (p_prep, :372-374); ``Pp`` = (nkv, hd,
    nk, 0, stride, window, 0, 0), ``vbuf`` the K buffer for k == v layers,
    ``dyn`` = (p0, MC, 0, 0). ``ld``, ``koff``, ``voff`` (elements): rows of
    K and V inside a wider buffer (the q/k/v GEMM's output, :func:`gemm_cat_ds`)."""
    nkv, hd, nk, _z, stride, window = (int(v) for v in np.asarray(Pp, np.uint32)[:6])
    ld = ld or nk
    esz = torch.empty((), dtype=kv_dtype).element_size()
    n = (MC - 1) * ld + nk
    kw = dict(M=MC, ld=ld, nkv=nkv, hd=hd, stride=stride, window=window, dyn=dyn.view(torch.int32, 4))
    return OpDesc(ops.pre_prepkv, (kbuf.view(kv_dtype, n, koff * esz), vbuf.view(kv_dtype, n, voff * esz),
                                   _f32v(knw, hd), _f32v(cosM, MC * hd), _f32v(sinM, MC * hd),
                                   kc.view(torch.float16), vc.view(torch.float16)), kw)


def pre_attn_ds(qbuf: Buf, qnw: Buf, cosM: Buf, sinM: Buf, kc: Buf, vc: Buf, out: Buf, Aa, dyn: Buf, nkv: int,
                max_keys: int | None = None, q_dtype=torch.float32, out_dtype=torch.float32,
                ldq: int | None = None) -> OpDesc:
    """Causal attention of the chunk (p_attn, :375-377); ``Aa`` = (nH, nq, hd,
    stride, window, grp, 0, 0). ``max_keys`` bounds the keys a token will
    see (default: the ring for sliding layers, the cache for global ones);
    the split-key scratch is allocated here, before any recording. ``ldq``:
    the q rows' stride inside a wider buffer (:func:`gemm_cat_ds`)."""
    nH, nq, hd, stride, window, grp = (int(v) for v in np.asarray(Aa, np.uint32)[:6])
    if nH // grp != nkv:
        raise ValueError(f"grp={grp} does not match nH={nH} / nkv={nkv}")
    mk = max_keys or (window if window > 0 else stride)
    ws = ops.pre_attn_workspace(MC, nH, nkv, hd, mk, qbuf.t.device)
    KEEP.append(ws)
    ldq = ldq or nq
    kw = dict(M=MC, ldq=ldq, nH=nH, nkv=nkv, hd=hd, stride=stride, window=window, max_keys=mk,
              dyn=dyn.view(torch.int32, 4), ws=ws)
    return OpDesc(ops.pre_attn, (qbuf.view(q_dtype, (MC - 1) * ldq + nq), _f32v(qnw, hd), _f32v(cosM, MC * hd),
                                 _f32v(sinM, MC * hd), kc.view(torch.float16), vc.view(torch.float16),
                                 out.view(out_dtype, MC * nH * hd)), kw)


def record_prefill(layers, fuse: bool = True, gemm_norms: bool = False, profile: bool | None = None) -> ops.Graph:
    """Record the prefill of one ``MC``-token chunk through ``layers`` in the
    reference's order (rec_layer, src/vk_engine.py:410-424): per layer
    p_in, the q/k/v GEMMs, p_prep, p_attn, the o GEMM, p_na, p_pfn, the
    gate/up GEMMs, p_gm, the down GEMM, p_nas. ``layers`` holds the
    reference's per-layer keys (``p_in`` ... ``p_nas``; ``p_v`` may be None;
    GEMM entries are :func:`gemm_ds` tuples); a layer with a ``p_gu``
    descriptor (:func:`pre_gate_up_ds`) runs it in place of ``p_g``, ``p_u``
    and ``p_gm``, and one with ``p_qkv`` (:func:`gemm_cat_ds`) in place of
    the q/k/v GEMMs. With ``gemm_norms``, a GEMM whose fp16 output only
    feeds the pre_na after it (the o and down projections) runs with that
    normadd as :func:`ops.gemm_w4a16_normadd`, and the stacked q/k/v GEMM
    with the pre_prepkv after it as :func:`ops.gemm_w4a16_qkv_prepkv`. The
    reference submits one
    command buffer per layer; one graph holds them all here (the chunk's
    buffers persist between layers either way). With ``fuse``, each
    pre_na and the pre_norm of the same rows after it run as one launch.
    With ``profile`` (default: ``PREPROF=1``) a GPU timestamp follows every
    launch (src/vk_engine.py:491-504; see :func:`record_decode`)."""
    seq = []
    for L in layers:
        if L.get("p_qkv") is not None:
            seq += [L["p_in"], ("gmm", L["p_qkv"])]
        else:
            seq += [L["p_in"], ("gmm", L["p_q"]), ("gmm", L["p_k"])] + \
                   ([("gmm", L["p_v"])] if L.get("p_v") is not None else [])
        seq += [L["p_prep"], L["p_attn"], ("gmm", L["p_o"]), L["p_na"], L["p_pfn"]] + \
            ([L["p_gu"]] if L.get("p_gu") is not None else [("gmm", L["p_g"]), ("gmm", L["p_u"]), L["p_gm"]]) + \
            [("gmm", L["p_d"]), L["p_nas"]]
    if fuse:
        seq = _fuse_pre_norms(seq)
    if gemm_norms:
        seq = _fuse_gemm_prepkv(_fuse_gemm_normadd(seq))

    def run(op):
        if isinstance(op, tuple) and op and op[0] == "gmm":
            gmm(None, op[1])
        else:
            disp(op)

    g = _record_seq(seq, run, PREPROF if profile is None else profile)
    g.seq = seq          # the recorded descriptor sequence, for inspection
    return g


def _op_tensors(op):
    """Every tensor an op of a prefill sequence passes (OpDesc args and
    keywords, or the cast/GEMM/cast tuples of a ``("gmm", ...)`` entry)."""
    if isinstance(op, OpDesc):
        items = list(op.args) + list(op.kw.values())
    elif isinstance(op, tuple) and op and op[0] == "gmm":
        items = [t for part in op[1][:3] if part is not None for t in part[1:]]
    else:
        items = []
    return [t for t in items if isinstance(t, torch.Tensor)]


def _overlap(t: torch.Tensor, u: torch.Tensor) -> bool:
    a0, b0 = t.data_ptr(), u.data_ptr()
    return a0 < b0 + u.numel() * u.element_size() and b0 < a0 + t.numel() * t.element_size()


def _read_later(seq, start: int, y: torch.Tensor) -> bool:
    """Whether an op from ``seq[start]`` on passes memory of ``y`` before a
    GEMM writes ``y`` again (conservative: passing it counts as reading)."""
    nbytes = y.numel() * y.element_size()
    for op in seq[start:]:
        if isinstance(op, tuple) and op and op[0] == "gmm":
            cin, gem = op[1][0], op[1][1]
            reads = list(cin[1:] if cin is not None else ()) + list(gem[1:4] if gem[0] == "w4a16" else gem[1:5])
            if any(isinstance(t, torch.Tensor) and _overlap(t, y) for t in reads):
                return True
            out = gem[5]
            if out.data_ptr() == y.data_ptr() and out.numel() * out.element_size() >= nbytes:
                return False        # overwritten: later readers see the new values
            continue
        if any(_overlap(t, y) for t in _op_tensors(op)):
            return True
    return False


def _fuse_gemm_normadd(seq):
    """A W4A16 prefill GEMM with fp16 input and output followed by a pre_na
    (or pre_na + pre_norm) that reads its output: one GEMM into split-K
    partials and one normadd launch that sums them (:func:`ops.gemm_w4a16_normadd`).
    The fused launch never writes the GEMM's output buffer, so the pair is
    fused only when no later op reads that buffer before a GEMM writes it
    again."""
    out, i = [], 0
    while i < len(seq):
        a = seq[i]
        b = seq[i + 1] if i + 1 < len(seq) else None
        gem = a[1][1] if isinstance(a, tuple) and a and a[0] == "gmm" else None
        if (gem is not None and gem[0] == "w4a16" and a[1][0] is None and a[1][2] is None and
                isinstance(b, OpDesc) and b.fn is ops.pre_normadd and b.args[0].dtype == torch.float16 and
                b.args[0].data_ptr() == gem[5].data_ptr() and b.kw["D"] == gem[4] and
                not _read_later(seq, i + 2, gem[5])):
            _k, x16, wq, sc16, N, _y16, _ws = gem
            M, K = x16.shape
            need = ops.gemm_normadd_workspace_bytes(M, N, K)
            ws = _stage("W4nws", need).view(torch.uint8, need)
            _x, w, h = b.args
            kw = dict(scale=b.kw.get("scale", 0.0), ws=ws)
            if b.kw.get("w2") is not None:
                kw.update(w2=b.kw["w2"], y=b.kw["y"])
            out.append(OpDesc(ops.gemm_w4a16_normadd, (x16, wq, sc16, N, w, h.view(M, N)), kw))
            i += 2
        else:
            out.append(a)
            i += 1
    return out


def _fuse_gemm_prepkv(seq):
    """The stacked q/k/v GEMM (fp16 in and out) followed by the pre_prepkv
    that reads its k/v columns: one GEMM into split-K partials and one
    launch that stores the q columns and writes the caches
    (:func:`ops.gemm_w4a16_qkv_prepkv`). The k/v columns of the GEMM's
    output are then never written: the caller's later ops must read k and v
    from the caches only (the attention does; :func:`record_prefill`'s
    layer order guarantees it), while q is read from the output as before."""
    out, i = [], 0
    while i < len(seq):
        a = seq[i]
        b = seq[i + 1] if i + 1 < len(seq) else None
        gem = a[1][1] if isinstance(a, tuple) and a and a[0] == "gmm" else None
        if (gem is not None and gem[0] == "w4a16" and a[1][0] is None and a[1][2] is None and
                isinstance(b, OpDesc) and b.fn is ops.pre_prepkv and b.args[0].dtype == torch.float16 and
                b.kw["ld"] == gem[4]):
            _k, x16, wq, sc16, N, y16, _ws = gem
            k, v = b.args[0], b.args[1]
            same = all(t.untyped_storage().data_ptr() == y16.untyped_storage().data_ptr() for t in (k, v))
            koff = (k.data_ptr() - y16.data_ptr()) // 2 if same else -1
            voff = (v.data_ptr() - y16.data_ptr()) // 2
            nk = b.kw["nkv"] * b.kw["hd"]
            keqv = voff == koff
            if koff > 0 and N == koff + nk * (1 if keqv else 2) and (keqv or voff == koff + nk):
                M, K = x16.shape
                need = ops.gemm_normadd_workspace_bytes(M, N, K)
                ws = _stage("W4nws", need).view(torch.uint8, need)
                kw = {kk: b.kw[kk] for kk in ("nkv", "hd", "stride", "window", "dyn")}
                out.append(OpDesc(ops.gemm_w4a16_qkv_prepkv, (x16, wq, sc16, N, y16.view(-1)) + tuple(b.args[2:]),
                                  dict(kw, nq=koff, ldq=N, keqv=keqv, ws=ws)))
                i += 2
                continue
        out.append(a)
        i += 1
    return out


def _fuse_pre_norms(seq):
    """A pre_na followed by a pre_norm of the same rows: one launch."""
    out, i = [], 0
    while i < len(seq):
        a = seq[i]
        b = seq[i + 1] if i + 1 < len(seq) else None
        if (isinstance(a, OpDesc) and isinstance(b, OpDesc) and a.fn is ops.pre_normadd and b.fn is ops.pre_rmsnorm
                and a.args[2].data_ptr() == b.args[0].data_ptr() and a.kw["D"] == b.kw["D"]):
            x, w, h = a.args
            _, w2, y = b.args
            out.append(OpDesc(ops.pre_normadd, (x, w, h), dict(a.kw, w2=w2, y=y)))
            i += 2
        else:
            out.append(a)
            i += 1
    return out


# ------------------------------------------------------- record-once submit
def record(body) -> ops.Graph:
    """Capture everything ``body()`` enqueues into one hipGraph
    (the command buffer recorded once, src/vk_engine.py:254-290)."""
    g = ops.Graph()
    with g.capture():
        body()
    return g


def op_label(op) -> str:
    """Profile label of a recorded descriptor: the op's name, or a GEMV's
    (stacked) rows x K."""
    if isinstance(op, tuple) and op and op[0] in ("gemvs", "gemvs_nx"):
        ds = op[1] if op[0] == "gemvs" else op[2]
        return ("gemv+norm " if op[0] == "gemvs_nx" else "gemv ") + f"{sum(d.N for d in ds)}x{ds[0].dp[7]}"
    if isinstance(op, tuple) and op and op[0] == "gmm":
        return "gemm"
    fn = getattr(op, "fn", None)
    if fn is ops.gemv_normadd:
        return f"gemv+norm {op.args[7]}x{op.args[8]}"
    return getattr(fn, "__name__", "op").lstrip("_")


def _record_seq(seq, run, profile: bool) -> ops.Graph:
    """Record ``run(op)`` for every op of ``seq``. With ``profile``, a GPU
    timestamp before the first op and after each one (the reference's
    ts(label) after each dispatch, src/vk_engine.py:263-265). Each stamp is
    a small launch of its own, so an op's time includes one launch gap."""
    if not profile:
        return record(lambda: [run(op) for op in seq])
    ts = ops.Timestamps(len(seq) + 1)

    def body():
        ts.record(0)
        for i, op in enumerate(seq):
            run(op)
            ts.record(i + 1)
    g = record(body)
    g.ts, g.labels, g.prof, g.prof_runs = ts, [op_label(op) for op in seq], {}, 0
    return g


def read_profile(g: ops.Graph) -> None:
    """After a submit of a profiled graph: add each op's time (us) to its
    label's total (src/vk_engine.py:321-327)."""
    ts = getattr(g, "ts", None)
    if ts is None:
        return
    ms = ts.read_ms()
    for i, lab in enumerate(g.labels):
        g.prof[lab] = g.prof.get(lab, 0.0) + 1e3 * (ms[i + 1] - ms[i])
    g.prof_runs += 1


def profile_report(g: ops.Graph) -> dict:
    """Per-label GPU time per submit (us), largest first, and their TOTAL
    (src/vk_engine.py:329-335)."""
    n = max(1, getattr(g, "prof_runs", 0))
    rep = {k: v / n for k, v in sorted(getattr(g, "prof", {}).items(), key=lambda kv: -kv[1])}
    rep["TOTAL"] = sum(rep.values())
    return rep


def print_profile(g: ops.Graph, what: str = "token") -> None:
    """The reference's profile printout (src/vk_engine.py:329-335)."""
    if not getattr(g, "prof_runs", 0):
        return
    rep = profile_report(g)
    tot = rep.pop("TOTAL")
    print(f"\n=== GPU profile (per {what}, avg of {g.prof_runs}) ===", flush=True)
    for k, us in rep.items():
        print(f"  {k:24} {us:9.1f} us  {100 * us / tot:5.1f}%", flush=True)
    print(f"  {'TOTAL':24} {tot:9.1f} us", flush=True)


def token_inputs_ds(step: torch.Tensor, emb: Buf, h: Buf, dyn: Buf, tables=(), *, vocab: int, H: int,
                    max_pos: int) -> OpDesc:
    """The host writes of the reference's forward() (src/vk_engine.py:312-314:
    ``B["h"].write(EMB[tid])``, the DYN position words, ``set_rope(pos)``) as
    the first launch of a decode graph (:func:`ops.token_inputs`): ``step``
    is a pinned int32 host tensor of (tid, pos) that :func:`forward` fills
    before each launch; ``emb`` holds the pre-scaled fp32 embedding rows
    [vocab, H] in device memory; ``tables`` = ``[(cos_tab, sin_tab, hd,
    cosb, sinb)]``, per layer type, fp32 RoPE rows [max_pos, hd] (Buf) and
    the row buffers the layers read."""
    tabs = [(_f32v(ct, max_pos * hd), _f32v(st, max_pos * hd), hd, _f32v(co, hd), _f32v(so, hd))
            for ct, st, hd, co, so in tables]
    return OpDesc(ops.token_inputs, (step, _f32v(emb, vocab * H), _f32v(h, H), dyn.view(torch.int32, 4), tabs),
                  dict(vocab=vocab, H=H, max_pos=max_pos))


def forward(g: ops.Graph, step: torch.Tensor, tid: int, pos: int, *, vocab: int, max_pos: int, label: str = "",
            timeout_ms: int | None = None) -> None:
    """One decode token (src/vk_engine.py:312-319) through a graph recorded
    with a :func:`token_inputs_ds` head: (tid, pos) into the pinned step
    buffer (no device synchronization), one graph launch, one bounded wait.
    The logits are in the graph's lm_head output buffer afterwards."""
    if not (0 <= tid < vocab and 0 <= pos < max_pos):
        raise ValueError(f"token {tid} or position {pos} out of range (vocab {vocab}, max_pos {max_pos})")
    step[0] = tid
    step[1] = pos
    submit(g, label or f"decode pos={pos}", timeout_ms)


def record_decode(layers, d_fin: OpDesc, d_lm: GemvDesc, fuse: bool = True, fuse_gemv: bool = True,
                  d_tok: OpDesc | None = None, profile: bool | None = None) -> ops.Graph:
    """Record one decode token in the reference's dispatch order
    (src/vk_engine.py:274-287): per layer norm, q/k/v (one batched launch),
    prepkv, attention, o, normadd, norm, gate/up (one launch), gelumul,
    down, normadd (layer scale); then the final norm and lm_head. ``layers``
    holds the reference's per-layer descriptor keys (``d_in``, ``d_q``,
    ``d_k``, ``d_v`` (may be None), ``d_prep``, ``d_attn``, ``d_o``, ``d_na``,
    ``d_pfn``, ``d_g``, ``d_u``, ``d_gm``, ``d_d``, ``d_nas``); a layer with a
    ``d_gu`` descriptor (:func:`gate_up_ds`) runs it in place of ``d_g``,
    ``d_u`` and ``d_gm``.

    With ``fuse`` (default), every normadd that is followed by an rmsnorm of
    the same residual vector (the post-attention normadd and the MLP norm;
    a layer's last normadd and the next layer's input norm or the final
    norm) runs as one :func:`ops.normadd_rmsnorm` launch, and prepkv with
    the attention after it as :func:`ops.prepkv_attn`: three launches fewer
    per layer, same arithmetic. With ``fuse_gemv`` too, each such fused
    norm with an fp16 output runs inside the GEMV launch that reads it
    (q/k/v, gate/up; :func:`ops.gemv_batch_normadd`, :func:`ops.gemv_normadd`),
    two launches fewer per layer. ``d_tok`` (:func:`token_inputs_ds`), when
    given, is the graph's first launch: the token's embedding row, position
    and RoPE rows come from the step buffer that :func:`forward` writes.
    With ``profile`` (default: ``PROFILE=1``) a GPU timestamp follows every
    launch; :func:`submit` then adds each op's time to its label
    (:func:`profile_report`, :func:`print_profile`)."""
    seq = [d_tok] if d_tok is not None else []
    for L in layers:
        seq += [L["d_in"], ("gemvs", [L["d_q"], L["d_k"]] + ([L["d_v"]] if L.get("d_v") is not None else [])),
                L["d_prep"], L["d_attn"], ("gemvs", [L["d_o"]]), L["d_na"], L["d_pfn"],
                *([L["d_gu"]] if L.get("d_gu") is not None else [("gemvs", [L["d_g"], L["d_u"]]), L["d_gm"]]),
                ("gemvs", [L["d_d"]]), L["d_nas"]]
    seq += [d_fin, ("gemvs", [d_lm])]
    if fuse:
        seq = _fuse_norms(seq)
        if fuse_gemv:
            seq = _fuse_norm_gemvs(seq)

    def run(op):
        if isinstance(op, tuple) and op and op[0] == "gemvs":
            gemv_many(op[1])
        elif isinstance(op, tuple) and op and op[0] == "gemvs_nx":
            a, w, h, h_out, w2, sc = op[1]
            d0 = op[2][0].dp
            ops.gemv_batch_normadd(a, w, h, h_out, w2, [(d.dp[1], d.dp[2], d.dp[6], d.dp[5], d.dp[4])
                                                        for d in op[2]], d0[7], scale=sc, scale_fmt=d0[3])
        else:
            disp(op)

    g = _record_seq(seq, run, PROFILE if profile is None else profile)
    g.seq = seq          # the recorded descriptor sequence, for inspection
    return g


# GEMVs this tall keep their own norm launch: every workgroup of a fused
# launch forms the whole x, which a grid of thousands of workgroups (lm_head)
# would repeat thousands of times.
_NX_MAX_ROWS = 65536


def _copy_into(dst: torch.Tensor, src: torch.Tensor) -> None:
    dst.copy_(src)


def _aligned(*ts) -> bool:
    return all(t.data_ptr() % 16 == 0 for t in ts)


def _fuse_norm_gemvs(seq):
    """A :func:`ops.normadd_rmsnorm` with an fp16 output and the GEMV launch
    after it that reads that output (a ``("gemvs", descs)`` group or a gated
    gate/up descriptor) become one launch. The norm output is read by that
    launch only (src/vk_engine.py:231-234, 243-244: the norm buffer is
    rewritten before its next use). The fused launch writes the new residual
    to a second buffer (other workgroups still read the old one), so the
    residual alternates between its buffer and a twin; later descriptors
    that use the residual are pointed at the buffer that holds it, and a
    copy at the end puts it back where the reference keeps it."""
    out, cur, home = [], {}, {}
    twin: dict = {}

    def sub(t):
        return cur.get(t.data_ptr(), t) if isinstance(t, torch.Tensor) else t

    i = 0
    while i < len(seq):
        a = seq[i]
        b = seq[i + 1] if i + 1 < len(seq) else None
        fused = None
        if isinstance(a, OpDesc) and a.fn is ops.normadd_rmsnorm:
            x, w, h, w2, sc, y = a.args
            D = x.numel()
            h_in = sub(h)
            ok = (y.dtype == torch.float16 and D <= ops.GEMV_NORMADD_MAX_K and _aligned(x, w, h, w2)
                  and y.data_ptr() not in cur)
            if ok and isinstance(b, tuple) and b and b[0] == "gemvs":
                ds = b[1]
                d0 = ds[0].dp
                if (len(ds) <= ops.GEMV_MAX_BATCH and sum(d.dp[6] for d in ds) <= _NX_MAX_ROWS
                        and all(d.dp[0].data_ptr() == y.data_ptr() and d.dp[0].dtype == torch.float16
                                and d.dp[7] == D and d.dp[3] == d0[3] and d.dp[5].dtype == d0[5].dtype for d in ds)):
                    fused = lambda h_out: ("gemvs_nx", (x, w, h_in, h_out, w2, sc), ds)  # noqa: E731
            elif (ok and isinstance(b, OpDesc) and b.fn is ops.gemv_gated and b.args[0].data_ptr() == y.data_ptr()
                  and b.args[4] == D and b.args[3] <= _NX_MAX_ROWS):
                _x, wo, so, N, K = b.args
                kw = b.kw
                fused = lambda h_out: OpDesc(ops.gemv_normadd, (x, w, h_in, h_out, w2, wo, so, N, K),  # noqa: E731
                                             dict(scale=sc, scale_fmt=kw["scale_fmt"], inv=kw["inv"], y=kw["act"],
                                                  gated=True))
            if fused is not None:
                key = h.data_ptr()
                home.setdefault(key, h)
                if key not in twin:
                    twin[key] = torch.empty_like(h)
                    KEEP.append(twin[key])
                h_out = twin[key] if h_in.data_ptr() == key else home[key]
                out.append(fused(h_out))
                cur[key] = h_out
                if h_out.data_ptr() == key:
                    del cur[key]
                i += 2
                continue
        if isinstance(a, OpDesc):
            a = OpDesc(a.fn, tuple(sub(t) for t in a.args), {k: sub(v) for k, v in a.kw.items()})
        out.append(a)
        i += 1
    for key, t in cur.items():
        out.append(OpDesc(_copy_into, (home[key], t), {}))
    return out


def _fuse_norms(seq):
    """Pairs of adjacent descriptors that run as one launch: a normadd and
    the rmsnorm of the same residual vector after it; a prepkv and the
    attention that reads the same caches and position after it."""
    out, i = [], 0
    while i < len(seq):
        a = seq[i]
        b = seq[i + 1] if i + 1 < len(seq) else None
        if (isinstance(a, OpDesc) and isinstance(b, OpDesc) and a.fn is ops.normadd and b.fn is ops.rmsnorm
                and a.args[2].data_ptr() == b.args[0].data_ptr() and a.args[2].numel() == b.args[0].numel()):
            x, w, h, sc = a.args
            _, w2, y = b.args
            out.append(OpDesc(ops.normadd_rmsnorm, (x, w, h, w2, sc, y), {}))
            i += 2
        elif (isinstance(a, OpDesc) and isinstance(b, OpDesc) and a.fn is ops.prepkv and b.fn is ops.attn
              and a.args[0].data_ptr() == b.args[0].data_ptr() and a.args[4].data_ptr() == b.args[4].data_ptr()
              and a.args[5].data_ptr() == b.args[5].data_ptr() and a.kw["dyn"].data_ptr() == b.kw["dyn"].data_ptr()
              and a.kw["hd"] == b.kw["hd"] and a.kw["nkv"] == b.kw["nkv"] and a.kw["stride"] == b.kw["stride"]
              and a.kw["window"] == b.kw["window"] and a.args[2].data_ptr() == b.args[2].data_ptr()
              and a.args[3].data_ptr() == b.args[3].data_ptr()):
            qkv, knw, cosb, sinb, kc, vc = a.args
            _, qnw, _, _, _, _, outt = b.args
            kw = dict(b.kw, koff=a.kw["koff"], voff=a.kw["voff"], keqv=a.kw["keqv"], out_dtype=outt.dtype)
            out.append(OpDesc(ops.prepkv_attn, (qkv, knw, qnw, cosb, sinb, kc, vc, outt), kw))
            i += 2
        else:
            out.append(a)
            i += 1
    return out


def wait(stream=None, label: str = "", timeout_ms: int | None = None) -> None:
    """Bounded wait (src/vk_engine.py:293-302); infinite when the bound is 0."""
    ops.stream_wait(stream, _FENCE_MS if timeout_ms is None else timeout_ms, label)


def submit(g: ops.Graph, label: str = "", timeout_ms: int | None = None) -> None:
    """Replay a recorded graph and wait for it (src/vk_engine.py:312-319);
    a profiled graph's op times are added to its labels (:func:`read_profile`)."""
    g.launch()
    wait(g.stream, label, timeout_ms)
    read_profile(g)
